// Shared helpers for the gfx950 kernels and their C-ABI launchers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <cstdarg>
#include <cstdio>

#include "../../include/unum_ops_amd.h"

namespace unum {

// Thread-local message of the last failing C-ABI call (capi.hip owns it).
void set_error(const char* fmt, ...);
void clear_error();

// Validation helper: record the message and return `code`.
#define UNUM_FAIL(code, ...)          \
  do {                                \
    ::unum::set_error(__VA_ARGS__);   \
    return (code);                    \
  } while (0)

#define UNUM_REQUIRE(cond, ...)                                        \
  do {                                                                 \
    if (!(cond)) UNUM_FAIL(UNUM_ERR_INVALID_ARGUMENT, __VA_ARGS__);    \
  } while (0)

// Check the launch that was just enqueued.
inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return UNUM_ERR_LAUNCH;
  }
  return UNUM_OK;
}

constexpr int kWave = 64;  // CDNA wavefront width

// Lane i takes v from lane i-1 and lane 0 takes `fill`: a DPP wave_shr:1
// move (one VALU instruction, no LDS round trip as for a shuffle).
__device__ __forceinline__ float wave_shr1(float v, float fill) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(fill), __float_as_int(v), 0x138,
                                                    0xF, 0xF, false));
}

// The device the launch runs on, for the entry points whose plan depends
// on it (CU count, per-device scratch): the current device, which `stream`
// must belong to (the null stream is the current device's).  Sets *dev and
// returns UNUM_OK, or returns UNUM_ERR_INVALID_ARGUMENT (the stream is
// another device's) / UNUM_ERR_LAUNCH (no usable device) with the error set.
inline int launch_device(void* stream, const char* op, int* dev) {
  int cur = -1;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess || cur < 0)
    UNUM_FAIL(UNUM_ERR_LAUNCH, "%s: no usable current device (%s)", op, hipGetErrorString(e));
  if (stream != nullptr) {
    int sdev = -1;
    e = hipStreamGetDevice(static_cast<hipStream_t>(stream), &sdev);
    if (e != hipSuccess)
      UNUM_FAIL(UNUM_ERR_LAUNCH, "%s: hipStreamGetDevice failed: %s", op, hipGetErrorString(e));
    if (sdev != cur)
      UNUM_FAIL(UNUM_ERR_INVALID_ARGUMENT,
                "%s: the stream belongs to device %d, the current device is %d (make the "
                "stream's device current)", op, sdev, cur);
  }
  *dev = cur;
  return UNUM_OK;
}

// Compute units of device `dev` (cached per device; 256 if the query fails).
// The cache is read and written by any host thread that launches: relaxed
// atomics make that race-free (every writer stores the same value).
inline int num_cus(int dev) {
  static std::atomic<int> cached[64];
  if (dev < 0 || dev >= 64) return 256;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Compute units of the current device.
inline int num_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  return num_cus(dev);
}

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Round-to-nearest-even fp32 -> bf16 (NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) {
  _Float16 h;
  __builtin_memcpy(&h, &b, 2);
  return static_cast<float>(h);
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  _Float16 h = static_cast<_Float16>(f);
  uint16_t b;
  __builtin_memcpy(&b, &h, 2);
  return b;
}

}  // namespace unum
