"""unum_ops_amd: the InfLLM-v2 sparse-attention selection path on MI355X (gfx950).

A from-scratch, MI355X-native replacement for the selection path of
``Yanguan619/unum_ops``:

* ``unum_ops_amd.infllm_v2.infllmv2_attn_stage1``       (bf16 MFMA stage-1 scores)
* ``unum_ops_amd.infllm_v2.max_pooling_1d_varlen``      (HBM-bound varlen max-pool)
* ``unum_ops_amd.sparse_kernel_extension.get_block_table`` (integer slot gather)
* ``unum_ops_amd.pipeline.select_blocks``               (stage1 -> pool -> top-k -> table)
* ``unum_ops_amd.pipeline.maxpool_topk``                (fused pool + block top-k)
* ``unum_ops_amd.compression.compress_keys``            (raw keys -> compressed keys)
* ``unum_ops_amd.sparse_attention.sparse_paged_attention`` (stage 2 over the block table)

Each op keeps the reference's names, argument lists and output layouts and
runs hand-written HIP kernels through the C ABI in ``include/unum_ops_amd.h``.
"""

import torch  # noqa: F401  -- load torch's HIP runtime before the native library

from . import (compression, infllm_v2, pipeline, sparse_attention,  # noqa: E402
               sparse_kernel_extension)

__version__ = "0.1.0"

__all__ = ["compression", "infllm_v2", "pipeline", "sparse_attention", "sparse_kernel_extension",
           "__version__"]
