"""CPU oracle for the InfLLM-v2 selection path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference algorithm of each op on the
path (Yanguan619/unum_ops):

* ``get_block_table``        -- numpy restatement of
  ``src/unum_ops/sparse_kernel_extension/get_table_torch.py:4-44``.
* ``max_pooling_1d_varlen``  -- numpy restatement of the Triton kernel
  ``src/unum_ops/infllm_v2/max_pooling_1d_varlen.py:33-183`` (the reference
  ships no torch version of this op).
* ``infllmv2_attn_stage1``   -- fp32 torch-CPU restatement of the Triton v2
  kernel ``src/unum_ops/infllm_v2/infllmv2_attn_stage1_triton_v2.py:20-228``
  (the exported ``infllmv2_attn_stage1``).
* ``topk_blocks``            -- the block selection over pooled scores
  (top-k, ids sorted ascending as in ``test/test_sparse_kernel.py:42-43``),
  with the build's tie-break (equal scores by ascending id).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker / the timed CPU
baseline.  The product path (``unum_ops_amd``) never imports it and never falls
back to it.

How each function is pinned (so that a plausible mistake in the restatement
fails a check that does not retype the same formula):

* block table: a pure-Python scalar brute force on tiny inputs, hand-computed
  known answers, and closed forms (parity of entries with the head index,
  zeros for negative ids and past the limits, the clamp to ``L-1``).
* max-pool: reduction to ``torch.nn.functional.max_pool1d(k=5, s=4, p=1)`` on
  rows gathered through the flat-stride view and masked to ``-inf`` past the
  key length, plus a scalar brute force and hand-computed known answers.
* stage 1: reduction to ``torch.nn.functional.scaled_dot_product_attention``
  with an identity value matrix (which returns the probability matrix), the
  uniform-softmax closed form ``G / vis`` that pins the causal visible count,
  a hand-derived table of visible counts (truncating division), and row-sum
  invariants.
* top-k: a Python ``sorted`` brute force over (score, id) pairs, and
  ``torch.topk`` (a library routine) on rows with distinct scores.

All three functions are pinned; none is "parity unpinned".
"""

from .block_table import get_block_table
from .maxpool import max_pooling_1d_varlen
from .stage1 import infllmv2_attn_stage1, visible_counts, tdiv
from .topk import topk_blocks

__all__ = [
    "get_block_table",
    "max_pooling_1d_varlen",
    "infllmv2_attn_stage1",
    "visible_counts",
    "tdiv",
    "topk_blocks",
]
