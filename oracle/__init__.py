"""CPU oracle for the mini-sglang-mlx attention hot path.

TEST INFRASTRUCTURE ONLY. This package checks results and is never the product:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it. The HIP backend under ``mini-sglang-mlx_amd/`` never
imports it and has no CPU fallback.

It restates, in numpy, the reference's algorithm for the attention path
(paths relative to the reference's ``python/minisgl_mlx/``):

- index work (bit-exact, int32): ``scheduler/scheduler.py:154-157``,
  ``scheduler/cache.py:53-72,138-143``, ``attention/naive.py:36-48``,
  ``attention/metal.py:145-152``, ``attention/base.py:70-83``;
- KV store (bit-exact copy): ``kvcache/pool.py:47-50``;
- attention (fp64 accumulation): ``attention/naive.py:50-60`` (decode),
  ``attention/base.py:85-105`` (prefill, bottom-right causal);
- rotary embedding and the rotate-then-store order: ``layers.py:19-74, 107-109``
  (``rope.py``);
- an fp8 (e4m3) KV cache with one scale per token and kv head, the extension
  docs/09-exercises.md:81-82 describes (``kv_quant.py``).

Every function is pinned by a check in ``tests/test_oracle.py`` that does not
retype its formula: closed forms (one key gives that key's value row, equal
keys give the mean of the values), brute-force Python loops on tiny inputs,
an independent library routine (``torch.nn.functional.scaled_dot_product_attention``
on the CPU), the rotary embedding of ``transformers`` (``apply_rotary_pos_emb`` and its
llama3 / linear frequency initialisers), torch's ``float8_e4m3fn`` casts, the reference test's fixture construction
(``tests/test_attention.py:19-39``) and the page-layout assertion of
``tests/test_cache_manager.py:66-75``, plus mutation tests that plant a
mistake in a copy of the oracle and show the checks catch it.
"""

from .attention import (  # noqa: F401
    align_up,
    allocate_paged,
    csr_decode_metadata,
    div_ceil,
    expand_page_indices,
    forward_prefill,
    naive_decode_metadata,
    naive_forward_decode,
    page_to_token,
    paged_decode,
    prefill_metadata,
    prepare_batch_indices,
    sdpa,
    store_kv,
)
from .rope import (  # noqa: F401
    rope,
    rope_angles,
    rope_inv_freq,
    rope_periods,
    rope_position_scale,
    rope_store_kv,
)
from .kv_quant import (  # noqa: F401
    E4M3_MAX,
    dequantize_fp8,
    e4m3_decode,
    e4m3_encode,
    quantize_fp8,
    store_kv_fp8,
)
