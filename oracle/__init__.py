"""CPU oracle for the QwenForge attention hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in ``qwenforge_amd`` imports this package;
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may use it, and only as the checker (or the timed CPU baseline),
never as the measured or shipped path.

Each function restates, in plain torch-on-CPU (fp32 or fp64) or numpy code, the
reference behaviour it cites (``student_engine.py`` = ``SE``).  The pins that
make the restatement trustworthy live in ``tests/test_oracle_*.py``:

* ``eager_attention`` / ``grouped_decode_attention`` / ``causal_prefill``:
  checked against ``torch.nn.functional.scaled_dot_product_attention`` (a
  library routine), against fp64 brute-force loops, and against the
  reference's whiteboard known-answer logits (causal attention + split-half
  RoPE).
* ``grouped_decode_attention_fp16`` and ``eager_attention_fp16`` (the
  reference's fp16 forms, timed as CPU baselines only): within fp16 rounding
  of fp64 SDPA, exact on uniform V (and, causal, on the first query row,
  which sees only key 0), fp16 output.
* ``split_partials`` / ``combine_partials``: invariants (independence of the
  split count, S=1 equals the unsplit path, empty and fully masked splits,
  single valid key, uniform V, key permutation).
* ``apply_rope_fp16``: torch-CPU half arithmetic and numpy float16
  arithmetic (two independent correctly-rounded implementations), position-0
  identity, fp64 norm preservation, and the whiteboard split-half KAT.
* ``rope_cos_sin``: fp64 closed form at positions up to 131071 (rotate-half
  layout, theta, the fp32 angle), and through the whiteboard KAT and the
  model pin below, which both build their RoPE from it.
* ``model.prefill`` / ``model.decode_step``: ``transformers.Qwen2ForCausalLM``
  on a tiny random config, live and through committed logits.
* ``append_*`` / ``capacity`` / ``decode_slots``: brute-force loops.
* ``pages_to_dense`` / ``dense_to_pages`` / ``paged_location``: the identity
  block table reduces to a reshape of the dense cache (closed form), and the
  two are inverse on random tables.

No function is "parity unpinned".
"""

from .attention import (  # noqa: F401
    FP16_MIN,
    causal_prefill,
    combine_partials,
    eager_attention,
    eager_attention_fp16,
    flash_decode,
    grouped_decode_attention,
    grouped_decode_attention_fp16,
    split_partials,
)
from .rope import (  # noqa: F401
    apply_rope_fp16,
    inv_freq,
    rope_cos_sin,
    rotate_half,
)
from .kv import (  # noqa: F401
    append_decode,
    append_prefill,
    append_rows,
    capacity,
    dense_to_pages,
    pages_to_dense,
    paged_location,
    decode_bias,
    decode_slots,
)
