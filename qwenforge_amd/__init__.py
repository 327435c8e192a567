"""MI355X-native (gfx950) attention hot path of the QwenForge engine.

Hand-written HIP kernels behind a C ABI (``include/qf_attn.h``), reached from
Python with ctypes.  See ``qwenforge_amd.ops`` for the drop-in functions.
"""

from . import ops  # noqa: F401  (registers the student_qwen:: custom ops)
from .ops import (  # noqa: F401
    choose_splits,
    decode_attention,
    decode_plan,
    flash_decode_attention,
    gqa_flash_prefill,
    gqa_flash_prefill_rope_append,
    make_flash_scratch,
    rope_append,
)

__version__ = "0.1.0"
