"""The C-ABI library loads and exports every entry point the header declares.

Runs without a GPU: only argument rejections (which return before any HIP
call) are exercised.
"""

import ctypes
import re
from pathlib import Path

import pytest

from qwenforge_amd import _lib

INCLUDE = Path(__file__).resolve().parents[1] / "include"
HEADERS = sorted(INCLUDE.glob("*.h"))


def _declared():
    names = set()
    for header in HEADERS:
        text = header.read_text()
        names.update(re.findall(r"^\s*(?:const\s+char\*|int|int64_t)\s+(qf_\w+)\s*\(", text, re.M))
    return sorted(names)


def test_header_declares_the_three_kernels():
    names = _declared()
    for n in ("qf_decode_attn", "qf_prefill_attn", "qf_rope_append", "qf_error_string",
              "qf_abi_version", "qf_rms_qkv_rope_append", "qf_gemv_residual",
              "qf_rms_gate_up_swiglu", "qf_rms_lm_head", "qf_argmax_step"):
        assert n in names


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in _declared():
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"


def test_version_and_error_strings():
    lib = _lib.load()
    assert lib.qf_abi_version() == 301
    assert lib.qf_error_string(0) == b"success"
    assert b"invalid" in lib.qf_error_string(-1)
    assert b"unsupported" in lib.qf_error_string(-2)


def _decode_call(lib, **over):
    args = dict(q=16, k=16, v=16, acc=16, m=16, l=16, out=16, splits=1, B=1, KVH=2, G=7, D=64, cap=8)
    args.update(over)
    a = args
    return lib.qf_decode_attn(a["q"], 0, 0, 0, a["k"], 0, 0, 0, a["v"], 0, 0, 0, None, 0, None, 0,
                              a["acc"], a["m"], a["l"], a["splits"], None, a["out"], 0, 0, 0,
                              a["B"], a["KVH"], a["G"], a["D"], a["cap"], 0.125, None)


def test_decode_rejects_bad_arguments_without_launching():
    lib = _lib.load()
    assert _decode_call(lib, D=128) == -2
    assert _decode_call(lib, G=17) == -2
    assert _decode_call(lib, G=0) == -2
    assert _decode_call(lib, q=None) == -1
    assert _decode_call(lib, splits=0) == -1
    assert _decode_call(lib, cap=0) == -1
    assert _decode_call(lib, q=18) == -1  # misaligned pointer


def test_decode_launch_plan_names_the_kernel():
    from qwenforge_amd import ops

    # Config 2 (B=4, cap 2048, 16 splits, single-launch merge, vector bias).
    assert ops.decode_kernel_name(4, 2, 7, 2048, 16, True) == "qf::decode_split_kernel<8, 1, 2, false>"
    # One workgroup per kv head streams everything with 16 waves.
    assert _lib.load().qf_decode_waves(1, 2, 7, 512, 1, 0) == 16
    assert _lib.load().qf_decode_waves(1, 2, 0, 512, 1, 0) == -1


@pytest.mark.parametrize("b,cap,splits,fused,waves", [
    (1, 512, 16, 1, 8),      # config 1: the single-launch merge gives each of 7 queries a wave
    (4, 2048, 16, 1, 8),     # config 2: same, although each split has only 4 tiles
    (1, 32768, 128, 0, 4),   # config 3: 256 workgroups, 8 tiles each -> two tiles per wave
    (4, 4096, 32, 0, 4),     # 256 workgroups, 4 tiles each -> four waves
    (1, 256, 1, 0, 8),       # one split over 2 workgroups: one tile per wave
    (12, 256, 1, 0, 4),      # one split over 24 workgroups: at least two tiles per wave
    (16, 32768, 8, 1, 8),    # bandwidth regime, one workgroup per CU
    (64, 4096, 2, 1, 8),
    (12, 5760, 10, 1, 8),    # the reference's benchmark shape
])
def test_decode_waves_at_benchmark_shapes(b, cap, splits, fused, waves):
    """Waves per decode workgroup as the library launches them (host code, no GPU)."""
    assert _lib.load().qf_decode_waves(b, 2, 7, cap, splits, fused) == waves


def test_stream_read_rejects_bad_arguments():
    lib = _lib.load()
    assert lib.qf_stream_read(None, 1024, 16, 4, None) == -1
    assert lib.qf_stream_read(16, 1000, 16, 4, None) == -1   # not a multiple of 16 bytes
    assert lib.qf_stream_read(8, 1024, 16, 4, None) == -1    # misaligned source
    assert lib.qf_stream_read(16, 1024, 16, 0, None) == -1


def test_launch_probe_rejects_bad_arguments():
    lib = _lib.load()
    assert lib.qf_launch_probe(16, 1024, 16, 16, 4, 100, 1, None) == -1   # threads not x64
    assert lib.qf_launch_probe(16, 1024, 16, 16, 4, 2048, 1, None) == -1  # > 1024 threads
    assert lib.qf_launch_probe(16, 1024, 16, 16, 0, 256, 1, None) == -1   # no workgroups
    assert lib.qf_launch_probe(16, 1024, 16, 16, 4, 256, 3, None) == -1   # round trips > 2
    assert lib.qf_launch_probe(None, 1024, 16, 16, 4, 256, 1, None) == -1  # no source
    assert lib.qf_launch_probe(16, 1000, 16, 16, 4, 256, 1, None) == -1   # bytes not x16
    assert lib.qf_launch_probe(16, 1024, None, 16, 4, 256, 2, None) == -1  # no index


def test_noalloc_decode_rejects_before_any_hip_call():
    """Shape, size and pointer checks of qf_decode_attn_noalloc return before the
    library touches the device (no GPU here)."""
    lib = _lib.load()

    def call(splits=8, B=1, KVH=2, G=7, D=64, cap=64, q=16):
        return lib.qf_decode_attn_noalloc(q, 0, 0, 0, 16, 0, 0, 0, 16, 0, 0, 0, None, 0, None, 0,
                                          splits, 16, 0, 0, 0, B, KVH, G, D, cap, 0.125, None)

    assert call(D=128) == -2
    assert call(G=17) == -2
    assert call(splits=0) == -1
    # 64 x 2 x 64 x 7 partial rows of 66 floats = 15 MB > QF_NOALLOC_PARTIAL_BYTES (4 MiB).
    assert call(B=64, splits=64) == -3
    assert call(q=None) == -1
    assert b"no-allocation scratch" in lib.qf_error_string(-3)


def test_prefill_and_append_reject_bad_arguments():
    lib = _lib.load()
    rc = lib.qf_prefill_attn(16, 0, 0, 0, 16, 0, 0, 0, 16, 0, 0, 0, None, None, 0, 0,
                             None, 0, 0, 0, None, 0, 0, 0, 0, 0, 16, 0, 0, 0,
                             1, 14, 2, 8, 32, 0.125, None)
    assert rc == -2
    rc = lib.qf_prefill_attn(16, 0, 0, 0, 16, 0, 0, 0, 16, 0, 0, 0, 16, None, 0, 0,
                             None, 0, 0, 0, None, 0, 0, 0, 0, 0, 16, 0, 0, 0,
                             1, 14, 2, 8, 64, 0.125, None)
    assert rc == -1  # cos without sin
    rc = lib.qf_prefill_attn(16, 0, 0, 0, 16, 0, 0, 0, 16, 0, 0, 0, None, None, 0, 0,
                             16, 0, 0, 0, 16, 0, 0, 0, 5, 8, 16, 0, 0, 0,
                             1, 14, 2, 8, 64, 0.125, None)
    assert rc == -1  # start_pos + S > cap
    rc = lib.qf_rope_append(16, 0, 0, 16, 0, 0, 16, 0, 0, 16, 16, 0, 16, 0, 0, 0, 16, 0, 0, 0,
                            None, 16, 0, 0, 1, 14, 2, 64, 8, None)
    assert rc == -1  # no write_index


def test_ops_refuse_cpu_tensors():
    torch = pytest.importorskip("torch")
    from qwenforge_amd import ops

    q = torch.zeros(1, 2, 7, 64, dtype=torch.float16)
    k = torch.zeros(1, 2, 16, 64, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="no CPU path"):
        ops.decode_attention(q, k, k)
    with pytest.raises(RuntimeError, match="no CPU path"):
        torch.ops.student_qwen.gqa_flash_prefill(torch.zeros(1, 14, 8, 64, dtype=torch.float16),
                                                 torch.zeros(1, 2, 8, 64, dtype=torch.float16),
                                                 torch.zeros(1, 2, 8, 64, dtype=torch.float16))


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "absent.so")
    with pytest.raises(RuntimeError, match="missing"):
        _lib.load()
    assert ctypes  # keeps the import used


def test_step_kernels_reject_bad_arguments():
    lib = _lib.load()
    # B outside 1..4 and hidden > 1024 are unsupported; null pointers invalid.
    assert lib.qf_gemv_residual(16, 896, 16, 16, 896, 5, 896, 896, None) == -2
    assert lib.qf_gemv_residual(16, 896, 16, 16, 896, 1, 8200, 896, None) == -2
    assert lib.qf_gemv_residual(None, 896, 16, 16, 896, 1, 896, 896, None) == -1
    assert lib.qf_gemv_residual(18, 896, 16, 16, 896, 1, 896, 896, None) == -1  # misaligned
    assert lib.qf_rms_gate_up_swiglu(16, 896, 16, 1e-6, 16, 0, 16, 4864, 1, 2048, 4864, None) == -2
    assert lib.qf_rms_gate_up_swiglu(16, 896, None, 1e-6, 16, 0, 16, 4864, 1, 896, 4864, None) == -1
    assert lib.qf_rms_gate_up_swiglu(16, 896, 16, 1e-6, 16, 7, 16, 4864, 1, 896, 4864, None) == -1
    # tiles need hidden % 32 == 0 and I % 8 == 0
    assert lib.qf_rms_gate_up_swiglu(16, 888, 16, 1e-6, 16, 1, 16, 4864, 1, 888, 4864, None) == -2
    assert lib.qf_rms_gate_up_swiglu(16, 896, 16, 1e-6, 16, 1, 16, 4860, 1, 896, 4860, None) == -2
    assert lib.qf_rms_lm_head(16, 896, 16, 1e-6, 16, 0, 16, 100, 16, 0, 1, 896, 100, None) == -1
    assert lib.qf_rms_lm_head(16, 896, 16, 1e-6, 16, 0, 16, 100, 16, 8, 0, 896, 100, None) == -2
    assert lib.qf_rms_lm_head(16, 896, 16, 1e-6, 16, 3, 16, 100, 16, 8, 1, 896, 100, None) == -1
    # tiles need whole 16-row blocks and 8-byte logit stores
    assert lib.qf_rms_lm_head(16, 896, 16, 1e-6, 16, 1, 16, 104, 16, 8, 2, 896, 100, None) == -2
    assert lib.qf_rms_lm_head(16, 896, 16, 1e-6, 16, 1, 18, 112, 16, 8, 2, 896, 112, None) == -1
    assert lib.qf_argmax_step(16, 8, 1, 16, 16, 4, 4, None, None, None, None) == -1  # rows w/o step
    assert lib.qf_argmax_step(16, 8, 9, 16, None, 0, 0, None, None, None, None) == -2
    def qkv(cos=16, sin=16, pos=None, inv=None, kc=16, D=64, lay=0):
        return lib.qf_rms_qkv_rope_append(16, 896, None, None, 0, 16, 1e-6, 16, lay, None, cos, sin, 64,
                                          pos, inv, kc, 0, 0, 0, 16, 0, 0, 0, 16, 16, 0, 0,
                                          1, 896, 14, 2, D, 64, None)

    assert qkv(D=128) == -2                      # head_dim 128
    assert qkv(kc=None) == -1                    # no key cache
    assert qkv(pos=16, inv=16) == -1             # tables and positions together
    assert qkv(cos=None, sin=None) == -1         # neither RoPE source
    assert qkv(cos=None, sin=None, pos=16) == -1  # positions without inv_freq
    assert qkv(lay=2) == -1                      # unknown weight layout


def test_prefill_varlen_rejects_bad_arguments():
    lib = _lib.load()

    def call(cu=16, total=8, max_seqlen=8, cos=None, sin=None, kc=None, vc=None, cap=0):
        return lib.qf_prefill_varlen(16, 64, 896, 16, 64, 128, 16, 64, 128, cu, total, max_seqlen,
                                     cos, sin, 64, kc, 0, 0, 0, vc, 0, 0, 0, 0, cap,
                                     16, 64, 896, 2, 14, 2, 64, 0.125, None)

    assert call(cu=None) == -1                      # no row offsets
    assert call(total=0) == -1
    assert call(cos=16, sin=16) == -2               # RoPE needs the caches
    assert call(kc=16, vc=16, cap=4) == -1          # max_seqlen exceeds capacity


def test_paged_entry_points_reject_bad_arguments():
    lib = _lib.load()

    def decode(page=64, ppr=4, n_pages=8, table=16, bt_sb=4, kp_sp=2 * 64 * 64, out=16):
        return lib.qf_decode_attn_paged(16, 0, 0, 0, 16, kp_sp, 64 * 64, 64, 16, 2 * 64 * 64,
                                        64 * 64, 64, table, bt_sb, ppr, n_pages, page,
                                        None, 0, None, 0, 16, 16, 16, 1, None, out, 0, 0, 0,
                                        1, 2, 7, 64, 0.125, None)

    assert decode(page=32) == -2          # below the 64-slot minimum
    assert decode(page=96) == -2          # not a power of two
    assert decode(page=8192) == -2        # above the maximum
    assert decode(ppr=0) == -2
    assert decode(n_pages=0) == -2
    assert decode(table=None) == -1
    assert decode(bt_sb=2) == -1          # table rows overlap
    assert decode(kp_sp=2 * 64 * 64 + 4) == -1  # page stride breaks 16-byte rows
    assert decode(out=None) == -1

    def append(page=64, slots=16, table=16):
        return lib.qf_rope_append_paged(16, 0, 0, 16, 0, 0, 16, 0, 0, 16, 16, 0,
                                        16, 8192, 4096, 64, 16, 8192, 4096, 64,
                                        table, 4, 4, 8, page, slots, 1, 16, 0, 0,
                                        1, 14, 2, 64, None)

    assert append(page=48) == -2
    assert append(slots=None) == -1
    assert append(table=None) == -1

    def prefill(start=0, max_seqlen=8, ppr=4, table=16):
        return lib.qf_prefill_varlen_paged(16, 64, 896, 16, 64, 128, 16, 64, 128, 16, 8,
                                           max_seqlen, None, None, 0,
                                           16, 8192, 4096, 64, 16, 8192, 4096, 64,
                                           table, 4, ppr, 8, 64, start,
                                           16, 64, 896, 2, 14, 2, 64, 0.125, None)

    assert prefill(start=32) == -1        # start must be tile-aligned
    assert prefill(table=None) == -1
    assert prefill(start=256, max_seqlen=8) == -1  # past the row's 256 slots

    def qkv(page=64, slots=16, B=1):
        return lib.qf_rms_qkv_rope_append_paged(16, 896, None, None, 0, 16, 1e-6, 16, 0, None,
                                                16, 16, 64, None, None, 16, 8192, 4096, 64,
                                                16, 8192, 4096, 64, 16, 4, 4, 8, page,
                                                slots, 1, 16, 896, 64, B, 896, 14, 2, 64, None)

    assert qkv(page=100) == -2
    assert qkv(B=5) == -2
    assert qkv(slots=None) == -1


def test_pack_weight_rejects_bad_arguments():
    lib = _lib.load()
    assert lib.qf_pack_weight(16, 896, 16, 1152, 896, 3, None) == -1     # unknown row map
    assert lib.qf_pack_weight(16, 896, 16, 1150, 896, 0, None) == -2     # N % 16
    assert lib.qf_pack_weight(16, 888, 16, 1152, 888, 0, None) == -2     # K % 32
    assert lib.qf_pack_weight(16, 896, 16, 1136, 896, 2, None) == -2     # ROPE needs N % 64
    assert lib.qf_pack_weight(None, 896, 16, 1152, 896, 0, None) == -1
    assert lib.qf_pack_weight(16, 800, 16, 1152, 896, 0, None) == -1     # row stride < K
    assert lib.qf_pack_weight(18, 896, 16, 1152, 896, 0, None) == -1     # misaligned
