"""The no-allocation decode entry point (qf_decode_attn_noalloc) through the C ABI.

Its output must equal qf_decode_attn's (same kernels, same split count and
merge; the existing entry point gets torch-allocated scratch) bit for bit, on
two calls in a row where the second is smaller, for the single-launch merge
(2-32 splits), the two-launch merge (> 32 splits) and one split, and on four
calls that change the layout and the merge in turn; and stay within the
2e-3 max-abs-err of the CPU oracle.  A fresh process whose first
no-allocation call is made under graph capture replays the graph against the
existing entry point too.
"""

import os
import subprocess
import sys
import textwrap

import pytest
import torch

import oracle
from qwenforge_amd import _lib, ops, workloads

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _qkv(c, kv_last):
    g, k, v = c.grouped, c.key_cache, c.value_cache
    return (g.data_ptr(), g.stride(0), g.stride(1), g.stride(2),
            k.data_ptr(), k.stride(0), k.stride(1), k.stride(2),
            v.data_ptr(), v.stride(0), v.stride(1), v.stride(2),
            None if c.bias is None else c.bias.data_ptr(),
            0 if c.bias is None else c.bias.stride(0),
            None if kv_last is None else kv_last.data_ptr(),
            0 if kv_last is None or kv_last.numel() == 1 else 1)


def _noalloc(lib, c, splits, kv_last, dev):
    b, kvh, g, d = c.grouped.shape
    out = torch.full((b, kvh, g, d), float("nan"), dtype=torch.float16, device=dev)
    rc = lib.qf_decode_attn_noalloc(*_qkv(c, kv_last), splits,
                                    out.data_ptr(), out.stride(0), out.stride(1), out.stride(2),
                                    b, kvh, g, d, c.key_cache.shape[2], 0.125,
                                    torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "qf_decode_attn_noalloc")
    return out


def _existing(lib, c, splits, kv_last, dev):
    b, kvh, g, d = c.grouped.shape
    cap = c.key_cache.shape[2]
    flash = ops.make_flash_scratch(b, kvh, g, cap, dev, splits=splits,
                                   fused=1 < splits <= 32)
    acc, m, l, out = flash[:4]
    ticket = flash[4] if len(flash) > 4 else None
    rc = lib.qf_decode_attn(*_qkv(c, kv_last), acc.data_ptr(), m.data_ptr(), l.data_ptr(), splits,
                            None if ticket is None else ticket.data_ptr(),
                            out.data_ptr(), out.stride(0), out.stride(1), out.stride(2),
                            b, kvh, g, d, cap, 0.125, torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "qf_decode_attn")
    return out


CASES = {
    # name: [(case builder, splits, kv_last per row?), (smaller second call)]
    "fused": [(lambda: workloads.decode_ragged(4, seed=3), 16, True),
              (lambda: workloads.decode_uniform(1, 512, seed=4), 8, False)],
    "two_launch": [(lambda: workloads.decode_uniform(1, 32768, seed=5, heavy_frac=0.01), 128, False),
                   (lambda: workloads.decode_uniform(1, 4096, seed=6, cap=4160), 64, True)],
    # Layout changes in both directions and between the merges: each call
    # must find the partials the previous one used cleared.
    "mixed": [(lambda: workloads.decode_uniform(2, 8192, seed=10), 64, False),
              (lambda: workloads.decode_ragged(4, seed=11), 16, True),
              (lambda: workloads.decode_uniform(2, 2048, seed=12), 32, False),
              (lambda: workloads.decode_ragged(4, seed=13), 16, True)],
    "direct": [(lambda: workloads.decode_ragged(2, seed=7), 1, True),
               (lambda: workloads.decode_uniform(1, 100, seed=8, cap=128), 1, False)],
}


@pytest.mark.parametrize("name", list(CASES))
def test_noalloc_equals_existing_entry_point_on_two_calls(dev, name):
    lib = _lib.load()
    for i, (build, splits, per_row) in enumerate(CASES[name]):
        case = build()
        c = case.to(dev)
        kv_last = None
        if per_row:
            kv_last = torch.tensor([n - 1 for n in case.lengths], dtype=torch.int64, device=dev)
        print(f"[noalloc {name} call {i}] B={case.grouped.shape[0]} cap={case.key_cache.shape[2]} "
              f"splits={splits}", flush=True)
        got = _noalloc(lib, c, splits, kv_last, dev)
        want = _existing(lib, c, splits, kv_last, dev)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"call {i}"
        ref = oracle.grouped_decode_attention(case.grouped, case.key_cache, case.value_cache,
                                              case.bias)
        assert (got.float().cpu() - ref).abs().max().item() <= TOL


def test_noalloc_rejects_a_problem_beyond_its_scratch(dev):
    lib = _lib.load()
    case = workloads.decode_uniform(64, 64, seed=9).to(dev)
    # 64 rows x 2 kv heads x 64 splits x 7 queries x 66 floats = 15 MB > 4 MiB.
    out = torch.zeros(64, 2, 7, 64, dtype=torch.float16, device=dev)
    g, k, v = case.grouped, case.key_cache, case.value_cache
    rc = lib.qf_decode_attn_noalloc(g.data_ptr(), g.stride(0), g.stride(1), g.stride(2),
                                    k.data_ptr(), k.stride(0), k.stride(1), k.stride(2),
                                    v.data_ptr(), v.stride(0), v.stride(1), v.stride(2),
                                    None, 0, None, 0, 64,
                                    out.data_ptr(), out.stride(0), out.stride(1), out.stride(2),
                                    64, 2, 7, 64, 64, 0.125, torch.cuda.current_stream().cuda_stream)
    assert rc == -3
    assert b"no-allocation scratch" in lib.qf_error_string(rc)


_CAPTURE_FIRST = textwrap.dedent("""
    import torch
    from qwenforge_amd import _lib, ops, workloads
    lib = _lib.load()
    dev = torch.device("cuda:0")
    case = workloads.decode_ragged(4, seed=21)
    c = case.to(dev)
    b, kvh, g, d = c.grouped.shape
    cap = c.key_cache.shape[2]
    splits = 16
    kv_last = torch.tensor([n - 1 for n in case.lengths], dtype=torch.int64, device=dev)
    gq, k, v = c.grouped, c.key_cache, c.value_cache
    qkv = (gq.data_ptr(), gq.stride(0), gq.stride(1), gq.stride(2),
           k.data_ptr(), k.stride(0), k.stride(1), k.stride(2),
           v.data_ptr(), v.stride(0), v.stride(1), v.stride(2),
           c.bias.data_ptr(), c.bias.stride(0), kv_last.data_ptr(), 1)
    want = ops.flash_decode_attention(gq, k, v, c.bias, ops.make_flash_scratch(
        b, kvh, g, cap, dev, splits=splits, fused=True), kv_last=kv_last).clone()
    out = torch.full((b, kvh, g, d), float("nan"), dtype=torch.float16, device=dev)
    torch.cuda.synchronize()
    print("capturing the first no-allocation call", flush=True)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = lib.qf_decode_attn_noalloc(*qkv, splits, out.data_ptr(), out.stride(0),
                                        out.stride(1), out.stride(2), b, kvh, g, d, cap, 0.125,
                                        torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "qf_decode_attn_noalloc (first call, under capture)")
    for i in range(3):
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {i}"
        # Eager work between replays, the same entry point included.
        eager = torch.empty_like(out)
        _lib.check(lib.qf_decode_attn_noalloc(*qkv, splits, eager.data_ptr(), eager.stride(0),
                                              eager.stride(1), eager.stride(2), b, kvh, g, d,
                                              cap, 0.125, torch.cuda.current_stream().cuda_stream),
                   "qf_decode_attn_noalloc (eager)")
        torch.cuda.synchronize()
        assert torch.equal(eager, want), f"eager call after replay {i}"
    print("capture-first ok", flush=True)
""")


def test_noalloc_first_call_under_graph_capture(dev):
    """The first no-allocation call of a process made inside torch.cuda.graph
    capture (the counter fill is then recorded into the graph): three replays,
    each followed by an eager call, all equal to qf_decode_attn's output."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    print("[noalloc capture-first] fresh process", flush=True)
    proc = subprocess.run([sys.executable, "-c", _CAPTURE_FIRST], cwd=root, capture_output=True,
                          text=True, timeout=240)
    print(proc.stdout[-2000:], proc.stderr[-2000:], flush=True)
    assert proc.returncode == 0 and "capture-first ok" in proc.stdout
