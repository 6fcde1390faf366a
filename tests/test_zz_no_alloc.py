"""The no-allocation attention entry point (qd_attention_decode_noalloc)
against qd_attention_decode with a caller-allocated workspace: same kernels,
same inputs, so the outputs must be bit-identical.  Two calls in a row on the
library's per-GPU scratch array, the second smaller, on both merge paths (a
split count <= 16 merges in the partial kernel through the arrival counters
that the first call leaves at zero; more splits take the merge launch), then
a request too large for the array, which must be refused with a clear error
and no launch.  Run alone or after the other GPU tests."""

from __future__ import annotations

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def _call(lib, name, q, kc, vc, L, T, n_split, out, ws=None):
    from qwen3vl_hip import _lib

    hq, hkv, d = 16, 8, 128
    cp = torch.full((1,), L - 1, dtype=torch.int64, device=q.device)
    args = [_lib.ptr(q), _lib.QD_F16, d, _lib.ptr(kc), _lib.ptr(vc), T * d, d, T, _lib.ptr(cp),
            ctypes.c_float(d ** -0.5), _lib.ptr(out), _lib.QD_F16, hq, hkv, n_split]
    if ws is not None:
        args.append(_lib.ptr(ws))
    st = getattr(lib, name)(*args, _lib.stream())
    torch.cuda.synchronize()
    return st


@pytest.mark.parametrize("first,second", [((4096, 16), (700, 8)), ((8192, 64), (1024, 20))])
def test_noalloc_attention_matches_workspace_entry_point(cuda, first, second):
    from qwen3vl_hip import _lib

    lib = _lib.lib()
    gen = torch.Generator(device=cuda).manual_seed(71)
    T = 8192
    kc = torch.randn(8, T, 128, generator=gen, device=cuda, dtype=torch.float16)
    vc = torch.randn(8, T, 128, generator=gen, device=cuda, dtype=torch.float16)
    for L, n_split in (first, second):
        print(f"case noalloc L={L} n_split={n_split}", flush=True)
        q = torch.randn(16, 128, generator=gen, device=cuda, dtype=torch.float16)
        ws = torch.zeros(int(lib.qd_attention_workspace_bytes(16, 8, n_split)), dtype=torch.uint8, device=cuda)
        ref = torch.full((16, 128), float("nan"), dtype=torch.float16, device=cuda)
        got = torch.full((16, 128), float("nan"), dtype=torch.float16, device=cuda)
        assert _call(lib, "qd_attention_decode", q, kc, vc, L, T, n_split, ref, ws) == 0
        assert _call(lib, "qd_attention_decode_noalloc", q, kc, vc, L, T, n_split, got) == 0, _lib.last_error()
        assert torch.isfinite(got).all()
        assert torch.equal(got, ref), f"L={L} n_split={n_split}: max diff {(got.float() - ref.float()).abs().max()}"


def test_noalloc_attention_refuses_oversized_requests(cuda):
    from qwen3vl_hip import _lib

    lib = _lib.lib()
    q = torch.zeros(16, 128, dtype=torch.float16, device=cuda)
    kc = torch.zeros(8, 64, 128, dtype=torch.float16, device=cuda)
    out = torch.full((16, 128), 7.0, dtype=torch.float16, device=cuda)
    # 16 heads x 128 splits need 1 057 024 bytes, more than the 1 MiB array
    st = _call(lib, "qd_attention_decode_noalloc", q, kc, kc, 64, 64, 128, out)
    assert st == -3 and "scratch" in _lib.last_error()
    assert (out == 7.0).all()   # nothing was launched
