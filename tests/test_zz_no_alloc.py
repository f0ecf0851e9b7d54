"""linatt_kata_bwd_noalloc (workspace from the library's fixed per-device
scratch, no allocation) against linatt_kata_bwd with a caller workspace, both
through the C ABI: the same kernels on the same inputs, so results must be
bit-identical.  Two calls in a row, the second smaller, so the second reads
scratch the first left behind."""

import ctypes

import pytest
import torch

from linatt_amd import _lib

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _inputs(B, T, H, D, seed):
    g = torch.Generator().manual_seed(seed)
    q, k, v = ((torch.randn(B, T, H, D, generator=g) / 8).to(torch.bfloat16) for _ in range(3))
    do = torch.randn(B, T, H, D, generator=g).to(torch.bfloat16)
    return [x.to(DEV) for x in (q, k, v, do)]


def _bwd_pair(B, T, H, D, M, seed):
    L = _lib.load()
    q, k, v, do = _inputs(B, T, H, D, seed)
    scale = (D // M) ** -0.5
    o = torch.empty_like(v)
    den = torch.empty(B, T, H, device=DEV, dtype=torch.float32)
    s = _lib.stream_of(q)
    _lib.check("linatt_kata_fwd", L.linatt_kata_fwd(
        _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), None, _lib.ptr(o), _lib.ptr(den),
        B, T, H, H, D, D, M, scale, 0, _lib.LINATT_BFLOAT16, s))
    outs = []
    for noalloc in (False, True):
        dq, dk, dv = torch.full_like(q, 7.0), torch.full_like(k, 7.0), torch.full_like(v, 7.0)
        if noalloc:
            st = L.linatt_kata_bwd_noalloc(
                _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(o), _lib.ptr(den), _lib.ptr(do),
                _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv), B, T, H, H, D, D, M, scale, 0,
                _lib.LINATT_BFLOAT16, s)
            _lib.check("linatt_kata_bwd_noalloc", st)
        else:
            ws = torch.empty(L.linatt_kata_bwd_workspace_bytes(B, T, H, D, _lib.LINATT_BFLOAT16),
                             device=DEV, dtype=torch.uint8)
            _lib.check("linatt_kata_bwd", L.linatt_kata_bwd(
                _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(o), _lib.ptr(den), _lib.ptr(do),
                _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv), _lib.ptr(ws), B, T, H, H, D, D, M,
                scale, 0, _lib.LINATT_BFLOAT16, s))
        torch.cuda.synchronize()
        outs.append((dq, dk, dv))
    return outs


def test_noalloc_matches_workspace_entry_point_twice():
    # first call: config-2 heads at full length (workspace ~6.4 MiB of the 32 MiB);
    # second call smaller, reusing the scratch the first call left behind
    for (B, T, H), seed in (((2, 2048, 12), 11), ((1, 333, 3), 12)):
        print(f"noalloc case B={B} T={T} H={H} seed={seed}", flush=True)
        ref, got = _bwd_pair(B, T, H, 64, 4, seed)
        for name, a, b in zip(("dq", "dk", "dv"), ref, got):
            assert torch.equal(a, b), f"{name} differs (B={B} T={T} H={H})"
            assert torch.isfinite(b.float()).all()


def test_noalloc_rejects_oversized():
    L = _lib.load()
    st = L.linatt_kata_bwd_noalloc(None, None, None, None, None, None, None, None, None,
                                   8, 4096, 12, 12, 64, 64, 4, 0.25, 0, 1, None)
    assert st == -1 and b"exceeds" in L.linatt_last_error()
