"""The allocation-free prologue backward (``sbda_backward_prologue_noalloc``,
C ABI) against the existing ``sbda_backward_prologue`` with a caller
workspace: two calls in a row on one GPU, the second smaller, must give the
same gradients bit for bit (the kernels are the same and deterministic); a
call needing more than the static scratch is refused before any launch."""

from __future__ import annotations

import ctypes

import pytest
import torch

from sbda_amd import _lib
import sbda_amd

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _p(t):
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def _problem(b, t, h, d, layer, seed):
    gen = torch.Generator(device=DEV).manual_seed(seed)
    q, k, v, g = (torch.randn(b, t, h, d, generator=gen, device=DEV).to(torch.bfloat16)
                  .permute(0, 2, 1, 3) for _ in range(4))
    wq = (1 + 0.1 * torch.randn(d, generator=gen, device=DEV)).float()
    wk = (1 + 0.1 * torch.randn(d, generator=gen, device=DEV)).float()
    cos, sin = sbda_amd.rope_tables(t, d, 10000.0, DEV)
    jump = 1 << (layer - 1)
    offs = (0, jump) if layer <= 2 else (0, 1, 2, jump)
    return q, k, v, g, wq, wk, cos, sin, offs


def _shape(q, offs):
    b, h, t, d = q.shape
    return (b, h, h, t, d, 0, _lib.offsets_array(offs), len(offs))


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream(DEV).cuda_stream)


def _forward_lse(lib, q, k, v, wq, wk, cos, sin, offs):
    b, h, t, d = q.shape
    out = torch.empty_like(q)
    lse = torch.empty(b, t, h, dtype=torch.float32, device=DEV)
    _lib.check(lib.sbda_forward_prologue(
        _p(q), _lib.strides(q), _p(k), _lib.strides(k), _p(v), _lib.strides(v),
        _p(out), _lib.strides(out), _p(lse), _p(wq), _p(wk), _p(cos), _p(sin), 1e-6,
        *_shape(q, offs), None, _stream()))
    return lse


def _backward(lib, noalloc, q, k, v, g, lse, wq, wk, cos, sin, offs):
    d = q.shape[-1]
    dq, dk, dv = (torch.empty_like(x) for x in (q, k, v))
    dwq = torch.empty(d, dtype=torch.float32, device=DEV)
    dwk = torch.empty_like(dwq)
    head = (_p(q), _lib.strides(q), _p(k), _lib.strides(k), _p(v), _lib.strides(v),
            _p(g), _lib.strides(g), _p(lse), _p(wq), _p(wk), _p(cos), _p(sin), 1e-6,
            _p(dq), _lib.strides(dq), _p(dk), _lib.strides(dk), _p(dv), _lib.strides(dv),
            _p(dwq), _p(dwk))
    if noalloc:
        rc = lib.sbda_backward_prologue_noalloc(*head, *_shape(q, offs), None, _stream())
    else:
        need = lib.sbda_backward_workspace_for(
            1, *(_lib.strides(x) for x in (q, k, v, g, dq, dk, dv)), *_shape(q, offs), None)
        assert need >= 0
        ws = torch.empty(max(need, 16), dtype=torch.uint8, device=DEV)
        rc = lib.sbda_backward_prologue(*head, _p(ws), ws.numel(), *_shape(q, offs), None,
                                        _stream())
    _lib.check(rc)
    torch.cuda.synchronize()
    return dq, dk, dv, dwq, dwk


def test_noalloc_backward_matches_workspace_backward_twice():
    lib = _lib.load()
    assert lib.sbda_noalloc_scratch_bytes() == 128 << 20
    # First a config-3 far layer (row chains + finishing pass: partial rows
    # and deferred slots fill ~65 MiB of the scratch), then a smaller call
    # (T = 3000, a 2-pass far-4 layer) that reuses the same scratch.
    for b, t, layer, seed in ((4, 32768, 5, 11), (1, 3000, 3, 12)):
        print(f"no-alloc backward: B={b} T={t} layer {layer}", flush=True)
        prob = _problem(b, t, 8, 64, layer, seed)
        q, k, v, g, wq, wk, cos, sin, offs = prob
        lse = _forward_lse(lib, q, k, v, wq, wk, cos, sin, offs)
        want = _backward(lib, False, q, k, v, g, lse, wq, wk, cos, sin, offs)
        got = _backward(lib, True, q, k, v, g, lse, wq, wk, cos, sin, offs)
        for name, a, w in zip(("dq", "dk", "dv", "dwq", "dwk"), got, want):
            assert torch.equal(a, w), f"B={b} T={t} layer {layer}: {name} differs"


def test_noalloc_backward_refuses_more_than_its_scratch():
    lib = _lib.load()
    # T = 2^20, layer 5: the chained prologue backward needs ~525 MiB.
    b, t, h, d = 1, 1 << 20, 8, 64
    print("no-alloc backward: refusal at T=2^20 layer 5", flush=True)
    q, k, v, g, dq, dk, dv = (torch.empty(b, t, h, d, dtype=torch.bfloat16, device=DEV)
                              .permute(0, 2, 1, 3) for _ in range(7))
    lse = torch.empty(b, t, h, dtype=torch.float32, device=DEV)
    w = torch.ones(d, dtype=torch.float32, device=DEV)
    cs = torch.empty(t, d // 2, dtype=torch.float32, device=DEV)
    dw = torch.empty(d, dtype=torch.float32, device=DEV)
    offs = (0, 1, 2, 16)
    rc = lib.sbda_backward_prologue_noalloc(
        _p(q), _lib.strides(q), _p(k), _lib.strides(k), _p(v), _lib.strides(v),
        _p(g), _lib.strides(g), _p(lse), _p(w), _p(w), _p(cs), _p(cs), 1e-6,
        _p(dq), _lib.strides(dq), _p(dk), _lib.strides(dk), _p(dv), _lib.strides(dv),
        _p(dw), _p(dw), *_shape(q, offs), None, _stream())
    assert rc == _lib.ERR_VALUE
    assert "scratch" in lib.sbda_last_error().decode()
