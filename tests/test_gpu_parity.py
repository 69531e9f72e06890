"""GPU parity of the HIP kernels against the CPU oracle (through the C ABI).

Bars (from the build's north star): fp32 outputs within 1e-5 relative;
bf16/fp16 outputs and gradients within 2e-2 relative and 1e-2 absolute of an
fp32 oracle run on the same (rounded) inputs; source indexing and masks
bit-exact (checked by exact-integer probes).  Inputs are generated on the CPU
from fixed seeds, so both sides see identical bits.
"""

from __future__ import annotations

import math

import pytest
import torch

import sbda_amd
from oracle import sbda_oracle as ref
from tests.sampled import sampled_oracle as _sampled_oracle

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
FP32_TOL = dict(rtol=1e-5, atol=1e-5)
LOW_TOL = dict(rtol=2e-2, atol=1e-2)


def _inputs(b, t, h, d, dtype, seed, hkv=None, n=4):
    """n tensors ``[B, T, heads, D]`` (CPU, ``dtype``), N(0, 1) from one seed."""
    g = torch.Generator().manual_seed(seed)
    heads = [h, hkv or h, hkv or h, h][:n]
    return [torch.randn(b, t, hh, d, generator=g).to(dtype) for hh in heads]


def _dev(x):
    """CPU [B,T,H,D] -> device [B,H,T,D] view (the left_v2 layout)."""
    return x.to(DEV).permute(0, 2, 1, 3)


def _fused(q, k, v, offs, grad):
    qd, kd, vd = (_dev(x).requires_grad_() for x in (q, k, v))
    off = torch.tensor(offs, dtype=torch.int32, device=DEV)
    out = sbda_amd.fused_sbda_gqa_key_backward(qd, kd, vd, off)
    out.backward(_dev(grad))
    torch.cuda.synchronize()
    return [x.detach().float().cpu() for x in (out, qd.grad, kd.grad, vd.grad)]


def _oracle(q, k, v, offs, grad, dtype=torch.float32):
    rq, rk, rv = (x.to(dtype).permute(0, 2, 1, 3).requires_grad_() for x in (q, k, v))
    out = ref.gather_attention(rq, rk, rv, offs)
    out.backward(grad.to(dtype).permute(0, 2, 1, 3))
    return [x.detach().float() for x in (out, rq.grad, rk.grad, rv.grad)]


def _close(got, want, tol, what):
    for name, a, b in zip(("out", "dq", "dk", "dv"), got, want):
        torch.testing.assert_close(a, b, **tol, msg=lambda m: f"{what} {name}: {m}")


# ------------------------------------------------------------ fp32 parity

@pytest.mark.parametrize("layer", [1, 2, 3])
def test_config1_fp32_matches_oracle(layer):
    # B=1, T=32, H=2, head_dim=8, fp32, layers 1..3.
    q, k, v, g = _inputs(1, 32, 2, 8, torch.float32, seed=100 + layer)
    offs = ref.sbda_layer_offsets(layer)
    got = _fused(q, k, v, offs, g)
    want = _oracle(q, k, v, offs, g, torch.float64)
    _close(got, [w.float() for w in want], FP32_TOL, f"config1 layer {layer}")
    out, lse = sbda_amd.sbda_forward(_dev(q), _dev(k), _dev(v), offs)
    want_lse = ref.attention_lse(q.double().permute(0, 2, 1, 3), k.double().permute(0, 2, 1, 3), offs)
    torch.testing.assert_close(lse.cpu().double(), want_lse, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("offs", [(0, 1, 2, 64), (0, 1, 2, 4096), (0, 2), (0, 5, 1, 300)])
def test_fp32_head_dim_64(offs):
    q, k, v, g = _inputs(2, 300, 4, 64, torch.float32, seed=7)
    _close(_fused(q, k, v, offs, g), _oracle(q, k, v, offs, g), FP32_TOL, f"fp32 {offs}")


# ------------------------------------------------------------ bf16 / fp16

@pytest.mark.parametrize("layer", range(1, 13))
def test_config2_bf16_forward_sweep(layer):
    # B=8, T=4096, H=8, D=64, bf16, layers 1..12.
    q, k, v = _inputs(8, 4096, 8, 64, torch.bfloat16, seed=200 + layer, n=3)
    offs = ref.sbda_layer_offsets(layer)
    out, lse = sbda_amd.sbda_forward(_dev(q), _dev(k), _dev(v), offs)
    rq, rk, rv = (x.float().permute(0, 2, 1, 3) for x in (q, k, v))
    want = ref.gather_attention(rq, rk, rv, offs)
    torch.testing.assert_close(out.float().cpu(), want, **LOW_TOL)
    torch.testing.assert_close(lse.cpu(), ref.attention_lse(rq, rk, offs), rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("layer", [1, 2, 3, 5, 8, 11, 12])
def test_bf16_fwd_bwd_layers(layer):
    q, k, v, g = _inputs(2, 2048, 8, 64, torch.bfloat16, seed=300 + layer)
    offs = ref.sbda_layer_offsets(layer)
    _close(_fused(q, k, v, offs, g), _oracle(q, k, v, offs, g), LOW_TOL, f"bf16 layer {layer}")


@pytest.mark.parametrize("layer", [1, 2])
def test_far_free_full_tiles_at_t_2_17(layer):
    # B = 1, T = 2^17: enough tiles that the far-free walks keep their full
    # tile sizes (64-position forward tiles, 32-position backward tiles, as
    # at the metric shape), checked in full against the oracle.
    q, k, v, g = _inputs(1, 1 << 17, 8, 64, torch.bfloat16, seed=320 + layer)
    offs = ref.sbda_layer_offsets(layer)
    _close(_fused(q, k, v, offs, g), _oracle(q, k, v, offs, g), LOW_TOL, f"T=2^17 layer {layer}")


@pytest.mark.parametrize("b,t,h,offs", [(2, 40000, 16, (0, 1, 2, 16384)), (1, 70000, 8, (0, 32768)),
                                         (3, 16385, 8, (0, 1, 2, 16384))])
def test_large_far_offsets_with_partial_rows(b, t, h, offs):
    # Far offsets >= 16384 over a few column rows: the forward's 2-row groups
    # and the backward's row pairs with an odd row count (a pair padded with a
    # row past T), partial last rows, a last row of one position, several
    # head groups and batches, far-only patterns.
    q, k, v, g = _inputs(b, t, h, 64, torch.bfloat16, seed=t + h + offs[-1])
    _close(_fused(q, k, v, offs, g), _oracle(q, k, v, offs, g), LOW_TOL, f"far rows B={b} T={t} {offs}")


def test_fp16_fwd_bwd():
    q, k, v, g = _inputs(1, 1000, 8, 64, torch.float16, seed=17)
    offs = (0, 1, 2, 16)
    _close(_fused(q, k, v, offs, g), _oracle(q, k, v, offs, g), LOW_TOL, "fp16")


@pytest.mark.parametrize("length,offs", [(1, (0, 1)), (7, (0, 1, 2, 1024)), (129, (0, 1, 2, 4))])
def test_reference_kernel_test_cases_gqa_head_dim_40(length, offs):
    # tests/test_model.py:46-68: GQA 4 query / 2 kv heads, head_dim 40, bf16.
    q, k, v, g = _inputs(1, length, 4, 40, torch.bfloat16, seed=42, hkv=2)
    got = _fused(q, k, v, offs, g)
    want = _oracle(q, k, v, offs, g)
    _close(got, want, LOW_TOL, f"gqa T={length}")
    _close(got, want, dict(rtol=0.015, atol=0.015), f"gqa T={length} (reference tol)")


# ------------------------------------------------- indexing and mask probes

@pytest.mark.parametrize("offs", [(0, 1), (0, 2), (0, 1, 2, 4), (0, 1, 2, 512), (0, 1, 2, 4096),
                                  (3, 1, 0, 7)])
def test_source_indexing_is_exact(offs):
    # q = 0 gives uniform weights over the valid sources, so with integer
    # position codes in v the output times the source count is an exact
    # integer sum of source positions, and exp(lse) is the exact count.
    t, d = 2048, 8
    q = torch.zeros(1, t, 2, d)
    k = _inputs(1, t, 2, d, torch.float32, seed=5, n=1)[0]
    pos = torch.arange(t, dtype=torch.float32)
    v = torch.zeros(1, t, 2, d)
    v[0, :, :, 0] = pos[:, None]
    v[0, :, :, 1] = (pos * pos)[:, None]
    v[0, :, :, 2] = 1.0
    out, lse = sbda_amd.sbda_forward(_dev(q), _dev(k), _dev(v), offs)
    out, lse = out.cpu().double(), lse.cpu().double()
    _, valid = ref.path_tables(t, offs)
    idx = torch.arange(t)[:, None] - torch.tensor(offs)[None, :]
    count = valid.sum(-1).double()
    s1 = (idx * valid).sum(-1).double()
    s2 = (idx * idx * valid).sum(-1).double()
    got_count = torch.exp(lse[0, 0]).round()
    assert torch.equal(got_count, count)
    assert torch.equal((out[0, 0, :, 0] * count).round(), s1)
    # Sums of squared positions reach ~1.7e7, past fp32's exact integers:
    # compare them to within 2 (a wrong source moves them by >= 2 * i).
    assert ((out[0, 0, :, 1] * count) - s2).abs().max().item() < 2.0
    torch.testing.assert_close(out[0, 0, :, 2], torch.ones(t, dtype=torch.float64), rtol=0, atol=1e-6)


def test_empty_rows_are_zero_with_infinite_lse():
    q, k, v, g = _inputs(1, 16, 2, 64, torch.float32, seed=9)
    offs = (1, 2)                                   # row 0 has no source
    got = _fused(q, k, v, offs, g)
    assert got[0][:, :, 0].abs().max().item() == 0
    _, lse = sbda_amd.sbda_forward(_dev(q), _dev(k), _dev(v), offs)
    assert torch.isinf(lse[:, :, 0]).all() and (lse[:, :, 0] > 0).all()
    _close(got, _oracle(q, k, v, offs, g), FP32_TOL, "empty rows")


# -------------------------------------------------- layout and determinism

def test_strided_and_contiguous_layouts_agree():
    q, k, v, g = _inputs(2, 512, 8, 64, torch.bfloat16, seed=11)
    offs = (0, 1, 2, 32)
    a = _fused(q, k, v, offs, g)
    qc, kc, vc = (_dev(x).contiguous().requires_grad_() for x in (q, k, v))
    out = sbda_amd.fused_sbda_key_backward(qc, kc, vc, torch.tensor(offs, dtype=torch.int32, device=DEV))
    assert out.is_contiguous()
    out.backward(_dev(g))                           # non-contiguous grad_out
    b = [x.detach().float().cpu() for x in (out, qc.grad, kc.grad, vc.grad)]
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_output_keeps_query_strides():
    q, k, v, _ = _inputs(1, 64, 8, 64, torch.bfloat16, seed=12)
    out = sbda_amd.fused_sbda_key_backward(_dev(q), _dev(k), _dev(v),
                                           torch.tensor((0, 1), dtype=torch.int32, device=DEV))
    assert out.stride() == _dev(q).stride()


def test_backward_is_bitwise_deterministic():
    q, k, v, g = _inputs(1, 4096, 8, 64, torch.bfloat16, seed=13)
    offs = (0, 1, 2, 256)
    out, lse = sbda_amd.sbda_forward(_dev(q), _dev(k), _dev(v), offs)
    first = sbda_amd.sbda_backward(_dev(q), _dev(k), _dev(v), _dev(g), lse, offs)
    for _ in range(2):
        again = sbda_amd.sbda_backward(_dev(q), _dev(k), _dev(v), _dev(g), lse, offs)
        for x, y in zip(first, again):
            assert torch.equal(x, y)


# ------------------------------------------------------------ prologue

@pytest.mark.parametrize("dtype,tol", [(torch.float32, FP32_TOL),
                                       (torch.bfloat16, LOW_TOL)])
@pytest.mark.parametrize("layer", [1, 2, 3, 7, 12])
def test_prologue_matches_oracle(dtype, tol, layer):
    # Config 3 style: q/k head-RMS-normalised, then RoPE base 10000.
    theta = 10000.0
    b, t, h, d = 2, 2048, 8, 64
    q, k, v, g = _inputs(b, t, h, d, dtype, seed=400 + layer)
    gen = torch.Generator().manual_seed(401)
    wq = (1 + 0.1 * torch.randn(d, generator=gen))
    wk = (1 + 0.1 * torch.randn(d, generator=gen))
    offs = ref.sbda_layer_offsets(layer)
    qd, kd, vd = (_dev(x).requires_grad_() for x in (q, k, v))
    wqd, wkd = wq.to(DEV).requires_grad_(), wk.to(DEV).requires_grad_()
    out = sbda_amd.fused_sbda_prologue(qd, kd, vd, torch.tensor(offs, dtype=torch.int32, device=DEV),
                                       wqd, wkd, theta=theta)
    out.backward(_dev(g))
    torch.cuda.synchronize()
    rq, rk, rv = (x.float().requires_grad_() for x in (q, k, v))
    rwq, rwk = wq.clone().requires_grad_(), wk.clone().requires_grad_()
    qq, kk = ref.prologue(rq, rk, rwq, rwk, theta)
    want = ref.gather_attention(qq.permute(0, 2, 1, 3), kk.permute(0, 2, 1, 3), rv.permute(0, 2, 1, 3), offs)
    want.backward(g.float().permute(0, 2, 1, 3))
    pairs = [("out", out, want), ("dq", qd.grad, rq.grad.permute(0, 2, 1, 3)),
             ("dk", kd.grad, rk.grad.permute(0, 2, 1, 3)), ("dv", vd.grad, rv.grad.permute(0, 2, 1, 3))]
    for name, a, w in pairs:
        torch.testing.assert_close(a.detach().float().cpu(), w.detach(), **tol,
                                   msg=lambda m: f"prologue {name}: {m}")
    # Weight gradients sum over B*T*H rows: compare relative to their scale.
    for name, a, w in (("dwq", wqd.grad, rwq.grad), ("dwk", wkd.grad, rwk.grad)):
        a = a.float().cpu()
        scale = w.abs().max().item() + 1e-6
        assert (a - w).abs().max().item() / scale < (2e-2 if dtype != torch.float32 else 1e-5), name


@pytest.mark.parametrize("dtype,h,d", [(torch.bfloat16, 16, 32), (torch.bfloat16, 4, 128),
                                       (torch.float16, 8, 64), (torch.float32, 8, 32),
                                       (torch.float32, 16, 16)])
@pytest.mark.parametrize("layer", [1, 3, 9])
def test_prologue_across_head_dims(dtype, h, d, layer):
    # Rows of 4, 8 and 16 lanes in the prologue walks (the head dimension is
    # a compile-time function of the lane count there), far-free and far.
    theta = 10000.0
    b, t = 1, 3000
    q, k, v, g = _inputs(b, t, h, d, dtype, seed=900 + layer + d)
    gen = torch.Generator().manual_seed(901 + d)
    wq = (1 + 0.1 * torch.randn(d, generator=gen))
    wk = (1 + 0.1 * torch.randn(d, generator=gen))
    offs = ref.sbda_layer_offsets(layer)
    qd, kd, vd = (_dev(x).requires_grad_() for x in (q, k, v))
    wqd, wkd = wq.to(DEV).requires_grad_(), wk.to(DEV).requires_grad_()
    out = sbda_amd.fused_sbda_prologue(qd, kd, vd, torch.tensor(offs, dtype=torch.int32, device=DEV),
                                       wqd, wkd, theta=theta)
    out.backward(_dev(g))
    torch.cuda.synchronize()
    rq, rk, rv = (x.float().requires_grad_() for x in (q, k, v))
    rwq, rwk = wq.clone().requires_grad_(), wk.clone().requires_grad_()
    qq, kk = ref.prologue(rq, rk, rwq, rwk, theta)
    want = ref.gather_attention(qq.permute(0, 2, 1, 3), kk.permute(0, 2, 1, 3), rv.permute(0, 2, 1, 3), offs)
    want.backward(g.float().permute(0, 2, 1, 3))
    tol = FP32_TOL if dtype == torch.float32 else LOW_TOL
    pairs = [("out", out, want), ("dq", qd.grad, rq.grad.permute(0, 2, 1, 3)),
             ("dk", kd.grad, rk.grad.permute(0, 2, 1, 3)), ("dv", vd.grad, rv.grad.permute(0, 2, 1, 3))]
    for name, a, w in pairs:
        torch.testing.assert_close(a.detach().float().cpu(), w.detach(), **tol,
                                   msg=lambda m: f"prologue {name} ({dtype}, h={h}, d={d}): {m}")
    for name, a, w in (("dwq", wqd.grad, rwq.grad), ("dwk", wkd.grad, rwk.grad)):
        a = a.float().cpu()
        scale = w.abs().max().item() + 1e-6
        assert (a - w).abs().max().item() / scale < (2e-2 if dtype != torch.float32 else 1e-5), name


def _check_prologue_against_oracle(q, k, v, g, offs, dtype, *, width=None, what=""):
    """fused_sbda_prologue (autograd) against the oracle's prologue + gather
    attention.  ``width``: place q/k/v as the first H heads of a ``width``-head
    buffer, so their position stride is ``width * D`` elements."""
    theta = 10000.0
    b, t, h, d = q.shape
    gen = torch.Generator().manual_seed(31 + d + t)
    wq = (1 + 0.1 * torch.randn(d, generator=gen))
    wk = (1 + 0.1 * torch.randn(d, generator=gen))

    def place(x):
        if width is None:
            return _dev(x)
        buf = torch.zeros(b, t, width, d, dtype=x.dtype, device=DEV)
        buf[:, :, :h] = x.to(DEV)
        return buf[:, :, :h].permute(0, 2, 1, 3)

    qd, kd, vd = (place(x).detach().requires_grad_() for x in (q, k, v))
    wqd, wkd = wq.to(DEV).requires_grad_(), wk.to(DEV).requires_grad_()
    out = sbda_amd.fused_sbda_prologue(qd, kd, vd, torch.tensor(offs, dtype=torch.int32, device=DEV),
                                       wqd, wkd, theta=theta)
    out.backward(_dev(g))
    torch.cuda.synchronize()
    rq, rk, rv = (x.float().requires_grad_() for x in (q, k, v))
    rwq, rwk = wq.clone().requires_grad_(), wk.clone().requires_grad_()
    qq, kk = ref.prologue(rq, rk, rwq, rwk, theta)
    want = ref.gather_attention(qq.permute(0, 2, 1, 3), kk.permute(0, 2, 1, 3), rv.permute(0, 2, 1, 3), offs)
    want.backward(g.float().permute(0, 2, 1, 3))
    tol = FP32_TOL if dtype == torch.float32 else LOW_TOL
    pairs = [("out", out, want), ("dq", qd.grad, rq.grad.permute(0, 2, 1, 3)),
             ("dk", kd.grad, rk.grad.permute(0, 2, 1, 3)), ("dv", vd.grad, rv.grad.permute(0, 2, 1, 3))]
    for name, a, w in pairs:
        torch.testing.assert_close(a.detach().float().cpu(), w.detach(), **tol,
                                   msg=lambda m: f"prologue {what} {name}: {m}")
    for name, a, w in (("dwq", wqd.grad, rwq.grad), ("dwk", wkd.grad, rwk.grad)):
        a = a.float().cpu()
        scale = w.abs().max().item() + 1e-6
        assert (a - w).abs().max().item() / scale < (2e-2 if dtype != torch.float32 else 1e-5), \
            f"{what} {name}"


@pytest.mark.parametrize("b,t,h,d,dtype,offs", [
    (1, 1000, 8, 64, torch.bfloat16, (0, 1, 2, 16)),     # 63 rows of 16, last one partial
    (2, 2048, 16, 64, torch.bfloat16, (0, 1, 2, 512)),   # 4 rows: 4-wave chains, 2 head groups
    (1, 700, 8, 64, torch.bfloat16, (0, 1, 2, 512)),     # 2 rows, the second partial
    (1, 300, 8, 64, torch.bfloat16, (0, 1, 2, 512)),     # 1 row: far source never valid
    (1, 3000, 8, 64, torch.float16, (0, 64)),            # self + far only
    (1, 2500, 8, 32, torch.float32, (0, 1, 2, 32)),
    (3, 1200, 8, 64, torch.bfloat16, (0, 1, 2, 64)),     # 19 rows: chains of 8, 8 and 3
])
def test_chained_prologue_backward_edges(b, t, h, d, dtype, offs):
    q, k, v, g = _inputs(b, t, h, d, dtype, seed=1300 + t + offs[-1])
    _check_prologue_against_oracle(q, k, v, g, offs, dtype, what=f"b={b} t={t} offs={offs}")


def test_chained_prologue_backward_wide_row_stride():
    # q/k/v are 8 of 64 heads of their buffers: an 8 KiB position stride, so
    # rows F = 4096 positions apart are 32 MiB apart and chains hold 4 rows.
    b, t, h, d = 1, 8 * 4096, 8, 64
    q, k, v, g = _inputs(b, t, h, d, torch.bfloat16, seed=1400)
    _check_prologue_against_oracle(q, k, v, g, (0, 1, 2, 4096), torch.bfloat16, width=64,
                                   what="wide stride")


# ---------------------------------------------------------------- config 3

@pytest.fixture(scope="module")
def config3_inputs():
    """BASELINE config 3's seeded inputs: raw q/k, v and dO ~ N(0, 1) at
    B = 4, T = 32768, H = 8, D = 64, bf16 ([B, T, H, D], CPU), and the two
    head-norm weights."""
    b, t, h, d = 4, 32768, 8, 64
    q, k, v, g = _inputs(b, t, h, d, torch.bfloat16, seed=3000)
    gen = torch.Generator().manual_seed(3001)
    wq = 1 + 0.1 * torch.randn(d, generator=gen)
    wk = 1 + 0.1 * torch.randn(d, generator=gen)
    return q, k, v, g, wq, wk


@pytest.mark.parametrize("layer", range(1, 16))
def test_config3_prologue_stack_layer(layer, config3_inputs):
    # the 15-layer stack with head-RMSNorm + RoPE (theta
    # 10^4) fused, forward + backward, each layer on the seeded inputs; every
    # element of out, dq, dk, dv and both norm-weight gradients against the
    # CPU oracle (fp32) run on the same bf16 inputs.
    q, k, v, g, wq, wk = config3_inputs
    theta = 10000.0
    offs = ref.sbda_layer_offsets(layer)
    print(f"config 3: layer {layer} offsets {offs}", flush=True)
    qd, kd, vd = (_dev(x).requires_grad_() for x in (q, k, v))
    wqd, wkd = wq.to(DEV).requires_grad_(), wk.to(DEV).requires_grad_()
    out = sbda_amd.fused_sbda_prologue(qd, kd, vd, torch.tensor(offs, dtype=torch.int32, device=DEV),
                                       wqd, wkd, theta=theta)
    out.backward(_dev(g))
    torch.cuda.synchronize()
    got = [x.detach().float().cpu() for x in (out, qd.grad, kd.grad, vd.grad)]
    del qd, kd, vd, out
    rq, rk, rv = (x.float().requires_grad_() for x in (q, k, v))
    rwq, rwk = wq.clone().requires_grad_(), wk.clone().requires_grad_()
    qq, kk = ref.prologue(rq, rk, rwq, rwk, theta)
    want = ref.gather_attention(qq.permute(0, 2, 1, 3), kk.permute(0, 2, 1, 3),
                                rv.permute(0, 2, 1, 3), offs)
    want.backward(g.float().permute(0, 2, 1, 3))
    wants = [want.detach(), rq.grad.permute(0, 2, 1, 3), rk.grad.permute(0, 2, 1, 3),
             rv.grad.permute(0, 2, 1, 3)]
    _close(got, wants, LOW_TOL, f"config 3 layer {layer}")
    for name, a, w in (("dwq", wqd.grad, rwq.grad), ("dwk", wkd.grad, rwk.grad)):
        a = a.float().cpu()
        scale = w.abs().max().item() + 1e-6
        assert (a - w).abs().max().item() / scale < 2e-2, f"config 3 layer {layer} {name}"


# --------------------------------------------------- metric-size properties

def _device_rows(*xs):
    """fetch() over device ``[1, T, H, D]`` tensors: fp32 CPU rows at positions."""
    def fetch(pos):
        idx = pos.to(xs[0].device)
        return tuple(x[0].index_select(0, idx).float().cpu() for x in xs)
    return fetch


def _check_sampled_rows(q, k, v, g, offs, out, dq_, dk_, dv_, rows):
    """Rows ``rows`` of out and of each gradient ([B=1,H,T,D] views) against
    the oracle evaluated on those rows' sources (q/k/v/g: [1, T, H, D])."""
    t, d = q.shape[1], q.shape[3]
    rows = rows.unique()
    want = _sampled_oracle(_device_rows(q, k, v, g), offs, rows, t, d)
    idx = rows.to(out.device)
    for name, a, w in zip(("out", "dq", "dk", "dv"), (out, dq_, dk_, dv_), want):
        got = a.detach()[0].index_select(1, idx).permute(1, 0, 2).float().cpu()
        torch.testing.assert_close(got, w, **LOW_TOL, msg=lambda m: f"{name}: {m}")


def _metric_rows(t, seed, n=2040):
    """Sampled positions: the first 8, the last 4, and n uniform ones."""
    return torch.cat([torch.arange(0, 8), torch.arange(t - 4, t),
                      torch.randint(0, t, (n,), generator=torch.Generator().manual_seed(seed))]).unique()


@pytest.fixture(scope="module")
def metric_inputs():
    """One seeded q/k/v/dO set at the metric shape (T = 2**20, H = 8, D = 64,
    bf16, [1, T, H, D] memory), shared by the per-layer metric-size tests."""
    t, h, d = 1 << 20, 8, 64
    gen = torch.Generator(device=DEV).manual_seed(500)
    xs = [torch.randn(1, t, h, d, generator=gen, device=DEV).to(torch.bfloat16) for _ in range(4)]
    yield xs
    del xs
    torch.cuda.empty_cache()


@pytest.mark.parametrize("layer", range(1, 21))
def test_metric_shape_sampled_rows(layer, metric_inputs):
    # T = 2**20, H = 8, D = 64 bf16, every layer of the timed schedule (each
    # runs its own launch configuration at this size): ~2k sampled rows of the
    # output and of each gradient against the oracle on those rows' sources.
    q, k, v, g = metric_inputs
    t = q.shape[1]
    offs = ref.sbda_layer_offsets(layer)
    print(f"metric shape: layer {layer} offsets {offs}", flush=True)
    qd, kd, vd = (x.permute(0, 2, 1, 3).detach().requires_grad_() for x in (q, k, v))
    out = sbda_amd.fused_sbda_key_backward(qd, kd, vd, torch.tensor(offs, dtype=torch.int32, device=DEV))
    out.backward(g.permute(0, 2, 1, 3))
    torch.cuda.synchronize()
    _check_sampled_rows(q, k, v, g, offs, out, qd.grad, kd.grad, vd.grad, _metric_rows(t, 3 + layer))


@pytest.mark.parametrize("layer", range(1, 21))
def test_metric_shape_prologue_sampled_rows(layer, metric_inputs):
    # The fused norm + RoPE route (the backbone's attention) at T = 2**20 for
    # every layer: sampled rows of out / dq / dk / dv (gradients w.r.t. the
    # raw q/k) against the oracle's prologue + attention on those rows.
    q, k, v, g = metric_inputs
    t, d = q.shape[1], q.shape[3]
    theta = 10000.0
    offs = ref.sbda_layer_offsets(layer)
    print(f"metric shape, prologue: layer {layer} offsets {offs}", flush=True)
    gen = torch.Generator().manual_seed(600 + layer)
    wq = 1 + 0.1 * torch.randn(d, generator=gen)
    wk = 1 + 0.1 * torch.randn(d, generator=gen)
    qd, kd, vd = (x.permute(0, 2, 1, 3).detach().requires_grad_() for x in (q, k, v))
    out = sbda_amd.fused_sbda_prologue(qd, kd, vd, torch.tensor(offs, dtype=torch.int32, device=DEV),
                                       wq.to(DEV), wk.to(DEV), theta=theta)
    out.backward(g.permute(0, 2, 1, 3))
    torch.cuda.synchronize()
    raw = _device_rows(q, k, v, g)

    def fetch(pos):
        rq, rk, rv, rg = raw(pos)
        qq, kk = ref.prologue(rq[None], rk[None], wq, wk, theta, positions=pos)
        return qq[0], kk[0], rv, rg

    rows = _metric_rows(t, 7 + layer, n=1020)
    o_w, dq_w, dk_w, dv_w = _sampled_oracle(fetch, offs, rows, t, d)
    # Gradients w.r.t. the raw rows: back through the per-row prologue.
    rq, rk, _, _ = raw(rows)
    rq, rk = rq.requires_grad_(), rk.requires_grad_()
    qq, kk = ref.prologue(rq[None], rk[None], wq, wk, theta, positions=rows)
    dq_w, dk_w = torch.autograd.grad((qq[0], kk[0]), (rq, rk), (dq_w, dk_w))
    idx = rows.to(DEV)
    for name, a, w in zip(("out", "dq", "dk", "dv"), (out, qd.grad, kd.grad, vd.grad),
                          (o_w, dq_w, dk_w, dv_w)):
        got = a.detach()[0].index_select(1, idx).permute(1, 0, 2).float().cpu()
        torch.testing.assert_close(got, w, **LOW_TOL, msg=lambda m: f"layer {layer} {name}: {m}")


@pytest.mark.parametrize("layer", [3, 20])
def test_row_span_past_4_gib_runs_generic_kernels(layer):
    # q, k, v and grad_out are 8-head slices of one [1, 2^20, 64, 64] bf16
    # buffer: an 8 KiB position stride, so a head group spans 8 GiB -- past the
    # walk kernels' 32-bit offsets.  The generic kernels run, with the
    # workspace the stride-aware query sizes.
    t, d = 1 << 20, 64
    offs = ref.sbda_layer_offsets(layer)
    gen = torch.Generator(device=DEV).manual_seed(700 + layer)
    buf = torch.randn(1, t, 64, d, generator=gen, device=DEV).to(torch.bfloat16)
    q, k, v, g = (buf[:, :, 8 * i:8 * i + 8] for i in range(4))
    qd, kd, vd = (x.permute(0, 2, 1, 3).detach().requires_grad_() for x in (q, k, v))
    out = sbda_amd.fused_sbda_key_backward(qd, kd, vd, torch.tensor(offs, dtype=torch.int32, device=DEV))
    out.backward(g.permute(0, 2, 1, 3))
    torch.cuda.synchronize()
    _check_sampled_rows(q, k, v, g, offs, out, qd.grad, kd.grad, vd.grad, _metric_rows(t, 5, n=400))
    del buf


def test_rope_table_matches_fp32_reference_angles():
    # Angles are fp32 products position * inv_freq (bit-identical to the
    # reference's torch.outer); cos/sin then agree to a few fp32 ulps, also
    # at the metric length where the angle reaches ~1e6 rad.
    t, d = 1 << 20, 64
    for theta in (10000.0, 1_000_000.0):
        cos, sin = sbda_amd.rope_tables(t, d, theta, DEV)
        want_c, want_s = ref.rope_tables(t, d, theta, torch.float32)
        torch.testing.assert_close(cos.cpu(), want_c[:, : d // 2], rtol=0, atol=3e-7)
        torch.testing.assert_close(sin.cpu(), want_s[:, : d // 2], rtol=0, atol=3e-7)


@pytest.mark.parametrize("t", [1, 2, 3, 5, 17, 300, 3000])
@pytest.mark.parametrize("offs", [(0, 1), (0, 2), (0, 1, 2, 3), (0, 1, 2, 4), (0, 1, 2, 8),
                                  (0, 1, 2, 16), (0, 1, 2, 1024), (0, 4), (0, 8),
                                  (2, 0, 1, 64)])
def test_tile_edges_and_offset_patterns(t, offs):
    # Lengths that are not multiples of the tile, the 3-step unroll or the far
    # offset; far offsets below, at and above the tile size (linear and
    # column tile orders); near-only, near+far and far-only patterns.
    q, k, v, g = _inputs(2, t, 8, 64, torch.bfloat16, seed=t * 31 + sum(offs))
    _close(_fused(q, k, v, offs, g), _oracle(q, k, v, offs, g), LOW_TOL, f"T={t} {offs}")
    q, k, v, g = _inputs(1, t, 8, 64, torch.float32, seed=t * 37 + sum(offs))
    _close(_fused(q, k, v, offs, g), _oracle(q, k, v, offs, g), FP32_TOL, f"fp32 T={t} {offs}")


@pytest.mark.parametrize("dtype,tol", [(torch.bfloat16, LOW_TOL), (torch.float16, LOW_TOL),
                                       (torch.float32, FP32_TOL)])
@pytest.mark.parametrize("b,h,d", [(2, 16, 64), (1, 32, 32), (1, 8, 128)])
@pytest.mark.parametrize("offs", [(0, 1, 2, 4), (0, 1, 2, 8), (0, 1, 2, 16), (0, 1, 2, 256),
                                  (0, 1, 2, 2048), (0, 8)])
def test_walk_kernels_across_head_groups_and_row_widths(dtype, tol, b, h, d, offs):
    # The walk kernels for every lanes-per-row width (16-byte chunks per row:
    # 4, 8 or 16) and several head groups per position / batches, so each
    # workgroup decode path (independent waves, lockstep column chains,
    # transposed chains for far offsets 4 and 8) runs with more than one head
    # group; T = 4100 is not a multiple of any tile, row or chain length.
    t = 4100
    q, k, v, g = _inputs(b, t, h, d, dtype, seed=h * 7 + d + sum(offs))
    _close(_fused(q, k, v, offs, g), _oracle(q, k, v, offs, g), tol,
           f"{dtype} B={b} H={h} D={d} {offs}")


@pytest.mark.parametrize("t,offs", [(16384, (0, 1, 2, 4096)), (32768, (0, 1, 2, 8192)),
                                    (20000, (0, 1, 2, 4096))])
def test_walk_forward_row_groups_at_4_to_8_mib_strides(t, offs):
    # Far rows 4-8 MiB apart (1 KiB positions): the forward walks 8 rows x 1
    # band per workgroup there instead of 2 rows x 4 bands; T = 20000 leaves
    # a partial last row.
    q, k, v, g = _inputs(1, t, 8, 64, torch.bfloat16, seed=t + offs[-1])
    _close(_fused(q, k, v, offs, g), _oracle(q, k, v, offs, g), LOW_TOL, f"T={t} {offs}")


# ------------------------------------------------------------ module level

def _oracle_module_forward(m, x, valid_mask=None, seam_reset=None, path_indices=None,
                           path_valid=None):
    """The reference module's forward (left_v2.py:234-306 fused route, or the
    eager masked gather of :313-405 for holes / seams), restated with the
    oracle's prologue and gather attention."""
    b, t, dim = x.shape
    q = (x @ m.q.weight.T).view(b, t, m.heads, m.head_dim)
    k = (x @ m.k.weight.T).view(b, t, m.kv_heads, m.head_dim)
    v = (x @ m.v.weight.T).view(b, t, m.kv_heads, m.head_dim)
    q, k = ref.prologue(q, k, m.q_norm.weight, m.k_norm.weight, m.rope_theta)
    qh, kh, vh = (x_.permute(0, 2, 1, 3) for x_ in (q, k, v))
    prefix = valid_mask is None or bool(torch.all(~valid_mask[:, 1:] | valid_mask[:, :-1]))
    if path_indices is not None:
        att = ref.gather_attention_tables(qh, kh, vh, path_indices, path_valid, valid_mask,
                                          seam_reset)
    elif prefix and seam_reset is None:
        att = ref.gather_attention(qh, kh, vh, m.offsets)
    else:
        att = ref.gather_attention_masked(qh, kh, vh, m.offsets, valid_mask, seam_reset)
    out = att.transpose(1, 2).reshape(b, t, dim) @ m.out.weight.T
    if valid_mask is not None:
        out = out * valid_mask[:, :, None].to(out.dtype)
    return out


@pytest.mark.parametrize("layer,kv_heads", [(1, None), (3, None), (9, None), (4, 4)])
def test_sbdattention_module_matches_oracle_module(layer, kv_heads):
    torch.manual_seed(50 + layer)
    dim, heads, t = 512, 8, 700
    m = sbda_amd.SBDAttention(dim, heads, layer, kv_heads=kv_heads, rope_theta=10000.0,
                              total_layers=12)
    with torch.no_grad():
        m.q_norm.weight.mul_(1 + 0.1 * torch.randn(m.head_dim))
        m.k_norm.weight.mul_(1 + 0.1 * torch.randn(m.head_dim))
    x = torch.randn(2, t, dim)
    valid = torch.ones(2, t, dtype=torch.bool)
    valid[1, 650:] = False                         # right padding: fused-eligible
    g = torch.randn(2, t, dim)
    md = m.to(DEV)
    xd = x.to(DEV).requires_grad_()
    out = md(xd, valid.to(DEV))
    out.backward(g.to(DEV))
    torch.cuda.synchronize()
    mc = sbda_amd.SBDAttention(dim, heads, layer, kv_heads=kv_heads, rope_theta=10000.0,
                               total_layers=12)
    mc.load_state_dict({k_: v_.cpu() for k_, v_ in md.state_dict().items()})
    xc = x.clone().requires_grad_()
    want = _oracle_module_forward(mc, xc, valid)
    want.backward(g)
    tol = FP32_TOL
    torch.testing.assert_close(out.detach().cpu(), want.detach(), **tol)
    torch.testing.assert_close(xd.grad.cpu(), xc.grad, **tol)
    for (name, p), (_, pc) in zip(md.named_parameters(), mc.named_parameters()):
        scale = pc.grad.abs().max().item() + 1e-6
        err = (p.grad.cpu() - pc.grad).abs().max().item()
        assert err / scale < 1e-5, f"{name}: {err} vs scale {scale}"


def test_sbdattention_module_rejects_eager_only_inputs():
    m = sbda_amd.SBDAttention(64, 4, 3).to(DEV)
    x = torch.randn(1, 8, 64, device=DEV)
    off = sbda_amd.SBDAttention(64, 4, 3, use_fused=False).to(DEV)
    with pytest.raises(NotImplementedError, match="use_fused"):
        off(x)
    bad = torch.full((1, 8, 2), 8, dtype=torch.long, device=DEV)
    with pytest.raises(ValueError, match="out-of-range"):
        m(x, None, None, bad)


# ------------------------------------------------------------ masks

def _masks(b, t, seed):
    """Holes, a padded tail and seams, the masks of left_v2.py:329-378."""
    g = torch.Generator().manual_seed(seed)
    valid = torch.rand(b, t, generator=g) > 0.15
    valid[0, t - t // 5:] = False
    seam = torch.rand(b, t, generator=g) < 0.03
    seam[:, 0] = False
    return valid, seam


@pytest.mark.parametrize("dtype,tol", [(torch.float32, FP32_TOL), (torch.bfloat16, LOW_TOL)])
@pytest.mark.parametrize("offs,hkv,d", [((0, 1), None, 64), ((0, 1, 2, 4), None, 64),
                                        ((0, 1, 2, 64), None, 64), ((0, 1, 2, 16), 2, 64),
                                        ((0, 2), 4, 40), ((0, 1, 2, 128), None, 128)])
@pytest.mark.parametrize("which", ["holes", "seams", "both"])
def test_masked_op_matches_oracle(dtype, tol, offs, hkv, d, which):
    b, t, h = 2, 300, 8
    q, k, v, g = _inputs(b, t, h, d, dtype, seed=hash((offs, d, which)) % 1000, hkv=hkv)
    valid, seam = _masks(b, t, seed=len(offs) * 7 + d)
    vm = None if which == "seams" else valid
    sr = None if which == "holes" else seam
    keep = torch.ones(b, t, dtype=torch.bool) if vm is None else vm
    g = g * keep[:, :, None, None].to(dtype)        # padded rows get no gradient
    key = sbda_amd.segment_keys(None if vm is None else vm.to(DEV),
                                None if sr is None else sr.to(DEV))
    qd, kd, vd = (_dev(x).requires_grad_() for x in (q, k, v))
    off = torch.tensor(offs, dtype=torch.int32, device=DEV)
    out = sbda_amd.fused_sbda_gqa_key_backward(qd, kd, vd, off, seg_key=key)
    out.backward(_dev(g))
    torch.cuda.synchronize()
    got = [x.detach().float().cpu() for x in (out, qd.grad, kd.grad, vd.grad)]
    rq, rk, rv = (x.float().permute(0, 2, 1, 3).requires_grad_() for x in (q, k, v))
    want = ref.gather_attention_masked(rq, rk, rv, offs, vm, sr)
    want.backward(g.float().permute(0, 2, 1, 3))
    rows = keep[:, None, :, None].expand_as(got[0])
    # Padded query rows: zeros here, slot 0 forced valid in the reference;
    # both are multiplied by valid_mask by the caller.
    assert torch.all(got[0][~rows] == 0)
    torch.testing.assert_close(got[0][rows], want.detach()[rows], **tol)
    for name, a, r in zip(("dq", "dk", "dv"), got[1:], (rq.grad, rk.grad, rv.grad)):
        torch.testing.assert_close(a, r, **tol, msg=lambda m: f"{which} {offs} {name}: {m}")


def test_masked_prologue_matches_unmasked_on_independent_segments():
    # seam_reset splits a batch row into segments that attend as separate
    # sequences would (RoPE positions stay global): the second segment's
    # results must not change when everything before the seam does, and the
    # first segment's must equal the unmasked op on the prefix.
    b, t, h, d = 1, 512, 8, 64
    q, k, v, g = _inputs(b, t, h, d, torch.bfloat16, seed=91)
    offs = (0, 1, 2, 32)
    seam = torch.zeros(b, t, dtype=torch.bool)
    seam[0, 256] = True
    wq = (1 + 0.1 * torch.randn(d)).to(DEV)
    wk = (1 + 0.1 * torch.randn(d)).to(DEV)
    off = torch.tensor(offs, dtype=torch.int32, device=DEV)
    key = sbda_amd.segment_keys(None, seam.to(DEV))

    def run(seg_key, qx, kx, vx, gx):
        qd, kd, vd = (_dev(x).requires_grad_() for x in (qx, kx, vx))
        out = sbda_amd.fused_sbda_prologue(qd, kd, vd, off, wq, wk, theta=10000.0,
                                           seg_key=seg_key)
        out.backward(_dev(gx))
        torch.cuda.synchronize()
        return [x.detach().float().cpu() for x in (out, qd.grad, kd.grad, vd.grad)]

    masked = run(key, q, k, v, g)
    # Second segment alone: the first segment's k/v replaced by values that
    # would change every result if any of them were read as a source.
    k2, v2 = k.clone(), v.clone()
    k2[:, :256] = 50.0
    v2[:, :256] = -50.0
    second = run(key, q, k2, v2, g)
    for a, bb in zip(masked, second):
        torch.testing.assert_close(a[:, :, 256:], bb[:, :, 256:], rtol=0, atol=0)
    # and the first segment equals the unmasked op cut at the seam (another
    # kernel family, so within the bf16 tolerance rather than bit for bit).
    plain = run(None, q[:, :256], k[:, :256], v[:, :256], g[:, :256])
    for a, bb in zip(masked, plain):
        torch.testing.assert_close(a[:, :, :256], bb, **LOW_TOL)


@pytest.mark.parametrize("layer", [3, 8])
def test_sbdattention_module_with_holes_and_seams_matches_oracle(layer):
    torch.manual_seed(70 + layer)
    dim, heads, t = 256, 4, 400
    m = sbda_amd.SBDAttention(dim, heads, layer, rope_theta=10000.0, total_layers=12)
    with torch.no_grad():
        m.q_norm.weight.mul_(1 + 0.1 * torch.randn(m.head_dim))
        m.k_norm.weight.mul_(1 + 0.1 * torch.randn(m.head_dim))
    x = torch.randn(2, t, dim)
    valid, seam = _masks(2, t, seed=layer)
    g = torch.randn(2, t, dim)
    md = m.to(DEV)
    xd = x.to(DEV).requires_grad_()
    out = md(xd, valid.to(DEV), seam.to(DEV))
    out.backward(g.to(DEV))
    torch.cuda.synchronize()
    mc = sbda_amd.SBDAttention(dim, heads, layer, rope_theta=10000.0, total_layers=12)
    mc.load_state_dict({k_: v_.cpu() for k_, v_ in md.state_dict().items()})
    xc = x.clone().requires_grad_()
    want = _oracle_module_forward(mc, xc, valid, seam)
    want.backward(g)
    tol = FP32_TOL
    torch.testing.assert_close(out.detach().cpu(), want.detach(), **tol)
    torch.testing.assert_close(xd.grad.cpu(), xc.grad, **tol)
    for (name, p), (_, pc) in zip(md.named_parameters(), mc.named_parameters()):
        scale = pc.grad.abs().max().item() + 1e-6
        err = (p.grad.cpu() - pc.grad).abs().max().item()
        assert err / scale < 1e-5, f"{name}: {err} vs scale {scale}"


def test_backbone_forward_backward_matches_oracle_composition():
    # BiAttnLM with SBDA layers (the reference's caller, BiAttn/model.py:248-502)
    # against the same weights run through the oracle module forward on the CPU.
    torch.manual_seed(60)
    cfg = sbda_amd.BiAttnConfig(vocab_size=64, dim=256, layers=5, heads=4, rope_theta=10000.0,
                                ff_hidden=512)
    m = sbda_amd.BiAttnLM(cfg)
    ids = torch.randint(0, 64, (2, 300))
    valid = torch.ones(2, 300, dtype=torch.bool)
    valid[0, 280:] = False
    md = m.to(DEV)
    out = md(ids.to(DEV), valid.to(DEV))
    out.float().square().mean().backward()
    torch.cuda.synchronize()
    mc = sbda_amd.BiAttnLM(cfg)
    mc.load_state_dict({k_: v_.cpu() for k_, v_ in md.state_dict().items()})

    def oracle_forward(model, input_ids, vm):
        x = model.embedding(input_ids)
        for blk in model.layers:
            x = x + _oracle_module_forward(blk.attn, blk.norm1(x), vm)
            ff = blk.ff(blk.norm2(x)) * vm[:, :, None].to(x.dtype)
            x = x + ff
        return model.lm_head(model.norm(x))

    want = oracle_forward(mc, ids, valid)
    want.float().square().mean().backward()
    torch.testing.assert_close(out.detach().cpu(), want.detach(), **FP32_TOL)
    for (name, p), (_, pc) in zip(md.named_parameters(), mc.named_parameters()):
        scale = pc.grad.abs().max().item() + 1e-8
        err = (p.grad.cpu() - pc.grad).abs().max().item()
        assert err / scale < 1e-5, f"{name}: {err} vs scale {scale}"


# ------------------------------------------------------------ source tables

def _tables(b, t, s, seed):
    """Mostly near-causal source tables with some future entries, a
    duplicate, and random path_valid flags."""
    g = torch.Generator().manual_seed(seed)
    anywhere = torch.randint(0, t, (b, t, s), generator=g)
    near = (torch.arange(t)[None, :, None]
            - torch.randint(0, 40, (b, t, s), generator=g)).clamp_min(0)
    idx = torch.where(torch.rand(b, t, s, generator=g) < 0.8, near, anywhere)
    if s > 2:
        idx[:, 5, 1:3] = 2
    valid = torch.rand(b, t, s, generator=g) > 0.15
    return idx, valid


def _table_run(fn, q, k, v, g):
    qd, kd, vd = (_dev(x).requires_grad_() for x in (q, k, v))
    out = fn(qd, kd, vd)
    out.backward(_dev(g))
    torch.cuda.synchronize()
    return [x.detach().float().cpu() for x in (out, qd.grad, kd.grad, vd.grad)]


@pytest.mark.parametrize("dtype,tol", [(torch.float32, FP32_TOL), (torch.bfloat16, LOW_TOL)])
@pytest.mark.parametrize("s,hkv,d", [(1, None, 64), (3, None, 64), (5, 2, 64), (8, 4, 40),
                                     (4, None, 128)])
@pytest.mark.parametrize("masked", [False, True])
def test_table_op_matches_oracle(dtype, tol, s, hkv, d, masked):
    b, t, h = 2, 300, 8
    q, k, v, g = _inputs(b, t, h, d, dtype, seed=s * 13 + d + int(masked), hkv=hkv)
    idx, valid = _tables(b, t, s, seed=s + d)
    vm, sr = _masks(b, t, seed=s) if masked else (None, None)
    keep = torch.ones(b, t, dtype=torch.bool) if vm is None else vm
    g = g * keep[:, :, None, None].to(dtype)
    key = sbda_amd.segment_keys(vm.to(DEV), sr.to(DEV)) if masked else None
    pidx, pval = idx.to(DEV), valid.to(DEV)
    got = _table_run(lambda a, bb, c: sbda_amd.fused_sbda_paths(a, bb, c, pidx, pval, seg_key=key),
                     q, k, v, g)
    rq, rk, rv = (x.float().permute(0, 2, 1, 3).requires_grad_() for x in (q, k, v))
    want = ref.gather_attention_tables(rq, rk, rv, idx, valid, vm, sr)
    want.backward(g.float().permute(0, 2, 1, 3))
    rows = keep[:, None, :, None].expand_as(got[0])
    assert torch.all(got[0][~rows] == 0)
    torch.testing.assert_close(got[0][rows], want.detach()[rows], **tol)
    for name, a, r in zip(("dq", "dk", "dv"), got[1:], (rq.grad, rk.grad, rv.grad)):
        torch.testing.assert_close(a, r, **tol, msg=lambda m: f"S={s} {name}: {m}")


def test_tables_from_offsets_match_the_offset_op():
    b, t, h, d = 1, 1000, 8, 64
    q, k, v, g = _inputs(b, t, h, d, torch.bfloat16, seed=123)
    for offs in ((0, 2), (0, 1, 2, 16), (0, 1, 2, 512)):
        idx, ok = ref.path_tables(t, offs)
        pidx = idx.unsqueeze(0).to(DEV).contiguous()
        pval = ok.unsqueeze(0).to(DEV).contiguous()
        off = torch.tensor(offs, dtype=torch.int32, device=DEV)
        a = _table_run(lambda x, y, z: sbda_amd.fused_sbda_paths(x, y, z, pidx, pval), q, k, v, g)
        w = _table_run(lambda x, y, z: sbda_amd.fused_sbda_key_backward(x, y, z, off), q, k, v, g)
        _close(a, w, LOW_TOL, f"tables vs offsets {offs}")


def test_table_backward_is_bitwise_deterministic():
    b, t, h, d, s = 2, 700, 8, 64, 6
    q, k, v, g = _inputs(b, t, h, d, torch.bfloat16, seed=7)
    idx, valid = _tables(b, t, s, seed=8)
    pidx, pval = idx.to(DEV), valid.to(DEV)
    fn = lambda x, y, z: sbda_amd.fused_sbda_paths(x, y, z, pidx, pval)  # noqa: E731
    first = _table_run(fn, q, k, v, g)
    second = _table_run(fn, q, k, v, g)
    for a, bb in zip(first, second):
        assert torch.equal(a, bb)


def test_table_module_reference_known_answers():
    # tests/test_model.py:19-42 on the module: a slot pointing at a future
    # position is masked, and all-invalid tables give zero output and gradient.
    torch.manual_seed(42)
    attn = sbda_amd.SBDAttention(32, 4, 3, kv_heads=2).to(DEV)
    x = torch.randn(1, 8, 32, device=DEV, requires_grad=True)
    paths = torch.arange(8, device=DEV).view(1, 8, 1).expand(1, 8, 2).clone()
    paths[:, :, 1] = 7
    y = attn(x, path_indices=paths)
    changed = x.detach().clone()
    changed[:, 4:] += 10
    torch.testing.assert_close(y[:, :4], attn(changed, path_indices=paths)[:, :4])
    y[:, :4].square().sum().backward()
    assert x.grad[:, 4:].abs().max().item() == 0
    attn2 = sbda_amd.SBDAttention(32, 4, 3).to(DEV)
    x2 = torch.randn(1, 8, 32, device=DEV, requires_grad=True)
    zeros = torch.zeros(1, 8, 2, dtype=torch.long, device=DEV)
    y2 = attn2(x2, path_indices=zeros, path_valid=torch.zeros_like(zeros, dtype=torch.bool))
    assert y2.abs().max().item() == 0
    y2.sum().backward()
    assert x2.grad.abs().max().item() == 0


@pytest.mark.parametrize("masked", [False, True])
def test_sbdattention_module_with_tables_matches_oracle(masked):
    torch.manual_seed(80)
    dim, heads, t, s = 256, 4, 300, 5
    m = sbda_amd.SBDAttention(dim, heads, 6, kv_heads=2, rope_theta=10000.0, total_layers=12)
    with torch.no_grad():
        m.q_norm.weight.mul_(1 + 0.1 * torch.randn(m.head_dim))
        m.k_norm.weight.mul_(1 + 0.1 * torch.randn(m.head_dim))
    x = torch.randn(2, t, dim)
    idx, valid = _tables(2, t, s, seed=81)
    vm, sr = _masks(2, t, seed=82) if masked else (None, None)
    g = torch.randn(2, t, dim)
    md = m.to(DEV)
    xd = x.to(DEV).requires_grad_()
    out = md(xd, None if vm is None else vm.to(DEV), None if sr is None else sr.to(DEV),
             idx.to(DEV), valid.to(DEV))
    out.backward(g.to(DEV))
    torch.cuda.synchronize()
    mc = sbda_amd.SBDAttention(dim, heads, 6, kv_heads=2, rope_theta=10000.0, total_layers=12)
    mc.load_state_dict({k_: v_.cpu() for k_, v_ in md.state_dict().items()})
    xc = x.clone().requires_grad_()
    want = _oracle_module_forward(mc, xc, vm, sr, idx, valid)
    want.backward(g)
    tol = FP32_TOL
    torch.testing.assert_close(out.detach().cpu(), want.detach(), **tol)
    torch.testing.assert_close(xd.grad.cpu(), xc.grad, **tol)
    for (name, p), (_, pc) in zip(md.named_parameters(), mc.named_parameters()):
        scale = pc.grad.abs().max().item() + 1e-6
        err = (p.grad.cpu() - pc.grad).abs().max().item()
        assert err / scale < 1e-5, f"{name}: {err} vs scale {scale}"


def test_backbone_with_tables_and_path_active_matches_oracle():
    # BiAttn/model.py:397-466: per-layer tables; path_active skips a layer for
    # some rows (those rows pass through unchanged).
    torch.manual_seed(61)
    layers, t, s = 3, 200, 4
    cfg = sbda_amd.BiAttnConfig(vocab_size=64, dim=128, layers=layers, heads=2,
                                rope_theta=10000.0, ff_hidden=256)
    m = sbda_amd.BiAttnLM(cfg)
    ids = torch.randint(0, 64, (3, t))
    idx = torch.stack([_tables(3, t, s, seed=90 + l)[0] for l in range(layers)], dim=1)
    valid = torch.stack([_tables(3, t, s, seed=90 + l)[1] for l in range(layers)], dim=1)
    active = torch.tensor([[True, True, True], [True, False, True], [False, False, True]])
    md = m.to(DEV)
    out = md(ids.to(DEV), None, None, idx.to(DEV), valid.to(DEV), active.to(DEV))
    out.float().square().mean().backward()
    torch.cuda.synchronize()
    mc = sbda_amd.BiAttnLM(cfg)
    mc.load_state_dict({k_: v_.cpu() for k_, v_ in md.state_dict().items()})

    def oracle_forward(model):
        x = model.embedding(ids)
        for li, blk in enumerate(model.layers):
            y = x + _oracle_module_forward(blk.attn, blk.norm1(x), None, None,
                                           idx[:, li], valid[:, li])
            y = y + blk.ff(blk.norm2(y))
            x = torch.where(active[:, li, None, None], y, x)
        return model.lm_head(model.norm(x))

    want = oracle_forward(mc)
    want.float().square().mean().backward()
    torch.testing.assert_close(out.detach().cpu(), want.detach(), **FP32_TOL)
    for (name, p), (_, pc) in zip(md.named_parameters(), mc.named_parameters()):
        scale = pc.grad.abs().max().item() + 1e-8
        err = (p.grad.cpu() - pc.grad).abs().max().item()
        assert err / scale < 1e-5, f"{name}: {err} vs scale {scale}"


# ------------------------------------------------------------ block kernels

@pytest.mark.parametrize("dtype,tol", [(torch.float32, FP32_TOL), (torch.bfloat16, LOW_TOL),
                                       (torch.float16, LOW_TOL)])
@pytest.mark.parametrize("dim", [64, 512, 1000, 2048])
def test_fused_add_rms_norm_matches_fp32_reference(dtype, tol, dim):
    if dtype == torch.float32 and dim > 2048:
        pytest.skip("fp32 rows are limited to 8 KiB")
    g = torch.Generator().manual_seed(dim)
    x, r, gs, gy = (torch.randn(3, 129, dim, generator=g).to(dtype) for _ in range(4))
    w = (1 + 0.1 * torch.randn(dim, generator=g)).to(dtype)
    xd, rd, wd = (t.to(DEV).requires_grad_() for t in (x, r, w))
    s, y = sbda_amd.fused_add_rms_norm(xd, rd, wd, 1e-6)
    torch.autograd.backward((s, y), (gs.to(DEV), gy.to(DEV)))
    # The sum is the eager `x + r` bit for bit.
    assert torch.equal(s.detach(), x.to(DEV) + r.to(DEV))
    xc, rc, wc = (t.float().requires_grad_() for t in (x, r, w))
    sc = (xc + rc).to(dtype).float()                   # eager rounding of the sum
    yc = torch.nn.functional.rms_norm(sc, (dim,), wc, 1e-6)
    torch.autograd.backward((sc, yc), (gs.float(), gy.float()))
    torch.testing.assert_close(y.detach().float().cpu(), yc.detach(), **tol)
    torch.testing.assert_close(xd.grad.float().cpu(), xc.grad, **tol)
    torch.testing.assert_close(rd.grad.float().cpu(), rc.grad, **tol)
    scale = wc.grad.abs().max().item()
    assert (wd.grad.float().cpu() - wc.grad).abs().max().item() <= 2e-2 * scale + 1e-3


def test_fused_rms_norm_alone_and_deterministic_weight_grad():
    g = torch.Generator().manual_seed(5)
    x = torch.randn(4000, 512, generator=g).to(torch.bfloat16)
    w = torch.randn(512, generator=g).to(torch.bfloat16)
    gy = torch.randn(4000, 512, generator=g).to(torch.bfloat16)
    grads = []
    for _ in range(2):
        xd, wd = x.to(DEV).requires_grad_(), w.to(DEV).requires_grad_()
        y = sbda_amd.fused_rms_norm(xd, wd)
        y.backward(gy.to(DEV))
        grads.append((y.detach().cpu(), xd.grad.cpu(), wd.grad.cpu()))
    for a, b in zip(*grads):
        assert torch.equal(a, b)
    yc = torch.nn.functional.rms_norm(x.float(), (512,), w.float(), 1e-6)
    torch.testing.assert_close(grads[0][0].float(), yc, **LOW_TOL)


@pytest.mark.parametrize("dtype,tol", [(torch.float32, FP32_TOL), (torch.bfloat16, LOW_TOL)])
@pytest.mark.parametrize("hidden", [64, 200, 2048])
def test_fused_swiglu_matches_fp32_reference(dtype, tol, hidden):
    g = torch.Generator().manual_seed(hidden)
    gu = (2 * torch.randn(5, 77, 2 * hidden, generator=g)).to(dtype)
    dh = torch.randn(5, 77, hidden, generator=g).to(dtype)
    gud = gu.to(DEV).requires_grad_()
    h = sbda_amd.fused_swiglu(gud)
    h.backward(dh.to(DEV))
    guc = gu.float().requires_grad_()
    hc = torch.nn.functional.silu(guc[..., :hidden]) * guc[..., hidden:]
    hc.backward(dh.float())
    torch.testing.assert_close(h.detach().float().cpu(), hc.detach(), **tol)
    torch.testing.assert_close(gud.grad.float().cpu(), guc.grad, **tol)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,dim,hidden,with_bias", [
    (1, 64, 128, True),          # one token: a single, mostly clamped token tile
    (257, 128, 384, False),      # ragged token tail, three hidden tiles, no bias
    (300, 512, 256, True),
    (1000, 2048, 128, True),     # 32 k stages
    (4096, 512, 2048, True),     # the config-5 feed-forward shape (16 x 16 tiles)
])
def test_fused_swiglu_gemm_matches_fp32_reference(dtype, rows, dim, hidden, with_bias):
    g = torch.Generator().manual_seed(rows + dim + hidden)
    x = torch.randn(rows, dim, generator=g).to(dtype)
    w = (torch.randn(2 * hidden, dim, generator=g) / math.sqrt(dim)).to(dtype)
    b = (0.1 * torch.randn(2 * hidden, generator=g)).to(dtype) if with_bias else None
    xd, wd = x.to(DEV), w.to(DEV)
    bd = None if b is None else b.to(DEV)
    assert sbda_amd.swiglu_gemm_supported(xd, wd)
    got = sbda_amd.fused_swiglu_gemm(xd, wd, bd)
    assert got.shape == (rows, hidden) and got.dtype == dtype
    gu = x.float() @ w.float().t()
    if b is not None:
        gu = gu + b.float()
    want = torch.nn.functional.silu(gu[:, :hidden]) * gu[:, hidden:]
    torch.testing.assert_close(got.float().cpu(), want, **LOW_TOL)
    # Against the unfused device path (GEMM rounded to the dtype, then the
    # activation kernel): the same rounding points, so within two units in
    # the last place.
    unfused = sbda_amd.fused_swiglu(torch.nn.functional.linear(xd, wd, bd))
    ulp = 2.0 ** (-7 if dtype == torch.bfloat16 else -10)
    torch.testing.assert_close(got.float(), unfused.float(), rtol=2 * ulp, atol=1e-3)


def test_swiglu_module_uses_the_fused_gemm_without_grad():
    torch.manual_seed(3)
    ff = sbda_amd.model.SwiGLU(512, 4.0, hidden_size=2048).to(device=DEV, dtype=torch.bfloat16)
    x = torch.randn(3, 333, 512, device=DEV).to(torch.bfloat16)
    with torch.no_grad():
        fused = ff(x)
    eager = ff(x.requires_grad_())              # the grad-recording path
    eager.sum().backward()
    assert fused.shape == eager.shape
    torch.testing.assert_close(fused.float(), eager.detach().float(), rtol=2e-2, atol=2e-3)


def test_bf16_backbone_tracks_the_fp32_oracle_composition():
    # The config-5 layer shape (d=512, 8 x 64 heads, FFN 2048) in bf16 on the
    # GPU -- fused QKV GEMM, add+RMSNorm and SwiGLU kernels -- against the same
    # weights in fp32 through the oracle on the CPU.
    torch.manual_seed(62)
    cfg = sbda_amd.BiAttnConfig(vocab_size=256, dim=512, layers=3, heads=8, ff_hidden=2048)
    m = sbda_amd.BiAttnLM(cfg)
    ids = torch.randint(0, 256, (1, 700))
    md = sbda_amd.BiAttnLM(cfg)
    md.load_state_dict(m.state_dict())
    md = md.to(device=DEV, dtype=torch.bfloat16)
    with torch.no_grad():
        got = md.forward_hidden(ids.to(DEV)).float().cpu()
        x = m.embedding(ids)
        for blk in m.layers:
            x = x + _oracle_module_forward(blk.attn, blk.norm1(x))
            x = x + blk.ff(blk.norm2(x))
        want = m.norm(x)
    rel = ((got - want).norm() / want.norm()).item()
    assert rel < 2e-2, rel
