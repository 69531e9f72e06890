"""Host-side checks that need no GPU: the C ABI library loads and exports
exactly what ``include/sbda_amd.h`` declares, argument validation maps to the
reference's error classes, the schedule matches the reference's known answers
and the module mirrors the reference's constructor/parameter surface."""

from __future__ import annotations

import ctypes
import json
import re
from pathlib import Path

import pytest
import torch

import sbda_amd
from sbda_amd import _lib
from oracle import sbda_oracle as ref

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "sbda_amd.h"
KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def _declared_functions() -> set[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(sbda_[a-z_0-9]+)\s*\(", text))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    declared = _declared_functions()
    assert declared == set(_lib.SIGNATURES), "binding and header disagree"
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.sbda_abi_version() == _lib.ABI_VERSION


def _shape_call(lib, **kw):
    args = dict(batch=1, heads=2, kv_heads=2, length=8, head_dim=64, dtype=0,
                offsets=(0, 1, 2, 4))
    args.update(kw)
    offs = args["offsets"]
    return lib.sbda_backward_prologue_workspace(
        args["batch"], args["heads"], args["kv_heads"], args["length"], args["head_dim"],
        args["dtype"], _lib.offsets_array(offs), len(offs), None)


def test_validation_errors_without_launching():
    lib = _lib.load()
    assert _shape_call(lib) > 0
    assert _shape_call(lib, dtype=7) == -_lib.ERR_DTYPE
    assert "dtype" in lib.sbda_last_error().decode()
    assert _shape_call(lib, head_dim=12) == -_lib.ERR_VALUE       # 24 bytes per row
    assert _shape_call(lib, heads=3, kv_heads=2) == -_lib.ERR_VALUE
    assert _shape_call(lib, offsets=(0, -1)) == -_lib.ERR_VALUE
    assert _shape_call(lib, offsets=(0, 1, 2, 3, 4)) == -_lib.ERR_VALUE
    assert _shape_call(lib, length=0) == -_lib.ERR_VALUE
    # A null tensor is rejected before anything is launched.
    z = ctypes.c_void_p(0)
    st = (ctypes.c_int64 * 4)(0, 0, 0, 1)
    rc = lib.sbda_forward(z, st, z, st, z, st, z, st, z, 1, 1, 1, 8, 64, 0,
                          _lib.offsets_array((0, 1)), 2, z, z)
    assert rc == _lib.ERR_VALUE and "null" in lib.sbda_last_error().decode()
    with pytest.raises(ValueError):
        _lib.check(_lib.ERR_VALUE)
    with pytest.raises(TypeError):
        _lib.check(_lib.ERR_DTYPE)


def test_python_op_rejects_cpu_tensors_like_the_reference():
    q = torch.zeros(1, 2, 8, 64)
    with pytest.raises(RuntimeError):
        sbda_amd.fused_sbda_key_backward(q, q, q, torch.tensor([0, 1], dtype=torch.int32))


def test_segment_keys_encode_the_reference_masks():
    valid = torch.tensor([[True, True, False, True, True], [True, True, True, True, True]])
    seam = torch.tensor([[False, False, False, True, False], [False, True, False, False, True]])
    assert sbda_amd.segment_keys(None, None) is None
    assert sbda_amd.segment_keys(valid, None).tolist() == [[0, 0, -1, 0, 0], [0] * 5]
    assert sbda_amd.segment_keys(None, seam).tolist() == [[0, 0, 0, 1, 1], [0, 1, 1, 1, 2]]
    keys = sbda_amd.segment_keys(valid, seam)
    assert keys.dtype == torch.int32 and keys.is_contiguous()
    assert keys.tolist() == [[0, 0, -1, 1, 1], [0, 1, 1, 1, 2]]
    # The key test "key[j] == key[i] >= 0" is the oracle's source-valid table
    # for every valid query row (padded rows differ only in the forced slot 0).
    offs = (0, 1, 2, 4)
    idx, ok = ref.masked_source_valid(5, offs, valid, seam)
    in_range = torch.tensor([[i - o >= 0 for o in offs] for i in range(5)])
    for b in range(2):
        for i in range(5):
            if not valid[b, i]:
                continue
            for s in range(4):
                mine = bool(in_range[i, s]) and keys[b, i] >= 0 and \
                    keys[b, int(idx[i, s])] == keys[b, i]
                assert mine == bool(ok[b, i, s]), (b, i, s)


def test_host_offsets_cache():
    t = torch.tensor([0, 1, 2, 8], dtype=torch.int32)
    assert sbda_amd.host_offsets(t) == (0, 1, 2, 8)
    t[3] = 16                                   # bumps the version counter
    assert sbda_amd.host_offsets(t) == (0, 1, 2, 16)
    assert sbda_amd.host_offsets([0, 2]) == (0, 2)
    with torch.inference_mode():                # no version counter: read each time
        u = torch.tensor([0, 1, 2, 4], dtype=torch.int32)
        assert sbda_amd.host_offsets(u) == (0, 1, 2, 4)
        u[3] = 32
        assert sbda_amd.host_offsets(u) == (0, 1, 2, 32)


def test_backward_workspace_queries():
    # Host-only calls.  Position-major [B,T,H,D] strides: the walk kernels
    # need no workspace without the prologue; a row span past 4 GiB (64 heads
    # x 64 x bf16 at T = 2^20) sends the call to the generic kernels, which
    # need their weight table; the stride-less queries bound every case.
    lib = _lib.load()
    offs = _lib.offsets_array((0, 1, 2, 4096))

    def strides(t, h, d):          # [1,T,H,D] memory seen as [1,H,T,D]
        return (ctypes.c_int64 * 4)(t * h * d, d, h * d, 1)

    def exact(pro, t, h, d):
        s = strides(t, h, d)
        return lib.sbda_backward_workspace_for(pro, *([s] * 7), 1, h, h, t, d, 0, offs, 4, None)

    t = 1 << 20
    assert exact(0, t, 8, 64) == 0
    big = exact(0, t, 64, 64)
    assert big == t * 64 * 2 * 4 * 4                          # fp32 (p, dS) per row and slot
    assert lib.sbda_backward_workspace(1, 64, 64, t, 64, 0, offs, 4, None) >= big
    assert lib.sbda_backward_workspace(1, 8, 8, t, 64, 0, offs, 4, None) >= exact(0, t, 8, 64)
    for h in (8, 64):
        assert 0 < exact(1, t, h, 64) <= lib.sbda_backward_prologue_workspace(1, h, h, t, 64, 0,
                                                                               offs, 4, None)
    bad = lib.sbda_backward_workspace_for(0, *([strides(t, 8, 64)] * 7), 1, 8, 8, t, 64, 7, offs,
                                          4, None)
    assert bad < 0                                            # unknown dtype code


def test_outputs_keep_the_inputs_position_major_layout():
    # Outputs and gradients are allocated dense in the input's stride order:
    # [B,T,H,D] memory seen as [B,H,T,D] (the reference's empty_like(q)), a
    # q sliced out of a fused [B,T,3,H,D] projection, and a plain [B,H,T,D].
    S = sbda_amd.sbda
    x = torch.randn(2, 5, 3, 4)                                  # [B,T,H,D]
    views = [x.permute(0, 2, 1, 3),
             torch.randn(2, 5, 3, 3, 4)[:, :, 0].permute(0, 2, 1, 3),
             torch.randn(2, 3, 5, 4)]
    for v in views:
        out = S._dense_like(v)
        assert out.shape == v.shape
        order = sorted(range(4), key=lambda i: -v.stride(i))
        assert sorted(range(4), key=lambda i: -out.stride(i)) == order
        assert out.is_contiguous() or out.permute(order).is_contiguous()
    lse = S._lse_storage(2, 3, 5, "cpu")
    assert lse.shape == (2, 3, 5) and lse.permute(0, 2, 1).is_contiguous()


def test_topology_matches_oracle_and_reference_statistics():
    for layer in range(1, 24):
        assert sbda_amd.topology_offsets(layer, topology="sbda") == ref.sbda_layer_offsets(layer)
        assert sbda_amd.sbda_stage(layer) == ref.sbda_stage(layer)
    stats = KATS["route_graph_statistics"]
    for name, length, layers, cov, auc, total, unique in stats["rows"]:
        offs = [sbda_amd.topology_offsets(l, topology=name, total_layers=layers)
                for l in range(1, layers + 1)]
        assert ref.valid_cell_count(length, offs) == total, name
        assert ref.unique_cell_count(length, offs) == unique, name
        reach, area = {0}, 0
        for o in offs:
            reach = {r + x for r in reach for x in o if r + x < length}
            area += len(reach)
        assert (len(reach), area) == (cov, auc), name
    with pytest.raises(ValueError):
        sbda_amd.topology_offsets(0, topology="sbda")
    with pytest.raises(ValueError):
        sbda_amd.topology_offsets(1, topology="nope")


def test_module_surface_matches_reference():
    m = sbda_amd.SBDAttention(64, 4, 3, kv_heads=2)
    assert sorted(m.state_dict()) == sorted(
        ["q.weight", "k.weight", "v.weight", "q_norm.weight", "k_norm.weight", "out.weight"])
    assert m.topology == "sbda" and m.backward_mode == "key"
    assert m._fused_offsets.tolist() == [0, 1, 2, 4]
    assert m._fused_offsets.dtype == torch.int32
    with pytest.raises(ValueError):
        sbda_amd.SBDAttention(30, 4, 1)
    with pytest.raises(ValueError):
        sbda_amd.SBDAttention(32, 4, 0)
    with pytest.raises(ValueError):
        sbda_amd.BinaryPathAttention(32, 4, 1, backward_mode="other")
    with pytest.raises(ValueError):
        sbda_amd.SBDAttention(32, 4, 1, kv_heads=3)
    x = torch.randn(1, 5, 64)
    with pytest.raises(NotImplementedError, match="CPU tensor"):
        m(x)
    with pytest.raises(ValueError):
        m(torch.randn(1, 5, 32))
    assert sbda_amd.SBDAAttention is sbda_amd.SBDAttention


def test_backbone_surface_matches_reference():
    cfg = sbda_amd.BiAttnConfig(vocab_size=32, layers=4, dim=64, heads=4)
    assert cfg.window_schedule() == (2, 4, 8, 16)
    m = sbda_amd.BiAttnLM(cfg)
    assert isinstance(m.layers[0].attn, sbda_amd.SBDAttention)
    assert m.layers[3].attn.offsets == (0, 1, 2, 8)
    assert m.lm_head.weight is m.embedding.weight
    names = {n for n, _ in m.named_parameters()}
    assert "layers.0.attn.q_norm.weight" in names and "layers.0.ff.gate.weight" in names
    assert m.layers[0].ff.hidden_size == 256          # ceil(64 * pi / 64) * 64
    with pytest.raises(ValueError):
        sbda_amd.BiAttnConfig(vocab_size=32, attention_backend="left").validate()
    with pytest.raises(NotImplementedError, match="CPU tensor"):
        m(torch.tensor([[1, 2, 3]]))


def test_swiglu_gemm_validation_without_launching():
    lib = _lib.load()
    ok = lib.sbda_swiglu_gemm_supported
    assert ok(1 << 20, 512, 2048, 0) == 1 and ok(1, 64, 128, 1) == 1
    assert ok(1 << 20, 512, 2048, 2) == 0          # fp32: no MFMA path
    assert ok(100, 96, 128, 0) == 0                # dim not a multiple of 64
    assert ok(100, 512, 200, 0) == 0               # hidden not a multiple of 128
    assert ok(1 << 22, 1024, 128, 0) == 0          # rows * dim reaches 2^31
    z = ctypes.c_void_p(0)
    assert lib.sbda_swiglu_gemm_forward(z, z, None, z, 8, 64, 128, 2, z) == _lib.ERR_DTYPE
    assert lib.sbda_swiglu_gemm_forward(z, z, None, z, 8, 64, 128, 0, z) == _lib.ERR_VALUE
    assert "null" in lib.sbda_last_error().decode()
    with pytest.raises(ValueError):
        sbda_amd.fused_swiglu_gemm(torch.zeros(4, 64, dtype=torch.bfloat16),
                                   torch.zeros(256, 64, dtype=torch.bfloat16))
    assert not sbda_amd.swiglu_gemm_supported(torch.zeros(4, 64), torch.zeros(256, 64))


def test_stacked_rows_cache_matches_cat_and_its_gradient():
    from sbda_amd._weights import StackedRows

    g = torch.Generator().manual_seed(3)
    a = torch.randn(4, 6, generator=g, requires_grad=True)
    b = torch.randn(2, 6, generator=g, requires_grad=True)
    rows = StackedRows()
    x = torch.randn(5, 6, generator=g)
    w = rows(a, b)
    assert torch.equal(w, torch.cat((a, b)))
    up = torch.randn(5, 6, generator=g)
    (x @ w.T).mul(up[:, :6]).sum().backward()
    ga, gb = a.grad.clone(), b.grad.clone()
    a.grad = b.grad = None
    (x @ torch.cat((a, b)).T).mul(up[:, :6]).sum().backward()
    assert torch.allclose(ga, a.grad) and torch.allclose(gb, b.grad)
    # Served from the cache until a parameter changes in place.
    first = rows._buf
    before = torch.cat((a, b)).detach().clone()
    rows(a, b)
    assert rows._buf is first
    with torch.no_grad():
        a.add_(1.0)
    w2 = rows(a, b)
    assert rows._buf is not first and torch.equal(w2, torch.cat((a, b)))
    # The earlier output keeps its values (the cache is rebuilt, not overwritten).
    assert torch.equal(w.detach(), before)
    with torch.no_grad():
        assert not rows(a, b).requires_grad
