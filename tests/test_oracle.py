"""Pin the CPU oracle before trusting it (CPU only).

Each oracle function is checked against something that does not restate its
own formula: the reference's known answers (``tests/golden/reference_kats.json``),
closed forms, fp64 brute-force loops, fp64 gradcheck, invariants of the maths
(causality, empty rows, relative-position property of RoPE) and special cases
whose answer is exact.  ``test_planted_mistakes_are_caught`` shows that the
checks fail for plausible mistakes planted in a copy of the oracle.
"""

from __future__ import annotations

import json
import math
from pathlib import Path

import pytest
import torch

from oracle import sbda_oracle as ref
from tests.sampled import sampled_oracle

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def _rand(*shape, seed=0, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=torch.float64).to(dtype)


# ---------------------------------------------------------------- schedule

def test_stage_and_slot_counts_match_reference_tests():
    for layer, stage in KATS["sbda_stage"]["cases"]:
        assert ref.sbda_stage(layer) == stage
    kc = KATS["sbda_slot_counts"]
    for layer, count in zip(kc["layers"], kc["counts"]):
        offs = ref.sbda_layer_offsets(layer)
        assert len(offs) == count and offs[0] == 0 and all(o >= 0 for o in offs)
    with pytest.raises(ValueError):
        ref.sbda_layer_offsets(0)
    assert ref.sbda_layer_offsets(1) == (0, 1)
    assert ref.sbda_layer_offsets(2) == (0, 2)
    assert ref.sbda_layer_offsets(3) == (0, 1, 2, 4)
    assert ref.sbda_layer_offsets(20) == (0, 1, 2, 1 << 19)


def test_path_tables_known_answer():
    kat = KATS["binary_path_indices_len8_layer3"]
    idx, valid = ref.path_tables(kat["length"], kat["offsets"])
    assert idx.dtype == torch.int64 and valid.dtype == torch.bool
    assert idx.tolist() == kat["indices"]
    assert valid[:, 1].tolist() == [False] * 4 + [True] * 4


def test_path_tables_exhaustive_small():
    # Bit-exact against a direct definition for every length <= 40 and
    # every SBDA layer whose jump reaches past the end.
    for length in range(1, 41):
        for layer in range(1, 8):
            offs = ref.sbda_layer_offsets(layer)
            idx, valid = ref.path_tables(length, offs)
            for i in range(length):
                for s, o in enumerate(offs):
                    assert bool(valid[i, s]) == (o <= i)
                    assert int(idx[i, s]) == (i - o if o <= i else 0)


def test_graph_statistics_match_recorded_csv():
    for row in KATS["h8_graph_statistics"]["rows"]:
        offs = [ref.sbda_layer_offsets(l) for l in range(1, row["layers"] + 1)]
        n = row["length"]
        assert ref.valid_cell_count(n, offs) == row["total_cells"]
        assert ref.unique_cell_count(n, offs) == row["unique_cells"]
        reach = {0}
        auc = 0
        for o in offs:
            reach = {r + x for r in reach for x in o if r + x < n}
            auc += len(reach)
        assert len(reach) == row["coverage"] and auc == row["coverage_auc"]


def test_edge_count_closed_form_and_masks_agree():
    for layers, expected in KATS["edge_count_closed_form"]["cases"]:
        assert ref.sbda_edge_count_closed_form(1 << layers, layers) == expected
    for layers in range(2, 13):
        n = 1 << layers
        total = sum(int(ref.path_tables(n, ref.sbda_layer_offsets(l))[1].sum())
                    for l in range(1, layers + 1))
        assert total == ref.sbda_edge_count_closed_form(n, layers)
    # The metric shape, through the same masks.
    n, layers = 1 << 20, 20
    total = sum(int(ref.path_tables(n, ref.sbda_layer_offsets(l))[1].sum())
                for l in range(1, layers + 1))
    assert total == KATS["edge_count_closed_form"]["cases"][0][1]


# ------------------------------------------------------------- attention

CASES = [
    # (B, H, Hkv, T, D, offsets)
    (1, 2, 2, 9, 4, (0, 1)),
    (2, 2, 2, 11, 6, (0, 1, 2, 4)),
    (1, 4, 2, 7, 5, (0, 1, 2, 1024)),   # far offset beyond T, GQA
    (1, 2, 1, 6, 3, (0, 3, 3, 1)),      # duplicate slot, unsorted
]


@pytest.mark.parametrize("b,h,hkv,t,d,offs", CASES)
def test_gather_attention_matches_brute_force(b, h, hkv, t, d, offs):
    q = _rand(b, h, t, d, seed=1)
    k = _rand(b, hkv, t, d, seed=2)
    v = _rand(b, hkv, t, d, seed=3)
    want_o, want_lse = ref.brute_force_attention(q, k, v, offs)
    for route in (True, False):
        got = ref.gather_attention(q, k, v, offs, matmul_route=route)
        torch.testing.assert_close(got, want_o, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(ref.attention_lse(q, k, offs), want_lse, rtol=1e-12, atol=1e-12)


def test_matmul_and_elementwise_routes_agree_fp32():
    # Mirrors tests/test_model.py:148-166 (1e-5 in fp32).
    q, k, v = (_rand(2, 4, 17, 8, seed=s, dtype=torch.float32) for s in (4, 5, 6))
    a = ref.gather_attention(q, k, v, (0, 1, 2, 8), matmul_route=True)
    b = ref.gather_attention(q, k, v, (0, 1, 2, 8), matmul_route=False)
    torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-5)


def test_zero_query_gives_exact_mean_of_valid_sources():
    t, d = 12, 4
    offs = (0, 1, 2, 4)
    q = torch.zeros(1, 1, t, d, dtype=torch.float64)
    k = _rand(1, 1, t, d, seed=7)
    pos = torch.arange(t, dtype=torch.float64)
    v = torch.stack([pos, pos * pos, torch.ones(t), -pos], dim=-1)[None, None]
    out = ref.gather_attention(q, k, v, offs)
    lse = ref.attention_lse(q, k, offs)
    for i in range(t):
        srcs = [i - o for o in offs if o <= i]
        n = len(srcs)
        assert out[0, 0, i, 0].item() * n == pytest.approx(sum(srcs), abs=1e-12)
        assert out[0, 0, i, 1].item() * n == pytest.approx(sum(j * j for j in srcs), abs=1e-9)
        assert out[0, 0, i, 2].item() == pytest.approx(1.0, abs=1e-15)
        assert lse[0, 0, i].item() == pytest.approx(math.log(n), abs=1e-15)


def test_first_row_and_dominant_score():
    q = _rand(1, 1, 8, 4, seed=8)
    k = _rand(1, 1, 8, 4, seed=9)
    v = _rand(1, 1, 8, 4, seed=10)
    out = ref.gather_attention(q, k, v, (0, 1))
    assert torch.equal(out[0, 0, 0], v[0, 0, 0])      # only the self source
    k2 = k.clone()
    q2 = torch.zeros_like(q)
    q2[..., 0] = 1e3
    k2[..., 0] = 0
    k2[0, 0, 5, 0] = 1.0                              # source 5 dominates query 6
    out2 = ref.gather_attention(q2, k2, v, (0, 1))
    torch.testing.assert_close(out2[0, 0, 6], v[0, 0, 5], rtol=0, atol=1e-12)


def test_empty_source_rows_have_zero_output_and_gradient():
    # Invariant of tests/test_model.py:34-42: with no valid source, the row's
    # output and every gradient through it are exactly zero.
    q, k, v = (_rand(1, 2, 6, 4, seed=s).requires_grad_() for s in (11, 12, 13))
    out = ref.gather_attention(q, k, v, (1, 2))       # row 0 has no source
    assert out[:, :, 0].abs().max().item() == 0
    out[:, :, 0].sum().backward()
    for x in (q, k, v):
        assert x.grad.abs().max().item() == 0
    assert math.isinf(ref.attention_lse(q.detach(), k.detach(), (1, 2))[0, 0, 0].item())


def test_causality():
    t = 16
    q, k, v = (_rand(1, 2, t, 4, seed=s).requires_grad_() for s in (14, 15, 16))
    offs = (0, 1, 2, 8)
    out = ref.gather_attention(q, k, v, offs)
    k2 = k.detach().clone()
    v2 = v.detach().clone()
    k2[:, :, 9:] += 5
    v2[:, :, 9:] -= 3
    out2 = ref.gather_attention(q.detach(), k2, v2, offs)
    torch.testing.assert_close(out[:, :, :9], out2[:, :, :9], rtol=0, atol=0)
    out[:, :, :9].square().sum().backward()
    assert k.grad[:, :, 9:].abs().max().item() == 0
    assert v.grad[:, :, 9:].abs().max().item() == 0


def test_gradcheck_fp64():
    for offs, hkv in (((0, 1, 2, 4), 2), ((0, 1, 2, 64), 1)):
        q = _rand(1, 2, 7, 3, seed=17).requires_grad_()
        k = _rand(1, hkv, 7, 3, seed=18).requires_grad_()
        v = _rand(1, hkv, 7, 3, seed=19).requires_grad_()
        assert torch.autograd.gradcheck(
            lambda a, b, c: ref.gather_attention(a, b, c, offs), (q, k, v))


@pytest.mark.parametrize("b,h,hkv,t,d,offs", CASES + [(1, 2, 2, 5, 4, (1, 2))])
def test_key_gather_backward_matches_autograd(b, h, hkv, t, d, offs):
    q = _rand(b, h, t, d, seed=20).requires_grad_()
    k = _rand(b, hkv, t, d, seed=21).requires_grad_()
    v = _rand(b, hkv, t, d, seed=22).requires_grad_()
    g = _rand(b, h, t, d, seed=23)
    ref.gather_attention(q, k, v, offs).backward(g)
    dq, dk, dv = ref.key_gather_backward(q.detach(), k.detach(), v.detach(), g, offs)
    for got, want in ((dq, q.grad), (dk, k.grad), (dv, v.grad)):
        torch.testing.assert_close(got, want, rtol=1e-11, atol=1e-12)


# ---------------------------------------------------------------- prologue

def test_head_rmsnorm_closed_form():
    x = _rand(2, 5, 3, 8, seed=24, dtype=torch.float32)
    w = _rand(8, seed=25, dtype=torch.float32)
    got = ref.head_rmsnorm(x, w)
    xd = x.double()
    want = xd / torch.sqrt((xd * xd).sum(-1, keepdim=True) / 8 + 1e-6) * w.double()
    torch.testing.assert_close(got.double(), want, rtol=1e-6, atol=1e-6)
    xb = x.to(torch.bfloat16)
    assert ref.head_rmsnorm(xb, w).dtype == torch.bfloat16


def test_rope_frequencies_and_invariants():
    d, theta = 8, 10000.0
    inv = ref.rope_inverse_frequencies(d, theta)
    want = torch.tensor([theta ** (-2 * i / d) for i in range(d // 2)], dtype=torch.float64)
    torch.testing.assert_close(inv.double(), want, rtol=1e-6, atol=0)
    x = _rand(1, 40, 2, d, seed=26)
    y = ref.apply_rope(x, theta)
    # Position 0 is the identity; each (i, i + D/2) pair keeps its norm.
    torch.testing.assert_close(y[:, 0], x[:, 0], rtol=0, atol=0)
    half = d // 2
    nx = x[..., :half] ** 2 + x[..., half:] ** 2
    ny = y[..., :half] ** 2 + y[..., half:] ** 2
    torch.testing.assert_close(nx, ny, rtol=1e-6, atol=1e-6)
    # Relative-position property: <rope(a)_i, rope(b)_j> depends on i - j
    # only (angles are fp32, so compare at the fp32-angle resolution).
    a = _rand(d, seed=27)
    bb = _rand(d, seed=28)
    qa = ref.apply_rope(a.expand(1, 40, 1, d).contiguous(), theta)[0, :, 0]
    kb = ref.apply_rope(bb.expand(1, 40, 1, d).contiguous(), theta)[0, :, 0]
    for lag in (0, 1, 5):
        dots = [(qa[i] @ kb[i - lag]).item() for i in range(lag, 40)]
        assert max(dots) - min(dots) < 1e-4
    # Odd head_dim: identity.
    xo = _rand(1, 4, 1, 5, seed=29)
    assert torch.equal(ref.apply_rope(xo, theta), xo)


# RoFormer's rotation (Su et al. 2021, eq. 34, half-split pairing): the pair
# (x[d], x[d + D/2]) at position m is multiplied by R(m * theta_d) =
# [[cos, -sin], [sin, cos]].  D = 4, theta = 100: theta_0 = 1, theta_1 = 0.1.
# cos/sin of the angles 1, 3, 0.1, 0.3 written out (not recomputed here).
_C1, _S1 = 0.5403023058681398, 0.8414709848078965
_C3, _S3 = -0.9899924966004454, 0.1411200080598672
_C01, _S01 = 0.9950041652780258, 0.09983341664682815
_C03, _S03 = 0.955336489125606, 0.29552020666133955
ROPE_KAT = {
    # (position, one-hot coordinate): expected output row
    (1, 0): [_C1, 0.0, _S1, 0.0],
    (1, 2): [-_S1, 0.0, _C1, 0.0],
    (3, 0): [_C3, 0.0, _S3, 0.0],
    (3, 2): [-_S3, 0.0, _C3, 0.0],
    (1, 1): [0.0, _C01, 0.0, _S01],
    (1, 3): [0.0, -_S01, 0.0, _C01],
    (3, 1): [0.0, _C03, 0.0, _S03],
    (3, 3): [0.0, -_S03, 0.0, _C03],
}


def _rope_kat_holds() -> bool:
    theta = 100.0
    for (m, coord), want in ROPE_KAT.items():
        x = torch.zeros(1, 4, 1, 4, dtype=torch.float64)
        x[0, :, 0, coord] = 1.0                      # the same one-hot at every position
        y = ref.apply_rope(x, theta)[0, m, 0]
        # fp32 angles and cos/sin (the reference's tables): agree to ~1e-7.
        if not torch.allclose(y, torch.tensor(want, dtype=torch.float64), rtol=0, atol=1e-6):
            return False
    return True


def test_rope_rotation_direction_known_answer():
    assert ref.rope_inverse_frequencies(4, 100.0).tolist() == [1.0, 0.10000000149011612]
    assert _rope_kat_holds()
    # Rows at explicit positions (the sampled-row checks) are the same rows
    # of the whole-sequence rotation, bit for bit.
    x = _rand(2, 50, 3, 8, seed=34, dtype=torch.float32)
    idx = torch.tensor([0, 3, 17, 49, 4])
    full = ref.apply_rope(x, 10000.0)
    torch.testing.assert_close(ref.apply_rope(x[:, idx], 10000.0, positions=idx), full[:, idx],
                               rtol=0, atol=0)


def test_prologue_gradcheck_fp64():
    theta = 10000.0
    q = _rand(1, 6, 2, 4, seed=30).requires_grad_()
    k = _rand(1, 6, 2, 4, seed=31).requires_grad_()
    wq = _rand(4, seed=32).requires_grad_()
    wk = _rand(4, seed=33).requires_grad_()

    def f(a, b, c, e):
        qq, kk = ref.prologue(a, b, c, e, theta)
        return ref.gather_attention(qq.permute(0, 2, 1, 3), kk.permute(0, 2, 1, 3),
                                    kk.permute(0, 2, 1, 3), (0, 1, 2, 4))

    assert torch.autograd.gradcheck(f, (q, k, wq, wk))


# ----------------------------------------------------------- planted bugs

def test_planted_mistakes_are_caught():
    """Plausible slips in a copy of the oracle fail the checks above."""
    t = 9
    q, k, v = (_rand(1, 1, t, 4, seed=s) for s in (40, 41, 42))
    offs = (0, 1, 2, 4)
    want, _ = ref.brute_force_attention(q, k, v, offs)

    orig = ref.path_tables

    def off_by_one_mask(length, offsets):
        idx, _ = orig(length, offsets)
        pos = torch.arange(length)[:, None]
        return idx, pos > torch.tensor(offsets)[None, :]   # '>' instead of '>='

    try:
        ref.path_tables = off_by_one_mask
        bad = ref.gather_attention(q, k, v, offs)
    finally:
        ref.path_tables = orig
    assert not torch.allclose(bad, want, atol=1e-6)

    # A dropped softmax scale or a transposed (k <-> v) operand also differs.
    assert not torch.allclose(ref.gather_attention(q * 8, k, v, offs), want, atol=1e-6)
    assert not torch.allclose(ref.gather_attention(q, v, k, offs), want, atol=1e-6)

    # RoPE turned the other way (rotate_half as cat(x2, -x1): a rotation by
    # -m*theta) keeps every invariant of test_rope_frequencies_and_invariants
    # but fails the known answer.
    orig_rot = ref.rotate_half

    def flipped(x):
        half = x.shape[-1] // 2
        return torch.cat((x[..., half:], -x[..., :half]), dim=-1)

    try:
        ref.rotate_half = flipped
        assert not _rope_kat_holds()
        x = _rand(1, 40, 2, 8, seed=26)
        y = ref.apply_rope(x, 10000.0)
        torch.testing.assert_close(y[:, 0], x[:, 0], rtol=0, atol=0)   # still the identity at 0
    finally:
        ref.rotate_half = orig_rot
    assert _rope_kat_holds()


# ----------------------------------------------------------------- masks

def test_seam_reset_equals_independent_segments():
    # A seam at position s makes [0, s) and [s, T) two independent sequences:
    # the masked attention on the whole equals plain attention on each part.
    t, s_ = 23, 9
    q, k, v = (_rand(1, 2, t, 4, seed=s) for s in (60, 61, 62))
    seam = torch.zeros(1, t, dtype=torch.bool)
    seam[0, 0] = True
    seam[0, s_] = True
    for offs in ((0, 1), (0, 1, 2, 4), (0, 1, 2, 16)):
        got = ref.gather_attention_masked(q, k, v, offs, seam_reset=seam)
        left = ref.gather_attention(q[:, :, :s_], k[:, :, :s_], v[:, :, :s_], offs)
        right = ref.gather_attention(q[:, :, s_:], k[:, :, s_:], v[:, :, s_:], offs)
        torch.testing.assert_close(got, torch.cat((left, right), dim=2), rtol=1e-12, atol=1e-12)


def test_holes_are_skipped_and_prefix_masks_change_nothing():
    t = 17
    offs = (0, 1, 2, 8)
    q, k, v = (_rand(2, 2, t, 4, seed=s) for s in (63, 64, 65))
    prefix = torch.ones(2, t, dtype=torch.bool)
    prefix[1, 12:] = False
    got = ref.gather_attention_masked(q, k, v, offs, valid_mask=prefix)
    plain = ref.gather_attention(q, k, v, offs)
    # Causal sources of a valid query are valid under a prefix mask.
    torch.testing.assert_close(got[1, :, :12], plain[1, :, :12], rtol=0, atol=0)
    torch.testing.assert_close(got[0], plain[0], rtol=0, atol=0)
    holes = torch.ones(1, t, dtype=torch.bool)
    holes[0, 5] = False
    h_out = ref.gather_attention_masked(q[:1], k[:1], v[:1], offs, valid_mask=holes)
    # Brute force: drop source 5 from every query's softmax.
    for i in range(t):
        if not holes[0, i]:
            continue
        srcs = [i - o for o in offs if o <= i and i - o != 5]
        for hh in range(2):
            sc = torch.stack([(q[0, hh, i] * k[0, hh, j]).sum() / 2 for j in srcs])
            w = torch.softmax(sc, 0)
            want = sum(w[n] * v[0, hh, j] for n, j in enumerate(srcs))
            torch.testing.assert_close(h_out[0, hh, i], want, rtol=1e-12, atol=1e-12)


def test_masked_gradcheck_fp64():
    t = 9
    valid = torch.ones(1, t, dtype=torch.bool)
    valid[0, 3] = False
    seam = torch.zeros(1, t, dtype=torch.bool)
    seam[0, 6] = True
    q, k, v = (_rand(1, 2, t, 3, seed=s).requires_grad_() for s in (66, 67, 68))
    assert torch.autograd.gradcheck(
        lambda a, b, c: ref.gather_attention_masked(a, b, c, (0, 1, 2, 4), valid, seam), (q, k, v))


# ------------------------------------------------------------ source tables

def _random_tables(b, t, s, seed):
    g = torch.Generator().manual_seed(seed)
    idx = torch.randint(0, t, (b, t, s), generator=g)
    idx[:, :, 0] = torch.arange(t)                     # self in slot 0
    idx[:, 3, 1] = idx[:, 3, 2] = 1                    # a duplicate source
    valid = torch.rand(b, t, s, generator=g) > 0.2
    return idx, valid


def test_tables_match_brute_force_with_duplicates_and_future_entries():
    b, h, t, d, s = 2, 2, 9, 4, 4
    q, k, v = (_rand(b, h, t, d, seed=70 + i) for i in range(3))
    idx, valid = _random_tables(b, t, s, seed=71)
    got = ref.gather_attention_tables(q, k, v, idx, valid)
    sources = [[[int(idx[bb, i, ss]) for ss in range(s)
                 if bool(valid[bb, i, ss]) and int(idx[bb, i, ss]) <= i]
                for i in range(t)] for bb in range(b)]
    torch.testing.assert_close(got, ref.brute_force_sources(q, k, v, sources),
                               rtol=1e-12, atol=1e-12)


def test_tables_from_offsets_equal_the_offset_route():
    b, h, t, d = 2, 4, 37, 8
    q, k, v = (_rand(b, h, t, d, seed=80 + i) for i in range(3))
    valid_mask = torch.rand(b, t, generator=torch.Generator().manual_seed(81)) > 0.2
    seam = torch.zeros(b, t, dtype=torch.bool)
    seam[1, 20] = True
    for offs in ((0, 1), (0, 1, 2, 8), (0, 1, 2, 64)):
        idx, ok = ref.path_tables(t, offs)
        tab = idx.unsqueeze(0).expand(b, -1, -1).contiguous()
        okb = ok.unsqueeze(0).expand(b, -1, -1).contiguous()
        torch.testing.assert_close(ref.gather_attention_tables(q, k, v, tab, okb),
                                   ref.gather_attention(q, k, v, offs), rtol=0, atol=0)
        torch.testing.assert_close(
            ref.gather_attention_tables(q, k, v, tab, okb, valid_mask, seam),
            ref.gather_attention_masked(q, k, v, offs, valid_mask, seam), rtol=0, atol=0)


def test_tables_reference_known_answers():
    # tests/test_model.py:19-42: slot 1 points at position 7 for every row, so
    # rows before 7 see only themselves; all-invalid tables give zero rows.
    t, d = 8, 4
    q, k, v = (_rand(1, 2, t, d, seed=90 + i) for i in range(3))
    paths = torch.arange(t).view(1, t, 1).expand(1, t, 2).clone()
    paths[:, :, 1] = 7
    out = ref.gather_attention_tables(q, k, v, paths)
    torch.testing.assert_close(out[:, :, :7], v[:, :, :7], rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(out[:, :, 7], v[:, :, 7], rtol=1e-12, atol=1e-12)
    qg = q.clone().requires_grad_()
    none = ref.gather_attention_tables(qg, k, v, paths, torch.zeros_like(paths, dtype=torch.bool))
    assert none.abs().max().item() == 0
    none.sum().backward()
    assert qg.grad.abs().max().item() == 0


def test_duplicate_source_is_a_log2_score_bias():
    # Listing j twice weighs it like one entry with score + log 2.
    b, h, t, d = 1, 1, 6, 4
    q, k, v = (_rand(b, h, t, d, seed=95 + i) for i in range(3))
    i = 5
    idx = torch.tensor([[[r, max(r - 1, 0), max(r - 1, 0)] for r in range(t)]])
    ok = idx <= torch.arange(t)[None, :, None]
    got = ref.gather_attention_tables(q, k, v, idx, ok)[0, 0, i]
    s_self = (q[0, 0, i] @ k[0, 0, i]) / math.sqrt(d)
    s_prev = (q[0, 0, i] @ k[0, 0, i - 1]) / math.sqrt(d) + math.log(2)
    w = torch.softmax(torch.stack([s_self, s_prev]), 0)
    torch.testing.assert_close(got, w[0] * v[0, 0, i] + w[1] * v[0, 0, i - 1],
                               rtol=1e-12, atol=1e-12)


def test_tables_gradcheck_fp64():
    b, h, hkv, t, d, s = 1, 2, 1, 6, 3, 3
    q, k, v = (_rand(b, hh, t, d, seed=99 + i).requires_grad_() for i, hh in enumerate((h, hkv, hkv)))
    idx, valid = _random_tables(b, t, s, seed=98)
    assert torch.autograd.gradcheck(
        lambda a, bb, c: ref.gather_attention_tables(a, bb, c, idx, valid), (q, k, v))


# ------------------------------------------------ sampled-row helper

@pytest.mark.parametrize("offs", [(0, 1), (0, 2), (0, 1, 2, 4), (0, 1, 2, 32), (0, 1, 2, 64)])
@pytest.mark.parametrize("prologue", [False, True])
def test_sampled_oracle_equals_whole_sequence_oracle(offs, prologue):
    """The sampled-row evaluation used by the metric-size GPU tests gives the
    whole-sequence oracle's rows (forward, and autograd's gradients, also
    through the norm + RoPE prologue)."""
    b, t, h, d = 1, 70, 3, 8
    theta = 10000.0
    q, k, v, g = (_rand(b, t, h, d, seed=60 + i, dtype=torch.float32) for i in range(4))
    wq = 1 + 0.1 * _rand(d, seed=64, dtype=torch.float32)
    wk = 1 + 0.1 * _rand(d, seed=65, dtype=torch.float32)
    rq, rk, rv = (x.clone().requires_grad_() for x in (q, k, v))
    qq, kk = ref.prologue(rq, rk, wq, wk, theta) if prologue else (rq, rk)
    out = ref.gather_attention(qq.permute(0, 2, 1, 3), kk.permute(0, 2, 1, 3),
                               rv.permute(0, 2, 1, 3), offs)
    out.backward(g.permute(0, 2, 1, 3))
    rows = torch.tensor([0, 1, 2, 5, 31, 32, 33, 40, 68, 69])

    def fetch(pos):
        a, c = q[0, pos], k[0, pos]
        if prologue:
            a, c = ref.prologue(a[None], c[None], wq, wk, theta, positions=pos)
            a, c = a[0], c[0]
        return a, c, v[0, pos], g[0, pos]

    o_w, dq_w, dk_w, dv_w = sampled_oracle(fetch, offs, rows, t, d)
    if prologue:
        a, c = q[0, rows].clone().requires_grad_(), k[0, rows].clone().requires_grad_()
        aa, cc = ref.prologue(a[None], c[None], wq, wk, theta, positions=rows)
        dq_w, dk_w = torch.autograd.grad((aa[0], cc[0]), (a, c), (dq_w, dk_w))
    want = (out.detach()[0].permute(1, 0, 2)[rows], rq.grad[0, rows], rk.grad[0, rows],
            rv.grad[0, rows])
    for got, w in zip((o_w, dq_w, dk_w, dv_w), want):
        torch.testing.assert_close(got, w, rtol=1e-5, atol=1e-6)
