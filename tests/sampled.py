"""Oracle values at sampled positions of a long sequence (test helper).

At the metric length (T = 2**20) the whole oracle does not fit a test's time,
so the GPU tests check sampled rows: ``sampled_oracle`` evaluates the
oracle's maths (``oracle/sbda_oracle.py``: scores, masked softmax, the
gather-form gradients of ``key_gather_backward``) on only the rows the
sampled outputs depend on.  ``tests/test_oracle.py`` pins it against the
whole-sequence oracle and autograd on small inputs.
"""

from __future__ import annotations

import math

import torch


def sampled_oracle(fetch, offs, rows, t, d):
    """Oracle out, dq, dk, dv ([n, H, D] each) at positions ``rows`` (sorted
    1-D int64), evaluated on only the rows they depend on: the queries
    ``rows`` and ``rows + o_s`` and those queries' sources.
    ``fetch(positions) -> (q, k, v, g)``: fp32 CPU ``[m, H, D]`` rows at those
    positions (after the prologue where it is fused)."""
    offs_t = torch.tensor(offs, dtype=torch.int64)
    scale = d ** -0.5
    qpos = torch.cat([rows, (rows[:, None] + offs_t[None, :]).reshape(-1)])
    qpos = qpos[qpos < t].unique()
    src = qpos[:, None] - offs_t[None, :]                         # [n, S]
    ok = src >= 0
    need = torch.cat([qpos, src.clamp_min(0).reshape(-1)]).unique()
    qq, kk, vv, gg = fetch(need)
    qi = torch.searchsorted(need, qpos)
    si = torch.searchsorted(need, src.clamp_min(0))
    ks, vs = kk[si], vv[si]                                        # [n, S, H, D]
    sc = (qq[qi][:, None] * ks).sum(-1) * scale                    # [n, S, H]
    sc = sc.masked_fill(~ok[:, :, None], -math.inf)
    p = torch.softmax(sc, dim=1)
    dp = (gg[qi][:, None] * vs).sum(-1) * ok[:, :, None]
    ds = p * (dp - (p * dp).sum(1, keepdim=True))
    ri = torch.searchsorted(qpos, rows)
    out = (p[..., None] * vs).sum(1)[ri]
    dq = scale * (ds[..., None] * ks).sum(1)[ri]
    dk = torch.zeros_like(out)
    dv = torch.zeros_like(out)
    for s_, o_s in enumerate(offs):
        i = rows + o_s
        live = (i < t)[:, None, None]
        ii = torch.searchsorted(qpos, i.clamp(max=t - 1))
        dk += torch.where(live, scale * ds[ii, s_][..., None] * qq[qi[ii]], 0.0)
        dv += torch.where(live, p[ii, s_][..., None] * gg[qi[ii]], 0.0)
    return out, dq, dk, dv
