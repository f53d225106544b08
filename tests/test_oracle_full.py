"""Pins the chunked full-size oracle (oracle/full.py) to the oracle it
restates for large shapes (oracle/na.py, itself pinned by brute force and
finite differences in tests/test_oracle_na.py): outputs, LSE and every
gradient agree to 1e-12 on small problems of each kind, with chunk sizes
that split the query rows unevenly."""

import pytest
import torch

from oracle import full as F
from oracle import na as O


def _r(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float64)


CASES = [
    # (B, spatial, H, Hk, D, ks, dil, caus, st, n_extra)
    (2, (11,), 2, 2, 5, (3,), (2,), (False,), (1,), 0),
    (1, (10,), 4, 1, 4, (4,), (1,), (True,), (2,), 3),
    (1, (6, 7), 2, 2, 3, (3, 3), (1, 2), (False, True), (1, 1), 0),
    (2, (7, 9), 4, 2, 4, (5, 3), (1, 2), (False, False), (1, 1), 5),
    (1, (5, 6), 4, 2, 4, (3, 2), (1, 1), (True, False), (2, 3), 2),
    (1, (4, 5, 6), 2, 1, 3, (3, 3, 3), (1, 1, 2), (True, False, False), (1, 1, 1), 0),
    (1, (3, 4, 5), 2, 2, 3, (2, 3, 3), (1, 1, 1), (True, False, False), (1, 1, 2), 4),
]


def _close(a, b, what):
    torch.testing.assert_close(a, b, rtol=1e-12, atol=1e-12, msg=what)


@pytest.mark.parametrize("chunk", [7, 1024])
@pytest.mark.parametrize("case", CASES)
def test_full_matches_oracle(case, chunk):
    B, sp, H, Hk, D, ks, dil, caus, st, ne = case
    q, k, v = _r((B, *sp, H, D), 1), _r((B, *sp, Hk, D), 2), _r((B, *sp, Hk, D), 3)
    ek = _r((B, ne, Hk, D), 4) if ne else None
    ev = _r((B, ne, Hk, D), 5) if ne else None
    scale = 0.6

    def f(a, b, c, *x):
        return O.na_functional(a, b, c, ks, st, dil, caus, scale, return_lse=True,
                               additional_keys=x[0] if x else None,
                               additional_values=x[1] if x else None)

    out, lse = f(q, k, v, *((ek, ev) if ne else ()))
    go, gl = _r(out.shape, 6), _r(lse.shape, 7)
    ins = (q, k, v) + ((ek, ev) if ne else ())
    ref = O.grads(f, ins, (go, gl))
    res = F.fused(q, k, v, ks, st, dil, caus, scale, go, gl, ek, ev, chunk=chunk)
    _close(res["out"], out, "out")
    _close(res["lse"], lse, "lse")
    names = ["dq", "dk", "dv"] + (["dek", "dev"] if ne else [])
    for n, r in zip(names, ref):
        _close(res[n], r, n)


@pytest.mark.parametrize("chunk", [5, 1024])
def test_full_varlen_matches_oracle(chunk):
    """Per-sample extents: equality with per-sample oracle calls (GQA and
    additional tokens included), zero rows past each sample."""
    B, L, H, Hk, D, ne = 3, 23, 4, 2, 4, 3
    q, k, v = _r((B, L, H, D), 11), _r((B, L, Hk, D), 12), _r((B, L, Hk, D), 13)
    ek, ev = _r((B, ne, Hk, D), 14), _r((B, ne, Hk, D), 15)
    lens = torch.tensor([23, 14, 9])
    go, gl = _r((B, L, H, D), 16), _r((B, L, H), 17)
    res = F.fused(q, k, v, 5, 1, 2, False, None, go, gl, ek, ev, sizes=lens, chunk=chunk)
    for b in range(B):
        n = int(lens[b])
        sl = (slice(b, b + 1), slice(0, n))

        def f(a, c, d, e, g):
            return O.na_functional(a, c, d, 5, 1, 2, False, None, return_lse=True,
                                   additional_keys=e, additional_values=g)

        out, lse = f(q[sl], k[sl], v[sl], ek[b:b + 1], ev[b:b + 1])
        _close(res["out"][sl], out, "out")
        _close(res["lse"][sl], lse, "lse")
        ref = O.grads(f, (q[sl], k[sl], v[sl], ek[b:b + 1], ev[b:b + 1]), (go[sl], gl[sl]))
        for nm, r, s in zip(("dq", "dk", "dv", "dek", "dev"), ref,
                            (sl, sl, sl, slice(b, b + 1), slice(b, b + 1))):
            _close(res[nm][s], r, nm)
        for nm in ("out", "lse", "dq", "dk", "dv"):
            assert (res[nm][b, n:] == 0).all(), nm
    # 2D extents against oracle.na.na_varlen
    q2, k2, v2 = _r((2, 9, 8, 2, 3), 21), _r((2, 9, 8, 2, 3), 22), _r((2, 9, 8, 2, 3), 23)
    sizes = torch.tensor([[9, 8], [6, 7]])
    res2 = F.fused(q2, k2, v2, (3, 5), 1, (2, 1), False, None, sizes=sizes, chunk=chunk)
    _close(res2["out"], O.na_varlen(q2, k2, v2, sizes, (3, 5), (2, 1)), "2d out")
