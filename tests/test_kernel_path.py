"""Kernel selection (na_kernel_path, no GPU needed): which family each
BASELINE configuration and each eligibility boundary dispatches to.  The
lean workgroup kernels take the common problems (rank 3 staging its box a
few layers at a time when it is too large for LDS), varlen problems (when
the caller has checked d * K <= L_b) and additional tokens, forward and
backward; unchecked varlen and over-budget rank-1/2 boxes stay on the
32-query matrix-core kernels; fp32, even kernels and strides on the generic
kernels."""

import torch

from natten_amd._core import hip


def _path(shape_q, hkv, ks, dil, caus, dtype=torch.bfloat16, stride=None, backward=False,
          **kw):
    q = torch.empty(shape_q, dtype=dtype)
    k = torch.empty((*shape_q[:-2], hkv, shape_q[-1]), dtype=dtype)
    st = stride or (1,) * len(ks)
    return hip.kernel_path(q, k, ks, st, dil, caus, backward=backward, **kw)


def test_config2_runs_lean_both_ways():
    for d in ((1, 1), (4, 4)):
        for bwd in (False, True):
            assert _path((4, 56, 56, 4, 32), 4, (7, 7), d, (False, False), backward=bwd) == "lean"


def test_config3_runs_lean_in_depth_slabs():
    # the whole box exceeds the LDS budget; rank 3 stages it layer by layer
    for bwd in (False, True):
        assert _path((1, 16, 32, 32, 8, 64), 8, (3, 7, 7), (1, 1, 1), (True, False, False),
                     backward=bwd) == "lean"


def test_rank2_box_beyond_lds_budget_stays_on_mfma():
    assert _path((1, 64, 64, 2, 128), 2, (31, 31), (1, 1), (False, False)) == "mfma"


def test_config4_runs_lean_both_ways():
    # 1-D varlen GQA, k 63 d 2, 16 additional tokens (the functional entry
    # point checks d * K <= L_b on the host and says so)
    ext = torch.tensor([[4096], [1024]], dtype=torch.int32)
    kw = dict(n_extra=16, sample_extent=ext, dtype=torch.float16)
    for bwd in (False, True):
        assert _path((2, 4096, 16, 64), 4, (63,), (2,), (False,), varlen_clamped=True,
                     backward=bwd, **kw) == "lean"
        assert _path((2, 4096, 16, 64), 4, (63,), (2,), (False,), backward=bwd,
                     **kw) == "mfma"


def test_lean_boundaries():
    base = ((2, 40, 40, 4, 32), 4, (7, 7), (1, 1), (False, False))
    assert _path(*base) == "lean"
    assert _path(*base, dtype=torch.float32) == "generic"       # fp32: vector ALU
    assert _path(*base, stride=(2, 1)) == "generic"             # strided
    assert _path((2, 40, 40, 4, 32), 4, (6, 7), (1, 1), (False, False)) == "generic"  # even K
    assert _path((2, 40, 40, 4, 48), 4, (7, 7), (1, 1), (False, False)) == "generic"  # head_dim 48
    ext = torch.tensor([[40, 40], [20, 30]], dtype=torch.int32)
    for bwd, want in ((False, "lean"), (True, "lean")):
        assert _path(*base, n_extra=3, backward=bwd) == want     # additional tokens
        assert _path(*base, sample_extent=ext, varlen_clamped=True,
                     backward=bwd) == want                       # checked varlen
        assert _path(*base, sample_extent=ext, n_extra=16, varlen_clamped=True,
                     backward=bwd) == want
    assert _path(*base, sample_extent=ext) == "mfma"             # unchecked varlen
    # d * K > L on a non-causal axis (the legacy boundary windows)
    assert _path((2, 40, 12, 4, 32), 4, (7, 7), (1, 2), (False, False)) == "mfma"
    with hip.generic_kernels():
        assert _path(*base) == "generic"
    with hip.no_lean_kernels():
        assert _path(*base) == "mfma"
        assert _path(*base, backward=True) == "mfma"


def test_split_ops_run_lean():
    for d in ((1, 1), (4, 4)):
        assert _path((4, 56, 56, 4, 32), 4, (7, 7), d, (False, False), split=True) == "lean"
    assert _path((1, 16, 32, 32, 8, 64), 8, (3, 7, 7), (1, 1, 1), (True, False, False),
                 split=True) == "lean"
    assert _path((2, 300, 2, 128), 1, (63,), (2,), (False,), split=True) == "lean"
    assert _path((2, 40, 40, 4, 32), 4, (7, 7), (1, 1), (False, False), dtype=torch.float32,
                 split=True) == "generic"
    with hip.no_lean_kernels():
        assert _path((4, 56, 56, 4, 32), 4, (7, 7), (1, 1), (False, False),
                     split=True) == "mfma"


def _plan(shape_q, hkv, ks, dil, caus, dtype=torch.bfloat16, backward=False, **kw):
    q = torch.empty(shape_q, dtype=dtype)
    k = torch.empty((*shape_q[:-2], hkv, shape_q[-1]), dtype=dtype)
    return hip.kernel_plan(q, k, ks, (1,) * len(ks), dil, caus, backward=backward, **kw)


def test_plans_of_the_benchmarked_configs():
    """The launch shapes the benchmark lines time: config 3 stages its key
    box in several depth slabs both ways; config 4 at its full size groups
    the four query heads of a key/value head in the forward and reduces the
    additional tokens' gradients on matrix cores; config 2 stages its box
    whole."""
    for bwd in (False, True):
        p3 = _plan((1, 16, 32, 32, 8, 64), 8, (3, 7, 7), (1, 1, 1), (True, False, False),
                   backward=bwd)
        assert p3["path"] == "lean" and p3["slabs"] > 1, p3
        assert p3["lds_bytes"] <= 160 * 1024
        p2 = _plan((4, 56, 56, 4, 32), 4, (7, 7), (1, 1), (False, False), backward=bwd)
        assert p2["path"] == "lean" and p2["slabs"] == 1 and not p2["grouped_heads"], p2
        # the backward in seven-wave workgroups (14 x 8 queries: 448 of them,
        # at most 14 waves on a CU), the forward in four-wave ones (784)
        assert (p2["waves"], p2["workgroups"]) == ((7, 448) if bwd else (4, 784)), p2
    ext = torch.full((8, 1), 1024, dtype=torch.int32)
    kw = dict(n_extra=16, sample_extent=ext, dtype=torch.float16, varlen_clamped=True)
    f4 = _plan((8, 4096, 16, 64), 4, (63,), (2,), (False,), **kw)
    assert f4["path"] == "lean" and f4["grouped_heads"], f4
    b4 = _plan((8, 4096, 16, 64), 4, (63,), (2,), (False,), backward=True, **kw)
    assert b4["path"] == "lean" and b4["extra_reduction"] == "matrix", b4
    # a small varlen launch keeps one query head per workgroup
    small = _plan((3, 300, 8, 64), 2, (63,), (2,), (False,),
                  **dict(kw, sample_extent=torch.full((3, 1), 300, dtype=torch.int32)))
    assert small["path"] == "lean" and not small["grouped_heads"], small


def _box_need(L, K, d, t, inverse):
    """Largest box over the tiles [t0, t0 + t) (t0 = 0, t, 2t, ..) of every
    dilation phase of a sample of L points, by enumeration of the window
    rules: forward, the keys of the tile's queries; inverse, the queries
    whose windows hold the tile's keys (non-causal axis)."""
    nh = K // 2
    best = 0
    for r in range(min(d, L)):
        Lr = (L - 1 - r) // d + 1
        for t0 in range(0, Lr, t):
            t1 = min(t0 + t, Lr) - 1
            if inverse:
                lo = 0 if t0 <= K - 1 else t0 - nh
                hi = Lr if t1 >= Lr - K else t1 + nh + 1
            else:
                lo = min(max(t0 - nh, 0), Lr - K)
                hi = min(max(t1 - nh, 0), Lr - K) + K
            best = max(best, hi - lo)
    return best


def test_varlen_backward_box_covers_every_sample_length():
    """With per-sample extents the staged box is planned for any sample
    length the caller may pass (d K <= L_b <= L): it must hold the forward
    and inverse boxes of every tile of every such length."""
    for L, K, d, H in ((4096, 63, 2, 16), (700, 15, 1, 4), (900, 31, 3, 8)):
        ext = torch.full((2, 1), L, dtype=torch.int32)
        kw = dict(sample_extent=ext, dtype=torch.float16, varlen_clamped=True)
        p = _plan((2, L, H, 64), H // 4 if H >= 4 else 1, (K,), (d,), (False,),
                  backward=True, **kw)
        assert p["path"] == "lean", p
        t = p["tile"][2] * p["waves"]
        need = max(max(_box_need(Lb, K, d, t, True), _box_need(Lb, K, d, t, False))
                   for Lb in range(d * K, L + 1, 7 if L > 1000 else 1))
        assert p["box"][2] >= need, (L, K, d, p, need)


# ---- allin1 kernel families (na_rpb_kernel_plan, host only) ----

def _rpb_plan(B, L, H, D, K, d, dtype=None, heads_first=False):
    import ctypes

    from natten_amd._core import _lib

    lib = _lib.load()
    p = _lib.make_rpb_params(1, B, H, D, (L,), K, d, heads_first,
                             _lib.NA_F32 if dtype is None else dtype, 0.288)
    plan = _lib.NaRpbPlan()
    assert lib.na_rpb_kernel_plan(ctypes.byref(p), ctypes.byref(plan)) == 0
    return {f: getattr(plan, f) for f, _ in plan._fields_}


def test_config5_allin1_kernels():
    """Config 5 ([8, 2048, 12, 12] fp32): the staged rank-1 kernels for
    every K x d except K = 5 and 7 at d = 8, whose contiguous halos are too
    wide and which run phase-major; the dq pass (staged or phase-major)
    forms the bias partials; the backward's pairs run phase-major where
    the dilated span is wide."""
    from natten_amd._core import _lib

    for K in (3, 5, 7):
        for d in (1, 2, 4, 8):
            pl = _rpb_plan(8, 2048, 12, 12, K, d)
            want = _lib.RPB_PHASE if (K >= 5 and d == 8) else _lib.RPB_STAGED
            assert pl["qk"] == want and pl["av"] == want, (K, d, pl)
            assert pl["fused_bias"], (K, d, pl)  # staged or phase-major dq pass
            # the backward's phase-major pairs (dq with dk, dattn with dv)
            # where K >= 5 and (K - 1) d >= 12
            qk_pair = av_pair = d > 1 and K >= 5 and (K - 1) * d >= 12
            assert pl["dq"] == (_lib.RPB_PHASE if qk_pair else want), (K, d, pl)
            assert pl["dk"] == (_lib.RPB_PHASE if qk_pair else _lib.RPB_STAGED), (K, d, pl)
            assert pl["dattn"] == (_lib.RPB_PHASE if av_pair else want), (K, d, pl)
            assert pl["dv"] == (_lib.RPB_PHASE if av_pair else _lib.RPB_STAGED), (K, d, pl)


def test_allin1_low_precision_takes_generic_kernels():
    from natten_amd._core import _lib

    for dt in (_lib.NA_BF16, _lib.NA_F16):
        pl = _rpb_plan(2, 203, 12, 12, 5, 2, dtype=dt)
        assert all(pl[f] == _lib.RPB_GENERIC for f in ("qk", "av", "dq", "dk", "dattn", "dv"))
        assert pl["fused_bias"] == 0


def test_allin1_32bit_offset_limit():
    """The rank-1 kernels index with 32-bit integers: a problem whose rows
    times max(K, head_dim) reach 2^31 takes the generic kernels (64-bit row
    offsets); one just below keeps the staged kernels."""
    from natten_amd._core import _lib

    big = _rpb_plan(1, 15_000_000, 12, 12, 7, 1)        # 180M rows x 12 >= 2^31
    assert all(big[f] == _lib.RPB_GENERIC for f in ("qk", "av", "dq", "dk", "dattn", "dv"))
    assert big["fused_bias"] == 0
    ok = _rpb_plan(1, 10_000_000, 12, 12, 7, 1)         # 120M rows x 12 < 2^31
    assert ok["qk"] == _lib.RPB_STAGED and ok["dk"] == _lib.RPB_STAGED
    # the phase-major kernels obey the same limit
    assert _rpb_plan(1, 15_000_000, 12, 12, 7, 8)["qk"] == _lib.RPB_GENERIC


def test_plan_cache_returns_the_computed_plans():
    """The host planner caches its launch choice per problem (a few per
    thread): plans of more problems than the cache holds, asked for in
    interleaved order, equal the plans computed first, forward and
    backward, and two problems that differ only in batch or key/value
    heads get their own plans."""
    probs = [((b, 56, 56, 4, 32), 4, (7, 7), (d, d), (False, False))
             for b in (1, 2, 4) for d in (1, 2, 4)]
    probs += [((2, 300, 8, 64), 2, (9,), (2,), (False,)),
              ((1, 16, 32, 32, 8, 64), 8, (3, 7, 7), (1, 1, 1), (True, False, False)),
              ((8, 4096, 16, 64), 4, (63,), (2,), (False,))]
    first = {}
    for rep in range(3):
        order = probs if rep % 2 == 0 else probs[::-1]
        for pr in order:
            for bwd in (False, True):
                got = _plan(*pr, backward=bwd)
                key = (pr, bwd)
                if key in first:
                    assert got == first[key], (pr, bwd)
                else:
                    first[key] = got
    # batch and kv heads enter the backward's rank-2 wave rule
    a = _plan((4, 56, 56, 4, 32), 4, (7, 7), (1, 1), (False, False), backward=True)
    b = _plan((1, 56, 56, 4, 32), 4, (7, 7), (1, 1), (False, False), backward=True)
    assert a["workgroups"] != b["workgroups"]
