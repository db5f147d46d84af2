"""Pins for the CPU oracle itself (no GPU).

Each check is chosen so a plausible oracle mistake (wrong rounding direction,
dropped zero-point, transposed operand, division instead of reciprocal-multiply)
fails it: torch's independent fp8 casts, exact midpoints, closed forms,
brute-force loops, integer special cases, and the reference's own
test_quant.cu case with its +-1 acceptance criterion.
"""
import os

import numpy as np
import pytest
import torch

import oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# ---------------------------------------------------------------- fp8 codec
@pytest.mark.parametrize("fmt,tdt", [(O.E4M3, torch.float8_e4m3fn), (O.E5M2, torch.float8_e5m2)])
def test_fp8_decode_matches_torch_all_codes(fmt, tdt):
    c = np.arange(256, dtype=np.uint8)
    ours = O.fp8_decode(c, fmt)
    theirs = torch.from_numpy(c).view(tdt).float().numpy()
    assert np.array_equal(np.isnan(ours), np.isnan(theirs))
    fin = ~np.isnan(ours)
    assert np.array_equal(ours[fin], theirs[fin])


@pytest.mark.parametrize("fmt", [O.E4M3, O.E5M2])
def test_fp8_roundtrip_every_finite_code(fmt):
    c = np.arange(256, dtype=np.uint8)
    d = O.fp8_decode(c, fmt)
    fin = np.isfinite(d)
    assert np.array_equal(O.fp8_encode(d[fin], fmt), c[fin])


@pytest.mark.parametrize("fmt,tdt", [(O.E4M3, torch.float8_e4m3fn), (O.E5M2, torch.float8_e5m2)])
def test_fp8_midpoints_round_half_even(fmt, tdt):
    # Exact midpoints between consecutive positive finite values: RNE picks the
    # code with an even mantissa LSB. Checked against the rule and torch.
    c = np.arange(0, 0x7F, dtype=np.uint8)
    d = O.fp8_decode(c, fmt).astype(np.float64)
    fin = np.isfinite(d)
    c, d = c[fin], d[fin]
    mids = ((d[:-1] + d[1:]) / 2).astype(np.float32)
    assert np.array_equal(mids.astype(np.float64), (d[:-1] + d[1:]) / 2)  # exact in fp32
    enc = O.fp8_encode(mids, fmt)
    even = np.where(c[:-1] % 2 == 0, c[:-1], c[1:])
    assert np.array_equal(enc, even)
    assert np.array_equal(enc, torch.from_numpy(mids).to(tdt).view(torch.uint8).numpy())
    # and just either side of each midpoint rounds to the nearer code
    lo = np.nextafter(mids, np.float32(0))
    hi = np.nextafter(mids, np.float32(np.inf))
    assert np.array_equal(O.fp8_encode(lo, fmt), c[:-1])
    assert np.array_equal(O.fp8_encode(hi, fmt), c[1:])


@pytest.mark.parametrize("fmt,tdt,fmax", [(O.E4M3, torch.float8_e4m3fn, 448.0),
                                          (O.E5M2, torch.float8_e5m2, 57344.0)])
def test_fp8_random_in_range_matches_torch(fmt, tdt, fmax):
    rng = np.random.default_rng(1)
    x = np.concatenate([
        rng.standard_normal(200_000) * fmax / 3,
        rng.standard_normal(50_000) * 1e-2,
        rng.standard_normal(50_000) * 1e-5,
    ]).astype(np.float32)
    x = np.clip(x, -fmax, fmax)
    ours = O.fp8_encode(x, fmt)
    theirs = torch.from_numpy(x).to(tdt).view(torch.uint8).numpy()
    assert np.array_equal(ours, theirs)


def test_fp8_saturation_and_nan():
    big = np.array([448.5, 463.9, 464.0, 1e6, np.inf], np.float32)
    assert np.array_equal(O.fp8_encode(big, O.E4M3), np.full(5, 0x7E, np.uint8))
    assert np.array_equal(O.fp8_encode(-big, O.E4M3), np.full(5, 0xFE, np.uint8))
    big5 = np.array([57345.0, 61439.0, 61440.0, 1e9, np.inf], np.float32)
    assert np.array_equal(O.fp8_encode(big5, O.E5M2), np.full(5, 0x7B, np.uint8))
    assert O.fp8_encode(np.array([np.nan], np.float32), O.E4M3)[0] == 0x7F
    assert O.fp8_encode(np.array([-0.0], np.float32), O.E4M3)[0] == 0x80


# ------------------------------------------------------------- quantizers
def _np_scale(amax, qmax):
    return np.maximum(np.float32(amax) / np.float32(qmax), np.float32(1e-12)).astype(np.float32)


def test_int8_ties_and_extremes():
    # amax = 127 -> scale exactly 1, inv exactly 1: codes are rint(x), half-even
    x = np.array([[127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -127.0, 126.5]], np.float32)
    q, s = O.quant_row(x, O.INT8)
    assert s[0] == np.float32(1.0)
    assert q.view(np.int8).tolist() == [[127, 0, 2, 2, 0, -2, -127, 126]]


def test_all_zero_row_scale_floor():
    q, s = O.quant_row(np.zeros((2, 10), np.float32), O.INT8)
    assert np.all(s == np.float32(1e-12)) and np.all(q == 0)
    q, s = O.quant_group(np.zeros((1, 300), np.float32), 128, O.E4M3)
    assert np.all(s == np.float32(1e-12)) and np.all(q == 0)


def test_amax_maps_to_qmax():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((16, 256)).astype(np.float32)
    q, s = O.quant_row(x, O.E4M3)
    arg = np.abs(x).argmax(axis=1)
    codes = q[np.arange(16), arg]
    assert np.all((codes & 0x7F) == 0x7E)  # +-448
    q8, _ = O.quant_row(x, O.INT8)
    assert np.all(np.abs(q8.view(np.int8)[np.arange(16), arg].astype(int)) == 127)


def test_reference_int8_case_xorshift():
    # kernels/tests/test_quant.cu:34-139 on the same generated inputs: scales
    # match max(amax/127, eps) and codes are within +-1 of rint(x / scale)
    # (the reference's own acceptance), and exactly equal to the reciprocal-
    # multiply form the reference kernel uses (quant_int8.cu:44).
    x = O.xorshift32_uniform(6 * 130, 11, -5.0, 5.0).reshape(6, 130)
    for dt in ("f32", "f16", "bf16"):
        xs = O.round_to(x, dt)
        q, s = O.quant_row(xs, O.INT8)
        exp_s = _np_scale(np.abs(xs).max(axis=1), 127.0)
        assert np.array_equal(s, exp_s)
        div = np.clip(np.rint(xs / exp_s[:, None]), -127, 127)
        assert np.abs(q.view(np.int8) - div).max() <= 1
        inv = (np.float32(1.0) / exp_s).astype(np.float32)
        mul = np.rint(np.clip((xs * inv[:, None]).astype(np.float32), -127, 127))
        assert np.array_equal(q.view(np.int8).astype(np.float32), mul)
        qt, st = O.quant_tensor(xs, O.INT8)
        assert st[0] == _np_scale(np.abs(xs).max(), 127.0)


def test_fp8_group_closed_form_numpy():
    rng = np.random.default_rng(4)
    x = O.round_bf16(rng.standard_normal((5, 200)).astype(np.float32) * 3)
    q, s = O.quant_group(x, 64, O.E4M3)
    for g in range(4):
        blk = x[:, g * 64:(g + 1) * 64]
        sc = _np_scale(np.abs(blk).max(axis=1), 448.0)
        assert np.array_equal(s[:, g], sc)
        inv = (np.float32(1.0) / sc).astype(np.float32)
        expect = torch.from_numpy((blk * inv[:, None]).astype(np.float32)).to(
            torch.float8_e4m3fn).view(torch.uint8).numpy()
        assert np.array_equal(q[:, g * 64:(g + 1) * 64], expect)


def test_golden_fixtures_regenerate_identically():
    import importlib.util
    spec = importlib.util.spec_from_file_location("mg", os.path.join(GOLDEN, "make_golden.py"))
    mg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mg)
    for name, fn in mg.FIXTURES.items():
        fresh = fn()
        saved = np.load(os.path.join(GOLDEN, name + ".npz"))
        assert set(saved.files) == set(fresh)
        for key in saved.files:
            assert np.array_equal(saved[key], fresh[key]), (name, key)


# ----------------------------------------------------------- int4 formats
def test_repack_brute_force():
    rng = np.random.default_rng(6)
    k, n = 24, 5
    codes = rng.integers(0, 16, (k, n), dtype=np.uint8)
    words = O.pack_k8_int32(codes)
    for kk in range(k):  # the int32 layout: nibble kk % 8 of word kk // 8
        for c in range(n):
            assert (int(words.view(np.uint32)[kk // 8, c]) >> (4 * (kk % 8))) & 0xF == codes[kk, c]
    out = O.repack_int4(words)
    for kp in range(k // 2):
        for c in range(n):
            assert out[kp, c] == (codes[2 * kp, c] | (codes[2 * kp + 1, c] << 4))
    assert np.array_equal(O.unpack_k2_uint8(out), codes)
    perm = rng.permutation(k).astype(np.int32)
    assert np.array_equal(O.unpack_k2_uint8(O.repack_int4(words, perm)), codes[perm])


def test_dequant_int4_closed_form():
    rng = np.random.default_rng(8)
    k, n, gs = 32, 6, 16
    codes = rng.integers(0, 16, (k, n), dtype=np.uint8)
    s = rng.uniform(0.01, 0.1, (k // gs, n)).astype(np.float32)
    z = rng.integers(6, 10, (k // gs, n)).astype(np.float32)
    out = O.dequant_int4(O.pack_k8_int32(codes), s, z, gs)
    g = np.arange(k) // gs
    assert np.array_equal(out, ((codes.astype(np.float32) - z[g]) * s[g]).astype(np.float32))


# ------------------------------------------------------------------ GEMMs
def test_w4a16_integer_special_case_exact():
    # z = 8, s = 1 and small integer activations: the product is an exact
    # integer matmul of (q - 8); the oracle must reproduce it exactly.
    rng = np.random.default_rng(10)
    m, k, n, gs = 4, 128, 24, 32
    a = rng.integers(-3, 4, (m, k)).astype(np.float32)
    codes = rng.integers(0, 16, (k, n), dtype=np.uint8)
    s = np.ones((k // gs, n), np.float32)
    z = np.full((k // gs, n), 8.0, np.float32)
    exact = a.astype(np.int64) @ (codes.astype(np.int64) - 8)
    b = O.pack_k2_uint8(codes)
    assert np.array_equal(O.w4a16_scalar(a, b, s, z, gs), exact.astype(np.float32))
    assert np.array_equal(O.w4a16_ref(a, b, s, z, gs), exact.astype(np.float32))
    # zeros = None means zero-point 0
    assert np.array_equal(O.w4a16_scalar(a, b, s, None, gs),
                          (a.astype(np.int64) @ codes.astype(np.int64)).astype(np.float32))


def test_w4a16_scalar_vs_bench_reference():
    f = np.load(os.path.join(GOLDEN, "w4a16_small.npz"))
    ref = O.w4a16_ref(f["a"], f["b_packed"], f["scales"], f["zeros"], int(f["gs"]),
                      bias=f["bias"])
    assert O.rel_err(f["c_f32"], ref) < 1e-2
    # a zero-point error of one code unit would move the result far more
    ref_bad = O.w4a16_ref(f["a"], f["b_packed"], f["scales"], f["zeros"] + 1, int(f["gs"]),
                          bias=f["bias"])
    assert O.rel_err(f["c_f32"], ref_bad) > 5e-2


def test_fp8_blockwise_integer_special_case_exact():
    rng = np.random.default_rng(12)
    m, n, k = 9, 20, 70
    a_int = rng.integers(-8, 9, (m, k)).astype(np.float32)  # exactly representable
    b_int = rng.integers(-8, 9, (k, n)).astype(np.float32)
    a8, b8 = O.fp8_encode(a_int), O.fp8_encode(b_int)
    ones_a = np.ones((m, -(-k // 32)), np.float32)
    ones_b = np.ones((-(-k // 32), -(-n // 16)), np.float32)
    exact = (a_int.astype(np.int64) @ b_int.astype(np.int64)).astype(np.float32)
    assert np.array_equal(O.fp8_blockwise_scalar(a8, b8, ones_a, ones_b, 16, 32), exact)
    assert np.array_equal(O.fp8_blockwise_ref(a8, b8, ones_a, ones_b, 16, 32), exact)


def test_fp8_blockwise_scalar_vs_dequant_reference():
    f = np.load(os.path.join(GOLDEN, "fp8_blockwise_small.npz"))
    bn, bk = int(f["bn"]), int(f["bk"])
    ref = O.fp8_blockwise_ref(f["a8"], f["b8"], f["a_scale"], f["b_scale"], bn, bk)
    assert O.rel_err(f["c_f32"], ref) < 1e-5
    # transposing the weight-scale grid must be caught
    bad = O.fp8_blockwise_ref(f["a8"], f["b8"], f["a_scale"], f["b_scale"][:, ::-1].copy(), bn, bk)
    assert O.rel_err(f["c_f32"], bad) > 1e-2


def test_fp8_gemm_integer_special_case_exact():
    # gemm_fp8.cu with unit scales and integer-valued e4m3 operands is an exact
    # integer matmul (every partial sum is an integer below 2^24).
    rng = np.random.default_rng(21)
    m, n, k = 6, 11, 90
    a_int = rng.integers(-8, 9, (m, k)).astype(np.float32)
    b_int = rng.integers(-8, 9, (k, n)).astype(np.float32)
    a8, b8 = O.fp8_encode(a_int), O.fp8_encode(b_int)
    exact = (a_int.astype(np.int64) @ b_int.astype(np.int64)).astype(np.float32)
    for per_tok, per_ch in ((True, True), (False, False), (True, False)):
        sa = np.ones(m if per_tok else 1, np.float32)
        sb = np.ones(n if per_ch else 1, np.float32)
        assert np.array_equal(O.fp8_gemm_scalar(a8, b8, sa, sb, per_tok, per_ch), exact)
        assert np.array_equal(O.fp8_gemm_ref(a8, b8, sa, sb, per_tok, per_ch), exact)


def test_fp8_gemm_scales_and_modes():
    rng = np.random.default_rng(22)
    m, n, k = 5, 7, 64
    a8 = O.fp8_encode(rng.standard_normal((m, k)).astype(np.float32) * 4)
    b8 = O.fp8_encode(rng.standard_normal((k, n)).astype(np.float32) * 4)
    sa = rng.uniform(0.01, 0.1, m).astype(np.float32)
    sb = rng.uniform(0.01, 0.1, n).astype(np.float32)
    acc = O.fp8_gemm_scalar(a8, b8, np.ones(m, np.float32), np.ones(n, np.float32))
    # (acc * a_s) * b_s, left to right in fp32 (gemm_fp8.cu:154)
    exp = (acc * sa[:, None]).astype(np.float32) * sb[None, :]
    assert np.array_equal(O.fp8_gemm_scalar(a8, b8, sa, sb), exp.astype(np.float32))
    # per-tensor modes read element 0 only
    pt = O.fp8_gemm_scalar(a8, b8, sa, sb, False, False)
    assert np.array_equal(pt, ((acc * sa[0]).astype(np.float32) * sb[0]).astype(np.float32))
    # closed form agrees with the scalar order to fp32 rounding; swapping the
    # roles of the scales is caught
    assert O.rel_err(O.fp8_gemm_scalar(a8, b8, sa, sb), O.fp8_gemm_ref(a8, b8, sa, sb)) < 1e-5
    assert O.rel_err(O.fp8_gemm_scalar(a8, b8, sa, sb),
                     O.fp8_gemm_ref(a8, b8, sa[::-1].copy(), sb, True, True)) > 1e-2


def test_w8a8_accumulators_three_ways():
    rng = np.random.default_rng(14)
    a = rng.integers(-127, 128, (7, 50)).astype(np.int8)
    b = rng.integers(-127, 128, (50, 9)).astype(np.int8)
    brute = [[sum(int(a[i, t]) * int(b[t, j]) for t in range(50)) for j in range(9)]
             for i in range(7)]
    assert O.w8a8_acc_scalar(a, b).tolist() == brute
    assert O.w8a8_acc(a, b).tolist() == brute


def test_w8a8_epilogue_order():
    acc = np.array([[3, -5]], np.int32)
    a_s = np.array([0.1], np.float32)
    b_s = np.array([0.3, 0.7], np.float32)
    out = O.w8a8_epilogue(acc, a_s, b_s)
    exp = ((acc.astype(np.float32) * a_s[0]).astype(np.float32) * b_s).astype(np.float32)
    assert np.array_equal(out, exp)


def test_moe_topk_brute_force_and_ties():
    """moe_gate.cu:88-105: k largest logits, the lowest expert id wins a tie."""
    rng = np.random.default_rng(5)
    lg = rng.standard_normal((40, 16)).astype(np.float32)
    lg[0, [3, 7, 9]] = 5.0          # three-way tie at the top
    lg[1, :] = 1.0                  # everything tied
    ids = O.moe_topk_ids(lg, 4)
    assert list(ids[0][:3]) == [3, 7, 9]
    assert list(ids[1]) == [0, 1, 2, 3]
    for t in range(lg.shape[0]):
        best = sorted(range(16), key=lambda e: (-float(lg[t, e]), e))[:4]
        assert list(ids[t]) == best


def test_moe_group_rows_invariants():
    rng = np.random.default_rng(6)
    ids = O.moe_topk_ids(rng.standard_normal((33, 8)).astype(np.float32), 3)
    for pad in (1, 4, 16):
        src, offs = O.moe_group_rows(ids, 8, pad)
        assert offs[0] == 0 and offs[-1] == len(src) and np.all(np.diff(offs) % pad == 0)
        live = src[src >= 0]
        assert sorted(live.tolist()) == list(range(ids.size))   # each (token, slot) once
        flat = ids.reshape(-1)
        for e in range(8):
            blk = src[offs[e]:offs[e + 1]]
            assert np.all(flat[blk[blk >= 0]] == e)
            assert np.all(np.diff(blk[blk >= 0]) > 0)           # fixed (token, slot) order


def test_moe_ref_reduces_to_dense():
    """Identical experts make the grouped GEMM one dense W4A16 GEMM; each expert
    slice must equal the dense reference on that slice."""
    rng = np.random.default_rng(7)
    E, K, N, gs = 4, 64, 32, 32
    codes = rng.integers(0, 16, (K, N))
    b = O.pack_k2_uint8(codes)
    s = O.round_bf16(rng.uniform(0.002, 0.02, (K // gs, N)).astype(np.float32))
    z = np.full((K // gs, N), 8.0, np.float32)
    a = O.round_bf16(rng.standard_normal((20, K)).astype(np.float32))
    offs = np.array([0, 5, 5, 12, 20], np.int32)
    out = O.moe_w4a16_ref(a, np.stack([b] * E), np.stack([s] * E), np.stack([z] * E), offs, gs)
    dense = a @ O.w4a16_dequant_weight(b, s, z, gs)
    np.testing.assert_array_equal(out, dense)
    codes2 = rng.integers(0, 16, (E, K, N))
    b2 = np.stack([O.pack_k2_uint8(c) for c in codes2])
    out2 = O.moe_w4a16_ref(a, b2, np.stack([s] * E), None, offs, gs)
    for e in range(E):
        r0, r1 = offs[e], offs[e + 1]
        ref = a[r0:r1] @ O.w4a16_dequant_weight(b2[e], s, None, gs)
        np.testing.assert_array_equal(out2[r0:r1], ref)


def test_gate_softmax_ref_brute_force_and_ties():
    rng = np.random.default_rng(21)
    lg = rng.standard_normal((30, 16)).astype(np.float32)
    lg[0, [2, 5, 11]] = 4.0
    lg[1, :] = 0.5
    w, idx = O.gate_softmax_topk_ref(lg, 4, renormalize=True)
    assert list(idx[0][:3]) == [2, 5, 11] and list(idx[1]) == [0, 1, 2, 3]
    np.testing.assert_allclose(w.sum(1), 1.0, rtol=1e-6)
    w2, idx2 = O.gate_softmax_topk_ref(lg, 4, renormalize=False)
    assert np.array_equal(idx, idx2)
    for t in range(lg.shape[0]):
        p = np.exp(lg[t].astype(np.float64) - lg[t].max())
        p /= p.sum()
        best = sorted(range(16), key=lambda e: (-float(np.float32(p[e])), e))[:4]
        assert list(idx2[t]) == best
        np.testing.assert_allclose(w2[t], p[best], rtol=1e-6)


def _grouped_topk_vectorized(lg, bias, n_group, topk_group, top_k, rsf):
    """Independent formulation (sorting instead of scans) for cross-checking."""
    T, E = lg.shape
    epg = E // n_group
    score = 1.0 / (1.0 + np.exp(-lg.astype(np.float64)))
    sel = score + (0 if bias is None else bias.astype(np.float64))
    out_w, out_i = [], []
    for t in range(T):
        g = sel[t].reshape(n_group, epg)
        top2 = np.sort(g, axis=1)[:, ::-1][:, :2].sum(1) if epg >= 2 else g[:, 0]
        groups = sorted(range(n_group), key=lambda j: (-top2[j], j))[:topk_group]
        cand = [e for e in range(E) if e // epg in groups]
        pick = sorted(cand, key=lambda e: (-sel[t, e], e))[:top_k]
        ww = score[t, pick]
        out_w.append(ww / ww.sum() * rsf)
        out_i.append(pick)
    return np.array(out_w), np.array(out_i)


@pytest.mark.parametrize("E,ng,tg,k,bias", [(32, 4, 2, 4, True), (64, 8, 3, 6, False),
                                            (16, 1, 1, 5, True), (24, 24, 6, 3, False)])
def test_gate_sigmoid_group_ref_two_ways(E, ng, tg, k, bias):
    rng = np.random.default_rng(E + k)
    lg = rng.standard_normal((12, E)).astype(np.float32)
    b = rng.uniform(-0.3, 0.3, E).astype(np.float32) if bias else None
    w, idx = O.gate_sigmoid_group_topk_ref(lg, b, ng, tg, k, True, 2.5)
    w2, idx2 = _grouped_topk_vectorized(lg, b, ng, tg, k, 2.5)
    assert np.array_equal(idx, idx2)
    np.testing.assert_allclose(w, w2, rtol=1e-5)


def test_permutation_ref_matches_grouping_and_drops_invalid():
    rng = np.random.default_rng(22)
    ids = O.moe_topk_ids(rng.standard_normal((40, 12)).astype(np.float32), 3)
    srt, offs = O.compute_permutation_ref(ids, 12)
    row_src, offs2 = O.moe_group_rows(ids, 12, 1)
    assert np.array_equal(srt, row_src) and np.array_equal(offs, offs2)
    bad = ids.copy()
    bad[0, 0], bad[5, 2] = -1, 12
    srt, offs = O.compute_permutation_ref(bad, 12)
    assert offs[-1] == ids.size - 2 and 0 not in srt.tolist() and 17 not in srt.tolist()


def test_unpermute_ref_closed_forms():
    rng = np.random.default_rng(23)
    T, k, H = 6, 2, 8
    perm = O.round_bf16(rng.standard_normal((T * k, H)).astype(np.float32))
    ident = np.arange(T * k, dtype=np.int32)
    onehot = np.zeros((T, k), np.float32)
    onehot[:, 1] = 1.0
    out = O.unpermute_ref(perm, ident, onehot, T, k)
    assert np.array_equal(out, perm[1::2])
    x = O.round_bf16(rng.standard_normal((T, H)).astype(np.float32))
    p = O.permute_ref(x, ident, k)
    assert np.array_equal(p[::2], x) and np.array_equal(p[1::2], x)
    half = np.full((T, k), 0.5, np.float32)
    assert np.array_equal(O.unpermute_ref(p, ident, half, T, k), x)


# ---- dense grouped GEMM (moe_grouped_gemm.cu:68-127) ----------------------
def test_grouped_gemm_scalar_integer_case_is_exact():
    """Small integers make every fp32 partial sum exact in any order, so the
    scalar oracle must equal the int64 product of each expert's rows with that
    expert's [K, N] slab (a transposed slab, a wrong expert or a dropped k
    fails; K != N so a transpose cannot pass)."""
    rng = np.random.default_rng(11)
    E, K, N, rows = 5, 24, 17, 40
    a = rng.integers(-4, 5, (rows, K))
    b = rng.integers(-4, 5, (E, K, N))
    offs = np.array([3, 9, 9, 22, 30, 37], np.int32)  # rows 0-2 and 37-39 unrouted
    init = np.full((rows, N), -7.0, np.float32)
    out = O.grouped_gemm_scalar(a.astype(np.float32), b.astype(np.float32), offs, init)
    for e in range(E):
        r0, r1 = offs[e], offs[e + 1]
        np.testing.assert_array_equal(out[r0:r1], (a[r0:r1] @ b[e]).astype(np.float32))
    np.testing.assert_array_equal(out[:3], init[:3])
    np.testing.assert_array_equal(out[37:], init[37:])


def test_grouped_gemm_scalar_is_sequential_fma():
    """One expert, one output: the reference's k-ascending fp32 fma chain,
    checked against math.fsum-free hand evaluation with np.float32 fma via
    float64 (exact for one product plus one fp32 addend, then rounded)."""
    rng = np.random.default_rng(12)
    K = 50
    a = rng.standard_normal((1, K)).astype(np.float32)
    b = rng.standard_normal((1, K, 1)).astype(np.float32)
    acc = np.float32(0.0)
    for kk in range(K):  # fma(x, y, acc): x*y exact in float64, one rounding
        acc = np.float32(np.float64(a[0, kk]) * np.float64(b[0, kk, 0]) + np.float64(acc))
    out = O.grouped_gemm_scalar(a, b, np.array([0, 1], np.int32))
    assert out[0, 0] == acc


def test_grouped_gemm_ref_matches_scalar():
    rng = np.random.default_rng(13)
    E, K, N, rows = 3, 96, 40, 33
    a = rng.standard_normal((rows, K)).astype(np.float32)
    b = rng.standard_normal((E, K, N)).astype(np.float32)
    offs = np.array([0, 10, 10, 33], np.int32)
    s = O.grouped_gemm_scalar(a, b, offs)
    r = O.grouped_gemm_ref(a, b, offs)
    assert O.rel_err(s, r) < 1e-5
    # ranges are clamped to the rows that exist: [-5, 10) is rows 0-9, [10, 4)
    # is empty, [4, 50) is rows 4-32 (it overlaps expert 0 from row 4 on)
    offs2 = np.array([-5, 10, 4, 50], np.int32)
    out2 = O.grouped_gemm_scalar(a, b, offs2)
    np.testing.assert_array_equal(out2[:4], s[:4])
    np.testing.assert_array_equal(out2[4:], O.grouped_gemm_scalar(a[4:], b[2:], np.array([0, 29], np.int32)))
