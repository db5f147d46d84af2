"""GPU parity: MoE routing (ks_moe_gate_*, ks_moe_compute_permutation,
ks_moe_permute, ks_moe_unpermute) against the oracle restatements of
kernels/src/moe/moe_gate.cu and moe_permute.cu.

Bars: expert ids exact (ties go to the lowest id); routing weights within
rtol 1e-5 (the exponential is the device's, not bit-reproducible on the host);
the permutation exact (it is deterministic here: pair ids increase inside each
expert); permute exact; unpermute bit-exact in fp32 (one fused multiply-add per
slot in increasing k) and after rounding to bf16/f16.
"""
import numpy as np
import pytest
import torch

import kernel_set as ks
import oracle as O
from tests import helpers as H

pytestmark = pytest.mark.gpu


def softmax_gate(lg, k, renorm, dt):
    t = H.to_dev(lg, dt)[0]
    T, E = lg.shape
    w = torch.empty(T, k, device="cuda", dtype=torch.float32)
    i = torch.empty(T, k, device="cuda", dtype=torch.int32)
    ks.moe.gate_softmax_topk(w, i, t, T, E, k, renorm)
    torch.cuda.synchronize()
    return w.cpu().numpy(), i.cpu().numpy()


@pytest.mark.parametrize("E,k", [(8, 2), (64, 8), (256, 8), (1000, 32), (1024, 6)])
@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_gate_softmax_topk(E, k, dt):
    rng = np.random.default_rng(E + k)
    lg = rng.standard_normal((77, E)).astype(np.float32) * 2
    lg = O.round_to(lg, dt)
    for renorm in (True, False):
        w, i = softmax_gate(lg, k, renorm, dt)
        rw, ri = O.gate_softmax_topk_ref(lg, k, renorm)
        assert np.array_equal(i, ri)
        np.testing.assert_allclose(w, rw, rtol=1e-5, atol=1e-7)


def test_gate_softmax_ties_and_f16():
    lg = np.zeros((3, 64), np.float32)
    lg[0, [7, 3, 40]] = 1.0
    lg[2, 10:20] = -2.0
    w, i = softmax_gate(lg, 5, True, "f16")
    rw, ri = O.gate_softmax_topk_ref(lg, 5, True)
    assert np.array_equal(i, ri) and list(i[0][:3]) == [3, 7, 40] and list(i[1]) == [0, 1, 2, 3, 4]
    np.testing.assert_allclose(w, rw, rtol=1e-5)


@pytest.mark.parametrize("E,ng,tg,k,bias,rsf", [(256, 8, 4, 8, True, 2.5), (256, 8, 4, 8, False, 1.0),
                                                (64, 4, 1, 3, True, 1.0), (96, 32, 7, 12, True, 0.5),
                                                (20, 20, 20, 20, False, 1.0)])
def test_gate_sigmoid_group_topk(E, ng, tg, k, bias, rsf):
    rng = np.random.default_rng(E + ng + k)
    T = 53
    lg = rng.standard_normal((T, E)).astype(np.float32)
    b = rng.uniform(-0.5, 0.5, E).astype(np.float32) if bias else None
    w = torch.empty(T, k, device="cuda", dtype=torch.float32)
    i = torch.empty(T, k, device="cuda", dtype=torch.int32)
    ks.moe.gate_sigmoid_group_topk(w, i, H.to_dev(lg, "f32")[0], T, E, ng, tg, k,
                                   None if b is None else H.to_dev(b, "f32")[0], True, rsf)
    torch.cuda.synchronize()
    rw, ri = O.gate_sigmoid_group_topk_ref(lg, b, ng, tg, k, True, rsf)
    assert np.array_equal(i.cpu().numpy(), ri)
    np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=1e-5, atol=1e-7)


def permutation(ids, E):
    T, k = ids.shape
    srt = torch.full((T * k,), -7, device="cuda", dtype=torch.int32)
    offs = torch.empty(E + 1, device="cuda", dtype=torch.int32)
    ks.moe.compute_permutation(srt, offs, H.np_i32_dev(ids), T, E, k)
    torch.cuda.synchronize()
    return srt.cpu().numpy(), offs.cpu().numpy()


@pytest.mark.parametrize("T,E,k", [(1, 4, 1), (256, 64, 8), (3000, 256, 8), (4096, 2048, 4),
                                   (100, 1500, 16)])
def test_compute_permutation(T, E, k):
    rng = np.random.default_rng(T + E)
    ids = O.moe_topk_ids(rng.standard_normal((T, E)).astype(np.float32), k)
    srt, offs = permutation(ids, E)
    rs, ro = O.compute_permutation_ref(ids, E)
    assert np.array_equal(offs, ro) and np.array_equal(srt, rs)


def test_compute_permutation_skewed_and_invalid():
    rng = np.random.default_rng(5)
    ids = rng.integers(0, 3, (500, 6)).astype(np.int32)  # three hot experts of 40
    ids[3, 1], ids[77, 0], ids[499, 5] = -1, 40, 1 << 20
    srt, offs = permutation(ids, 40)
    rs, ro = O.compute_permutation_ref(ids, 40)
    assert np.array_equal(offs, ro)
    assert np.array_equal(srt[:ro[-1]], rs)
    assert np.all(srt[ro[-1]:] == -7)  # slots of dropped pairs are left untouched


@pytest.mark.parametrize("dt,H_", [("bf16", 2048), ("f16", 136), ("f32", 100), ("bf16", 7)])
def test_permute_and_unpermute(dt, H_):
    rng = np.random.default_rng(H_)
    T, E, k = 129, 16, 4
    ids = O.moe_topk_ids(rng.standard_normal((T, E)).astype(np.float32), k)
    srt, _ = O.compute_permutation_ref(ids, E)
    x = O.round_to(rng.standard_normal((T, H_)).astype(np.float32), dt)
    xt = H.to_dev(x, dt)[0]
    perm = torch.empty(T * k, H_, device="cuda", dtype=xt.dtype)
    ks.moe.permute(perm, xt, H.np_i32_dev(srt), T, k, H_)
    torch.cuda.synchronize()
    assert np.array_equal(H.from_dev_f32(perm), O.permute_ref(x, srt, k))
    p = O.round_to(rng.standard_normal((T * k, H_)).astype(np.float32), dt)
    wts = rng.uniform(0, 1, (T, k)).astype(np.float32)
    out = torch.empty(T, H_, device="cuda", dtype=xt.dtype)
    ks.moe.unpermute(out, H.to_dev(p, dt)[0], H.np_i32_dev(srt), H.np_f32_dev(wts), T, k, H_)
    torch.cuda.synchronize()
    ref = O.round_to(O.unpermute_ref(p, srt, wts, T, k), dt)
    assert np.array_equal(H.from_dev_f32(out), ref)


def test_permute_invalid_rows_zero_and_unpermute_skips():
    T, k, H_ = 4, 2, 16
    x = np.arange(T * H_, dtype=np.float32).reshape(T, H_)
    srt = np.array([0, 1, -1, 3, 99, 5, 6, 7], np.int32)
    perm = torch.empty(T * k, H_, device="cuda", dtype=torch.float32)
    ks.moe.permute(perm, H.np_f32_dev(x), H.np_i32_dev(srt), T, k, H_)
    torch.cuda.synchronize()
    assert np.array_equal(perm.cpu().numpy(), O.permute_ref(x, srt, k))
    wts = np.ones((T, k), np.float32)
    out = torch.empty(T, H_, device="cuda", dtype=torch.float32)
    ks.moe.unpermute(out, perm, H.np_i32_dev(srt), H.np_f32_dev(wts), T, k, H_)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(),
                          O.unpermute_ref(perm.cpu().numpy(), srt, wts, T, k))


def test_moe_layer_end_to_end():
    # gate -> permutation -> permute -> grouped W4A16 GEMM -> unpermute, against
    # the same chain composed from the oracle (config 5 shapes, fewer tokens).
    rng = np.random.default_rng(9)
    T, E, k, K, N, gs = 64, 64, 8, 2048, 256, 128
    logits = rng.standard_normal((T, E)).astype(np.float32)
    hidden = O.round_bf16(rng.standard_normal((T, K)).astype(np.float32))
    codes = rng.integers(0, 16, (E, K, N), dtype=np.uint8)
    b = np.stack([O.pack_k2_uint8(codes[e]) for e in range(E)])
    s = O.round_bf16(rng.uniform(0.002, 0.02, (E, K // gs, N)).astype(np.float32))
    z = np.full((E, K // gs, N), 8.0, np.float32)

    w = torch.empty(T, k, device="cuda", dtype=torch.float32)
    i = torch.empty(T, k, device="cuda", dtype=torch.int32)
    ks.moe.gate_softmax_topk(w, i, H.np_f32_dev(logits), T, E, k, True)
    srt = torch.empty(T * k, device="cuda", dtype=torch.int32)
    offs = torch.empty(E + 1, device="cuda", dtype=torch.int32)
    ks.moe.compute_permutation(srt, offs, i, T, E, k)
    xt = H.to_dev(hidden, "bf16")[0]
    perm = torch.empty(T * k, K, device="cuda", dtype=torch.bfloat16)
    ks.moe.permute(perm, xt, srt, T, k, K)
    y = torch.empty(T * k, N, device="cuda", dtype=torch.bfloat16)
    ks.moe.grouped_gemm_w4a16(y, perm, H.np_u8_dev(b), H.to_dev(s, "bf16")[0],
                              H.to_dev(z, "bf16")[0], offs, E, T * k, N, K, gs)
    out = torch.empty(T, N, device="cuda", dtype=torch.bfloat16)
    ks.moe.unpermute(out, y, srt, w, T, k, N)
    torch.cuda.synchronize()

    rw, ri = O.gate_softmax_topk_ref(logits, k, True)
    assert np.array_equal(i.cpu().numpy(), ri)
    rs, ro = O.compute_permutation_ref(ri, E)
    rp = O.permute_ref(hidden, rs, k)
    ry = O.moe_w4a16_ref(rp, b, s, z, ro, gs)
    ref = O.unpermute_ref(ry, rs, rw, T, k)
    assert O.rel_err(H.from_dev_f32(out), ref) <= 1e-2
