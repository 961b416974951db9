"""Pins the CPU oracle (oracle/gptq_oracle.py) with closed forms, invariants,
hand-worked examples and brute force, so that a plausible mistake in it (a
dropped term, a wrong sign or index, a transposed operand) fails here.  The
reference ships no golden vectors for this path; these checks stand in."""
import itertools

import numpy as np
import pytest

from oracle import gptq_oracle as O


# ---------------------------------------------------------------- Hessian --

def test_hessian_bruteforce_loops():
    rng = np.random.default_rng(0)
    b1 = rng.standard_normal((2, 3, 4))
    b2 = rng.standard_normal((5, 4))  # 2-D input counts as one sequence
    H, n = O.hessian([b1, b2])
    toks = [b1[i, t] for i in range(2) for t in range(3)] + [b2[t] for t in range(5)]
    Hb = np.zeros((4, 4))
    for x in toks:
        for i in range(4):
            for j in range(4):
                Hb[i, j] += x[i] * x[j]
    assert n == 3
    np.testing.assert_allclose(H, Hb, rtol=1e-12, atol=1e-12)


def test_hessian_invariants():
    rng = np.random.default_rng(1)
    X = rng.standard_normal((3, 17, 6))
    H, n = O.hessian([X])
    assert n == 3
    np.testing.assert_allclose(H, H.T)
    assert np.all(np.linalg.eigvalsh(H) > -1e-9)
    np.testing.assert_allclose(np.trace(H), np.sum(X ** 2))
    H2, _ = O.hessian([X[:1], X[1:]])
    np.testing.assert_allclose(H, H2)
    H3, _ = O.hessian([2.5 * X])
    np.testing.assert_allclose(H3, 6.25 * H)


# ------------------------------------------------------- damping/inverse --

def test_damp_ref_closed_form():
    H = np.array([[4.0, 1.0], [1.0, 8.0]])
    Hd = O.damp_ref(H, 2, 0.5)
    # H/2 = [[2, .5], [.5, 4]], mean diag 3, lambda 1.5
    np.testing.assert_allclose(Hd, [[3.5, 0.5], [0.5, 5.5]])


def _spd(k, seed):
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((4 * k, k))
    X[:, rng.integers(0, k)] *= 20
    return X.T @ X


def test_full_inverse():
    H = O.damp_ref(_spd(12, 2), 3, 0.01)
    Hi = O.full_inverse(H)
    np.testing.assert_allclose(H @ Hi, np.eye(12), atol=1e-9)
    np.testing.assert_allclose(Hi, np.linalg.inv(H), rtol=1e-9, atol=1e-12)


def test_upper_chol_of_inverse():
    H = O.damp_ref(_spd(16, 3), 3, 0.01)
    U = O.upper_chol_of_inverse(H)
    assert np.allclose(np.tril(U, -1), 0)
    assert np.all(np.diag(U) > 0)
    np.testing.assert_allclose(U.T @ U, np.linalg.inv(H), rtol=1e-8, atol=1e-12)
    # textbook route: chol(inv(H)) is lower L with L L^T = inv(H); GPTQ's
    # upper factor satisfies U^T U = inv(H), which is NOT L^T in general.
    # numpy only gives lower factors, so compare with the reversal identity
    # computed independently by scipy's upper Cholesky on the inverse
    import scipy.linalg as sl
    Us = sl.cholesky(np.linalg.inv(H), lower=False)
    np.testing.assert_allclose(U, Us, rtol=1e-7, atol=1e-10)


def test_prepare_canonical_dead_and_scale():
    H = np.diag([4.0, 0.0, 2.0])
    Hd, dead = O.prepare_canonical_H(H, 2, 0.0)
    assert list(dead) == [False, True, False]
    np.testing.assert_allclose(np.diag(Hd), [4.0, 1.0, 2.0])
    Hd2, _ = O.prepare_canonical_H(H, 2, 0.3)
    np.testing.assert_allclose(np.diag(Hd2), np.array([4.0, 1.0, 2.0]) + 0.7)


# -------------------------------------------------------------- quantizers --

def test_ref_params_and_quantize_hand():
    g = np.array([[-1.0, 0.5, 2.0]], dtype=np.float32)
    s, z = O.ref_params(g, 3)
    assert s[0] == 1.0 and z[0] == 1.0
    q = O.ref_quantize(g[0], s[0], z[0], 3)
    # 0.5/1 + 1 = 1.5 -> round half to even -> 2
    assert list(q) == [0.0, 2.0, 3.0]


def test_tie_rounding_differs_between_formulas():
    # reference: round(w/s + z); canonical: round(w/s) + z.  At w/s = 0.5 and
    # odd z these differ: round(1.5) = 2 but round(0.5) + 1 = 1.
    assert O.ref_quantize(np.float64(0.5), 1.0, 1.0, 3) == 2.0
    assert O.canonical_codes(np.float64(0.5), 1.0, 1.0, 3) == 1.0


def test_ref_params_allows_negative_zero_point():
    # all-positive group: the reference does not force 0 into the range
    s, z = O.ref_params(np.array([[2.0, 5.0]]), 3)
    assert s[0] == 1.0 and z[0] == -2.0


def test_canonical_params_hand():
    x = np.array([[1.0, 2.0, 3.0],      # all positive -> xmin forced to 0
                  [0.0, 0.0, 0.0],      # all zero -> [-1, 1]
                  [-3.0, 0.0, 1.5]])
    s, z = O.canonical_params(x, 15)
    np.testing.assert_allclose(s, [3.0 / 15, 2.0 / 15, 4.5 / 15])
    np.testing.assert_allclose(z, [0.0, 8.0, 10.0])  # round(7.5)=8, round(10)=10
    q = O.canonical_codes(x, s[:, None], z[:, None], 15)
    np.testing.assert_array_equal(q[2], [0.0, 10.0, 15.0])


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
def test_codes_cover_range_and_clamp(bits):
    maxq = 2 ** bits - 1
    x = np.linspace(-1.0, 1.0, 4 * (maxq + 1))[None]
    s, z = O.canonical_params(x, maxq)
    q = O.canonical_codes(x, s[:, None], z[:, None], maxq)
    assert q.min() == 0 and q.max() == maxq
    assert set(np.unique(q)) == set(range(maxq + 1))
    qr = O.ref_quantize(x, *[v[:, None] for v in O.ref_params(x, maxq)], maxq)
    assert qr.min() == 0 and qr.max() == maxq


# ------------------------------------------------------ reference sweep --

W_HAND = np.array([[0.4, -1.0, 0.3], [3.0, 2.0, 0.4], [0.0, 0.25, 3.0]])
HINV_HAND = np.array([[2.0, -1.0, 0.5], [-1.0, 4.0, 1.0], [0.5, 1.0, 1.0]])


def test_gptq_ref_hand_worked_propagation():
    """Worked by hand (bits=2, g=3, one block): A = W^T rows
    [0.4,3,0], [-1,2,.25], [.3,.4,3]; row 2's middle weight is rounded to 0 by
    plain RTN but to 1 after the error of column 0 is propagated."""
    r = O.gptq_ref(W_HAND, HINV_HAND, bits=2, group_size=3, blocksize=3)
    np.testing.assert_array_equal(r["codes"], [[0, 0, 0], [3, 3, 1], [0, 1, 3]])
    np.testing.assert_allclose(r["scale"][:, 0], [1.0, 1.0, 0.9])
    np.testing.assert_allclose(r["zero"][:, 0], [0.0, 1.0, 0.0])
    np.testing.assert_allclose(r["total_error"], 0.2553125, rtol=1e-12)


def test_gptq_ref_no_cross_block_update():
    """Same input with blocksize 2: column 2 gets no propagation (the
    reference has no lazy-batch trailing update)."""
    r = O.gptq_ref(W_HAND, HINV_HAND, bits=2, group_size=3, blocksize=2)
    np.testing.assert_array_equal(r["codes"], [[0, 0, 0], [3, 3, 1], [0, 1, 3]])
    np.testing.assert_allclose(r["total_error"], 0.22515625, rtol=1e-12)


def test_gptq_ref_identity_hessian_is_rtn():
    rng = np.random.default_rng(4)
    W = rng.standard_normal((8, 16)) * 0.02
    r = O.gptq_ref(W, np.eye(16) * 0.7, bits=4, group_size=4, blocksize=4)
    A = W.T
    for g in range(2):
        s, z = O.ref_params(A[:, 4 * g:4 * g + 4], 15)
        q = O.ref_quantize(A[:, 4 * g:4 * g + 4], s[:, None], z[:, None], 15)
        np.testing.assert_array_equal(r["codes"].T[:, 4 * g:4 * g + 4], q)


def test_gptq_ref_rejects_wide_layers():
    with pytest.raises(ValueError):
        O.gptq_ref(np.zeros((8, 4)), np.eye(4), 4, 4, 4)


# ------------------------------------------------------ canonical sweep --

def _layer(n, k, seed, toks=64):
    rng = np.random.default_rng(seed)
    W = rng.standard_normal((n, k)) * 0.02
    X = rng.standard_normal((2, toks, k))
    X[..., rng.integers(0, k, 2)] *= 20
    H, ns = O.hessian([X])
    return W, X, H, ns


@pytest.mark.parametrize("bits,gs", [(4, 4), (3, -1), (2, 8), (8, 16)])
def test_canonical_equals_bruteforce_obs(bits, gs):
    W, X, H, ns = _layer(6, 16, 5)
    bs = 4 if gs in (4, -1) else gs  # g a multiple of blocksize (see obs_bruteforce)
    r = O.gptq_canonical(W, H, ns, bits, gs, bs, 0.01)
    Hd, _ = O.prepare_canonical_H(H, ns, 0.01)
    if gs == -1:
        # per-channel params come from the original W in both
        q = O.obs_bruteforce(W, Hd, bits, -1)
    else:
        q = O.obs_bruteforce(W, Hd, bits, gs)
    np.testing.assert_array_equal(r["codes"], q)


def test_canonical_blocksize_invariance():
    W, X, H, ns = _layer(10, 32, 6)
    a = O.gptq_canonical(W, H, ns, 4, 8, 8, 0.01)
    b = O.gptq_canonical(W, H, ns, 4, 8, 32, 0.01)
    # group statistics are taken at the start of the block that holds the
    # group start; with g a multiple of both blocksizes the two agree
    c = O.gptq_canonical(W, H, ns, 4, 32, 32, 0.01)
    d = O.gptq_canonical(W, H, ns, 4, 32, 8, 0.01)
    np.testing.assert_array_equal(c["codes"], d["codes"])
    # with g < blocksize every group of the first block takes its statistics
    # from the weights as they stood at the block start, i.e. the originals
    for g in range(4):
        s, z = O.canonical_params(W[:, 8 * g:8 * g + 8], 15)
        np.testing.assert_allclose(b["scale"][:, g], s, rtol=1e-13)
        np.testing.assert_array_equal(b["zero"][:, g], z)
    # while with g == blocksize the later groups see the propagated weights
    assert not np.allclose(a["scale"][:, 1], b["scale"][:, 1])
    np.testing.assert_allclose(a["scale"][:, 0], b["scale"][:, 0], rtol=1e-13)


def test_canonical_identity_hessian_is_rtn():
    rng = np.random.default_rng(7)
    W = rng.standard_normal((5, 12))
    H = np.eye(12) * 3.0
    r = O.gptq_canonical(W, H, 6, 4, 4, 4, 0.0)
    for g in range(3):
        blk = W[:, 4 * g:4 * g + 4]
        s, z = O.canonical_params(blk, 15)
        np.testing.assert_array_equal(
            r["codes"][:, 4 * g:4 * g + 4],
            O.canonical_codes(blk, s[:, None], z[:, None], 15))


def test_canonical_actorder_is_permuted_run():
    W, X, H, ns = _layer(6, 16, 8)
    r = O.gptq_canonical(W, H, ns, 4, 4, 4, 0.01, actorder=True)
    perm = np.argsort(-np.diag(H), kind="stable")
    rp = O.gptq_canonical(W[:, perm], H[perm][:, perm], ns, 4, 4, 4, 0.01)
    np.testing.assert_array_equal(r["codes"][:, perm], rp["codes"])
    np.testing.assert_array_equal(r["g_idx"][perm], np.arange(16) // 4)
    assert not np.array_equal(perm, np.arange(16))


def test_canonical_dead_column():
    W, X, H, ns = _layer(4, 8, 9)
    H[3, :] = 0
    H[:, 3] = 0
    r = O.gptq_canonical(W, H, ns, 4, -1, 4, 0.01)
    # a dead input is zeroed before quantization
    np.testing.assert_allclose(r["dequant"][:, 3],
                               O.canonical_dequant(r["codes"][:, 3], r["scale"][:, 0],
                                                   r["zero"][:, 0]))
    s, z = r["scale"][:, 0], r["zero"][:, 0]
    np.testing.assert_array_equal(r["codes"][:, 3], O.canonical_codes(0.0 * s, s, z, 15))


def test_layer_error_identity():
    W, X, H, ns = _layer(6, 16, 10)
    r = O.gptq_canonical(W, H, ns, 3, 8, 8, 0.01)
    Xf = X.reshape(-1, 16)
    direct = np.sum((Xf @ W.T - Xf @ r["dequant"].T) ** 2)
    np.testing.assert_allclose(O.layer_error(W, r["dequant"], H), direct, rtol=1e-10)
    # GPTQ beats round-to-nearest on its own objective
    rtn = np.zeros_like(W)
    for g in range(2):
        blk = W[:, 8 * g:8 * g + 8]
        s, z = O.canonical_params(blk, 7)
        rtn[:, 8 * g:8 * g + 8] = O.canonical_dequant(
            O.canonical_codes(blk, s[:, None], z[:, None], 7), s[:, None], z[:, None])
    assert O.layer_error(W, r["dequant"], H) < O.layer_error(W, rtn, H)


# ---------------------------------------------------------------- packing --

@pytest.mark.parametrize("bits", [2, 3, 4, 8])
def test_bitstream_roundtrip_exhaustive(bits):
    vals = np.arange(2 ** bits, dtype=np.uint8)
    K = 32 * max(1, (2 ** bits) // 32)
    codes = np.stack([np.roll(np.resize(vals, K), r) for r in range(5)])
    p = O.pack_bitstream(codes, bits)
    assert p.shape == (5, K * bits // 8)
    np.testing.assert_array_equal(O.unpack_bitstream(p, bits, K), codes)


def test_bitstream_4bit_is_quantizedlinear_layout():
    codes = np.array([[1, 2, 3, 4, 15, 0, 7, 9]], dtype=np.uint8)
    p = O.pack_bitstream(codes, 4)
    # byte = w[:, i] | (w[:, i+1] << 4)   (models/layers.py:87)
    assert list(p[0]) == [0x21, 0x43, 0x0F, 0x97]
    # ... and the dequantizer's low-nibble-first unpack (core/dequantizer.py:86-87)
    np.testing.assert_array_equal(O.ref_unpack_4bit(p), codes)


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_bitstream_words_match_lsb_first_int32(bits):
    epp = 32 // bits
    rng = np.random.default_rng(bits)
    codes = rng.integers(0, 2 ** bits, (3, 4 * epp)).astype(np.uint8)
    words = O.pack_bitstream(codes, bits).view("<u4")
    for r, w in itertools.product(range(3), range(4)):
        expect = 0
        for j in range(epp):  # packed |= val << (j * bits)  (triton_kernels.py:217)
            expect |= int(codes[r, w * epp + j]) << (j * bits)
        assert int(words[r, w]) == expect


def test_bitstream_3bit_word_straddle():
    codes = np.zeros((1, 32), dtype=np.uint8)
    codes[0, 10] = 5   # bits 30..32 = 1,0,1
    codes[0, 21] = 6   # bits 63..65 = 0,1,1
    w = O.pack_bitstream(codes, 3).view("<u4")[0]
    assert int(w[0]) == 1 << 30
    assert int(w[1]) == 1          # bit 32
    assert int(w[2]) == 0b11       # bits 64, 65
    codes[:] = 7
    assert list(O.pack_bitstream(codes, 3).view("<u4")[0]) == [0xFFFFFFFF] * 3


def test_ref_pack_weights_layouts():
    codes = np.array([[1], [2], [3], [4]], dtype=np.uint8)  # (N=4, K=1)
    assert list(O.ref_pack_weights(codes, 4)[0]) == [0x12, 0x34]
    assert list(O.ref_pack_weights(codes, 2)[0]) == [1 * 64 + 2 * 16 + 3 * 4 + 4]
    c8 = np.array([[0], [127], [128], [255]], dtype=np.uint8)
    assert list(O.ref_pack_weights(c8, 8)[0]) == [0, 127, -128, -1]
    c3 = np.array([[5], [7]], dtype=np.uint8)
    p3 = O.ref_pack_weights(c3, 3)
    assert p3.dtype == np.uint8 and list(p3[0]) == [5, 7]


def test_dequant_and_linear_hand():
    codes = np.array([[0, 15, 8, 3]], dtype=np.uint8)
    scales = np.array([[0.5, 2.0]], dtype=np.float16)
    zeros = np.array([[8.0, 1.0]], dtype=np.float16)
    g_idx = np.array([0, 0, 1, 1])
    Wd = O.dequant(codes, scales, zeros, g_idx)
    np.testing.assert_array_equal(Wd, [[-4.0, 3.5, 14.0, 4.0]])
    x = np.array([[1.0, 2.0, 0.5, -1.0]])
    y = O.linear(x, codes, scales, zeros, g_idx, bias=np.array([0.25]))
    np.testing.assert_allclose(y, [[-4.0 + 7.0 + 7.0 - 4.0 + 0.25]])


def test_bitstream_odd_k_lone_nibble():
    # QuantizedLinear.pack_weights: the last, unpaired code of an odd row
    # fills a byte's low nibble alone (models/layers.py:88-89)
    codes = np.array([[3, 9, 12]], dtype=np.uint8)
    p = O.pack_bitstream(codes, 4)
    assert list(p[0]) == [0x93, 0x0C]
    np.testing.assert_array_equal(O.unpack_bitstream(p, 4, 3), codes)
    c3 = np.array([[1, 2, 3, 4, 5, 6, 7]], dtype=np.uint8)  # 21 bits -> 3 bytes
    p3 = O.pack_bitstream(c3, 3)
    assert p3.shape == (1, 3)
    bits = sum(int(v) << (3 * i) for i, v in enumerate(c3[0]))
    assert int.from_bytes(bytes(p3[0]), "little") == bits


# ------------------------------------------------------ sweep replay --

def _replay_case(bits, gs, actorder, seed=0, K=96, N=24):
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((4 * K, K))
    X[:, :2] *= 8
    H = X.T @ X
    W = rng.standard_normal((N, K)) * 0.02
    r = O.gptq_canonical(W, H, 8, bits, gs, 32, 0.01, actorder=actorder)
    return W, H, r


@pytest.mark.parametrize("bits,gs,actorder", [(4, 32, True), (3, 16, False), (8, -1, True), (2, 24, False)])
def test_replay_of_own_trajectory_is_exact(bits, gs, actorder):
    """Replaying the oracle's own codes and parameters gives margin 0 and
    the same parameters (it is the same loop with the decisions forced)."""
    W, H, r = _replay_case(bits, gs, actorder)
    rep = O.gptq_canonical_replay(W, r["U"], r["perm"], np.diag(H) == 0, bits, gs, 32, r["codes"], r["scale"],
                                  r["zero"])
    assert rep["margin"].max() == 0.0
    np.testing.assert_allclose(rep["scale"], r["scale"], rtol=1e-12)
    np.testing.assert_array_equal(rep["zero"], r["zero"])


def test_replay_catches_a_wrong_code_and_a_wrong_update():
    """A code one step off is outside its cell by (distance to the cell),
    and a trajectory computed with a dropped update term (the trailing GEMM
    skipped) is caught at once."""
    W, H, r = _replay_case(4, 32, False, seed=1)
    dead = np.diag(H) == 0
    codes = r["codes"].copy()
    q = codes[5, 40]
    codes[5, 40] = q + 1 if q < 15 else q - 1
    rep = O.gptq_canonical_replay(W, r["U"], r["perm"], dead, 4, 32, 32, codes, r["scale"], r["zero"])
    assert rep["margin"][5, 40] > 0
    assert np.all(np.delete(rep["margin"], 5, axis=0) == 0)
    # decisions of a sweep that skipped the cross-block update (blocksize =
    # cols without trailing work is the same as eager; here: only
    # intra-block propagation, as the reference mode does)
    U = r["U"]
    Wb = W.copy()
    Q = np.zeros_like(Wb)
    s, z = r["scale"], r["zero"]
    for c in range(W.shape[1]):
        if c % 32 == 0:
            blk = Wb[:, c:c + 32].copy()
        j = c % 32
        g = c // 32
        q = np.clip(np.round(blk[:, j] / s[:, g]) + z[:, g], 0, 15)
        Q[:, c] = q
        e = (blk[:, j] - s[:, g] * (q - z[:, g])) / U[c, c]
        blk[:, j:] -= np.outer(e, U[c, c:c - j + 32])
    rep2 = O.gptq_canonical_replay(W, U, None, dead, 4, 32, 32, Q, s, z)
    assert rep2["margin"].max() > 0.05


def test_replay_zero_tie_detector():
    """A group whose -xmin / s is exactly k + 1/2 (a symmetric range at 8
    bits: 255 / 2) is flagged as a tie; an ordinary group is not."""
    W = np.zeros((2, 4))
    W[0] = [-0.5, 0.5, 0.25, -0.25]          # xmin = -xmax -> -xmin / s = 127.5
    W[1] = [-0.3, 0.6, 0.1, 0.2]             # -xmin / s = 85: half a step from a tie
    U = np.eye(4)
    r = O.gptq_canonical(W, np.eye(4) * 10, 2, 8, -1, 4, 0.0, U=U)
    rep = O.gptq_canonical_replay(W, U, None, None, 8, -1, 4, r["codes"], r["scale"], r["zero"])
    assert rep["zero_margin"][0, 0] == 0.0 and rep["zero_margin"][1, 0] > 0.01
    assert rep["margin"].max() == 0.0
