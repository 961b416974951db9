"""CPU oracle for the GPTQ per-layer quantization hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in ``distributed_gptq_amd`` imports this
module; only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py`` may call it, and there only as the checker (or as the
timed CPU baseline), never as a product code path.

It restates, in numpy, the algorithm of kambojvikram/Distributed_GPTQ for the
hot path, in two modes:

* ``ref`` mode follows ``src/distributed_gptq/core/gptq.py`` as written, with a
  single minimal repair: at ``core/gptq.py:175`` the column ``w`` is (K,) while
  ``scale``/``zero`` are (K,1), so ``w / scale + zero`` broadcasts to (K,K) and
  ``:176`` raises.  The repair treats ``w`` as (K,1).  Everything else is kept:
  transposed orientation (``W = weight.t()``, ``:107-108``), the full inverse
  (``:122``), intra-block rank-1 updates only (``:186-187``), group min/max from
  the original weights (``:162``), ``round(w/s + z)`` (``:175``), codes as output
  (``:194``).
* ``canonical`` mode is GPTQ Algorithm 1 (arXiv:2210.17323) in the form the
  north-star names ``fasterquant`` / ``Quantizer.find_params/quantize`` (names the
  reference lacks): rows = out_features, upper Cholesky factor of H^-1,
  lazy-batch trailing update, group parameters from the current weights at
  the group start, optional act-order permutation.

Every function cites the reference lines it follows.  How each function is
pinned (closed forms, invariants, brute force) is listed in
``PINNING`` at the bottom and exercised by ``tests/test_oracle.py``.
"""
from __future__ import annotations

import numpy as np

# ---------------------------------------------------------------------------
# Hessian accumulation
# ---------------------------------------------------------------------------


def add_batch(H, nsamples, inp, dtype=np.float64):
    """One ``GPTQ.add_batch`` call (core/gptq.py:63-89).

    ``inp`` is (B, T, K) or (T, K); 2-D inputs are unsqueezed (:71-72).
    ``nsamples`` counts leading batch entries, i.e. sequences (:74, :81).
    Returns the updated (H, nsamples) with H = H + X^T X over all tokens
    (:88-89); H is allocated lazily as zeros (:84-85).
    """
    x = np.asarray(inp)
    if x.ndim == 2:
        x = x[None]
    bsz = x.shape[0]
    x = x.reshape(-1, x.shape[-1]).astype(dtype)
    if H is None:
        H = np.zeros((x.shape[1], x.shape[1]), dtype=dtype)
    H = H + x.T @ x
    return H, nsamples + bsz


def hessian(batches, dtype=np.float64):
    """Sum of ``add_batch`` over a list of batches: (H_raw, nsamples)."""
    H, n = None, 0
    for b in batches:
        H, n = add_batch(H, n, b, dtype)
    return H, n


# ---------------------------------------------------------------------------
# Damping and inverses
# ---------------------------------------------------------------------------


def damp_ref(H_raw, nsamples, percdamp):
    """Normalise and damp as ``GPTQ.quantize`` does (core/gptq.py:112-119).

    H <- H / nsamples;  diag(H) += percdamp * mean(diag(H)).
    """
    H = H_raw / nsamples
    lam = percdamp * np.mean(np.diag(H))
    H = H.copy()
    H[np.diag_indices_from(H)] += lam
    return H


def full_inverse(Hd):
    """``cholesky_inverse(cholesky(H))`` (core/gptq.py:122): the full H^-1."""
    L = np.linalg.cholesky(Hd)
    Linv = np.linalg.inv(L)
    return Linv.T @ Linv


def upper_chol_of_inverse(Hd):
    """Upper Cholesky factor U of H^-1 (U^T U = H^-1, U upper, diag > 0).

    Canonical GPTQ computes chol(cholesky_inverse(chol(H)), upper=True).  Here
    it is formed directly: with J the reversal permutation and
    L' = chol(J H J), U = J L'^-1 J.  (H = R R^T with R = J L' J upper, so
    H^-1 = R^-T R^-1 and U = R^-1.)
    """
    J = slice(None, None, -1)
    Lp = np.linalg.cholesky(Hd[J, J])
    Lpinv = np.linalg.inv(Lp)
    return np.ascontiguousarray(np.tril(Lpinv)[J, J])


def prepare_canonical_H(H_raw, nsamples, percdamp):
    """Canonical damping (GPTQ fasterquant):

    H = 2/nsamples * sum x x^T (the canonical running scale; the reference
    stores sum x x^T and divides by nsamples, core/gptq.py:113, so
    H_canonical = 2 * H_ref); dead inputs (H_ii == 0) get H_ii = 1;
    H += percdamp * mean(diag(H)) * I.  Returns (H_damped, dead_mask).
    """
    H = (2.0 / nsamples) * H_raw
    dead = np.diag(H) == 0
    H = H.copy()
    H[dead, dead] = 1.0
    lam = percdamp * np.mean(np.diag(H))
    H[np.diag_indices_from(H)] += lam
    return H, dead


# ---------------------------------------------------------------------------
# Quantizers
# ---------------------------------------------------------------------------


def rne(x):
    """Round half to even, as ``torch.round`` (used at core/gptq.py:169,175)."""
    return np.round(x)


def ref_params(w_group, maxq):
    """Min-max group parameters of the reference (core/gptq.py:165-169).

    s = (max - min) / maxq;  z = round(-min / s).  No forcing of 0 into
    [min, max], exactly as the reference.  One divergence: a constant group
    (max == min) gives s = 0 and the reference then divides by zero
    (non-finite codes); here s = 1 is used instead, in the oracle and the
    GPU kernel alike.
    """
    wmax = w_group.max(axis=1)
    wmin = w_group.min(axis=1)
    dt = w_group.dtype.type
    s = (wmax - wmin) / dt(maxq)
    s = np.where(s == 0, dt(1), s)
    z = rne(-wmin / s)
    return s, z


def ref_quantize(w, s, z, maxq):
    """q = clamp(round(w / s + z), 0, maxq) (core/gptq.py:175)."""
    return np.clip(rne(w / s + z), 0, maxq)


def canonical_params(x, maxq):
    """``Quantizer.find_params(x, weight=True)`` (asymmetric, per row).

    xmin = min(min(x), 0), xmax = max(max(x), 0); an all-zero row gets
    [-1, +1]; s = (xmax - xmin) / maxq; z = round(-xmin / s).
    """
    dt = x.dtype.type
    xmin = np.minimum(x.min(axis=1), dt(0))
    xmax = np.maximum(x.max(axis=1), dt(0))
    both0 = (xmin == 0) & (xmax == 0)
    xmin = np.where(both0, dt(-1), xmin)
    xmax = np.where(both0, dt(1), xmax)
    s = (xmax - xmin) / dt(maxq)
    z = rne(-xmin / s)
    return s, z


def canonical_codes(x, s, z, maxq):
    """``Quantizer.quantize`` codes: clamp(round(x / s) + z, 0, maxq)."""
    return np.clip(rne(x / s) + z, 0, maxq)


def canonical_dequant(q, s, z):
    """``Quantizer.quantize`` value: s * (q - z)."""
    return s * (q - z)


# ---------------------------------------------------------------------------
# The column sweep, both modes
# ---------------------------------------------------------------------------


def gptq_ref(weight, Hinv, bits, group_size, blocksize):
    """Reference-mode column sweep (core/gptq.py:101-214, minimal repair at :175).

    weight: (N, K) as stored by nn.Linear.  A = weight^T is (K, N): "rows" are
    input features, "columns" output features (:107-108).  The sweep walks the
    N columns and indexes the K x K inverse by output index (:141-142, :153),
    so it requires N <= K and N % group_size == 0 (:125-126).

    Returns dict(codes (N, K), scale (K, N//g), zero (K, N//g), total_error).
    """
    dt = Hinv.dtype.type
    A = np.ascontiguousarray(weight.T.astype(Hinv.dtype))
    rows, cols = A.shape
    if cols > rows or cols % group_size:
        raise ValueError("reference semantics need N <= K and N % group_size == 0")
    maxq = 2 ** bits - 1
    A0 = A.copy()  # group statistics read the never-updated W (:162, :194)
    scale = np.zeros((rows, cols // group_size), dtype=Hinv.dtype)
    zero = np.zeros_like(scale)
    total_error = 0.0
    for i1 in range(0, cols, blocksize):
        i2 = min(i1 + blocksize, cols)
        B = A[:, i1:i2].copy()
        Q = np.zeros_like(B)
        Hb = Hinv[i1:i2, i1:i2]
        for j in range(i2 - i1):
            c = i1 + j
            d = Hb[j, j]
            g = c // group_size
            if c % group_size == 0:
                s, z = ref_params(A0[:, c:min(c + group_size, cols)], maxq)
                scale[:, g], zero[:, g] = s, z
            s, z = scale[:, g], zero[:, g]
            w = B[:, j]
            q = ref_quantize(w, s, z, maxq)
            Q[:, j] = q
            err = (w - (q - z) * s) / d
            if j < i2 - i1 - 1:
                B[:, j + 1:] -= np.outer(err, Hb[j, j + 1:])
            total_error += float(np.sum(err.astype(np.float64) ** 2))
        A[:, i1:i2] = Q
    return dict(codes=A.T.copy(), scale=scale, zero=zero,
                total_error=total_error)


def gptq_canonical(weight, H_raw, nsamples, bits, group_size, blocksize,
                   percdamp, actorder=False, dtype=np.float64, U=None, perm=None):
    """Canonical GPTQ (paper Alg. 1, ``fasterquant``) on weight (N, K).

    group_size = -1 means one group per row (per-channel).  Group parameters
    for a group starting at column c are computed, at the start of the block
    containing c, from the current (trailing-updated) weights over columns
    [c, c + group_size).  With act-order, columns are processed in order of
    decreasing H_ii and groups are contiguous in that order.

    If ``U`` is given it is used as the upper Cholesky factor of the damped,
    permuted H^-1 instead of computing it (so a GPU factor can be fed in);
    ``perm`` then gives the act-order permutation that factor belongs to
    (when diagonal entries nearly tie, the order computed here in ``dtype``
    can differ from the one the factor was built for).

    Returns dict(codes (N, K) in original column order, scale/zero
    (N, ngroups), g_idx (K,), perm (K,), dequant (N, K), losses (N, K),
    U).
    """
    W = np.array(weight, dtype=dtype, copy=True)
    rows, cols = W.shape
    maxq = 2 ** bits - 1
    if U is None:
        H, dead = prepare_canonical_H(np.asarray(H_raw, dtype=dtype), nsamples, 0.0)
        diag = np.diag(H)
    else:
        # a given factor needs only the diagonal (dead columns, act-order):
        # the same values prepare_canonical_H puts there, without K x K work
        diag = (2.0 / nsamples) * np.asarray(np.diag(H_raw), dtype=dtype)
        dead = diag == 0
        diag = np.where(dead, dtype(1), diag)
    # damping is applied after the permutation, on the permuted matrix;
    # mean(diag) is permutation invariant so the order does not matter
    if group_size == -1:
        s_pc, z_pc = canonical_params(W, maxq)
    W[:, dead] = 0
    if actorder and perm is not None:
        perm = np.asarray(perm, dtype=np.int64)
    elif actorder:
        perm = np.argsort(-diag, kind="stable")
    else:
        perm = np.arange(cols)
    if actorder:
        W = W[:, perm]
    if U is None:
        if actorder:
            H = H[perm][:, perm]
        H = H.copy()
        H[np.diag_indices_from(H)] += percdamp * np.mean(np.diag(H))
        U = upper_chol_of_inverse(H)
    U = np.asarray(U, dtype=dtype)
    gs = cols if group_size == -1 else group_size
    ngroups = (cols + gs - 1) // gs
    scale = np.zeros((rows, ngroups), dtype=dtype)
    zero = np.zeros_like(scale)
    if group_size == -1:
        scale[:, 0], zero[:, 0] = s_pc, z_pc
    Q = np.zeros_like(W)
    Qv = np.zeros_like(W)
    Losses = np.zeros_like(W)
    for i1 in range(0, cols, blocksize):
        i2 = min(i1 + blocksize, cols)
        if group_size != -1:
            for c in range(i1, i2):
                if c % gs == 0:
                    s, z = canonical_params(W[:, c:min(c + gs, cols)], maxq)
                    scale[:, c // gs], zero[:, c // gs] = s, z
        W1 = W[:, i1:i2].copy()
        Err1 = np.zeros_like(W1)
        for j in range(i2 - i1):
            c = i1 + j
            s, z = scale[:, c // gs], zero[:, c // gs]
            w = W1[:, j]
            d = U[c, c]
            q = canonical_codes(w, s, z, maxq)
            qv = canonical_dequant(q, s, z)
            Q[:, c] = q
            Qv[:, c] = qv
            Losses[:, c] = (w - qv) ** 2 / d ** 2 / 2
            e = (w - qv) / d
            W1[:, j:] -= np.outer(e, U[c, c:i2])
            Err1[:, j] = e
        W[:, i2:] -= Err1 @ U[i1:i2, i2:]
    invperm = np.argsort(perm)
    g_idx = (np.arange(cols) // gs)[invperm].astype(np.int32)
    return dict(codes=Q[:, invperm], dequant=Qv[:, invperm], scale=scale,
                zero=zero, g_idx=g_idx, perm=perm, losses=Losses[:, invperm],
                U=U)


def code_margin(y, q, maxq):
    """How far y = w / s + z lies outside the cell of values whose canonical
    code clamp(round(w / s) + z, 0, maxq) is q (z integral), in quantisation
    steps: 0 inside [q - 1/2, q + 1/2], the cell being open-ended at code 0
    and at maxq."""
    lo = np.where(q <= 0, -np.inf, q - 0.5)
    hi = np.where(q >= maxq, np.inf, q + 0.5)
    return np.maximum(np.maximum(lo - y, y - hi), 0.0)


def gptq_canonical_replay(weight, U, perm, dead, bits, group_size, blocksize, codes, scale, zero):
    """fp64 replay of the canonical sweep along given decisions.

    Runs ``gptq_canonical``'s loop (same order, same lazy-batch updates) with
    the factor ``U`` (sweep order), but takes the codes and the group
    parameters from ``codes`` (N x K, original column order) and
    ``scale``/``zero`` (N x ngroups, sweep group order) instead of deciding
    them, so one different decision cannot cascade.  Returns

    * ``margin`` (N x K, original order): per weight, how far the replayed
      w / s + z lies outside the rounding cell of the given code, in
      quantisation steps (0 = the given code is the correct rounding of the
      fp64 value along that trajectory);
    * ``scale``/``zero``: the group parameters the replay computes itself at
      each group start (per-channel: from the original weight), and
      ``zero_margin``: the distance of -xmin / s from the nearest rounding
      tie (a zero point within a hair of a tie may legitimately differ).
    """
    W = np.array(weight, dtype=np.float64, copy=True)
    rows, cols = W.shape
    maxq = 2 ** bits - 1
    perm = np.arange(cols) if perm is None else np.asarray(perm)
    dead = np.zeros(cols, bool) if dead is None else np.asarray(dead, bool)
    gs = cols if group_size == -1 else group_size
    ngroups = (cols + gs - 1) // gs
    s_own = np.zeros((rows, ngroups))
    z_own = np.zeros((rows, ngroups))
    z_tie = np.full((rows, ngroups), np.inf)

    def own_params(x, g):
        xmin = np.minimum(x.min(axis=1), 0.0)
        xmax = np.maximum(x.max(axis=1), 0.0)
        both0 = (xmin == 0) & (xmax == 0)
        xmin = np.where(both0, -1.0, xmin)
        xmax = np.where(both0, 1.0, xmax)
        s = (xmax - xmin) / maxq
        v = -xmin / s
        s_own[:, g], z_own[:, g] = s, np.round(v)
        z_tie[:, g] = np.abs(np.abs(v - np.floor(v)) - 0.5)

    if group_size == -1:
        own_params(W, 0)
    W[:, dead] = 0
    W = W[:, perm]
    Q = np.asarray(codes, np.float64)[:, perm]
    S = np.asarray(scale, np.float64)
    Z = np.asarray(zero, np.float64)
    U = np.asarray(U, np.float64)
    margin = np.zeros_like(W)
    for i1 in range(0, cols, blocksize):
        i2 = min(i1 + blocksize, cols)
        if group_size != -1:
            for c in range(i1, i2):
                if c % gs == 0:
                    own_params(W[:, c:min(c + gs, cols)], c // gs)
        W1 = W[:, i1:i2].copy()
        Err1 = np.zeros_like(W1)
        for j in range(i2 - i1):
            c = i1 + j
            s, z = S[:, c // gs], Z[:, c // gs]
            w = W1[:, j]
            q = Q[:, c]
            margin[:, c] = code_margin(w / s + z, q, maxq)
            e = (w - s * (q - z)) / U[c, c]
            W1[:, j:] -= np.outer(e, U[c, c:i2])
            Err1[:, j] = e
        W[:, i2:] -= Err1 @ U[i1:i2, i2:]
    inv = np.argsort(perm)
    return dict(margin=margin[:, inv], scale=s_own, zero=z_own, zero_margin=z_tie)


def obs_bruteforce(weight, Hd, bits, group_size, param_snapshot_cols=None):
    """Textbook sequential OBS quantization with explicit inverse downdating.

    Independent of the Cholesky formulation: keeps the full inverse of the
    Hessian over the not-yet-quantized columns and removes one column at a
    time (H^-1 <- H^-1 - H^-1[:, q] H^-1[q, :] / H^-1[q, q]).  Group
    parameters come from the fully updated weights at the group start.
    Used on tiny K to pin ``gptq_canonical`` (GPTQ's lazy-batch Cholesky
    form is an exact reordering of this).
    """
    W = np.array(weight, dtype=np.float64, copy=True)
    rows, cols = W.shape
    maxq = 2 ** bits - 1
    Hinv = np.linalg.inv(np.asarray(Hd, dtype=np.float64))
    gs = cols if group_size == -1 else group_size
    Q = np.zeros_like(W)
    s = z = None
    for c in range(cols):
        if c % gs == 0:
            s, z = canonical_params(W[:, c:min(c + gs, cols)], maxq)
        q = canonical_codes(W[:, c], s, z, maxq)
        Q[:, c] = q
        e = (W[:, c] - canonical_dequant(q, s, z)) / Hinv[c, c]
        W -= np.outer(e, Hinv[c, :])
        Hinv = Hinv - np.outer(Hinv[:, c], Hinv[c, :]) / Hinv[c, c]
    return Q


def layer_error(weight, dequant, H_raw):
    """||W X - Q X||^2 over the calibration tokens = tr(dW H_raw dW^T)."""
    dW = np.asarray(weight, np.float64) - np.asarray(dequant, np.float64)
    return float(np.einsum("ij,jk,ik->", dW, np.asarray(H_raw, np.float64), dW))


# ---------------------------------------------------------------------------
# Packing, unpacking, dequantisation
# ---------------------------------------------------------------------------


def pack_bitstream(codes, bits):
    """Native packed layout: each row of (N, K) codes as an LSB-first bit
    stream of ``bits``-bit fields, ceil(K * bits / 8) bytes per row.

    For 4-bit this is the ``QuantizedLinear.pack_weights`` byte layout
    (byte = c[2i] | c[2i+1] << 4, models/layers.py:85-89, a lone last nibble
    for odd K, :90); for 2/4/8-bit the bytes read as little-endian int32 equal
    ``pack_weights_kernel``'s words (word |= code_j << (j * bits),
    kernels/triton_kernels.py:212-217) over consecutive codes of a row.  For
    3-bit, 32 codes fill three 32-bit words (the reference defines no 3-bit
    packing; it stores 3-bit unpacked, core/gptq.py:256-257).
    """
    c = np.asarray(codes).astype(np.uint32) & ((1 << bits) - 1)
    N, K = c.shape
    pitch = (K * bits + 7) // 8
    out = np.zeros((N, pitch + 2), dtype=np.uint32)
    for k in range(K):
        byte, off = divmod(k * bits, 8)
        v = c[:, k] << np.uint32(off)      # at most 15 bits wide
        out[:, byte] |= v & np.uint32(0xFF)
        out[:, byte + 1] |= v >> np.uint32(8)
    return out[:, :pitch].astype(np.uint8)


def unpack_bitstream(packed, bits, K):
    """Inverse of ``pack_bitstream``: (N, ceil(K*bits/8)) uint8 -> (N, K)."""
    p = np.asarray(packed, dtype=np.uint8).astype(np.uint32)
    N = p.shape[0]
    p = np.concatenate([p, np.zeros((N, 1), np.uint32)], axis=1)
    out = np.zeros((N, K), dtype=np.uint8)
    for k in range(K):
        byte, off = divmod(k * bits, 8)
        v = (p[:, byte] | (p[:, byte + 1] << np.uint32(8))) >> np.uint32(off)
        out[:, k] = v & np.uint32((1 << bits) - 1)
    return out


def ref_pack_weights(codes_nk, bits):
    """``GPTQ.pack_weights`` (core/gptq.py:216-266) on codes (N, K).

    Works on W = weight^T (K, N) (:223-226).  4-bit: byte = 16*W[:, i] +
    W[:, i+1] (MSB-first pairs along N, :237-238).  2-bit: 64, 16, 4, 1
    weights (:248-254).  Other widths are returned unpacked, cast to int8
    for 8-bit (codes >= 128 wrap) and uint8 otherwise (:256-257).
    """
    W = np.asarray(codes_nk).T.astype(np.int64)
    if bits == 4:
        return (W[:, 0::2] * 16 + W[:, 1::2]).astype(np.uint8)
    if bits == 2:
        return (W[:, 0::4] * 64 + W[:, 1::4] * 16 + W[:, 2::4] * 4
                + W[:, 3::4]).astype(np.uint8)
    if bits == 8:
        return W.astype(np.uint8).view(np.int8)
    return W.astype(np.uint8)


def ref_unpack_4bit(qweight):
    """``GPTQDequantizer._unpack_4bit`` (core/dequantizer.py:68-89): low
    nibble -> even index, high nibble -> odd index."""
    q = np.asarray(qweight, dtype=np.uint8)
    out = np.zeros((q.shape[0], q.shape[1] * 2), dtype=np.uint8)
    out[:, 0::2] = q & 0xF
    out[:, 1::2] = (q >> 4) & 0xF
    return out


def dequant(codes, scales, zeros, g_idx):
    """(q - zero[g]) * scale[g] in fp32, no FMA (models/layers.py:136,
    core/dequantizer.py:64, kernels/triton_kernels.py:120).  ``g_idx[k]`` is the
    group of input column k; scales/zeros are (N, ngroups), any float dtype,
    promoted to fp32 as torch promotes an fp16 operand against fp32."""
    q = np.asarray(codes).astype(np.float32)
    s = np.asarray(scales).astype(np.float32)[:, g_idx]
    z = np.asarray(zeros).astype(np.float32)[:, g_idx]
    return ((q - z) * s).astype(np.float32)


def linear(x, codes, scales, zeros, g_idx, bias=None):
    """``QuantizedLinear`` fallback semantics F.linear(x, unpack(), bias)
    (models/layers.py:155-157), evaluated in fp64 on the fp32 dequantized
    weight; the GPU op returns this in x's dtype."""
    Wd = dequant(codes, scales, zeros, g_idx).astype(np.float64)
    y = np.asarray(x, np.float64) @ Wd.T
    if bias is not None:
        y = y + np.asarray(bias, np.float64)
    return y


PINNING = {
    "add_batch/hessian": "brute-force triple loop, symmetry, trace = ||X||_F^2, "
                         "additivity, H(aX) = a^2 H, nsamples counts sequences",
    "damp_ref": "closed form; diag shift equals percdamp * mean(diag)",
    "full_inverse": "H @ Hinv = I, equals numpy.linalg.inv",
    "upper_chol_of_inverse": "U upper, diag > 0, U^T U = H^-1, equals "
                             "chol(inv(H)).T from numpy",
    "ref_params/ref_quantize": "hand-computed groups, tie cases, exhaustive "
                               "code range",
    "canonical_params/codes": "hand-computed groups incl. all-positive, "
                              "all-zero rows, tie cases",
    "gptq_ref": "H = I reduces to min-max RTN; hand-worked 3-column example "
                "with propagation",
    "gptq_canonical": "obs_bruteforce (explicit inverse downdating) on K <= 16; "
                      "blocksize invariance; H = I reduces to RTN; act-order "
                      "equals running on permuted inputs; loss identity",
    "pack/unpack": "exhaustive code values, round trip, byte layout vs "
                   "hand-written words for each reference layout",
    "dequant/linear": "hand-computed values; equals dense float matmul",
}
