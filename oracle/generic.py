"""The reference's generic (jax.numpy) path restated in numpy -- TEST INFRASTRUCTURE.

Every function works on a batch (B, n, n) and keeps the input dtype (float32 in,
float32 arithmetic; slogdet / slogpf and lu_parts also take float64, complex64 and
complex128, the reference's other kinds), citing the reference function it follows. The LU is LAPACK
``?getrf`` (the routine ``lax.linalg.lu`` calls on the CPU) and the triangular solves
are LAPACK ``?trtrs`` (``lax.linalg.triangular_solve``'s CPU routine); the rest --
pivot bookkeeping, pairwise reductions, the masked Parlett-Reid, the gradient
assembly -- is the reference's own logic written out again from its description.
"""

import numpy as np
import scipy.linalg
import scipy.linalg.lapack as _lapack


# ------------------------------------------------------------------ reductions
def pairwise(x, op, fill):
    """Reduce the last axis by an explicit pairwise tree of ``op``, padding odd
    lengths with ``fill`` (reference ``_fallback.py:19-33``): halves [0, h) and [h, 2h)
    are combined elementwise until one entry is left."""
    x = np.asarray(x)
    n = x.shape[-1]
    if n == 0:
        return np.full(x.shape[:-1], fill, x.dtype)
    while n > 1:
        h = (n + 1) // 2
        if 2 * h != n:
            pad = np.full(x.shape[:-1] + (1,), fill, x.dtype)
            x = np.concatenate([x, pad], axis=-1)
        x = op(x[..., :h], x[..., h:])
        n = h
    return x[..., 0]


# ------------------------------------------------------------------ LU (getrf)
def lu_factor(A):
    """Batched LU with partial pivoting, P A = L U (``lax.linalg.lu``, reference
    ``_fallback.py:59,78``): LAPACK getrf per matrix. Returns (lu, piv, perm): the
    packed factors, the 0-based LAPACK swap sequence (row k swapped with piv[k]) and
    the permutation with (P A)[c] = A[perm[c]]."""
    A = np.asarray(A)
    B, n, _ = A.shape
    getrf = {
        np.dtype(np.float32): _lapack.sgetrf,
        np.dtype(np.float64): _lapack.dgetrf,
        np.dtype(np.complex64): _lapack.cgetrf,
        np.dtype(np.complex128): _lapack.zgetrf,
    }[A.dtype]
    lu = np.empty_like(A)
    piv = np.empty((B, n), np.int32)
    for b in range(B):
        f, p, _info = getrf(A[b])
        lu[b] = f
        piv[b] = p
    perm = np.broadcast_to(np.arange(n, dtype=np.int32), (B, n)).copy()
    rows = np.arange(B)
    for k in range(n):
        pk = piv[:, k]
        tmp = perm[rows, k].copy()
        perm[rows, k] = perm[rows, pk]
        perm[rows, pk] = tmp
    return lu, piv, perm


def slog_from_lu(lu, piv):
    """(sign, logabs) of P L U from the diagonal of U and the swap sequence (reference
    ``_fallback.py:36-55``): parity = number of non-trivial swaps + number of negative
    pivots (real), or the pairwise product of the pivots' unit phases d / |d| with the
    swap parity's sign flip (complex); a zero pivot gives (0, -inf); log|det| is a
    pairwise sum of log|d| in the real dtype."""
    d = np.diagonal(lu, axis1=-2, axis2=-1)
    iota = np.arange(lu.shape[-1])
    swaps = np.sum(piv != iota, axis=-1)
    zero = np.any(d == 0, axis=-1)
    dsafe = np.where(d == 0, np.ones_like(d), d)
    rdt = np.finfo(lu.dtype).dtype
    if np.iscomplexobj(lu):
        sign = pairwise((dsafe / np.abs(dsafe)).astype(lu.dtype), np.multiply, 1)
        sign = np.where(swaps % 2 == 1, -sign, sign)
    else:
        parity = swaps + np.sum(d < 0, axis=-1)
        sign = np.where(parity % 2 == 1, -1.0, 1.0).astype(lu.dtype)
    sign = np.where(zero, np.zeros_like(sign), sign)
    with np.errstate(divide="ignore"):
        logsum = pairwise(np.log(np.abs(dsafe)).astype(rdt), np.add, 0)
    logabs = np.where(zero, -np.inf, logsum).astype(rdt)
    return sign, logabs


def slogdet_generic(A):
    """Reference ``_slogdet_generic`` (``_fallback.py:58-60``)."""
    lu, piv, _ = lu_factor(A)
    return slog_from_lu(lu, piv)


def _tri_solve(T, X, lower, unit):
    """Batched T^-1 X (``lax.linalg.triangular_solve(left_side=True)``)."""
    out = np.empty_like(X)
    for b in range(T.shape[0]):
        out[b] = scipy.linalg.solve_triangular(
            T[b], X[b], lower=lower, unit_diagonal=unit, check_finite=False
        )
    return out


def lu_parts_generic(A, zero_singular=True):
    """(sign, logabs, invT, lu, perm, zero) of reference ``_lu_parts_generic``
    (``_fallback.py:63-97``, at N = n): invT = (U~^-1 L^-1 P)^T with the zero pivots of U
    replaced by 1 (U~); members whose result is non-finite -- and, with
    ``zero_singular``, members with an exact zero pivot -- get invT = 0."""
    A = np.asarray(A)
    B, n, _ = A.shape
    dt = A.dtype
    lu, piv, perm = lu_factor(A)
    sign, logabs = slog_from_lu(lu, piv)
    zero = np.diagonal(lu, axis1=-2, axis2=-1) == 0
    Ut = lu + zero.astype(dt)[..., None] * np.eye(n, dtype=dt)
    X = np.zeros((B, n, n), dt)
    X[np.arange(B)[:, None], np.arange(n)[None, :], perm] = 1  # row c of P I = e_perm[c]
    with np.errstate(all="ignore"):
        X = _tri_solve(lu, X, lower=True, unit=True)
        X = _tri_solve(Ut, X, lower=False, unit=False)
    bad = ~np.all(np.isfinite(X), axis=(-1, -2))
    if zero_singular:
        bad = bad | np.any(zero, axis=-1)
    invT = np.where(bad[:, None, None], np.zeros_like(X), np.swapaxes(X, -1, -2))
    return sign, logabs, invT, lu, perm, zero


# ------------------------------------------------------------ Parlett-Reid
def _pr_step(A, c, idx):
    """One masked pair step of the generic Parlett-Reid (reference
    ``_fallback.py:276-295``): pivot on column c over rows > c (first largest
    magnitude), swap it into c+1 (rows and columns), d = A[c, c+1], then
    A += tau w^T - w tau^T with tau = -A[:, c]/d, w = A[:, c+1] on rows > c+1."""
    B = A.shape[0]
    dt = A.dtype
    col = A[:, :, c]
    cand = np.where(idx > c, np.abs(col), -1.0)
    kp = np.argmax(cand, axis=1)
    moved = np.where(idx == kp[:, None], c + 1, idx)
    p = np.where(idx == c + 1, kp[:, None], moved)
    A = np.take_along_axis(A, p[:, :, None], axis=1)
    A = np.take_along_axis(A, p[:, None, :], axis=2)
    colc = A[:, :, c]
    colc1 = A[:, :, c + 1]
    d = colc1[np.arange(B), c]
    dsafe = np.where(d == 0, np.ones_like(d), d)
    inv = np.where(d == 0, np.zeros_like(d), (1 / dsafe).astype(dt))
    mask = (idx > c + 1).astype(dt)
    tau = -colc * inv[:, None] * mask
    w = colc1 * mask
    A = A + tau[:, :, None] * w[:, None, :] - w[:, :, None] * tau[:, None, :]
    return A, kp, p, d, tau, w


def slogpf_generic(S):
    """Reference ``_slogpf_generic`` (``_fallback.py:266-300``): n/2 masked pair steps;
    every non-trivial swap flips the sign, each pivot d contributes sign(d) and
    log|d| (a zero pivot gives sign 0 and logabs -inf)."""
    A = np.array(S)
    B, n, _ = A.shape
    dt = A.dtype
    idx = np.arange(n)[None, :]
    sign = np.ones(B, dt)
    log = np.zeros(B, np.finfo(dt).dtype)
    with np.errstate(divide="ignore", invalid="ignore"):
        for k in range(n // 2):
            c = 2 * k
            A, kp, _, d, _, _ = _pr_step(A, c, idx)
            sign = np.where(kp != c + 1, -sign, sign)
            # sign(d): d / |d| for complex d (numpy >= 2 and jnp.sign alike)
            sign = sign * np.sign(d)
            log = (log + np.log(np.abs(d))).astype(log.dtype)
    return sign.astype(dt), log


# pf gradient helpers (reference _fallback.py:101-192)
def pivot_index(d, n):
    """argmin |d| over the real pairs (reference ``_pivot_index``, :101-108)."""
    a = np.abs(d)
    h = d.shape[1]
    if n // 2 < h:
        a = a.copy()
        a[:, n // 2 :] = np.inf
    return np.argmin(a, axis=1)


def pair_scale(d, K):
    """d~: pivot K and every exact zero replaced by 1 (reference ``_pair_scale``)."""
    isK = np.arange(d.shape[1])[None, :] == K[:, None]
    return np.where(isK | (d == 0), np.ones_like(d), d)


def pf_value(d, sgnP):
    """sgnP * prod(d) by exp of a pairwise log sum (reference ``_pf_value``)."""
    dsafe = np.where(d == 0, np.ones_like(d), d)
    mag = np.exp(pairwise(np.log(np.abs(dsafe)), np.add, 0))
    return sgnP * pairwise(np.sign(d), np.multiply, 1) * mag


def second_zero(d, K):
    """(has2, is2): a zero pivot besides K and the mask of the first one (reference
    ``_second_zero``, :128-139)."""
    h = d.shape[1]
    others = (d == 0) & (np.arange(h)[None, :] != K[:, None])
    has2 = np.any(others, axis=1)
    first = np.argmax(others, axis=1)
    is2 = has2[:, None] & (np.arange(h)[None, :] == first[:, None])
    return has2, is2


def pf_adj_coeffs(d, sgnP, K, adjugate):
    """(a1, a2, d_K) (reference ``_pf_adj_coeffs``, :157-176)."""
    h = d.shape[1]
    isK = np.arange(h)[None, :] == K[:, None]
    dK = np.take_along_axis(d, K[:, None], axis=1)[:, 0]
    dsafe = np.where(d == 0, np.ones_like(d), d)
    logD = pairwise(np.where(isK, 0, np.log(np.abs(dsafe))).astype(d.dtype), np.add, 0)
    phase = pairwise(np.where(isK, 1, np.sign(d)).astype(d.dtype), np.multiply, 1)
    D = phase * np.exp(logD)
    if adjugate:
        return sgnP * D * dK, sgnP * D * (1 - dK), dK
    nz = dK != 0
    a2 = np.where(nz, (1 - dK) / np.where(nz, dK, 1), 0).astype(d.dtype)
    return np.ones_like(dK), a2, dK


def pf_parts_generic(S, adjugate):
    """(sign, logabs, G, pf) of reference ``_pf_parts_generic`` (``_fallback.py:195-263``):
    the masked Parlett-Reid keeping the factor L (w in column a = 2s, tau in column
    p = 2s+1 of each pair, rows permuted along), then with d~ = pair_scale(d, K),
    L~ = L with the a columns scaled by 1/d~ plus I, Y = L~^-1,
    DY = rows (Y[p], -Y[a]) / d~, R = Y^T DY and
    PT = -[a1 R + a2 (w v^T - v w^T)] (w = R e_aK, v = Y^T e_aK), scattered back through
    the permutation. adjugate=True gives pf(S) S^-1 (second zero pivot: mean of the
    lifted evaluations, reference ``_lifted_mean`` :142-154), False gives S^-1 zeroed for
    singular or non-finite members."""
    A = np.array(S)
    B, n, _ = A.shape
    dt = A.dtype
    idx = np.arange(n)[None, :]
    h = n // 2
    L0 = np.zeros_like(A)
    perm = np.broadcast_to(np.arange(n), (B, n)).copy()
    sign = np.ones(B, dt)
    log = np.zeros(B, dt)
    par = np.zeros(B, bool)
    with np.errstate(divide="ignore", invalid="ignore"):
        for k in range(h):
            c = 2 * k
            A, kp, p, d, tau, w = _pr_step(A, c, idx)
            L0 = np.take_along_axis(L0, p[:, :, None], axis=1)
            perm = np.take_along_axis(perm, p, axis=1)
            swapped = kp != c + 1
            sign = np.where(swapped, -sign, sign)
            L0[:, :, c] = w
            L0[:, :, c + 1] = tau
            sign = sign * np.sign(d)
            log = (log + np.log(np.abs(d))).astype(dt)
            par = par ^ swapped
    T = A
    d = np.stack([T[:, 2 * s, 2 * s + 1] for s in range(h)], axis=1)
    K = pivot_index(d, n)
    sgnP = np.where(par, -1.0, 1.0).astype(dt)
    eye = np.broadcast_to(np.eye(n, dtype=dt), (B, n, n)).copy()
    iperm = np.argsort(perm, axis=1)

    def evaluate(dd):
        dts = pair_scale(dd, K)
        scale = np.stack([1 / dts, np.ones_like(dts)], axis=2).reshape(B, n)
        Lt = L0 * scale[:, None, :] + np.eye(n, dtype=dt)
        with np.errstate(all="ignore"):
            Y = _tri_solve(Lt.astype(dt), eye, lower=True, unit=True)
        Yr = Y.reshape(B, h, 2, n)
        DY = np.stack([Yr[:, :, 1], -Yr[:, :, 0]], axis=2) / dts[:, :, None, None]
        R = np.matmul(np.swapaxes(Y, 1, 2), DY.reshape(B, n, n).astype(dt))
        a1, a2, _ = pf_adj_coeffs(dd, sgnP, K, adjugate)
        aK = 2 * K
        w_ = np.take_along_axis(R, aK[:, None, None], axis=2)[:, :, 0]
        v_ = np.take_along_axis(Y, aK[:, None, None], axis=1)[:, 0, :]
        outer = lambda x, y: x[:, :, None] * y[:, None, :]
        PT = -(a1[:, None, None] * R + a2[:, None, None] * (outer(w_, v_) - outer(v_, w_)))
        G = np.take_along_axis(PT, iperm[:, :, None], axis=1)
        return np.take_along_axis(G, iperm[:, None, :], axis=2).astype(dt)

    with np.errstate(all="ignore"):
        if adjugate:
            has2, is2 = second_zero(d, K)
            G = evaluate(d)
            if np.any(has2):
                lifted = 0.5 * (
                    evaluate(np.where(is2, 1, d).astype(dt))
                    + evaluate(np.where(is2, -1, d).astype(dt))
                )
                G = np.where(has2[:, None, None], lifted, G)
        else:
            G = evaluate(d)
            dK = np.take_along_axis(d, K[:, None], axis=1)[:, 0]
            bad = (dK == 0) | ~np.all(np.isfinite(G), axis=(1, 2))
            G = np.where(bad[:, None, None], np.zeros_like(G), G)
        pfv = pf_value(d, sgnP)
    return sign.astype(dt), log, G, pfv.astype(dt)


# ------------------------------------------------------- det gradient pieces
def perm_sign(g0):
    """sgn(P) of the row permutation g0 (B, N) as (-1)^(N - #cycles) (reference
    ``_perm_sign``, ``_diff.py:160-176``; here the cycles are counted by walking them)."""
    g0 = np.asarray(g0)
    B, N = g0.shape
    out = np.empty(B)
    for b in range(B):
        seen = np.zeros(N, bool)
        ncyc = 0
        for s in range(N):
            if not seen[s]:
                ncyc += 1
                j = s
                while not seen[j]:
                    seen[j] = True
                    j = g0[b, j]
        out[b] = 1.0 - 2.0 * ((N - ncyc) % 2)
    return out


def lu_det(d, g0):
    """sgn(P) prod(d) of the packed factors, 0 for a zero pivot (reference ``_lu_det``,
    ``_diff.py:184-202``)."""
    dsafe = np.where(d == 0, np.ones_like(d), d)
    logsum = pairwise(np.log(np.abs(dsafe)), np.add, 0)
    phase = pairwise(np.sign(dsafe), np.multiply, 1)
    det = (perm_sign(g0).astype(d.dtype) * phase * np.exp(logsum)).astype(d.dtype)
    return np.where(np.any(d == 0, axis=1), np.zeros_like(det), det)


def det_gradT(invT, LU, g0, zero, n):
    """d det / dA = adj(A)^T from the LU parts (reference ``_det_gradT``,
    ``_diff.py:205-246``): det * A^-T for regular members; with zero pivots at
    k1 <= ... <= km the Woodbury form sgn(P) d_K c (U~^-1 e_k1)(row k_m of U~^-1 L^-1 P),
    c = (U~^-1)[k1, km] for m = 2, 1 for m = 1, and 0 for m >= 3."""
    B, N = LU.shape[:2]
    dt = LU.dtype
    m = np.sum(zero, axis=1)
    d = np.diagonal(LU, axis1=1, axis2=2)
    det = lu_det(d, g0)
    G = det[:, None, None] * invT
    if not np.any(m >= 1):
        return G
    idx = np.arange(N)
    k1 = np.minimum(np.min(np.where(zero, idx, N), axis=1), N - 1)
    k2 = np.maximum(np.max(np.where(zero, idx, -1), axis=1), 0)
    dsafe = np.where(zero, np.ones_like(d), d)
    dK = (np.prod(np.sign(dsafe), axis=1) * np.exp(np.sum(np.log(np.abs(dsafe)), axis=1))).astype(dt)
    Ut = np.triu(LU) + zero.astype(dt)[:, :, None] * np.eye(N, dtype=dt)
    E = np.zeros((B, N, 2), dt)
    E[np.arange(B), k1, 0] = 1
    E[np.arange(B), k2, 1] = 1
    with np.errstate(all="ignore"):
        UE = _tri_solve(Ut, E, lower=False, unit=False)
    u1 = UE[:, :n, 0]
    c = np.take_along_axis(UE[:, :, 1], k1[:, None], axis=1)[:, 0]
    s = perm_sign(g0).astype(dt) * dK * np.where(m >= 2, c, 1.0)
    s = np.where(m >= 3, 0.0, s).astype(dt)
    col = np.take_along_axis(invT, k2[:, None, None], axis=2)[:, :, 0]
    Gs = s[:, None, None] * col[:, :, None] * u1[:, None, :]
    return np.where((m >= 1)[:, None, None], Gs, G).astype(dt)


def det_parts(A):
    """(det, G = adj(A)^T) as the reference's det jvp computes them on the generic
    path (``_diff.py:290-301`` with ``_lu_parts_generic(zero_singular=False)``)."""
    sign, logabs, invT, lu, perm, zero = lu_parts_generic(A, zero_singular=False)
    with np.errstate(all="ignore"):
        d = (sign * np.exp(logabs)).astype(A.dtype)
    return d, det_gradT(invT, lu, perm, zero, A.shape[-1])


# ------------------------------------------------------- tiny-n polynomials
def det_poly(A):
    """det for n <= 4 by explicit expansion (reference ``_det_poly``,
    ``_poly.py:10-37``)."""
    A = np.asarray(A)
    n = A.shape[-1]
    a = lambda i, j: A[..., i, j]
    m = lambda r, s, i, j: a(r, i) * a(s, j) - a(r, j) * a(s, i)
    if n == 0:
        return np.ones(A.shape[:-2], A.dtype)
    if n == 1:
        return a(0, 0)
    if n == 2:
        return m(0, 1, 0, 1)
    if n == 3:
        return a(0, 0) * m(1, 2, 1, 2) - a(0, 1) * m(1, 2, 0, 2) + a(0, 2) * m(1, 2, 0, 1)
    if n == 4:
        return (
            m(0, 1, 0, 1) * m(2, 3, 2, 3)
            - m(0, 1, 0, 2) * m(2, 3, 1, 3)
            + m(0, 1, 0, 3) * m(2, 3, 1, 2)
            + m(0, 1, 1, 2) * m(2, 3, 0, 3)
            - m(0, 1, 1, 3) * m(2, 3, 0, 2)
            + m(0, 1, 2, 3) * m(2, 3, 0, 1)
        )
    raise ValueError(n)


def pf_poly(S):
    """pf for even n <= 6 from the strict upper triangle (reference ``_pf_poly``,
    ``_poly.py:40-60``)."""
    S = np.asarray(S)
    n = S.shape[-1]
    s = lambda i, j: S[..., i, j]
    pf4 = lambda a, b, c, d: s(a, b) * s(c, d) - s(a, c) * s(b, d) + s(a, d) * s(b, c)
    if n == 0:
        return np.ones(S.shape[:-2], S.dtype)
    if n == 2:
        return s(0, 1)
    if n == 4:
        return pf4(0, 1, 2, 3)
    if n == 6:
        return (
            s(0, 1) * pf4(2, 3, 4, 5)
            - s(0, 2) * pf4(1, 3, 4, 5)
            + s(0, 3) * pf4(1, 2, 4, 5)
            - s(0, 4) * pf4(1, 2, 3, 5)
            + s(0, 5) * pf4(1, 2, 3, 4)
        )
    raise ValueError(n)
