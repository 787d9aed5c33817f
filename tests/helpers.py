"""Shared helpers for the tests: seeded inputs and tolerance checks."""
import numpy as np

from cpab import Cpab

_CACHE = {}


def cpab_for(tess):
    key = tuple(tess)
    if key not in _CACHE:
        _CACHE[key] = Cpab(list(tess))
    return _CACHE[key]


def seeded_theta(T, n, scale, seed):
    return (np.random.default_rng(seed).standard_normal((n, T.params.d)) * scale).astype(np.float32)


def uniform_points(ndim, n, seed):
    return np.random.default_rng(seed).random((ndim, n)).astype(np.float32)


def meshgrid(sizes):
    """uniform_meshgrid of the reference (coordinate 0 fastest), in float32."""
    lin = [np.linspace(0, 1, s, dtype=np.float32) for s in sizes]
    mesh = np.meshgrid(*lin[::-1], indexing="ij")
    return np.stack([m.reshape(-1) for m in mesh[::-1]]).astype(np.float32)


def edge_lattice(tess, seed):
    """Points on and just beyond the domain's faces, edges and corners.

    Each axis takes, in turn, an "edge" coordinate (0, -0, 1, a step outside,
    the float neighbours of 0 and 1, denormals of both signs, the smallest
    normal, the 2D lookup's clamp bound 1 - 2^-23, far outside) while the
    others take cell-face coordinates k/n, their float neighbours and random
    values; then every pair of axes, and (3D) all three, take edge coordinates
    together.  Returns [ndim, n] float32."""
    rng = np.random.default_rng(seed)
    tiny = np.nextafter(np.float32(0), np.float32(1))          # smallest denormal
    edge = np.array([0.0, -0.0, 1.0, -1e-3, 1.0 + 1e-3, np.nextafter(np.float32(1), 0),
                     np.nextafter(np.float32(1), 2), tiny, -tiny,
                     np.float32(2.0 ** -126) - tiny, np.float32(2.0 ** -126),
                     np.float32(1.0 - 1e-7), -0.4, 1.4], np.float32)
    nd = len(tess)

    def across(n):
        k = np.arange(n + 1, dtype=np.float32) / np.float32(n)
        m = 64 if nd == 2 else 8
        return np.concatenate([k, np.nextafter(k, np.float32(2)), np.nextafter(k, np.float32(-1)),
                               rng.random(m).astype(np.float32)]).astype(np.float32)

    parts = []
    for mask in range(1, 1 << nd):          # bit a set: axis a takes edge coordinates
        axes = [edge if (mask >> a) & 1 else across(tess[a]) for a in range(nd)]
        mesh = np.meshgrid(*axes, indexing="ij")
        parts.append(np.stack([m.ravel() for m in mesh]))
    return np.concatenate(parts, axis=1).astype(np.float32)


def rel_err(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def assert_grad_close(got, ref, rtol=2e-5, atol_frac=5e-6):
    """Moment parity: per element |got - ref| <= rtol*|ref| + atol_frac*max|ref|.

    The moments are sums of many per-trajectory contributions accumulated with
    float atomics in no fixed order, so elements whose contributions cancel
    carry an absolute (not relative) error of a few fp32 ulps of the summed
    magnitudes; atol_frac*max|ref| bounds that.  Measured on MI355X over the
    GPU suite: at rtol 2e-5 the largest absolute part needed is 1.2e-6 of
    max|ref| (the stage-wise chain cases), a quarter of the bound.
    """
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = np.abs(ref).max()
    bad = np.abs(got - ref) > rtol * np.abs(ref) + atol_frac * scale
    assert not bad.any(), (f"{bad.sum()} of {bad.size} elements off; max abs err "
                           f"{np.abs(got - ref).max():.3e}, scale {scale:.3e}")


def assert_adjoint_close(got, ref):
    """Point adjoints (grad_points) against the oracle.

    The HIP reverse sweep advances lambda as lambda + G^T lambda with the
    per-cell G = h A + (h^2/2) A^2, the reference's two half-steps
    (cpab_ops_2d.cu:374-381) multiplied out: the same number, rounded
    differently, so after T steps the two differ by a few fp32 ulps of the
    trajectory's adjoint.  Held per element to 1e-5 relative plus 1e-6 of the
    largest adjoint (measured on MI355X over the GPU suite: at most 4.1e-7 of
    it needed beyond the relative part).
    """
    assert_grad_close(got, ref, rtol=1e-5, atol_frac=1e-6)


def theta_grad_bound(got, mom, basis, scale=1.0, rtol=2e-5, atol_frac=5e-6):
    """(|got - ref|, bound) for a theta gradient; see assert_theta_grad_close."""
    import scipy.sparse as sp
    got = np.asarray(got, np.float64)
    m = np.asarray(mom, np.float64).reshape(got.shape[0], -1)
    Bc = sp.csc_matrix(basis, dtype=np.float64)
    Ba = abs(Bc)
    nnz = int(np.diff(Bc.indptr).max()) if Bc.nnz else 0
    ref = (Bc.T @ m.T).T * scale
    tol_m = rtol * np.abs(m) + atol_frac * np.abs(m).max()
    rounding = (nnz + 1) * 2.0 ** -24 * (Ba.T @ np.abs(m).T).T
    bound = ((Ba.T @ tol_m.T).T + rounding) * abs(scale)
    return np.abs(got - ref), bound


def assert_theta_grad_close(got, mom, basis, scale=1.0, rtol=2e-5, atol_frac=5e-6):
    """Theta-gradient parity, propagated from the moments' tolerance.

    got [rows, d] is the library's gradient; the reference is scale * B^T m
    per row, m [rows, D] being the oracle's moments and B the basis [D, d].
    The library's moments are held to rtol*|m| + atol_frac*max|m| (the moment
    bound of assert_grad_close); the projection carries that to each
    theta-gradient element as |B|^T of it, plus the projection's own fp32
    rounding (B rounded to float32 and at most nnz terms summed:
    (nnz + 1) 2^-24 |B|^T |m|).  A bound on the gradient alone, relative to
    its own largest element, would have to be ~30x looser than the moments':
    each element sums moment contributions of both signs that cancel, so it
    is small next to the moments it sums, and their rounding is not."""
    err, bound = theta_grad_bound(got, mom, basis, scale, rtol, atol_frac)
    bad = err > bound
    assert not bad.any(), (f"{bad.sum()} of {bad.size} elements off; worst err/bound "
                           f"{(err / np.maximum(bound, 1e-300)).max():.3f}")


def recover_growth(As, T=50):
    """Per theta row, the bound (max_c ||M_c||_2)^T on how much the register
    backward's recovered positions can amplify their rounding, M_c being the
    inverse of cell c's explicit-midpoint step map (the criterion the library
    applies to choose between recovering positions and replaying them from
    checkpoints, evaluated here in float64).  As: [rows, nC, nd, nd + 1]."""
    A = np.asarray(As, np.float64)
    nd = A.shape[-2]
    h = float(np.float32(1.0) / np.float32(T))
    h2 = h * float(np.float32(h * np.float32(0.5)))
    L = A[..., :nd]
    E = np.eye(nd) + h * L + h2 * (L @ L)
    s = np.linalg.norm(np.linalg.inv(E), ord=2, axis=(-2, -1))
    return s.max(axis=-1) ** T


def recover_error(points, As, nc, T=50):
    """Per theta row, the largest distance between the positions the register
    backward recovers and the replayed ones (CPU emulation, float32 data).

    Phase 1 replays the explicit-midpoint trajectory (the oracle's replay,
    which the kernels match bit for bit) and keeps its cells; phase 2 starts
    from the final position and steps back through each cell's inverse
    one-step map, p <- M_c p + m_c, with M_c and m_c formed in float64 from E_c
    = I + hA + (h^2/2)A^2 and e_c = hb + (h^2/2)Ab and rounded to float32, and
    each component accumulated from m_c by fmaf in the kernels' order (last
    coordinate first).  fmaf is emulated in float64: the product of two
    floats is exact there, the sum is rounded once to float64 and once to
    float32.  As: [rows, nC, nd, nd + 1]; points [nd, nP]."""
    from oracle import oracle as orc
    A64 = np.asarray(As, np.float64)
    nd = A64.shape[-2]
    h = np.float32(1.0) / np.float32(T)
    hd, h2 = float(h), float(h) * float(h * np.float32(0.5))
    L, b = A64[..., :nd], A64[..., nd]
    E = np.eye(nd) + hd * L + h2 * (L @ L)
    e = hd * b + h2 * (L @ b[..., None])[..., 0]
    M = np.linalg.inv(E)
    m = -(M @ e[..., None])[..., 0]
    M, m = M.astype(np.float32), m.astype(np.float32)
    final, cells, path = orc.forward_midpoint(points, As, nc, T, return_cells=True,
                                              return_path=True)
    err = np.zeros(A64.shape[0])
    for r in range(A64.shape[0]):
        p = final[r].astype(np.float64)
        for t in range(T - 1, -1, -1):
            c = cells[r, :, t]
            q = np.empty_like(p)
            for i in range(nd):
                acc = m[r, c, i].astype(np.float64)
                for j in range(nd - 1, -1, -1):
                    acc = (M[r, c, i, j].astype(np.float64) * p[j] + acc).astype(np.float32)
                    acc = acc.astype(np.float64)
                q[i] = acc
            p = q
            err[r] = max(err[r], float(np.abs(p - path[r, t]).max()))
    return err


def scatter_magnitude(data_shape, grid, outs, gout):
    """Per data pixel, the sum over its grad_data contributions of |g * w|
    (float64), w being the corner weight of the point's resampling.

    The reference clamps a corner index but not the fractional part
    (interpolation.py:3-159), so a point outside [0, 1] gives two weights of
    opposite sign and magnitude up to ~(size-1) that cancel in the sum (1 - t
    and t).  A summation-order bound has to scale with the terms' absolute
    values: summing the same n fp32 terms in two orders differs by at most
    ~2 n 2^-24 of this magnitude.  grid [B, nd, nP] lists points with
    coordinate 0 fastest; gout [B, C, *outs] has the last axis fastest."""
    B, C = data_shape[:2]
    ins = tuple(data_shape[2:])
    nd = len(ins)
    grid = np.asarray(grid, np.float64)
    gp = np.asarray(gout, np.float64).reshape(B, C, *outs)
    gp = gp.transpose(0, 1, *range(nd + 1, 1, -1)).reshape(B, C, -1)   # point order
    mag = np.zeros((B, C, int(np.prod(ins))))
    strides = [int(np.prod(ins[k + 1:])) for k in range(nd)]
    for b in range(B):
        lo, hi, wlo, whi = [], [], [], []
        for k in range(nd):
            x = grid[b, k] * (ins[k] - 1)
            f = np.floor(x)
            i0 = np.clip(f, 0, ins[k] - 1)
            lo.append(i0.astype(np.int64) * strides[k])
            hi.append(np.clip(f + 1, 0, ins[k] - 1).astype(np.int64) * strides[k])
            t = x - i0
            wlo.append(np.abs(1.0 - t))
            whi.append(np.abs(t))
        for corner in range(1 << nd):
            idx = np.zeros_like(lo[0])
            w = np.ones_like(wlo[0])
            for k in range(nd):
                up = (corner >> (nd - 1 - k)) & 1
                idx = idx + (hi[k] if up else lo[k])
                w = w * (whi[k] if up else wlo[k])
            for c in range(C):
                np.add.at(mag[b, c], idx, np.abs(gp[b, c]) * w)
    return mag.reshape(B, C, *ins)
