"""numpy restatement of the 2D domain-edge bound (fg-cpab_amd/csrc/cpab_device.hpp:
EdgeAcc, edge_bound_cell_2d, midpoint_step_err, midpoint_map_2d, pow_int,
edge_delta_2d; basis.hip: adjoint_table_kernel; backward_body.hpp: row_edge_delta),
in the device code's float64 operation order.  Test infrastructure only.

delta_T of a theta row: every point whose distance to each domain edge is at
least delta_T stays in (0, 1 - 2^-23]^2 for T computed explicit-midpoint replay
steps of that row's fields, so the backward's replay lookup takes the inside
rule at each of them.  Over the row's
cells and the four edges, with alpha the smallest contraction factor toward an
edge, beta the largest offset, reach the largest approach per step and err the
largest rounding bound of a computed step:
    delta_T = U (2^-23 + (T - 1)(beta + err)),  U = min(alpha, 1)^-(T-1),
valid when delta_T < r_lo = 1/(2 max(nx, ny)) and delta_T + reach + err <= r_lo.
"""
import numpy as np

ETA = 2.0 ** -20
ULP = 2.0 ** -24


def _ru(x):
    """float32 of the float64 x rounded toward +inf."""
    x = np.float64(x)
    f = np.float32(x)
    if np.isfinite(x) and np.float64(f) < x:
        f = np.nextafter(f, np.float32(np.inf))
    return np.float32(f)


def triangle_vertices(c, nx, ny):
    """Vertices of cell c: square (cx, cy), triangles 0 bottom, 1 right, 2 top,
    3 left, the square's centre last."""
    sq, t = c >> 2, c & 3
    cy, cx = divmod(sq, nx)
    x0, x1 = cx / nx, (cx + 1) / nx
    y0, y1 = cy / ny, (cy + 1) / ny
    xc, yc = 0.5 * (x0 + x1), 0.5 * (y0 + y1)
    vx = (x1 if t == 1 else x0, x0 if t == 3 else x1, xc)
    vy = (y1 if t == 2 else y0, y0 if t == 0 else y1, yc)
    return vx, vy


def midpoint_step_err(a, h, hh):
    S = 0.0
    for r in range(2):
        S = max(S, abs(float(a[3 * r])) + abs(float(a[3 * r + 1])) + abs(float(a[3 * r + 2])))
    dv = 2.02 * ULP * S
    pm = 1.0 + hh * S
    dpm = hh * dv + 1.01 * ULP * pm
    dvm = 2.02 * ULP * S * pm + S * dpm
    return 1.05 * (h * dvm + 1.01 * ULP * (1.0 + h * S * pm))


def midpoint_map(a, h):
    """The explicit-midpoint step of field a (2x3 row-major, float32) as the
    exact affine map [I + h A + h hh A^2 | h b + h hh A b]; h float32."""
    a = [float(v) for v in np.asarray(a, np.float32).ravel()]
    h32 = np.float32(h)
    hd = float(h32)
    h2 = hd * float(h32 * np.float32(0.5))
    m = [[0.0] * 3 for _ in range(2)]
    for i in range(2):
        ab = a[3 * i] * a[2] + a[3 * i + 1] * a[5]
        m[i][2] = hd * a[3 * i + 2] + h2 * ab
        for j in range(2):
            sq = a[3 * i] * a[j] + a[3 * i + 1] * a[3 + j]
            m[i][j] = (1.0 if i == j else 0.0) + hd * a[3 * i + j] + h2 * sq
    return m


class Acc:
    """Smallest alpha, largest beta, reach and err over a row's cells and edges."""

    def __init__(self):
        self.alpha, self.beta, self.reach, self.err = np.inf, 0.0, 0.0, 0.0

    def cell(self, m, c, nx, ny, err):
        vx, vy = triangle_vertices(c, nx, ny)
        if not (np.isfinite(err) and all(np.isfinite(m[a][j]) for a in range(2) for j in range(3))):
            self.alpha = -np.inf
            return
        self.err = max(self.err, err)
        for e in range(4):
            ax, far = e >> 1, e & 1
            rlo = 0.5 / (ny if ax else nx)
            d, dp = [], []
            for k in range(3):
                pos = vy[k] if ax else vx[k]
                img = m[ax][0] * vx[k] + m[ax][1] * vy[k] + m[ax][2]
                d.append(1.0 - pos if far else pos)
                dp.append(1.0 - img if far else img)
            slope = abs(m[ax][0]) + abs(m[ax][1])
            approach = max([0.0] + [d[k] - dp[k] for k in range(3)])
            self.reach = max(self.reach, approach + (slope + 1.0) * ETA)
            if min(d) < rlo:
                bv = max([0.0] + [-dp[k] for k in range(3) if d[k] == 0.0])
                al = min([np.inf] + [(dp[k] + bv) / d[k] for k in range(3) if d[k] > 0.0])
                self.alpha = min(self.alpha, al)
                self.beta = max(self.beta, bv + (slope + max(abs(al), 1.0)) * ETA)

    def delta(self, T, nx, ny):
        """edge_delta_2d: delta_T as float32 rounded up, or +inf."""
        U = (pow_int(1.0 / min(self.alpha, 1.0), T - 1) * (1.0 + 1e-12)
             if self.alpha > 0.0 else np.inf)
        E = self.err
        delta = U * (2.0 ** -23 + float(T - 1) * (self.beta + E)) * (1.0 + 1e-12)
        rlo = 0.5 / float(max(nx, ny))
        ok = T >= 1 and delta < rlo and (delta + self.reach + E) * (1.0 + 1e-12) <= rlo
        return _ru(delta) if ok else np.float32(np.inf)


def pow_int(x, n):
    """x^n by square and multiply (the device's sequence of double products)."""
    r = 1.0
    while n > 0:
        if n & 1:
            r *= x
        x *= x
        n >>= 1
    return r


def midpoint_delta(As_row, T, nx, ny):
    """delta_T of a row's explicit-midpoint replay maps (fields [nC, 6] float32,
    step 1.0f / T as the backward's replay takes it)."""
    h = np.float32(1.0) / np.float32(T)
    hh = float(h * np.float32(0.5))
    acc = Acc()
    for c, a in enumerate(np.asarray(As_row, np.float32).reshape(-1, 6)):
        acc.cell(midpoint_map(a, h), c, nx, ny, midpoint_step_err(a, float(h), hh))
    return acc.delta(T, nx, ny)


def safe_start(points, delta):
    """Per point: inside (0, 1) on both axes and at distance >= delta from each
    edge (edge_safe, in float32 as the device)."""
    x, y = points[0].astype(np.float32), points[1].astype(np.float32)
    one = np.float32(1.0)
    with np.errstate(invalid="ignore"):
        d = np.minimum(np.minimum(x, one - x), np.minimum(y, one - y))
        return (x == x) & (y == y) & (d >= np.float32(delta))
