"""CPU check of the backward's workgroup map (backward_body.hpp, wg_slot), restated
here: for every grid shape it must hand out each logical (part, row) exactly
once, whatever the number of workgroups modulo the 8 XCDs; and at C2's grid
(16 point ranges x 16 thetas) each XCD must serve 4 thetas over half the
ranges.  tests/test_gpu_launch_map.py runs the kernel's own map on the GPU
over grids of these kinds."""


def wg_slot(bx, by, nx, ny, row_block=4):
    n = nx * ny
    lin = by * nx + bx
    x, k, q, r = lin & 7, lin >> 3, n >> 3, n & 7
    L = x * (q + 1) + k if x < r else r * (q + 1) + (x - r) * q + k
    rb = min(ny, row_block)
    full = (ny // rb) * rb * nx
    if L < full:
        blk, rem = divmod(L, rb * nx)
        return rem // rb, blk * rb + rem % rb
    rr, rem = ny - (ny // rb) * rb, L - full
    return rem // rr, (ny // rb) * rb + rem % rr


def test_wg_slot_is_a_bijection():
    for nx in range(1, 41):
        for ny in range(1, 21):
            got = sorted(wg_slot(bx, by, nx, ny) for by in range(ny) for bx in range(nx))
            assert got == sorted((p, r) for p in range(nx) for r in range(ny)), (nx, ny)


def test_wg_slot_groups_rows_per_xcd_at_c2():
    nx = ny = 16
    for xcd in range(8):
        slots = [wg_slot(bx, by, nx, ny) for by in range(ny) for bx in range(nx)
                 if (by * nx + bx) % 8 == xcd]
        assert len({r for _, r in slots}) == 4
        assert len({p for p, _ in slots}) == 8
