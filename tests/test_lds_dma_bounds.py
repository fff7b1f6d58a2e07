"""
The LDS-DMA copies of the token-tile kernels, checked on the CPU.

Every expert kernel stages its token rows through `async_copy16` (gemm_core.h): one
`global_load_lds_dwordx4` per lane with the full 64-bit global address in a VGPR pair
(the "vaddr" form) and the wave-uniform LDS base in M0, the lane landing at M0 + 16 lane.
This file restates, lane by lane, the address arithmetic of the copies in
experts_async.hip -- the forward (`expert_fwd_reg_kernel`), the GLU backward
(`expert_bwd_reg_kernel`, with and without the saved pre-activations) and dX
(`expert_dx_reg_kernel`, and `expert_dx_res_kernel`, which keeps every k-step of its tile
resident) -- and checks for every tile height, wave, lane, copy and k-step:

  * the global source lies inside its tensor ([T, d] rows of x / dout, [rows, 2H] rows of
    dA1) or is the lane's 16 bytes of the 1 KiB zero buffer;
  * the LDS base is wave-uniform (a function of the wave, the copy and the stage only)
    and every lane's 16 bytes land inside the stage, no two lanes of a step on the same
    bytes;
  * the bytes land where the MFMA fragment reads look for them: chunk c of row r at
    r * 64 + ((c ^ swz(r)) << 4) (gemm_core.h sw_off);

and the saved pre-activations' block index (experts_common.h act_block) stays inside the
buffer the host sizes.  The fused router (router.hip) copies its weight whole into LDS the
same way; its copies and its transposed fragment reads are checked against its stage.  A forward variant with a producer-only wave, since removed, faulted
the GPU once; it used the scalar-base ("saddr") form of the copy, a 32-bit vector offset
from a 64-bit scalar base.  The copies kept use the 64-bit vaddr form, whose addresses are
exactly the ones checked here.
"""

import random

import pytest

NT = 256
ROWB = 64          # bytes of one 32-element row of a 16-bit k-step tile
VE = 8             # 16-bit elements per 16-byte chunk


def swz(r):
    """gemm_core.h swz for 16-bit types (4 chunks per row)."""
    return ((r >> 1) ^ (r >> 3)) & 3


def check_step(copies, stage_bytes, rows, T, d, k0):
    """copies: (wave, lane, lds_base, row r, chunk c, token) for one k-step."""
    seen = set()
    for wave, lane, base, r, c, tok in copies:
        off = base + 16 * lane
        assert 0 <= off and off + 16 <= stage_bytes, (wave, lane, off)
        assert off not in seen, ("two lanes on one slot", wave, lane)
        seen.add(off)
        # the fragment reads find chunk c of row r here
        assert off == r * ROWB + ((c ^ swz(r)) << 4), (wave, lane, r, c)
        if tok is not None and r < rows and k0 + c * VE < d:
            assert 0 <= tok < T and k0 + c * VE + VE <= d
    return seen


def fwd_copies(MB):
    """expert_fwd_reg_kernel's token copies of one step: (wave, lane, base, r, c)."""
    TM = 16 * MB
    XC = (TM * 4 + NT - 1) // NT
    XHALF = (TM * 4) % NT != 0
    out = []
    for x in range(XC):
        half = XHALF and x == XC - 1
        for wave in range(4):
            base = 4096 * x + wave * (512 if half else 1024)  # uniform: x, wave only
            for lane in range(64):
                if half and lane >= 32:
                    continue
                r = 64 * x + wave * 8 + lane // 4 if half else 64 * x + (wave * 64 + lane) // 4
                if r >= TM:
                    continue
                out.append((wave, lane, base, r, (lane & 3) ^ swz(r)))
    return out


def bwd_copies(MB):
    """expert_bwd_reg_kernel's copies of one token tile (x or dout) of one step."""
    TM = 16 * MB
    XC = (TM + 63) // 64
    out = []
    for x in range(XC):
        cl = min(64, TM - 64 * x)
        for wave in range(4):
            base = 4096 * x + wave * cl * 16
            for lane in range(cl):
                q = 256 * x + cl * wave + lane
                ar = q >> 2
                out.append((wave, lane, base, ar, (q & 3) ^ swz(ar)))
    return out


def dx_copies(MB):
    """expert_dx_reg_kernel's dA1 copies of one step."""
    out = []
    for wave in range(4):
        for lane in range(64):
            tid = wave * 64 + lane
            ar = tid >> 2
            out.append((wave, lane, wave * 1024, ar, (tid & 3) ^ swz(ar)))
    if MB == 6:
        for wave in range(4):
            for lane in range(32):
                r2 = 64 + wave * 8 + (lane >> 2)
                out.append((wave, lane, 4096 + wave * 512, r2, (lane & 3) ^ swz(r2)))
    return out


@pytest.mark.parametrize("kernel,MB", [("fwd", 2), ("fwd", 4), ("fwd", 6), ("bwd", 3), ("bwd", 4),
                                       ("bwd", 5), ("bwd", 6), ("dx", 4), ("dx", 6)])
@pytest.mark.parametrize("d", [64, 128, 576])
def test_copies_stay_in_bounds_and_match_the_fragment_layout(kernel, MB, d):
    TM = 16 * MB
    copies = {"fwd": fwd_copies, "bwd": bwd_copies, "dx": dx_copies}[kernel](MB)
    # the tile is covered: every (row, chunk) of the TM x 32 tile exactly once
    cover = {(r, c) for _, _, _, r, c in copies}
    assert cover == {(r, c) for r in range(TM) for c in range(4)}
    assert len(cover) == len(copies)
    rng = random.Random(MB * 1000 + d)
    T = 300
    for rows in (1, TM // 2 + 1, TM):
        toks = [rng.randrange(T) for _ in range(TM)]
        for k0 in range(0, d, 32):
            step = [(w, l, b, r, c, toks[r] if r < rows else None)
                    for w, l, b, r, c in copies]
            seen = check_step(step, TM * ROWB, rows, T, d, k0)
            assert len(seen) == len(copies)
    # the LDS base of a copy is one value per (wave, copy): M0 is wave-uniform
    per_wave = {}
    for w, l, b, r, c in copies:
        per_wave.setdefault((w, b), []).append(l)
    for (w, b), lanes in per_wave.items():
        assert sorted(lanes) == list(range(len(lanes)))


@pytest.mark.parametrize("two_h", [64, 128, 192, 256])
def test_dx_resident_tile_fits_its_stages(two_h):
    """expert_dx_res_kernel copies all 2H / 32 k-steps of its 96-row tile up front, k-step
    kk into stage kk of s_tile[8][96 x 64 B]: every copy stays inside the array, no two
    land on the same bytes, and each global chunk stays inside the tile's dA1 rows."""
    TM, KMAX = 96, 8
    nkk = two_h // 32
    assert nkk <= KMAX
    stage = TM * ROWB
    copies = dx_copies(6)
    seen = set()
    for kk in range(nkk):
        for wave, lane, base, r, c in copies:
            off = kk * stage + base + 16 * lane
            assert 0 <= off and off + 16 <= KMAX * stage
            assert off not in seen
            seen.add(off)
            assert off - kk * stage == r * ROWB + ((c ^ swz(r)) << 4)
            assert kk * 32 + c * VE + VE <= two_h  # inside the row's 2H elements
    assert len(seen) == nkk * TM * 4


RT_MAX_STEPS, RT_MAX_E, RT_WAVES = 18, 80, 16   # router_fused.h / router.hip


@pytest.mark.parametrize("d", [32, 64, 288, 576])
@pytest.mark.parametrize("E", [4, 12, 16, 64, 76, 80])
def test_router_weight_copies_and_fragment_reads_stay_in_the_stage(d, E):
    """router_fwd_kernel copies W_r [d, E] whole into s_stage (copy i of a wave: 16-byte
    chunks 64 i .. 64 i + 63 of the weight, landing at 1024 i + 16 lane; chunks past the
    weight read the zero page) and reads the MFMA B fragments with ds_read_b64_tr_b16 at
    row 32 ks + 8 g + 4 h + j / 4, byte 32 nb + 8 (j % 4) of E * 2-byte rows.  Every copy
    and every 8-byte read stays inside the stage; every byte of the weight is copied once
    to its own offset; reads past the weight (padding columns of the last rows) land in
    the zero-filled tail of the last copy or the stage's slack."""
    stage = max(RT_MAX_STEPS * 32 * RT_MAX_E * 2 + 64, RT_WAVES * 256 * 8)
    nb_blocks = (E + 15) // 16
    wbytes = d * E * 2
    assert wbytes % 256 == 0
    nw16 = wbytes // 16
    written = set()
    for wave in range(RT_WAVES):
        i = wave
        while i * 64 < nw16:
            for lane in range(64):
                c = i * 64 + lane
                off = i * 1024 + 16 * lane
                assert off + 16 <= stage
                if c < nw16:
                    assert off == c * 16  # chunk c of the weight at its own offset
                    written.add(c)
            i += RT_WAVES
    assert written == set(range(nw16))
    filled = -(-nw16 // 64) * 1024  # bytes the copies cover, zero-filled past the weight
    ep = E * 2
    nbh = -(-nb_blocks // 2)
    for cb0 in (0, nbh):
        for nb in range(cb0, min(cb0 + nbh, nb_blocks)):
            for ks in range(d // 32):
                for g in range(4):
                    for j in range(16):
                        for h in (0, 1):
                            off = (32 * ks + 8 * g + 4 * h + j // 4) * ep + 32 * nb + 8 * (j % 4)
                            assert off % 8 == 0 and off + 8 <= stage
                            col = 16 * nb + 4 * (j % 4)
                            if col < E:  # a real column: inside the weight's row
                                assert off + 8 <= (32 * ks + 8 * g + 4 * h + j // 4 + 1) * ep
                            else:      # padding column: read but dropped
                                assert off + 8 <= max(filled, wbytes + 64)


def test_backward_tiles_fit_their_ring_stages():
    """Without the saved pre-activations a stage holds x then dout (2 tiles); with them
    dout alone at offset 0.  Both stay inside S stages of the ring."""
    for MB in (3, 4, 5, 6):
        TM = 16 * MB
        for D in (2, 3, 4):
            S = D + 1
            for sa in (False, True):
                na = 1 if sa else 2
                doff = 0 if sa else TM * ROWB
                ring = S * na * TM * ROWB
                top = (S - 1) * na * TM * ROWB + doff + TM * ROWB
                assert top <= ring


def act_block(offs, E, l_cap, T, g, r):
    start = offs[g] if g < E else l_cap + (g - E) * (-(-T // 16) * 16)
    return (start + r) // 16


@pytest.mark.parametrize("T,E,S,k", [(1, 8, 2, 2), (300, 76, 2, 6), (8192, 76, 2, 6),
                                     (257, 12, 1, 4), (64, 76, 0, 6)])
def test_saved_pre_activation_blocks_stay_in_the_buffer(T, E, S, k):
    """Every 16-row block a tile of any height reads or writes (experts_common.h
    act_block) lies inside the l_cap / 16 + S ceil(T / 16) blocks the host allocates."""
    rng = random.Random(T + E)
    counts = [0] * E
    for _ in range(T * k):
        counts[rng.randrange(E)] += 1
    offs = [0]
    for c in counts:
        offs.append(offs[-1] + -(-c // 16) * 16)
    nonempty = min(T * k, E)
    l_cap = -(-(T * k + nonempty * 15) // 16) * 16
    assert offs[E] <= l_cap
    nblocks = l_cap // 16 + S * (-(-T // 16))
    for TM in (48, 64, 80, 96):
        for g in range(E + S):
            rows = counts[g] if g < E else T
            for m0 in range(0, rows, TM):
                for i in range(TM // 16):
                    if m0 + 16 * i >= rows:
                        break
                    assert 0 <= act_block(offs, E, l_cap, T, g, m0 + 16 * i) < nblocks
