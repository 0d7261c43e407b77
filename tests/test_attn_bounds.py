"""Index bounds of the decode attention kernels, modelled on the CPU (no GPU).

Every global and LDS index the kernels below compute is enumerated over the whole grid, every
thread and every unrolled load, for each model shape the library runs (the BASELINE configs and
the test models) and positions on both sides of each chunk boundary, and checked against the
extent of its buffer: the per-layer caches K [kvd][max_seq] and V [max_seq][kvd], the scores
att [n_heads][max_seq], q and out [n_heads*head_dim], and the dynamic LDS bytes the launcher
passes. The formulas restate the kernels' own index arithmetic, line by line:
  * k_attn_scores<HD>     quillm_amd/csrc/qmh_attn.hip:25-68 (launcher :70-88)
  * k_attn_scores_t<HD>   quillm_amd/csrc/qmh_ops.hip:431-464 (launcher :467-480): clamped float4 K
                          loads past the last position (t <= max_seq-4)
  * attn_pv_chunks<TC,M>  quillm_amd/csrc/qmh_attn.hip:100-257 (k_attn_pv :259-266): unconditional V
                          and score loads clamped to position n-1 / score 0, columns to head_dim-1
  * pv_mha_long<LA>       quillm_amd/csrc/qmh_attn.hip:274-379: exponentials of up to 8192 positions,
                          V pieces of 128 positions loaded LA pieces ahead (clamped to the last piece
                          and position n-1), two staged buffers
  * k_attn_pv_mha<640>    quillm_amd/csrc/qmh_attn.hip:502-553: one workgroup per query head, float4 V
                          loads of its kv head clamped to position n-1 and column head_dim-4
  * qmh_launch_attn_pv    quillm_amd/csrc/qmh_attn.hip:900-924: kernel choice and dynamic LDS
  * k_attn_fused<HD,TC,CW> quillm_amd/csrc/qmh_attn.hip:682-813, its V sum pv_short_flow :561-645 (the
                          one-launch attention for n <= TC, TC 640 for head_dim 48/64/128 and 1024
                          for head_dim 64/128 (48 too at CW 8), CW = 16 or 8 output columns per
                          workgroup): the K slice of each workgroup (clamped float4s), its LDS rows,
                          the epoch-tagged score words, and that the slices of a head's workgroups
                          cover its n positions exactly once (a position nobody writes would leave
                          its readers waiting until their bounded wait runs out)
This is a model: a kernel edit that changes an index must change it here too.
"""
import numpy as np
import pytest

WG, SC_T, CW = 256, 64, 16

# (n_heads, n_kv_heads, head_dim, max_seq): BASELINE configs c1-c5 and the test models
SHAPES = [
    (6, 6, 48, 256), (6, 2, 48, 256), (12, 12, 64, 1024), (32, 4, 64, 2048), (32, 32, 128, 4096),
    (4, 2, 16, 64), (6, 3, 12, 64), (3, 3, 32, 48), (12, 1, 8, 300), (4, 2, 48, 136),
    (2, 2, 128, 1300), (6, 6, 10, 700), (4, 2, 32, 700), (32, 32, 128, 640),
    (4, 2, 16, 9000), (2, 2, 16, 9000), (8, 1, 12, 8192), (4, 4, 64, 8193),
    # groups past 16 query heads per kv head: the kv-head P.V kernel in sub-groups of 16
    (20, 1, 10, 300), (32, 1, 64, 1040), (40, 2, 6, 700), (32, 1, 16, 9000),
]
POSITIONS = [0, 1, 2, 3, 63, 64, 65, 127, 128, 129, 255, 256, 257, 383, 384, 511, 512, 575, 639, 640, 641, 700,
             767, 768, 1023, 1024, 1279, 1280, 1281, 2047, 4095, 8191, 8192, 8193, 8900]


def positions(S):
    return sorted({p for p in POSITIONS if p < S} | {S - 2, S - 1} - {-1})


class Extents:
    def __init__(self, nh, nkv, hd, S):
        self.K = nkv * hd * S
        self.V = S * nkv * hd
        self.att = nh * S
        self.q = nh * hd
        self.out = nh * hd


def inb(what, idx, size):
    idx = np.asarray(idx)
    if idx.size == 0:
        return
    lo, hi = int(idx.min()), int(idx.max())
    assert lo >= 0 and hi < size, f"{what}: index range [{lo}, {hi}] outside [0, {size})"


def scores(nh, nkv, hd, S, pos, ext):
    """qmh_launch_attn_scores: the K-tile kernel for grouped heads, else the one-wave kernel."""
    group = nh // nkv
    t0 = np.arange(0, S, SC_T)  # blockIdx.y * 64
    t0 = t0[t0 <= pos]  # workgroups past pos return at once
    kvh = np.arange(nkv)
    if nh > nkv and S % 4 == 0 and S >= 4 and hd in (128, 64, 48):
        L4 = hd * SC_T // 4 // WG
        e = (np.arange(L4)[:, None] * WG + np.arange(WG)[None, :]).ravel()
        i, p4 = e // (SC_T // 4), e % (SC_T // 4)
        t = t0[:, None] + 4 * p4[None, :]
        tc = np.minimum(t, S - 4)
        for r in range(4):  # the float4's four floats
            inb("scores_t K", kvh[:, None, None] * hd * S + i[None, None, :] * S + tc[None, :, :] + r, ext.K)
        inb("scores_t LDS kt", i * SC_T + 4 * p4 + 3, hd * SC_T)
        lane = np.arange(64)
        inb("scores_t LDS read", (hd - 1) * SC_T + lane, hd * SC_T)
    else:
        lane = np.arange(SC_T)
        t = t0[:, None] + lane[None, :]
        tc = np.minimum(t, S - 1)
        d = np.arange(hd)
        inb("scores K", kvh[:, None, None] * hd * S + d[None, :, None] * S + tc.ravel()[None, None, :], ext.K)
    hl = np.arange(group)
    inb("scores q", (kvh[:, None] * group + hl[None, :]) * hd + hd - 1, ext.q)
    tw = (t0[:, None] + np.arange(SC_T)[None, :]).ravel()
    tw = tw[tw <= pos]
    inb("scores att", (kvh[:, None, None] * group + hl[None, :, None]) * S + tw[None, None, :], ext.att)


def pv_chunks(TC, MHA, nh, nkv, hd, S, n, ext, lds_floats):
    """attn_pv_chunks<TC, MHA> over grid (nkv * ceil(group/16), ceil(hd/16)) x 256 threads: workgroup x
    takes kv head x / nsub and query heads hb .. hb + gs - 1 of it, hb = kvh*group + 16*(x % nsub)."""
    group, kvd = nh // nkv, hd * nkv
    for sub in range((group + 15) // 16):
        pv_chunks_sub(TC, MHA, nh, nkv, hd, S, n, ext, lds_floats, sub)


def pv_chunks_sub(TC, MHA, nh, nkv, hd, S, n, ext, lds_floats, sub):
    group, kvd = nh // nkv, hd * nkv
    gsm = min(group, 16)
    gs = min(16, group - 16 * sub)
    assert gs >= 1 and gs * CW <= WG
    tid = np.arange(WG)
    kvh = np.arange(nkv)
    hb = kvh * group + 16 * sub  # first query head of each workgroup
    i0 = np.arange(0, hd, CW)
    # first head's scores, 4 per thread, clamped to 0
    t = tid[None, :] + WG * np.arange(4)[:, None]
    inb("pv sv", hb[:, None] * S + np.where(t < n, t, 0).ravel()[None, :], ext.att)
    LPT = TC * CW // WG
    e = (np.arange(LPT)[:, None] * WG + tid[None, :]).ravel()
    te, cce = e // CW, e % CW
    colc_e = np.minimum(i0[:, None] + (e % CW)[None, :], hd - 1)  # e % 16 == threadIdx % 16
    for T0 in range(0, n, TC):
        tcl = np.minimum(T0 + te, n - 1)
        inb("pv V", tcl[None, None, :] * kvd + kvh[:, None, None] * hd + colc_e[None, :, :], ext.V)
        nt = min(TC, n - T0)
        if not (MHA and T0 == 0):
            hl, tt = e[e < gs * TC] // TC, e[e < gs * TC] % TC
            inb("pv P", hl * TC + tt, gsm * TC)
            tt_on = tt < nt
            inb("pv att", (hb[:, None] + hl[None, tt_on]) * S + T0 + tt[None, tt_on], ext.att)
            # the sub-group's heads stay inside the kv head's group
            assert (hl < gs).all() and 16 * sub + gs <= group
        else:
            tp = tid[None, :] + WG * np.arange(4)[:, None]
            inb("pv P first", tp[tp < TC], gsm * TC)
        inb("pv Vs", gsm * TC + cce * (TC + 4) + te, lds_floats)
        n32 = (nt + 31) >> 5
        last = 4 * (8 * (n32 - 1) + 7) + 3
        chain = tid[tid < gs * CW]
        inb("pv chain P", (chain // CW) * TC + last, gsm * TC)
        inb("pv chain Vs", gsm * TC + (chain % CW) * (TC + 4) + last, lds_floats)
    ch = tid[tid < gs * CW]
    col = ch % CW
    ok = (i0[:, None] + col[None, :]) < hd
    outi = (hb[:, None, None] + (ch // CW)[None, None, :]) * hd + i0[None, :, None] + col[None, None, :]
    inb("pv out", outi[np.broadcast_to(ok[None], outi.shape)], ext.out)


def pv_mha(TC, nh, nkv, hd, S, n, ext, lds_floats):
    """k_attn_pv_mha<TC> for n <= TC over grid (nh, ceil(hd/16)) x 256 threads."""
    kvd = hd * nkv
    tid = np.arange(WG)
    h = np.arange(nh)
    kvh = h // (nh // nkv)
    i0 = np.arange(0, hd, CW)
    SK = (TC + WG - 1) // WG
    t = tid[None, :] + WG * np.arange(SK)[:, None]
    inb("mha sv", h[:, None] * S + np.where(t < n, t, 0).ravel()[None, :], ext.att)
    c = i0[:, None] + 4 * (tid & 3)[None, :]
    cc = np.where(c <= hd - 4, c, hd - 4)
    L4 = TC * CW // 4 // WG
    tv = np.arange(L4)[:, None] * (WG // 4) + (tid >> 2)[None, :]
    tcl = np.minimum(tv, n - 1)
    for r in range(4):  # the float4's four floats
        inb("mha V", tcl[None, None, :, :] * kvd + kvh[:, None, None, None] * hd + cc[None, :, None, :] + r, ext.V)
    inb("mha P", np.arange(n), TC)
    PC = 128
    npc = (n + PC - 1) // PC
    for j in range(npc):
        for u in range(2):
            ts = (2 * j + u) * (WG // 4) + (tid >> 2)
            assert ts.max() < TC
            for r in range(4):
                inb("mha Vs stage", TC + (4 * (tid & 3) + r) * (TC + 4) + ts, lds_floats)
        q = np.arange(PC // 4)
        inb("mha chain", TC + np.arange(CW)[:, None] * (TC + 4) + 4 * (j * (PC // 4) + q)[None, :] + 3, lds_floats)
    # float4 staging rows and chain rows stay 16-byte aligned
    assert (TC % 4, (TC + 4) % 4) == (0, 0)
    mha_out(nh, hd, ext)


def mha_out(nh, hd, ext):
    h, i0 = np.arange(nh), np.arange(0, hd, CW)
    ok = (i0[:, None] + np.arange(CW)[None, :]) < hd
    outi = h[:, None, None] * hd + i0[None, :, None] + np.arange(CW)[None, None, :]
    inb("mha out", outi[np.broadcast_to(ok[None], outi.shape)], ext.out)


PV_LONG, LA = 8192, 3


def pv_mha_long(nh, nkv, hd, S, n, ext, lds_floats):
    """pv_mha_long<3> for TC < n <= 8192, called by k_attn_pv_mha with P at LDS float 0 and the two
    staged buffers at float 8192."""
    kvd = hd * nkv
    tid = np.arange(WG)
    h = np.arange(nh)
    kvh = h // (nh // nkv)
    i0 = np.arange(0, hd, CW)
    PC, VS = 128, 132
    npc = (n + PC - 1) // PC
    c = i0[:, None] + 4 * (tid & 3)[None, :]
    cc = np.where(c <= hd - 4, c, hd - 4)
    # every piece index vload is given: the first LA (clamped to npc-1), then j+LA clamped
    js = sorted({min(k, npc - 1) for k in range(LA)} | {min(j + LA, npc - 1) for j in range(npc + LA)})
    for j in js:
        for u in range(2):
            t = (2 * j + u) * (WG // 4) + (tid >> 2)
            tcl = np.minimum(t, n - 1)
            for r in range(4):
                inb("long V", tcl[None, None, :] * kvd + (kvh[:, None] * hd)[:, :, None] + cc[None, :, :] + r, ext.V)
    inb("long scores", h[:, None] * S + np.arange(n)[None, :], ext.att)
    inb("long P", np.arange(n), PV_LONG)
    # staging of pieces 0 .. npc (the last piece's successor stages zeros); reads of P only below n
    for j in range(npc + 1):
        b = j & 1
        for u in range(2):
            tl = u * (WG // 4) + (tid >> 2)
            t = j * PC + tl
            inb("long P stage", t[t < n], PV_LONG)
            for r in range(4):
                inb("long stage", PV_LONG + b * CW * VS + (4 * (tid & 3) + r) * VS + tl, lds_floats)
    for j in range(npc):
        inb("long chain", PV_LONG + (j & 1) * CW * VS + np.arange(CW)[:, None] * VS + 4 * np.arange(PC // 4)[None, :] + 3,
            lds_floats)
    assert VS % 4 == 0 and PV_LONG % 4 == 0
    mha_out(nh, hd, ext)


LDS_MAX = 160 * 1024 - 1024  # per workgroup on gfx950, less the kernels' static LDS

AF_TC = 640
AF_TC2 = 1024  # the second instance (head_dim 64 and 128)


def af_instances(hd, cw=CW):
    """The instances (their TC) qmh_attn_fused_supported can return for a head size and column width
    (af_kernel_cw)."""
    if hd not in (48, 64, 128):
        return []
    return [AF_TC, AF_TC2] if hd in (64, 128) or cw == 8 else [AF_TC]


def af_lds_floats(hd, TC, cw=CW):
    ncg = hd // cw
    spm = ((TC + ncg - 1) // ncg + 3) // 4 * 4
    return max(spm * (hd + 4), TC + cw * (TC + 4))


def fused(nh, nkv, hd, S, n, ext, TC=AF_TC, cw=CW):
    """k_attn_fused<HD,TC,CW> over its (head, column group) workgroups x 256 threads (the grid's
    placement: af_grid_map), n <= TC positions: every thread loads its
    part of the K slice and its V float4s (as k_attn_pv_mha, TPP = CW/4 threads per position), the
    threads below the slice's position count run the score chains, every thread reads the head's
    scores, stages its products for all TC positions, and the first CW threads run the V sum's chains
    (pv_short_flow)."""
    assert cw in (16, 8) and TC in af_instances(hd, cw) and S % 4 == 0 and S >= 4 and n <= min(TC, S)
    AF_TC = TC
    ncg, kvd = hd // cw, hd * nkv
    TPP = cw // 4
    PR = WG // TPP
    spm = ((AF_TC + ncg - 1) // ncg + 3) // 4 * 4
    KS, KL4 = hd + 4, (spm // 4 * hd + WG - 1) // WG
    L4, SK, VS = AF_TC * cw // 4 // WG, (AF_TC + WG - 1) // WG, AF_TC + 4
    assert spm <= WG and L4 * PR == AF_TC
    lds = af_lds_floats(hd, TC, cw)
    assert 4 * lds <= LDS_MAX
    tid = np.arange(WG)
    inb("af q", np.arange(nh)[:, None] * hd + 4 * tid[tid < hd // 4][None, :] + 3, ext.q)
    sp = ((n + ncg - 1) // ncg + 3) & ~3
    covered = np.zeros(n, dtype=np.int64)
    for cg in range(ncg):
        p0 = cg * sp
        npos = max(min(n - p0, sp), 0)
        np4 = (npos + 3) >> 2
        np4d = max(np4, 1)
        assert 4 * np4 <= spm
        e = (np.arange(KL4)[:, None] * WG + tid[None, :]).ravel()
        d = np.minimum(e // np4d, hd - 1)
        t = p0 + 4 * (e % np4d)
        tc = np.minimum(t, S - 4)
        for kvh in range(nkv):
            for r in range(4):
                inb("af K", kvh * hd * S + d * S + tc + r, ext.K)
        on = e < np4 * hd
        for j in range(4):
            inb("af K LDS", (4 * (e[on] % np4d) + j) * KS + e[on] // np4d, lds)
        rows = tid[tid < npos]
        inb("af chain LDS", rows * KS + hd - 1, lds)
        for h in range(nh):
            inb("af score word", h * S + p0 + rows, ext.att)
        covered[p0 + rows] += 1
        # V: position k*PR + tid/TPP clamped to n-1, columns i0 + 4*(tid%TPP) clamped to hd-4
        c = cg * cw + 4 * (tid % TPP)
        cc = np.where(c <= hd - 4, c, hd - 4)
        tv = np.minimum(np.arange(L4)[:, None] * PR + (tid // TPP)[None, :], n - 1)
        for kvh in range(nkv):
            for r in range(4):
                inb("af V", tv * kvd + kvh * hd + cc[None, :] + r, ext.V)
    assert (covered == 1).all(), "every position's score is written by exactly one workgroup"
    t = tid[None, :] + WG * np.arange(SK)[:, None]
    inb("af poll", np.arange(nh)[:, None] * S + t[t < n][None, :], ext.att)
    inb("af P", t[t < n], AF_TC)
    # staging: every thread, positions k*PR + tid/TPP (all < TC), rows 4*(tid%TPP) + r of Vs
    ts = np.arange(L4)[:, None] * PR + (tid // TPP)[None, :]
    assert ts.max() < AF_TC
    inb("af P read", ts[ts < n], AF_TC)
    for r in range(4):
        inb("af stage", AF_TC + (4 * (tid % TPP) + r)[None, :] * VS + ts, lds)
    # every (column, position) cell below TC staged exactly once
    cells = np.zeros((cw, AF_TC), dtype=np.int64)
    for r in range(4):
        np.add.at(cells, (np.broadcast_to((4 * (tid % TPP) + r)[None, :], ts.shape), ts), 1)
    assert (cells == 1).all()
    # chains: CW lanes, 32-position steps up to the last holding a position below n
    nst = (n + 31) >> 5
    inb("af chain", AF_TC + np.arange(cw)[:, None] * VS + 4 * (8 * (nst - 1) + np.arange(8))[None, :] + 3, lds)
    assert 32 * nst <= AF_TC
    mha_out(nh, hd, ext)


def pv(nh, nkv, hd, S, pos, ext):
    """qmh_launch_attn_pv's choice of kernel and dynamic LDS bytes."""
    group = nh // nkv
    n = pos + 1
    if hd % 4 == 0 and (group == 1 or S <= PV_LONG):
        lds_floats = max(640 + CW * (640 + 4), PV_LONG + 2 * CW * (128 + 4))
        assert 4 * lds_floats <= LDS_MAX
        if n <= 640:
            pv_mha(640, nh, nkv, hd, S, n, ext, lds_floats)
        elif n <= PV_LONG:
            pv_mha_long(nh, nkv, hd, S, n, ext, lds_floats)
        else:
            assert group == 1  # the kernel's chunked fallback is for one query head per kv head
            pv_chunks(640, True, nh, nh, hd, S, n, ext, lds_floats)
        return
    TC, MHA = (640, True) if group == 1 else (640, False) if group <= 8 else (256, False)
    lds_floats = min(group, 16) * TC + CW * (TC + 4)
    assert 4 * lds_floats <= LDS_MAX
    pv_chunks(TC, MHA, nh, nkv, hd, S, n, ext, lds_floats)


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_decode_attention_indices_in_bounds(shape):
    nh, nkv, hd, S = shape
    ext = Extents(nh, nkv, hd, S)
    for pos in positions(S):
        scores(nh, nkv, hd, S, pos, ext)
        pv(nh, nkv, hd, S, pos, ext)
        # the one-launch kernel: shapes qmh_attn_fused_supported takes, each instance at the
        # positions the host gives it (below 640: the first; 640..1023: the second) and the first
        # at every position below 640
        if S % 4 == 0 and S >= 4:
            for cw in (16, 8):
                for TC in af_instances(hd, cw):
                    if pos + 1 <= TC:
                        fused(nh, nkv, hd, S, pos + 1, ext, TC, cw)


@pytest.mark.parametrize("cw", [16, 8])
@pytest.mark.parametrize("TC", [AF_TC, AF_TC2])
def test_fused_slices_cover_every_position(TC, cw):
    """Every n in 1..TC and every head_dim the instance takes: its workgroups' score slices
    cover positions 0..n-1 once each (fused() asserts it), here with the other checks too."""
    for hd in (48, 64, 128):
        if TC not in af_instances(hd, cw):
            continue
        ext = Extents(2, 1, hd, TC)
        for n in range(1, TC + 1):
            fused(2, 1, hd, TC, n, ext, TC, cw)


def af_grid_map(nh, hd, cw=CW):
    """k_attn_fused's one-dimensional grid: 8 * ceil(nh/8) * (hd/cw) workgroups; workgroup L takes
    head (L % 8) * ceil(nh/8) + (L / 8) / ncg, column group (L / 8) % ncg, and returns when the head
    is past nh. (h, cg) of each workgroup, -1 for the ones that return."""
    ncg = hd // cw
    hpx = (nh + 7) // 8
    G = 8 * hpx * ncg
    L = np.arange(G)
    h = (L & 7) * hpx + (L >> 3) // ncg
    cg = (L >> 3) % ncg
    return L, np.where(h < nh, h, -1), np.where(h < nh, cg, -1)


@pytest.mark.parametrize("cw", [16, 8])
@pytest.mark.parametrize("nh", [1, 2, 4, 6, 8, 12, 25, 32, 64])
@pytest.mark.parametrize("hd", [48, 64, 128])
def test_fused_grid_places_each_head_on_one_xcd(nh, hd, cw):
    """Every (head, column group) has exactly one workgroup, and a head's workgroups have one
    dispatch slot modulo 8 (the XCD the round-robin dispatcher gives them). The heads of one XCD
    are consecutive, so the query heads that share a kv head share as few XCDs as possible:
    ceil(group / heads per XCD) + 1 at most."""
    L, h, cg = af_grid_map(nh, hd, cw)
    live = h >= 0
    pairs = h[live] * (hd // cw) + cg[live]
    assert np.array_equal(np.sort(pairs), np.arange(nh * (hd // cw)))
    for head in range(nh):
        assert len(set((L[h == head] % 8).tolist())) == 1
    hpx = (nh + 7) // 8
    for x in range(8):
        hs = sorted(set(h[live & (L % 8 == x)].tolist()))
        assert hs == list(range(x * hpx, x * hpx + len(hs)))
    for group in (1, 2, 4, 8):
        if nh % group == 0:
            for kvh in range(nh // group):
                xcds = set((L[live & (h // group == kvh)] % 8).tolist())
                assert len(xcds) <= -(-group // hpx) + 1


def test_model_catches_an_out_of_range_clamp():
    """The check is not vacuous: in the K-tile kernel with max_seq = 136, the last tile's float4s
    start at positions 128 .. 188; clamped to max_seq-1 instead of max_seq-4 the last one reads
    three floats past the cache."""
    nh, nkv, hd, S = 4, 2, 48, 136
    t = 128 + 4 * np.arange(16)
    K = Extents(nh, nkv, hd, S).K
    inb("kept clamp", (nkv - 1) * hd * S + (hd - 1) * S + np.minimum(t, S - 4) + 3, K)
    with pytest.raises(AssertionError):
        inb("planted clamp", (nkv - 1) * hd * S + (hd - 1) * S + np.minimum(t, S - 1) + 3, K)


def test_model_catches_a_wrong_kv_head():
    """Grouped heads read V of kv head h // group with row stride head_dim * n_kv: taking the query
    head's index and stride instead runs past the cache."""
    nh, nkv, hd, S = 4, 2, 16, 700
    ext = Extents(nh, nkv, hd, S)
    pv_mha_long(nh, nkv, hd, S, S, ext, PV_LONG + 2 * CW * 132)
    with pytest.raises(AssertionError):
        pv_mha_long(nh, nh, hd, S, S, ext, PV_LONG + 2 * CW * 132)
