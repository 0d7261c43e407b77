"""Index bounds of the batched decode attention and the prefill attention tile kernels, modelled on
the CPU (no GPU), as tests/test_attn_bounds.py does for the single-sequence decode kernels.

Every global and LDS index is enumerated over the whole grid and every thread, for the model shapes
the batched paths take (head_dim <= 128, a multiple of 4), several sequence counts and mixed
positions, and checked against its buffer's extent:
  * qmh_launch_bt_attention  quillm_amd/csrc/qmh_batch.hip:222-248: the kernel choice by B, shape
                             and the largest position
  * k_attn_scores<HD> and k_attn_pv_mha<640> over blockIdx.z (qmh_launch_attn_batch,
                             quillm_amd/csrc/qmh_attn.hip:930-950): sequence z at q + z*n_heads*hd,
                             caches at + z*kv_stride, scores at + z*n_heads*max_seq, position pos[z]
  * k_bt_scores / k_bt_softmax / k_bt_pv  quillm_amd/csrc/qmh_batch.hip:16-117
  * k_bt_attn                quillm_amd/csrc/qmh_batch.hip:129-219 (V chunks of 128 positions
                             clamped to position n-1, the scores and probabilities in LDS after the
                             staged V, LDS of BT_FC*128 + max_pos + 1 floats)
  * qmh_launch_pf_attention  quillm_amd/csrc/qmh_prefill.hip:1461-1494, with k_pf_scores_rb<HD>
                             (:1057-1130), k_pf_softmax_r<R> (:1169-1209) and k_pf_pv_rb<HD>
                             (:1320-1459, the quadrant-reversed token groups and Wo's quantized
                             image)
The batched caches are [n_layers][B][kvd * max_seq] (qmh_batch_create, kv_stride = kvd*max_seq,
quillm_amd/host/qmh_host.c:1337): a sequence's index past its own stride would read the next
sequence's cache (or, for the last one, past the allocation), so the checks hold each sequence
to its own stride. This is a model: a kernel edit that changes an index must change it here too.
"""
import numpy as np
import pytest

from test_attn_bounds import CW, LDS_MAX, SC_T, WG, Extents, inb, pv, scores

BT_T, BT_FC, BT_FUSE_MAX, BT_DECODE_B, BT_VC = 1024, 128, 16384, 3, 64
PF_VC, PF_TOK = 64, 16

# (n_heads, n_kv_heads, head_dim, max_seq): the batched paths' shapes (head_dim <= 128, multiple of 4)
SHAPES = [
    (6, 6, 48, 256), (6, 2, 48, 256), (12, 12, 64, 1024), (32, 4, 64, 2048), (32, 32, 128, 640),
    (4, 2, 16, 64), (3, 3, 32, 48), (12, 1, 8, 300), (4, 2, 48, 136), (2, 2, 128, 1300), (4, 2, 32, 700),
]


def seq_positions(S, B, seed):
    """B positions in [0, S): mixed, with the first at S-1 and the second at 0 when B allows."""
    rng = np.random.default_rng(seed)
    p = rng.integers(0, S, size=B)
    p[0] = S - 1
    if B > 1:
        p[1] = 0
    return p


class BExt:
    """Extents of the batched step's buffers: B sequences of q/out (n_heads*hd), scores
    (n_heads*max_seq) and caches (one stride each)."""

    def __init__(self, nh, nkv, hd, S, B):
        self.stride = nkv * hd * S
        self.K = self.V = B * self.stride
        self.q = self.out = B * nh * hd
        self.att = B * nh * S


def in_seq(what, idx, b, stride):
    """the index of sequence b stays in its own cache region"""
    idx = np.asarray(idx)
    if idx.size:
        assert idx.min() >= b * stride and idx.max() < (b + 1) * stride, f"{what}: sequence {b} leaves its cache"


def attn_batch(nh, nkv, hd, S, pos, e):
    """qmh_launch_attn_batch: the single-sequence kernels with blockIdx.z = sequence. Each sequence's
    indices are the single-sequence kernels' (checked by their own models against one sequence's
    extents) plus the sequence's base offsets, which must keep it inside its own region."""
    one = Extents(nh, nkv, hd, S)
    assert one.K == e.stride and one.V == e.stride  # kv_stride = kvd * max_seq holds one sequence
    for z, p in enumerate(pos):
        scores(nh, nkv, hd, S, int(p), one)
        pv(nh, nkv, hd, S, int(p), one)
        # the z bases of the two kernels (k_attn_scores: q, Kt, att; k_attn_pv_mha: att, V, out)
        inb("batch q base", z * nh * hd + one.q - 1, e.q)
        inb("batch att base", z * nh * S + one.att - 1, e.att)
        inb("batch out base", z * nh * hd + one.out - 1, e.out)
        in_seq("batch K base", z * e.stride + np.array([0, one.K - 1]), z, e.stride)


def bt_scores(nh, nkv, hd, S, pos, e):
    """k_bt_scores over grid (n_heads, B, max_pos/256 + 1) x 256 threads."""
    group, D = nh // nkv, nh * hd
    nz = int(pos.max()) // WG + 1
    tid = np.arange(WG)
    assert hd <= 256  # qs[256]
    for b, p in enumerate(pos):
        for z in range(nz):
            if z * WG > p:
                continue
            t = z * WG + tid
            for h in range(nh):
                inb("bt q", b * D + h * hd + tid[tid < hd], e.q)
                tt = t[t <= p]
                kvh = h // group
                d = np.minimum(np.arange(((hd + 63) // 64) * 64), hd - 1)
                k = b * e.stride + kvh * hd * S + tt[None, :] + d[:, None] * S
                inb("bt K", k, e.K)
                in_seq("bt K", k, b, e.stride)
                inb("bt att", (b * nh + h) * S + tt, e.att)


def bt_softmax(nh, S, pos, e):
    """k_bt_softmax over grid (n_heads, B) x 256 threads: the row of (sequence, head) in place."""
    for b, p in enumerate(pos):
        n = int(p) + 1
        for h in range(nh):
            inb("bt softmax row", (b * nh + h) * S + np.arange(n), e.att)


def bt_pv(nh, nkv, hd, S, pos, e):
    """k_bt_pv over grid (n_heads, B) x 256 threads: V through LDS 64 positions at a time."""
    group, kvd, hd4 = nh // nkv, nkv * hd, hd // 4
    VR = BT_VC * 32 // WG
    tid = np.arange(WG)
    ek = (np.arange(VR)[:, None] * WG + tid[None, :]).ravel()
    t_l, c4 = ek >> 5, ek & 31
    inb("bt pv LDS vs", t_l * 128 + 4 * c4 + 3, BT_VC * 128)
    for b, p in enumerate(pos):
        n = int(p) + 1
        for h in range(nh):
            kvh = h // group
            for c0 in range(0, n, BT_VC):
                tc = np.minimum(c0 + t_l, n - 1)
                on = c4 < hd4
                v = b * e.stride + kvh * hd + tc[on] * kvd + 4 * c4[on] + 3
                inb("bt pv V", v, e.V)
                in_seq("bt pv V", v, b, e.stride)
                pr = c0 + tid[tid < BT_VC]
                inb("bt pv P", (b * nh + h) * S + pr[pr < n], e.att)
            inb("bt pv out", b * nh * hd + h * hd + tid[tid < hd], e.out)


def bt_attn(nh, nkv, hd, S, pos, e):
    """k_bt_attn over grid (n_heads, B) x 1024 threads, LDS BT_FC*128 + max_pos + 1 floats."""
    group, kvd, hd4 = nh // nkv, nkv * hd, hd // 4
    max_pos = int(pos.max())
    lds = BT_FC * 128 + max_pos + 1
    assert 4 * lds <= LDS_MAX
    VR = BT_FC * 32 // BT_T
    tid = np.arange(BT_T)
    ek = (np.arange(VR)[:, None] * BT_T + tid[None, :]).ravel()
    t_l, c4 = ek >> 5, ek & 31
    inb("bt attn LDS vs", t_l * 128 + 4 * c4 + 3, BT_FC * 128)
    for b, p in enumerate(pos):
        n = int(p) + 1
        assert n <= max_pos + 1
        inb("bt attn LDS P", BT_FC * 128 + np.arange(n), lds)
        for h in range(nh):
            kvh = h // group
            inb("bt attn q", b * nh * hd + h * hd + tid[tid < hd], e.q)
            for c0 in range(0, n, BT_FC):
                tc = np.minimum(c0 + t_l, n - 1)
                on = c4 < hd4
                v = b * e.stride + kvh * hd + tc[on] * kvd + 4 * c4[on] + 3
                inb("bt attn V", v, e.V)
                in_seq("bt attn V", v, b, e.stride)
                inb("bt attn P read", BT_FC * 128 + np.minimum(c0 + t_l, n - 1), lds)
            for t0 in range(0, n, BT_T):
                t = t0 + tid[(t0 + (tid & ~63)) < n]  # whole waves past n leave
                tc = np.minimum(t, n - 1)
                d = np.minimum(np.arange(((hd + 31) // 32) * 32), hd - 1)
                k = b * e.stride + kvh * hd * S + d[:, None] * S + tc[None, :]
                inb("bt attn K", k, e.K)
                in_seq("bt attn K", k, b, e.stride)
            inb("bt attn out", b * nh * hd + h * hd + tid[tid < hd], e.out)


def bt_attention(nh, nkv, hd, S, pos, split=0):
    """qmh_launch_bt_attention's choice for B sequences at positions pos."""
    B = len(pos)
    e = BExt(nh, nkv, hd, S, B)
    assert 4 <= hd <= 128 and hd % 4 == 0 and nh % nkv == 0 and 0 <= pos.max() < S
    if split == 0 and B <= BT_DECODE_B and nh == nkv and hd in (128, 64, 48):
        attn_batch(nh, nkv, hd, S, pos, e)
        return "single-sequence kernels"
    if split != 1 and pos.max() < BT_FUSE_MAX:
        bt_attn(nh, nkv, hd, S, pos, e)
        return "k_bt_attn"
    bt_scores(nh, nkv, hd, S, pos, e)
    bt_softmax(nh, S, pos, e)
    bt_pv(nh, nkv, hd, S, pos, e)
    return "three kernels"


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("B", [1, 2, 3, 4, 16])
def test_batched_decode_attention_indices_in_bounds(shape, B):
    nh, nkv, hd, S = shape
    for seed in range(2):
        pos = seq_positions(S, B, seed)
        bt_attention(nh, nkv, hd, S, pos)
        # the split paths too (split 1: three kernels; 2: the fused kernel past BT_DECODE_B's rule)
        bt_attention(nh, nkv, hd, S, pos, split=1)
        bt_attention(nh, nkv, hd, S, pos, split=2)


def test_batched_decode_kernel_choice():
    pos = np.array([5, 9, 100])
    assert bt_attention(32, 32, 128, 640, pos) == "single-sequence kernels"
    assert bt_attention(32, 4, 64, 2048, pos) == "k_bt_attn"  # grouped heads: not the z grid
    assert bt_attention(32, 32, 128, 640, np.arange(4)) == "k_bt_attn"  # past BT_DECODE_B sequences
    assert bt_attention(32, 32, 128, 640, pos, split=1) == "three kernels"


def test_batched_model_catches_a_sequence_leaving_its_cache():
    """Not vacuous: a V row index formed with the query head's index instead of its kv head's, in
    the three-kernel path of grouped heads, leaves the sequence's cache for the last heads."""
    nh, nkv, hd, S, B = 8, 2, 64, 256, 3
    e = BExt(nh, nkv, hd, S, B)
    b, h, tc = B - 1, nh - 1, S - 1
    kvd = nkv * hd
    with pytest.raises(AssertionError):
        in_seq("planted", b * e.stride + h * hd + tc * kvd + np.arange(hd), b, e.stride)


# ---------------------------------------------------------------------------- prefill tiles

def pf_scores_rb(HD, nh, nkv, S, P, pos0, e):
    """k_pf_scores_rb<HD> over grid (n_heads, ceil(P/64), ceil((pos0+P)/64)) x 256 threads."""
    DP = HD if HD < 64 else 64
    group, D = nh // nkv, nh * HD
    tid = np.arange(WG)
    tg, pg = tid >> 4, tid & 15
    assert 2 * 4 * DP * 64 <= 64 * 1024
    for p0 in range(0, P, 64):
        for c0 in range(0, pos0 + P, 64):
            if c0 > pos0 + min(p0 + 63, P - 1):
                continue
            for h in range(nh):
                kvh = h // group
                for d0 in range(0, HD, DP):
                    ek = (np.arange(DP * 64 // WG)[:, None] * WG + tid[None, :]).ravel()
                    inb("pf ks LDS", ek, DP * 64)
                    t = c0 + (ek & 63)
                    inb("pf K", (kvh * HD + d0) * S + (ek >> 6) * S + np.minimum(t, S - 1), e.K)
                    eq = (np.arange(DP * 64 // 4 // WG)[:, None] * WG + tid[None, :]).ravel()
                    tok, d4 = eq & 63, eq >> 6
                    p = np.minimum(p0 + tok, P - 1)
                    inb("pf Q", h * HD + d0 + p * D + 4 * d4 + 3, P * D)
                    inb("pf qs LDS", (4 * d4 + 3) * 64 + tok, DP * 64)
                    inb("pf qs/ks reads", (DP - 1) * 64 + 4 * np.maximum(tg, pg) + 3, DP * 64)
                for a in range(4):
                    p = p0 + 4 * tg + a
                    for b in range(4):
                        t = c0 + 4 * pg + b
                        on = (p < P) & (t <= pos0 + p)
                        inb("pf att", ((h * P + p) * S + t)[on], nh * P * S)


def pf_softmax(nh, S, P, pos0):
    """k_pf_softmax_r<R> (rows up to 64R) or k_pf_softmax: row (head, token) of n = pos0+p+1."""
    rlen = pos0 + P
    R = 4 if rlen <= 256 else 8 if rlen <= 512 else 16 if rlen <= 1024 else 0
    for p in range(P):
        n = pos0 + p + 1
        assert n <= S
        if R:
            assert n <= 64 * R  # the buffer range check zeroes the rest; stores are masked by n
        for h in range(nh):
            inb("pf softmax row", (h * P + p) * S + np.arange(n), nh * P * S)


def pf_pv_rb(HD, nh, nkv, S, P, pos0, e, PP):
    """k_pf_pv_rb<HD> over grid (n_heads, ceil(P / (2048/HD))) x 256 threads, with Wo's image."""
    T, VC = 2048 // HD, PF_VC
    VR, PR = VC * HD // 4 // WG, T * VC // WG
    group, kvd = nh // nkv, nkv * HD
    ng = (P + T - 1) // T
    q4 = ng // 4
    gy = np.arange(ng)
    grp = np.where((ng % 4 == 0) & ((gy // max(q4, 1)) % 2 == 1), (gy // max(q4, 1)) * q4 + (q4 - 1 - gy % max(q4, 1)), gy)
    assert np.array_equal(np.sort(grp), np.arange(ng)), "every token group once"
    tid = np.arange(WG)
    ev = (np.arange(VR)[:, None] * WG + tid[None, :]).ravel()
    inb("pf pv LDS vs", (ev // (HD // 4)) * HD + 4 * (ev % (HD // 4)) + 3, VC * HD)
    ep = (np.arange(PR)[:, None] * WG + tid[None, :]).ravel()
    inb("pf pv LDS ps", (ep % VC) * T + ep // VC, VC * T)
    tg, cg = tid // (HD // 2), tid % (HD // 2)
    assert 4 * tg.max() + 3 < T and 2 * cg.max() + 1 < HD
    nblk = nh * HD // 32
    for g in grp:
        p0 = int(g) * T
        np_ = min(T, P - p0)
        tmax = pos0 + p0 + np_
        for h in range(nh):
            kvh = h // group
            for c0 in range(0, tmax, VC):
                t = ev // (HD // 4)
                tc = np.minimum(c0 + t, tmax - 1)
                inb("pf pv V", kvh * HD + tc * kvd + 4 * (ev % (HD // 4)) + 3, e.V)
                kk, tt = ep // VC, c0 + ep % VC
                on = (kk < np_) & (tt <= pos0 + p0 + kk)
                inb("pf pv att", ((h * P + p0 + kk) * S + tt)[on], nh * P * S)
            for a in range(4):
                kk = 4 * tg + a
                on = kk < np_
                inb("pf pv out", ((p0 + kk) * nh * HD + h * HD + 2 * cg + 1)[on], P * nh * HD)
                b = h * (HD // 32) + (cg >> 4)
                assert b.max() < nblk
                j = cg & 15
                inb("pf pv image (Q4 order)", ((b * PP + p0 + kk) * 32 + 8 * (j >> 2) + 7)[on & ((j & 3) == 0)], nblk * PP * 32)
                inb("pf pv image (Q8 order)", ((b * PP + p0 + kk) * 32 + 2 * j + 3)[on & ((j & 1) == 0)], nblk * PP * 32)
                inb("pf pv image d", (b * PP + p0 + kk)[on & (j == 0)], nblk * PP)


@pytest.mark.parametrize("HD,nh,nkv,S", [(128, 32, 32, 640), (128, 2, 2, 1300), (64, 12, 12, 1024),
                                         (64, 32, 4, 2048), (64, 4, 1, 300)])
@pytest.mark.parametrize("P,pos0", [(1, 0), (5, 0), (64, 0), (65, 3), (130, 200), (512, 0), (300, 700)])
def test_prefill_tile_kernel_indices_in_bounds(HD, nh, nkv, S, P, pos0):
    if pos0 + P > S:
        pytest.skip("the launcher takes pos0 + P <= max_seq only")
    e = Extents(nh, nkv, HD, S)
    PP = (min(S, 512) + 127) // 128 * 128  # the model's pf_pp
    if P > PP:
        pytest.skip("a pass holds at most pf_cap tokens")
    pf_scores_rb(HD, nh, nkv, S, P, pos0, e)
    pf_softmax(nh, S, P, pos0)
    pf_pv_rb(HD, nh, nkv, S, P, pos0, e, PP)


def test_prefill_model_catches_an_unclamped_position():
    """Not vacuous: k_pf_scores_rb's K^T tile reads positions c0 .. c0+63 clamped to max_seq-1; without
    the clamp the last tile of a context ending at max_seq = 1300 reads past the last kv head's K."""
    HD, nkv, S = 128, 2, 1300
    K = Extents(2, nkv, HD, S).K
    c0 = 1280
    t = c0 + np.arange(64)
    inb("kept clamp", ((nkv - 1) * HD + HD - 1) * S + np.minimum(t, S - 1), K)
    with pytest.raises(AssertionError):
        inb("planted", ((nkv - 1) * HD + HD - 1) * S + t, K)
