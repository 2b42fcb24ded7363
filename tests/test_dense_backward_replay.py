"""CPU replay of fl_dense_sum_backward's launch sequence with every buffer
bounds-checked (flashlog_amd/csrc/fl_dense.hip).

Each kernel of the sequence is restated thread by thread -- its grid, its
index arithmetic and its loads and stores -- over buffers of exactly the
sizes the C-ABI entry point and its Python caller allocate.  Every access
is checked against its buffer's extent, and every read of a workspace
buffer (torch.empty memory) against the entries written before it.  The
arithmetic is float32 with round-to-nearest and no contraction, as the
kernels compute it (fl_mul / fl_add), so the replayed grad_A can also be
compared bit for bit with the CPU oracle of flashlog.cpp:216-278.

The sequence is k_bwd_identity (+ k_bwd_identity_fin) -> k_col_count with a
null out_ind -> k_frontier -> k_c2_hard -> k_row_count -> k_row_fill -> k_row_offsets ->
k_bwd_pairs -> k_bwd_gw, on the inputs of tests/test_gpu_dense.py's
test_dense_sum_backward.  An earlier k_col_count stored the identity output
without testing out_ind; the replay of that form stores through the null
pointer, which is what faulted, and the guarded form touches nothing out of
bounds anywhere in the sequence.
"""
import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import attention, bits, masks_for, small_graph, sparse_state

F32 = np.float32
WAVE = 64
COL_NT = 256
BWD_NT = 256
RL_NT = 1024
C2_NT = 256
GW_C = 32
BWD_SLICES_MAX = 32


class Buf:
    """A device buffer of `n` elements; `tracked` buffers start
    uninitialized and refuse reads of entries never written."""

    def __init__(self, name, n, dtype=np.float32, data=None, tracked=False):
        self.name = name
        self.a = np.zeros(max(int(n), 0), dtype)
        if data is not None:
            self.a[:] = np.asarray(data, dtype).reshape(-1)
        self.tracked = tracked
        self.init = np.zeros(self.a.size, bool) if tracked else None

    def _check(self, i, what):
        i = int(i)
        if not (0 <= i < self.a.size):
            raise IndexError("%s of %s[%d]: buffer holds %d elements" % (what, self.name, i, self.a.size))
        return i

    def __getitem__(self, i):
        i = self._check(i, "read")
        if self.tracked and not self.init[i]:
            raise IndexError("read of %s[%d] before any write" % (self.name, i))
        return self.a[i]

    def __setitem__(self, i, v):
        i = self._check(i, "write")
        self.a[i] = v
        if self.tracked:
            self.init[i] = True


def f2u(x):
    return int(np.array([x], F32).view(np.uint32)[0])


def u2f(u):
    return np.array([u], np.uint32).view(F32)[0]


class Side:
    def __init__(self, name, col, mask, gptr, grel, gstart, gcount):
        self.col_ind = Buf(name + ".col_ind", col.size, np.int32, col)
        self.mask = Buf(name + ".mask", mask.size, F32, mask)
        self.row_group_ptr = Buf(name + ".row_group_ptr", gptr.size, np.int32, gptr)
        self.group_rel = Buf(name + ".group_rel", grel.size, np.int16, grel)
        self.group_start = Buf(name + ".group_start", gstart.size, np.int32, gstart)
        self.group_count = Buf(name + ".group_count", gcount.size, np.int32, gcount)


def sides(csr, masks):
    ori = Side("ori", csr[1], masks[0], csr[8], csr[9], csr[10], csr[11])
    inv = Side("inv", csr[5], masks[1], csr[12], csr[13], csr[14], csr[15])
    return ori, inv


# ---------------------------------------------------------------------------
# kernels (one function per __global__, threads in launch order)

def k_bwd_identity(g_ind, A, w, E, n, wot_i, add_zero, nsl, gA, gw, BL):
    span = (E + nsl - 1) // nsl
    for bl in range(BL):
        for y in range(nsl):
            e0 = y * span
            e1 = min(e0 + span, E)
            wid = w[bl * n + (n - 1)]
            part = [F32(0)] * BWD_NT
            for t in range(BWD_NT):
                acc = F32(0)
                for e in range(e0 + t, e1, BWD_NT):
                    i = bl * E + e
                    if wot_i:
                        gA[i] = 0.0
                    else:
                        gi = g_ind[i]
                        t0 = F32(gi * wid)
                        gA[i] = F32(F32(0) + t0) if add_zero else t0
                        acc = F32(acc + F32(gi * A[i]))
                part[t] = acc
            st = BWD_NT // 2
            while st > 0:
                for t in range(st):
                    part[t] = F32(part[t] + part[t + st])
                st //= 2
            if nsl > 1:
                gw[bl * n + y] = F32(0) if wot_i else part[0]
                continue
            for r in range(n):
                gw[bl * n + r] = 0.0
            if not wot_i:
                gw[bl * n + (n - 1)] = part[0]


def k_bwd_identity_fin(n, nsl, wot_i, gw, BL):
    for bl in range(BL):
        s = F32(0)
        for c in range(nsl):
            s = F32(s + gw[bl * n + c])
        for r in range(n):
            gw[bl * n + r] = 0.0
        if not wot_i:
            gw[bl * n + (n - 1)] = s


def bwd_identity(g_ind, A, w, BL, E, n, wot_i, add_zero, gA, gw):
    nsl = (E + 4 * BWD_NT - 1) // (4 * BWD_NT)
    nsl = min(nsl, BWD_SLICES_MAX, n - 1)
    nsl = max(nsl, 1)
    k_bwd_identity(g_ind, A, w, E, n, wot_i, add_zero, nsl, gA, gw, BL)
    if nsl > 1:
        k_bwd_identity_fin(n, nsl, wot_i, gw, BL)


def k_col_count(A, w, BL, E, n, wot_i, out_ind, BM, hard_count, guard_out_ind):
    """out_ind is None for the null pointer; a store through it is a write
    to address 0 + offset, i.e. outside every buffer."""
    nw = (BL + 31) // 32
    nblk = (nw * E + COL_NT - 1) // COL_NT
    null = Buf("out_ind(null)", 0)
    for q in range(nblk * COL_NT):
        if q == 0:
            hard_count[0] = 0
        if q >= nw * E:
            continue
        wi, e = divmod(q, E)
        b0 = wi * 32
        nb = 32 if b0 + 32 < BL else BL - b0
        v = [A[(b0 + k) * E + e] if k < nb else F32(0) for k in range(32)]
        bitsw = 0
        for k in range(nb):
            if out_ind is not None or not guard_out_ind:
                dst = out_ind if out_ind is not None else null
                wid = w[(b0 + k) * n + (n - 1)]
                dst[(b0 + k) * E + e] = F32(0) if wot_i else F32(v[k] * wid)
            if v[k] != 0:
                bitsw |= 1 << k
        BM[wi * E + e] = bitsw


def row_positions(s, src):
    g0, g1 = int(s.row_group_ptr[src]), int(s.row_group_ptr[src + 1])
    if g1 > g0:
        return int(s.group_start[g0]), int(s.group_start[g1 - 1]) + int(s.group_count[g1 - 1])
    return 0, 0


def k_frontier(ori, inv, A, BL, E, K, do_topk, BM, PKa, PKt, hard_count, hard_e, hard_bl):
    """PK is float2 {a, theta}: PKa / PKt hold its two lanes."""
    nw = (BL + 31) // 32
    for e in range(E):
        cnt = sum(bin(int(BM[wi * E + e])).count("1") for wi in range(nw))
        if cnt == 0:
            continue
        dirmask = 0
        if do_topk:
            p0, p1 = row_positions(ori, e)
            if p1 - p0 > K:
                dirmask |= 1
            p0, p1 = row_positions(inv, e)
            if p1 - p0 > K:
                dirmask |= 2
        slot = 0
        if dirmask:
            slot = int(hard_count[0])
            hard_count[0] = slot + cnt
        for wi in range(nw):
            bw = int(BM[wi * E + e])
            while bw:
                b = (bw & -bw).bit_length() - 1
                bw &= bw - 1
                bl = wi * 32 + b
                a = A[bl * E + e]
                for base in (e * BL, (E + e) * BL):
                    PKa[base + bl] = a
                    PKt[base + bl] = 0.0
                if dirmask:
                    hard_e[slot] = e * 4 + dirmask
                    hard_bl[slot] = bl
                    slot += 1


def c2_select(s, g0, g1, w, wbase, K, hist):
    """The wave radix select of fl_c2.h: (found, theta key, cut)."""
    tot = 0
    for g in range(g0, g1):
        wv = w[wbase + int(s.group_rel[g])]
        if wv > 0:
            tot += int(s.group_count[g])
    if tot <= K:
        return False, 0, 0
    need, prefix, pmask = K, 0, 0
    for shift in (24, 16, 8, 0):
        hist.a[:256] = 0  # lanes zero entries 4*lane .. 4*lane+3 of the 256-entry LDS array
        for g in range(g0, g1):
            wv = w[wbase + int(s.group_rel[g])]
            k = f2u(wv)
            if wv > 0 and (k & pmask) == prefix:
                d = (k >> shift) & 255
                hist[d] = int(hist[d]) + int(s.group_count[g])
        # lane l reads entries 4*(63-l) .. 4*(63-l)+3: the digits from the top
        desc = hist.a[:256][::-1].astype(np.int64)
        cum = np.cumsum(desc)
        j = int(np.searchsorted(cum, need))  # first digit (from the top) whose cumulative count reaches need
        digit, nneed = 255 - j, need - (int(cum[j - 1]) if j > 0 else 0)
        prefix |= digit << shift
        pmask |= 0xFF << shift
        need = nneed
    run, cut = 0, 0x7FFFFFFF
    for g in range(g0, g1):
        wv = w[wbase + int(s.group_rel[g])]
        cnt = st = 0
        if wv > 0 and f2u(wv) == prefix:
            cnt, st = int(s.group_count[g]), int(s.group_start[g])
        if cnt > 0 and run + cnt > need:
            cut = st + (need - run)
            break
        run += cnt
    return True, prefix, cut


def k_c2_hard(ori, inv, w, BL, E, n, r_size, K, hard_count, hard_e, hard_bl, PKt, CUT):
    hist = Buf("c2 hist (LDS)", 256, np.int64)
    for j in range(int(hard_count[0])):
        src, dm = int(hard_e[j]) >> 2, int(hard_e[j]) & 3
        bl = int(hard_bl[j])
        for d in (0, 1):
            if not dm & (1 << d):
                continue
            s = inv if d else ori
            g0, g1 = int(s.row_group_ptr[src]), int(s.row_group_ptr[src + 1])
            ok, k2, c2 = c2_select(s, g0, g1, w, bl * n + (r_size if d else 0), K, hist)
            if ok:
                at = (d * E + src) * BL + bl
                PKt[at] = u2f(k2)
                CUT[at] = c2


def k_row_count(BM, BL, E, nch, ccnt):
    nw = (BL + 31) // 32
    for wi in range(nw):
        for c in range(nch):  # workgroup (chunk, word): thread t holds source c * RL_NT + t
            bits = [int(BM[wi * E + c * RL_NT + t]) if c * RL_NT + t < E else 0 for t in range(RL_NT)]
            for r in range(32):
                bl = wi * 32 + r
                if bl < BL:
                    ccnt[bl * nch + c] = sum((b >> r) & 1 for b in bits)


def k_row_fill(BM, BL, E, nch, ccnt, rowlist, rowcnt):
    nw = (BL + 31) // 32
    for wi in range(nw):
        for c in range(nch):
            bits = [int(BM[wi * E + c * RL_NT + t]) if c * RL_NT + t < E else 0 for t in range(RL_NT)]
            for r in range(32):
                bl = wi * 32 + r
                run = sum(int(ccnt[bl * nch + q]) for q in range(c)) if bl < BL else 0
                for t in range(RL_NT):  # waves in order, lanes in order
                    if (bits[t] >> r) & 1:
                        assert bl < BL
                        rowlist[bl * E + run] = c * RL_NT + t
                        run += 1
                if bl < BL and c == nch - 1:
                    rowcnt[bl] = run


def k_row_offsets(rowcnt, BL, rowoff):
    run = 0
    for b in range(BL):
        rowoff[b] = run
        run += int(rowcnt[b])
    rowoff[BL] = run


def group_take(wv, th, cut, start, count):
    if not wv > 0:
        return 0
    if wv > th:
        return count
    if wv == th:
        t = cut - start
        return 0 if t <= 0 else min(t, count)
    return 0


def bwd_side(s, src, bl, BL, E, n, off, d, a, w, grad, PKt, CUT, acc, pgl):
    """One side of a pair, lane by lane as the wave computes it: windows of
    64 groups, the inclusive take prefix, each item's group by the binary
    search over the lanes' prefixes, then the ordered additions."""
    at = (d * E + src) * BL + bl
    th = PKt[at]
    cut = int(CUT[at]) if th > 0 else 0
    g0, g1 = int(s.row_group_ptr[src]), int(s.row_group_ptr[src + 1])
    for gb in range(g0, g1, WAVE):
        rel, start, take, wv = [0] * WAVE, [0] * WAVE, [0] * WAVE, [F32(0)] * WAVE
        for lane in range(WAVE):
            g = gb + lane
            if g < g1:
                rel[lane] = int(s.group_rel[g])
                wv[lane] = w[bl * n + off + rel[lane]]
                start[lane] = int(s.group_start[g])
                take[lane] = group_take(wv[lane], th, cut, start[lane], int(s.group_count[g]))
        incl = [int(x) for x in np.cumsum(take)]
        total = incl[WAVE - 1]
        first = [start[j] - (incl[j] - take[j]) for j in range(WAVE)]
        gs = [F32(0)] * WAVE
        for q0 in range(0, total, WAVE):
            t1, t2, grp, contrib = [None] * WAVE, [None] * WAVE, [0] * WAVE, [False] * WAVE
            for lane in range(WAVE):
                k = q0 + lane
                j = 0
                step = WAVE // 2
                while step > 0:
                    if incl[j + step - 1] <= k:
                        j += step
                    step //= 2
                if k >= total:
                    continue
                assert 0 <= j < WAVE and incl[j] - take[j] <= k < incl[j]
                p = first[j] + k
                m = s.mask[p]
                dst = int(s.col_ind[p])
                go = grad[bl * E + dst] if m != 0 else F32(0)
                grp[lane] = j
                contrib[lane] = m != 0 and go != 0
                t1[lane] = F32(F32(go * wv[j]) * m)
                t2[lane] = F32(F32(go * a) * m)
            for lane in range(WAVE):
                if contrib[lane]:
                    acc = F32(acc + t1[lane])
                    gs[grp[lane]] = F32(gs[grp[lane]] + t2[lane])
        for lane in range(WAVE):
            if take[lane] > 0:
                pgl[off + rel[lane]] = gs[lane]
    return acc


BWDP_WAVES = BWD_NT // WAVE


def k_bwd_pairs(ori, inv, A, w, g_ori, g_inv, BL, E, n, r_size, PKt, CUT, rowlist, rowcnt, rowoff, pairs,
                gA, PG):
    nb = (pairs + BWDP_WAVES - 1) // BWDP_WAVES
    for q in range(nb * BWDP_WAVES):  # wave q of the grid
        if q >= pairs or q >= int(rowoff[BL]):
            continue
        lo, hi = 0, BL
        while hi - lo > 1:
            mid = (lo + hi) >> 1
            if int(rowoff[mid]) <= q:
                lo = mid
            else:
                hi = mid
        bl, k = lo, q - int(rowoff[lo])
        if k >= int(rowcnt[bl]):
            continue
        src = int(rowlist[bl * E + k])
        a = A[bl * E + src]
        pgl = Buf("pair relation row (LDS)", n, F32)
        for r in range(n):
            pgl[r] = F32(0)
        acc = gA[bl * E + src]
        acc = bwd_side(ori, src, bl, BL, E, n, 0, 0, a, w, g_ori, PKt, CUT, acc, pgl)
        acc = bwd_side(inv, src, bl, BL, E, n, r_size, 1, a, w, g_inv, PKt, CUT, acc, pgl)
        for r in range(n):
            PG[q * n + r] = pgl[r]
        gA[bl * E + src] = acc


def k_bwd_gw(PG, rowcnt, rowoff, pairs, n, nrel, gw, BL):
    stage = Buf("gw stage (LDS)", GW_C * n, F32, tracked=True)
    for bl in range(BL):
        cnt = int(rowcnt[bl])
        if int(rowoff[bl]) + cnt > pairs:
            cnt = max(pairs - int(rowoff[bl]), 0)
        base = int(rowoff[bl]) * n
        acc = [F32(0)] * (4 * BWD_NT)
        for k0 in range(0, cnt, GW_C):
            kc = min(cnt - k0, GW_C)
            for i in range(kc * n):
                stage[i] = PG[base + k0 * n + i]
            for r in range(min(nrel, 4 * BWD_NT)):
                for k in range(kc):
                    acc[r] = F32(acc[r] + stage[k * n + r])
        for r in range(min(nrel, 4 * BWD_NT)):
            gw[bl * n + r] = acc[r]


def replay(A, w, g, csr, masks, R, wot_i, K, guard_out_ind=True):
    """fl_dense_sum_backward's launch sequence over bounds-checked buffers;
    returns (grad_A, grad_w)."""
    BL, E = A.shape
    n = w.shape[1]
    ori, inv = sides(csr, masks)
    do_topk = 1 if 0 < K < (1 << 60) else 0
    K = K if do_topk else 0
    nw = (BL + 31) // 32
    cap = BL * E
    Ab = Buf("A", cap, F32, A)
    wb = Buf("w", BL * n, F32, w)
    gi, go, gv = (Buf(nm, cap, F32, x) for nm, x in zip(("grad_ind", "grad_ori", "grad_inv"), g))
    gA = Buf("grad_A", cap, F32, tracked=True)
    gw = Buf("grad_w", BL * n, F32, tracked=True)
    pairs = int(np.count_nonzero(A))  # the Python caller's torch.count_nonzero
    PG = Buf("pg", max(pairs, 1) * n, F32, tracked=True)
    # workspace (dense_ws_layout + the backward's row lists), uninitialized
    BM = Buf("ws.bm", nw * E, np.uint32, tracked=True)
    PKa = Buf("ws.pk.x", 2 * cap, F32, tracked=True)
    PKt = Buf("ws.pk.y", 2 * cap, F32, tracked=True)
    CUT = Buf("ws.cut", 2 * cap, np.int32, tracked=True)
    hard_e = Buf("ws.hard.x", cap, np.int32, tracked=True)
    hard_bl = Buf("ws.hard.y", cap, np.int32, tracked=True)
    hard_count = Buf("ws.hard_count", 1, np.int64, tracked=True)
    rowlist = Buf("rowlist", cap, np.int32, tracked=True)
    rowcnt = Buf("rowcnt", BL, np.int32, tracked=True)
    rowoff = Buf("rowoff", BL + 1, np.int64, tracked=True)
    nch = (E + RL_NT - 1) // RL_NT
    ccnt = Buf("row chunk counts", BL * nch, np.int32, tracked=True)

    bwd_identity(gi, Ab, wb, BL, E, n, wot_i, 1, gA, gw)
    k_col_count(Ab, wb, BL, E, n, wot_i, None, BM, hard_count, guard_out_ind)
    k_frontier(ori, inv, Ab, BL, E, K, do_topk, BM, PKa, PKt, hard_count, hard_e, hard_bl)
    if do_topk:
        k_c2_hard(ori, inv, wb, BL, E, n, R, K, hard_count, hard_e, hard_bl, PKt, CUT)
    k_row_count(BM, BL, E, nch, ccnt)
    k_row_fill(BM, BL, E, nch, ccnt, rowlist, rowcnt)
    k_row_offsets(rowcnt, BL, rowoff)
    if pairs > 0:
        k_bwd_pairs(ori, inv, Ab, wb, go, gv, BL, E, n, R, PKt, CUT, rowlist, rowcnt, rowoff, pairs, gA, PG)
        k_bwd_gw(PG, rowcnt, rowoff, pairs, n, 2 * R, gw, BL)
    return gA.a.reshape(BL, E), gw.a.reshape(BL, n), gA.init.all() and gw.init.all()


def _inputs(K, wot_i, scale=0.05, B=4):
    """tests/test_gpu_dense.py::test_dense_sum_backward's inputs (same seed
    and draw order), on a graph of the given scale."""
    rng = np.random.default_rng(300 + K + 11 * wot_i)
    h, r, t, E, R, csr = small_graph(2, scale)
    n = 2 * R + 1
    BL = B * 3
    A = sparse_state(BL, E, 60, rng, ties=True)
    w = attention(BL, n, rng)
    w[:, : n // 2] = w[:, :1]
    _, masks = masks_for(csr, h.shape[0], rng)
    g = [rng.standard_normal((BL, E)).astype(np.float32) for _ in range(3)]
    g[1][rng.random((BL, E)) < 0.3] = 0.0
    return A, w, g, csr, masks, R


def test_unguarded_identity_store_is_the_fault():
    """The earlier k_col_count (identity output stored without testing
    out_ind) writes through the null pointer the backward passes."""
    A, w, g, csr, masks, R = _inputs(2, False, scale=0.01, B=1)
    with pytest.raises(IndexError, match=r"out_ind\(null\)"):
        replay(A, w, g, csr, masks, R, False, 2, guard_out_ind=False)


@pytest.mark.parametrize("K", [0, 2, 7, 200])
@pytest.mark.parametrize("wot_i", [False, True])
def test_guarded_sequence_in_bounds_and_exact(K, wot_i):
    """The guarded sequence touches nothing out of bounds, reads no
    workspace entry before writing it, writes every entry of grad_A and
    grad_w, and its grad_A equals the CPU path's bits (grad_w within
    1e-5: per-(source, row) partials added in source order)."""
    A, w, g, csr, masks, R = _inputs(K, wot_i)
    gA, gw, complete = replay(A, w, g, csr, masks, R, wot_i, K if K > 0 else (1 << 60))
    assert complete
    gA_ref, gw_ref = O.dense_backward(*g, A, w, csr, masks, R, wot_i=wot_i,
                                      topk_edges=K if K > 0 else (1 << 60))
    assert np.array_equal(bits(gA), bits(gA_ref))
    np.testing.assert_allclose(gw, gw_ref, rtol=1e-5, atol=1e-6)
