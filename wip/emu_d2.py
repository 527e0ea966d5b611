"""CPU replay of the dot2 16-slot kernels (k_read_d2, k_write_d2, k_wgradz_d2): every global
and LDS index of every thread is bounds-checked, and the bf16 pair packing / dot2 data flow is
compared with float64 sums. Transcribes the kernels' index expressions literally (scratch)."""
import math, sys
import numpy as np

def bf16_bits(a):  # float32 array -> uint16 bits (round to nearest even)
    u = np.asarray(a, np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)
def bf(bits):
    return (np.asarray(bits, np.uint32) << 16).view(np.float32)
def lo16(w): return np.uint32(w) & np.uint32(0xFFFF)
def hi16(w): return np.uint32(w) >> np.uint32(16)
def pair_lo(a, b): return np.uint32((int(a) & 0xFFFF) | ((int(b) & 0xFFFF) << 16))
def pair_hi(a, b): return np.uint32((int(a) >> 16) | (int(b) & 0xFFFF0000))
def dot2(a, b, acc):
    a0 = bf(int(a) & 0xFFFF); a1 = bf(int(a) >> 16); b0 = bf(int(b) & 0xFFFF); b1 = bf(int(b) >> 16)
    return np.float32(np.float64(acc) + np.float64(a0) * np.float64(b0) + np.float64(a1) * np.float64(b1))

class Arr:  # bounds-checked flat array
    def __init__(self, n, name, dtype=np.uint32, data=None):
        self.a = np.zeros(n, dtype) if data is None else data
        self.name = name
    def chk(self, i):
        if not (0 <= i < len(self.a)):
            raise IndexError(f"{self.name}: index {i} outside [0, {len(self.a)})")
    def __getitem__(self, i):
        self.chk(i); return self.a[i]
    def __setitem__(self, i, v):
        self.chk(i); self.a[i] = v

def shape_for(C, V, bcg0, lds_per_channel, lds_cap=64 * 1024):
    CG = (C + V - 1) // V
    bcg = bcg0
    while bcg > 1 and bcg // 2 >= CG: bcg //= 2
    while bcg > 1 and lds_per_channel * bcg * V > lds_cap: bcg //= 2
    return bcg, 256 // bcg, (CG + bcg - 1) // bcg

def rw_tokens_per_lane(cell, events, read=False):
    assert cell == 4
    if read and 3 <= events <= 12: return 16 if events <= 4 else 32
    if not read and 8 < events <= 12: return 32
    return 8 if events <= 4 else (16 if events <= 16 else 64)

def logical_block(b, n, xcd):
    if not xcd: return b
    q, r = n >> 3, n & 7
    x, i = b & 7, b >> 3
    return x * (q + 1) + i if x < r else r * (q + 1) + (x - r) * q + i

class Geo:
    def __init__(s, B, G, K, C):
        s.B, s.G, s.K, s.C = B, G, K, C; s.GG = G * G; s.GK = G * K; s.M = B * G * G
def cell_pixel0(m, g, index):
    b = m // g.GG; n = m - b * g.GG
    if index is not None: n = min(int(index[m]), g.GG - 1)
    wy = n // g.G; wx = n - wy * g.G
    return (b * g.GK + wy * g.K) * g.GK + wx * g.K
def slot_offset(p0, s, g, c, K=4):
    return (p0 + (s // K) * g.GK + (s % K)) * g.C + c

# ---------------------------------------------------------------------------- read
def emu_read(xbits, abits, E, g, index, U=4):
    K, S, C, M = 4, 16, g.C, g.M
    bcg, tl, slices = shape_for(C, 2, 32, E * S * 2, 48 * 1024)
    tpb = tl * rw_tokens_per_lane(4, E, True); chunks = -(-M // tpb); gs = tpb
    lds_words = E * S * bcg * 2 * 2 // 4
    n = slices * chunks
    xw = Arr(len(xbits) // 2, "x", data=xbits.view(np.uint32))
    aw = Arr(len(abits) // 2, "alpha", data=abits.view(np.uint32))
    outs = [Arr(M * C // 2, f"out{e}") for e in range(E)]
    written = [np.zeros(M * C // 2, bool) for _ in range(E)]
    row_w = g.GK * (C >> 1); pix_w = C >> 1
    for b in range(n):
        blk = logical_block(b, n, True); sl = blk % slices; chunk = blk // slices
        cs = sl * bcg * 2; BC = 2 * bcg
        lds = Arr(lds_words, "lds")
        for i in range(E * BC * 8):
            e = i // (BC * 8); r = i - e * BC * 8; cl, pr = r >> 3, r & 7; c = cs + cl
            lds[((e * 4 + (pr >> 1)) * bcg + (cl >> 1)) * 4 + (pr & 1) * 2 + (cl & 1)] = aw[(e * C + c) * 8 + pr] if c < C else 0
        for ty in range(tl):
            for tx in range(bcg):
                c0 = cs + tx * 2
                if c0 >= C: continue
                for m0 in range(chunk * gs, M, chunks * gs):
                    m_end = min(m0 + gs, M)
                    for mi in range(m0, m_end, U * tl):
                        m = mi + ty
                        ok, zoff, xv = [], [], []
                        for u in range(U):
                            okk = m + u * tl < m_end; mu = m + u * tl if okk else mi
                            px = cell_pixel0(mu, g, index) * C + c0
                            assert px % 2 == 0; px //= 2
                            ok.append(okk); zoff.append(mu * C + c0)
                            xv.append([xw[px + uy * row_w + ux * pix_w] for uy in range(K) for ux in range(K)])
                        xp = [[(pair_lo(xv[u][2 * p], xv[u][2 * p + 1]), pair_hi(xv[u][2 * p], xv[u][2 * p + 1])) for p in range(8)] for u in range(U)]
                        for e in range(E):
                            acc = [[np.float32(0), np.float32(0)] for _ in range(U)]
                            for q in range(4):
                                base = ((e * 4 + q) * bcg + tx) * 4
                                w = [lds[base + k] for k in range(4)]
                                for u in range(U):
                                    acc[u][0] = dot2(xp[u][2 * q][0], w[0], acc[u][0]); acc[u][1] = dot2(xp[u][2 * q][1], w[1], acc[u][1])
                                    acc[u][0] = dot2(xp[u][2 * q + 1][0], w[2], acc[u][0]); acc[u][1] = dot2(xp[u][2 * q + 1][1], w[3], acc[u][1])
                            for u in range(U):
                                if ok[u]:
                                    bits = bf16_bits(np.array(acc[u], np.float32))
                                    wi = zoff[u] // 2
                                    outs[e][wi] = int(bits[0]) | (int(bits[1]) << 16); written[e][wi] = True
    return [o.a for o in outs], written, (bcg, tl, slices, chunks)

def ref_read(xbits, abits, E, g, index):
    K, S, C, M = 4, 16, g.C, g.M
    x = bf(xbits).astype(np.float64); a = bf(abits).astype(np.float64).reshape(E, C, S)
    out = np.zeros((E, M, C))
    for m in range(M):
        p0 = cell_pixel0(m, g, index)
        xs = np.stack([x[slot_offset(p0, s, g, 0):slot_offset(p0, s, g, 0) + C] for s in range(S)])  # [S, C]
        out[:, m, :] = np.einsum('ecs,sc->ec', a, xs)
    return out

# ---------------------------------------------------------------------------- write
def emu_write(xbits, zbits, bbits, E, g, index, add_x, U=2):
    K, S, C, M = 4, 16, g.C, g.M
    E4 = (E + 3) & ~3
    bcg, tl, slices = shape_for(C, 2, 32, E4 * S * 2, 48 * 1024)
    tpb = tl * rw_tokens_per_lane(4, E4); chunks = -(-M // tpb); gs = tpb
    lds_words = E4 * S * bcg * 2 * 2 // 4
    n = slices * chunks
    xw = Arr(len(xbits) // 2, "x", data=xbits.view(np.uint32))
    zw = [Arr(M * C // 2, f"z{e}", data=zbits[e].view(np.uint32)) for e in range(E)]
    bw = Arr(len(bbits), "beta16", dtype=np.uint16, data=bbits)
    out = Arr(len(xbits) // 2, "out")
    written = np.zeros(len(xbits) // 2, bool)
    row_w = g.GK * (C >> 1); pix_w = C >> 1
    J = (E + 1) // 2
    for b in range(n):
        blk = logical_block(b, n, True); sl = blk % slices; chunk = blk // slices
        cs = sl * bcg * 2; BC = 2 * bcg
        lds = Arr(lds_words, "lds")
        for i in range(J * BC * 16):
            j = i // (BC * 16); r = i - j * BC * 16; cl, sll = r >> 4, r & 15; c = cs + cl
            lo = hi = 0
            if c < C:
                lo = int(bw[(2 * j * C + c) * 16 + sll])
                if 2 * j + 1 < E: hi = int(bw[((2 * j + 1) * C + c) * 16 + sll])
            lds[((j * 8 + (sll >> 1)) * bcg + (cl >> 1)) * 4 + (sll & 1) * 2 + (cl & 1)] = lo | (hi << 16)
        for ty in range(tl):
            for tx in range(bcg):
                c0 = cs + tx * 2
                if c0 >= C: continue
                for m0 in range(chunk * gs, M, chunks * gs):
                    m_end = min(m0 + gs, M)
                    for mi in range(m0, m_end, U * tl):
                        m = mi + ty
                        ok, zoff, b0, acc = [], [], [], []
                        for u in range(U):
                            okk = m + u * tl < m_end; mu = m + u * tl if okk else mi
                            ok.append(okk)
                            p = cell_pixel0(mu, g, index) * C + c0; assert p % 2 == 0
                            b0.append(p >> 1); zoff.append(mu * C + c0)
                            a = []
                            for uy in range(K):
                                for ux in range(K):
                                    if add_x:
                                        v = int(xw[b0[u] + uy * row_w + ux * pix_w])
                                        a.append([bf(v & 0xFFFF), bf(v >> 16)])
                                    else:
                                        a.append([np.float32(0), np.float32(0)])
                            acc.append(a)
                        def issue(j):
                            return [[int(zw[min(2 * j + q, E - 1)][zoff[u] // 2]) for u in range(U)] for q in range(2)]
                        zr = issue(0)
                        for j in range(J):
                            second = 2 * j + 1 < E
                            d = []
                            for u in range(U):
                                w1 = zr[1][u] if second else 0
                                d.append((pair_lo(zr[0][u], w1), pair_hi(zr[0][u], w1)))
                            if j + 1 < J: zr = issue(j + 1)
                            for q in range(8):
                                base = ((j * 8 + q) * bcg + tx) * 4
                                w = [lds[base + k] for k in range(4)]
                                for u in range(U):
                                    acc[u][2 * q][0] = dot2(d[u][0], w[0], acc[u][2 * q][0]); acc[u][2 * q][1] = dot2(d[u][1], w[1], acc[u][2 * q][1])
                                    acc[u][2 * q + 1][0] = dot2(d[u][0], w[2], acc[u][2 * q + 1][0]); acc[u][2 * q + 1][1] = dot2(d[u][1], w[3], acc[u][2 * q + 1][1])
                        for u in range(U):
                            if ok[u]:
                                for uy in range(K):
                                    for ux in range(K):
                                        wi = b0[u] + uy * row_w + ux * pix_w
                                        bits = bf16_bits(np.array(acc[u][uy * K + ux], np.float32))
                                        out[wi] = int(bits[0]) | (int(bits[1]) << 16); written[wi] = True
    return out.a, written, (bcg, tl, slices, chunks)

def ref_write(xbits, zbits, bbits, E, g, index, add_x):
    K, S, C, M = 4, 16, g.C, g.M
    x = bf(xbits).astype(np.float64); bt = bf(bbits).astype(np.float64).reshape(E, C, S)
    z = np.stack([bf(zb).astype(np.float64).reshape(M, C) for zb in zbits])
    out = x.copy() if add_x else np.zeros_like(x)
    for m in range(M):
        p0 = cell_pixel0(m, g, index)
        for s in range(S):
            o = slot_offset(p0, s, g, 0)
            out[o:o + C] += np.einsum('ec,ec->c', bt[:, :, s], z[:, m, :])
    return out

# ---------------------------------------------------------------------------- weight gradient
def emu_wgradz(xbits, zbits, E, g, index, chunks, ep, nw, npq, TT=8):
    K, S, C, M = 4, 16, g.C, g.M
    L = 64; VS = 8; NV = L // VS; TP = TT // 2; NXP = TP * S * NV; NZK = (ep + 1) // 2
    slicesz = (C + L - 1) // L
    tpb = -(-M // chunks)
    n = slicesz * chunks
    xv = Arr(len(xbits) // 8, "x16B", dtype=object, data=None)
    X4 = xbits.view(np.uint32).reshape(-1, 4)
    Z4 = [zb.view(np.uint32).reshape(-1, 4) for zb in zbits]
    part = Arr(chunks * E * S * C, "part", dtype=np.float32)
    ldsw = TT * (S + E) * L * 2 // 4
    nthr = L * nw
    def ldx(elem_off):
        assert elem_off % 8 == 0
        i = elem_off // 8
        if not (0 <= i < len(X4)): raise IndexError(f"x vector {i}")
        return [int(v) for v in X4[i]]
    def ldz(e, elem_off):
        assert elem_off % 8 == 0
        i = elem_off // 8
        if not (0 <= i < len(Z4[e])): raise IndexError(f"z{e} vector {i}")
        return [int(v) for v in Z4[e][i]]
    def put_pairs(lds, dst, a, b, second):
        lo = [0] * 4; hi = [0] * 4
        for k in range(2):
            bl = b[k] if second else 0; bh = b[k + 2] if second else 0
            lo[2 * k] = pair_lo(a[k], bl); lo[2 * k + 1] = pair_hi(a[k], bl)
            hi[2 * k] = pair_lo(a[k + 2], bh); hi[2 * k + 1] = pair_hi(a[k + 2], bh)
        assert dst % 4 == 0
        for k in range(4): lds[dst + k] = lo[k]
        for k in range(4): lds[dst + 4 + k] = hi[k]
    for b in range(n):
        blk = b; sl = blk % slicesz; chunk = blk // slicesz
        cs = sl * L
        lds = Arr(ldsw, "lds")
        xt0, zt0 = 0, TP * S * L
        regs = {}
        def issue(t0, tn):
            for wave in range(nw):
                for lane in range(L):
                    tid = wave * L + lane
                    zh = lane // (L // 2); zp = (lane % (L // 2)) // NV; zj = lane % NV; zc = cs + zj * VS
                    xb = []
                    for k in range(npq):
                        i = min(tid + k * nthr, NXP - 1)
                        row = i // NV; tp = row // S; cc = cs + (i % NV) * VS
                        xb.append([ldx(slot_offset(cell_pixel0(t0 + min(2 * tp + h, tn - 1), g, index), row % S, g, cc if cc < C else cs)) for h in range(2)])
                    zoff = [(t0 + min(2 * zp + h, tn - 1)) * C + (zc if zc < C else cs) for h in range(2)]
                    zb = []
                    for k in range(NZK):
                        e = min(wave + (2 * k + zh) * nw, E - 1)
                        zb.append([ldz(e, zoff[h]) for h in range(2)])
                    regs[tid] = (xb, zb)
        def commit(tn):
            for wave in range(nw):
                for lane in range(L):
                    tid = wave * L + lane
                    xb, zb = regs[tid]
                    zh = lane // (L // 2); zp = (lane % (L // 2)) // NV; zj = lane % NV; zc = cs + zj * VS
                    for k in range(npq):
                        i = tid + k * nthr
                        row = i // NV; tp = row // S; j = i % NV; cc = cs + j * VS
                        if i < NXP and 2 * tp < tn and cc < C: put_pairs(lds, xt0 + row * L + j * VS, xb[k][0], xb[k][1], 2 * tp + 1 < tn)
                    for k in range(NZK):
                        e = wave + (2 * k + zh) * nw
                        if 2 * k + zh < ep and e < E and 2 * zp < tn and zc < C:
                            put_pairs(lds, zt0 + (zp * E + e) * L + zj * VS, zb[k][0], zb[k][1], 2 * zp + 1 < tn)
        acc = np.zeros((nw, L, ep, S), np.float32)
        m_begin = chunk * tpb; m_end = min(m_begin + tpb, M)
        if m_begin < m_end: issue(m_begin, min(TT, m_end - m_begin))
        for t0 in range(m_begin, m_end, TT):
            tn = min(TT, m_end - t0)
            commit(tn)
            if t0 + TT < m_end: issue(t0 + TT, min(TT, m_end - t0 - TT))
            for wave in range(nw):
                e0 = wave * ep
                for lane in range(L):
                    if cs + lane >= C: continue
                    zrow = [min(e0 + q, E - 1) for q in range(ep)]
                    tp = 0
                    while 2 * tp < tn:
                        zv = [lds[zt0 + (tp * E + zrow[q]) * L + lane] for q in range(ep)]
                        for s in range(S):
                            xs = lds[xt0 + (tp * S + s) * L + lane]
                            for q in range(ep): acc[wave, lane, q, s] = dot2(xs, zv[q], acc[wave, lane, q, s])
                        tp += 1
        for wave in range(nw):
            e0 = wave * ep
            for lane in range(L):
                c = cs + lane
                if c >= C: continue
                for q in range(ep):
                    if e0 + q < E:
                        for s in range(S): part[((chunk * E + e0 + q) * S + s) * C + c] = acc[wave, lane, q, s]
    res = part.a.reshape(chunks, E, S, C).sum(0)
    return res

def ref_wgrad(xbits, zbits, E, g, index):
    K, S, C, M = 4, 16, g.C, g.M
    x = bf(xbits).astype(np.float64)
    z = np.stack([bf(zb).astype(np.float64).reshape(M, C) for zb in zbits])
    out = np.zeros((E, S, C))
    for m in range(M):
        p0 = cell_pixel0(m, g, index)
        xs = np.stack([x[slot_offset(p0, s, g, 0):slot_offset(p0, s, g, 0) + C] for s in range(S)])
        out += z[:, m, None, :] * xs[None]
    return out

def ulps_ok(got_bits, ref):
    got = bf(got_bits).astype(np.float64)
    refb = bf(bf16_bits(ref.astype(np.float32))).astype(np.float64)
    ulp = np.maximum(np.abs(got), np.abs(refb)) * 2.0 ** -7 + 1e-30
    return np.max(np.abs(got - ref) / ulp)

def run(case):
    rng = np.random.default_rng(case.get("seed", 0))
    B, G, C, E = case["B"], case["G"], case["C"], case["E"]
    g = Geo(B, G, 4, C)
    index = None
    if case.get("index"):
        index = np.array([(m % g.GG * 7 + 3) % g.GG for m in range(g.M)], np.int32)
    xbits = bf16_bits(rng.standard_normal(B * g.GK * g.GK * C))
    kind = case["kind"]
    if kind == "read":
        abits = bf16_bits(0.25 + 0.02 * rng.standard_normal(E * C * 16))
        outs, written, shp = emu_read(xbits, abits, E, g, index)
        ref = ref_read(xbits, abits, E, g, index)
        worst = 0
        for e in range(E):
            assert written[e].all(), f"read: event {e} has unwritten outputs"
            ob = outs[e].view(np.uint16)
            worst = max(worst, ulps_ok(ob, ref[e].reshape(-1)))
        print(f"read  {case} shape(bcg,tl,slices,chunks)={shp}: all outputs written, worst {worst:.3f} bf16 ulp", flush=True)
        assert worst <= 1.0
    elif kind == "write":
        zbits = [bf16_bits(rng.standard_normal(g.M * C)) for _ in range(E)]
        bbits = bf16_bits(1.0 + 0.02 * rng.standard_normal(E * C * 16))
        add_x = case.get("add_x", True)
        out, written, shp = emu_write(xbits, zbits, bbits, E, g, index, add_x)
        ref = ref_write(xbits, zbits, bbits, E, g, index, add_x)
        if index is None or case.get("perm", True):
            assert written.all(), "write: unwritten carrier words"
        worst = ulps_ok(out.view(np.uint16)[np.repeat(written, 2)], ref[np.repeat(written, 2)])
        print(f"write {case} shape={shp}: all carrier words written, worst {worst:.3f} bf16 ulp", flush=True)
        assert worst <= 1.0
    else:
        zbits = [bf16_bits(0.1 * rng.standard_normal(g.M * C)) for _ in range(E)]
        res = emu_wgradz(xbits, zbits, E, g, index, case["chunks"], case["ep"], case["nw"], case["npq"])
        ref = ref_wgrad(xbits, zbits, E, g, index)
        err = np.max(np.abs(res - ref)) / np.max(np.abs(ref))
        print(f"wgrad {case}: max rel err {err:.2e}", flush=True)
        assert err < 1e-5

CASES = [
    dict(kind="read", B=3, G=7, C=72, E=24),
    dict(kind="read", B=3, G=7, C=72, E=3, index=True),
    dict(kind="read", B=2, G=4, C=6, E=1),
    dict(kind="write", B=3, G=7, C=72, E=24),
    dict(kind="write", B=3, G=7, C=72, E=7, add_x=False),
    dict(kind="write", B=2, G=4, C=6, E=1, index=True),
    dict(kind="wgrad", B=3, G=7, C=72, E=24, chunks=3, ep=3, nw=8, npq=1),
    dict(kind="wgrad", B=3, G=7, C=72, E=9, chunks=5, ep=3, nw=3, npq=3),
    dict(kind="wgrad", B=2, G=5, C=64, E=13, chunks=7, ep=4, nw=4, npq=2, index=True),
    dict(kind="wgrad", B=2, G=5, C=136, E=8, chunks=2, ep=4, nw=2, npq=4),
]
if __name__ == "__main__":
    sel = sys.argv[1:]
    for c in CASES:
        if not sel or c["kind"] in sel:
            run(c)
    print("all emulated cases passed")

# ---------------------------------------------------------------------------- per-event backward, 16 slots
def group_tokens(want, M, chunks, step):
    w = want if want > 0 else -(-M // max(chunks, 1))
    return -(-max(w, 1) // step) * step

def emu_event_bwd16(gxo, gzo, xo, dz, beta, alpha, E_parts, g, index, chunks=None):
    """gxo, xo: carrier bf16 bits; gzo, dz: workspace bits; beta, alpha: [C,16] bits.
    E_parts: (HAS_H, HAS_G, HAS_W, STORE_T)."""
    HAS_H, HAS_G, HAS_W, STORE_T = E_parts
    K, S, V, C, M = 4, 16, 2, g.C, g.M
    bcg, tl, slices = shape_for(C, 2, 32, 0)
    maxc = min(512, max(1, -(-M // 256)))
    chunks = chunks or maxc
    gs = group_tokens(64, M, chunks, 2 * tl)
    n = slices * chunks
    gxw = Arr(len(gxo) // 2, "gxo", data=gxo.view(np.uint32)) if HAS_H else None
    xow = Arr(len(xo) // 2, "xo", data=xo.view(np.uint32)) if HAS_G else None
    gzw = Arr(len(gzo) // 2, "gzo", data=gzo.view(np.uint32)) if HAS_G else None
    dzw = Arr(len(dz) // 2, "dz", data=dz.view(np.uint32)) if HAS_W else None
    bw16 = Arr(len(beta) // 2, "beta", data=beta.view(np.uint32)) if HAS_W else None
    aw16 = Arr(len(alpha) // 2, "alpha", data=alpha.view(np.uint32)) if HAS_G else None
    gx = Arr(len(xo) // 2 if HAS_G else len(gxo) // 2, "gx")
    gdz = Arr(M * C // 2, "gdz")
    part = Arr(maxc * 2 * S * C, "part", dtype=np.float64)
    lds_floats = tl * bcg * S * V
    row_w = g.GK * (C >> 1); pix_w = C >> 1
    for b in range(n):
        blk = logical_block(b, n, True); sl_ = blk % slices; chunk = blk // slices
        red = Arr(lds_floats, "red", dtype=np.float64)
        acc_db = np.zeros((tl, bcg, S, V)); acc_da = np.zeros((tl, bcg, S, V))
        for ty in range(tl):
            for tx in range(bcg):
                c0 = sl_ * bcg * V + tx * V
                if c0 >= C: continue
                bwords = [bw16[(c0 * S) // 2 + k] for k in range(16)] if HAS_W else None
                awords = [aw16[(c0 * S) // 2 + k] for k in range(16)] if HAS_G else None
                wget = lambda w, s_, v: bf((int(w[v * 8 + (s_ >> 1)]) >> 16) if (s_ & 1) else (int(w[v * 8 + (s_ >> 1)]) & 0xFFFF))
                for m0 in range(chunk * gs, M, chunks * gs):
                    m_end = min(m0 + gs, M)
                    for mi in range(m0, m_end, tl):
                        mt = mi + ty; ok = mt < m_end; mu = mt if ok else mi
                        p = cell_pixel0(mu, g, index) * C + c0; assert p % 2 == 0; b0 = p >> 1
                        zwi = (mu * C + c0) >> 1
                        gzr = int(gzw[zwi]) if HAS_G else 0
                        dr = int(dzw[zwi]) if HAS_W else 0
                        tr, xr = [], []
                        for uy in range(K):
                            for ux in range(K):
                                o = b0 + uy * row_w + ux * pix_w
                                tr.append(int(gxw[o]) if HAS_H else 0)
                                xr.append(int(xow[o]) if HAS_G else 0)
                        if not ok:
                            gzr = dr = 0; tr = [0] * S; xr = [0] * S
                        gz = [bf(gzr & 0xFFFF), bf(gzr >> 16)]; d = [bf(dr & 0xFFFF), bf(dr >> 16)]
                        gd = [np.float32(0), np.float32(0)]
                        for s_ in range(S):
                            t = [bf(tr[s_] & 0xFFFF), bf(tr[s_] >> 16)]
                            for v in range(V):
                                if HAS_G:
                                    xv = bf(xr[s_] >> 16) if v else bf(xr[s_] & 0xFFFF)
                                    acc_da[ty, tx, s_, v] += float(xv) * float(gz[v])
                                    t[v] = np.float32(float(wget(awords, s_, v)) * float(gz[v]) + float(t[v]))
                                if HAS_W:
                                    gd[v] = np.float32(float(wget(bwords, s_, v)) * float(t[v]) + float(gd[v]))
                                    acc_db[ty, tx, s_, v] += float(d[v]) * float(t[v])
                            if STORE_T and ok:
                                bits = bf16_bits(np.array(t, np.float32))
                                gx[b0 + (s_ // K) * row_w + (s_ % K) * pix_w] = int(bits[0]) | (int(bits[1]) << 16)
                        if HAS_W and ok:
                            bits = bf16_bits(np.array(gd, np.float32))
                            gdz[zwi] = int(bits[0]) | (int(bits[1]) << 16)
        # block reduction (index checks only; sums taken directly)
        W = bcg * S * V
        for ty in range(tl):
            for tx in range(bcg):
                for k in range(S * V): red[ty * W + tx * S * V + k] = 0.0
        for w in range(2):
            if (w == 0 and not HAS_W) or (w == 1 and not HAS_G): continue
            accs = acc_db if w == 0 else acc_da
            for i in range(W):
                lane = i // (S * V); r = i - lane * S * V; s_ = r // V; v = r - s_ * V
                c = sl_ * bcg * V + lane * V + v
                if c < C:
                    part[((chunk * 2 + w) * S + s_) * C + c] = accs[:, lane, s_, v].sum()
    P = part.a.reshape(maxc, 2, S, C)[:chunks].sum(0)
    return gx.a, gdz.a, P

def ref_event_bwd16(gxo, gzo, xo, dz, beta, alpha, parts, g, index):
    HAS_H, HAS_G, HAS_W, STORE_T = parts
    K, S, C, M = 4, 16, g.C, g.M
    G_ = bf(gxo).astype(np.float64) if HAS_H else np.zeros(len(xo))
    X = bf(xo).astype(np.float64) if HAS_G else None
    h = bf(gzo).astype(np.float64).reshape(M, C) if HAS_G else None
    d = bf(dz).astype(np.float64).reshape(M, C) if HAS_W else None
    b = bf(beta).astype(np.float64).reshape(C, S) if HAS_W else None
    a = bf(alpha).astype(np.float64).reshape(C, S) if HAS_G else None
    gx = np.zeros(len(G_)); gdz = np.zeros((M, C)); db = np.zeros((S, C)); da = np.zeros((S, C))
    for m in range(M):
        p0 = cell_pixel0(m, g, index)
        for s in range(S):
            o = slot_offset(p0, s, g, 0)
            t = G_[o:o + C].copy()
            if HAS_G:
                da[s] += X[o:o + C] * h[m]
                t += a[:, s] * h[m]
            if HAS_W:
                gdz[m] += b[:, s] * t
                db[s] += d[m] * t
            gx[o:o + C] = t
    return gx, gdz, np.stack([db, da])

def run_bwd16(B, G, C, parts, index=False, chunks=None, seed=0):
    rng = np.random.default_rng(seed)
    g = Geo(B, G, 4, C)
    idx = np.array([(m % g.GG * 7 + 3) % g.GG for m in range(g.M)], np.int32) if index else None
    ncar = B * g.GK * g.GK * C
    gxo = bf16_bits(0.01 * rng.standard_normal(ncar)); xo = bf16_bits(rng.standard_normal(ncar))
    gzo = bf16_bits(0.01 * rng.standard_normal(g.M * C)); dz = bf16_bits(rng.standard_normal(g.M * C))
    beta = bf16_bits(1 + 0.02 * rng.standard_normal(C * 16)); alpha = bf16_bits(0.25 + 0.02 * rng.standard_normal(C * 16))
    gx, gdz, P = emu_event_bwd16(gxo, gzo, xo, dz, beta, alpha, parts, g, idx, chunks)
    rgx, rgdz, rP = ref_event_bwd16(gxo, gzo, xo, dz, beta, alpha, parts, g, idx)
    HAS_H, HAS_G, HAS_W, STORE_T = parts
    if STORE_T:
        e1 = ulps_ok(gx.view(np.uint16), rgx)
        assert e1 <= 1.0, e1
    if HAS_W:
        e2 = ulps_ok(gdz.view(np.uint16), rgdz.reshape(-1))
        assert e2 <= 1.0, e2
    rows = [w for w in range(2) if (w == 0 and HAS_W) or (w == 1 and HAS_G)]
    err = max((np.max(np.abs(P[w] - rP[w])) / max(np.max(np.abs(rP[w])), 1e-30)) for w in rows) if rows else 0.0
    assert err < 1e-5, err
    print(f"event_bwd16 B={B} G={G} C={C} parts={parts} index={index} chunks={chunks}: bounds ok, outputs within 1 ulp, partial sums rel err {err:.1e}", flush=True)

def emu_event_fwd16(x, dz, beta, alpha, g, index, has_z=True, U=2, TPT=2):
    K, S, V, C, M = 4, 16, 2, g.C, g.M
    bcg, tl, slices = shape_for(C, 2, 32, 0)
    tpb = tl * TPT; chunks = -(-M // tpb); n = slices * chunks
    xw = Arr(len(x) // 2, "x", data=x.view(np.uint32)); dzw = Arr(M * C // 2, "dz", data=dz.view(np.uint32))
    bw16 = Arr(len(beta) // 2, "beta", data=beta.view(np.uint32)); aw16 = Arr(len(alpha) // 2, "alpha", data=alpha.view(np.uint32))
    xo = Arr(len(x) // 2, "xo"); zo = Arr(M * C, "zo", dtype=np.uint16)
    row_w = g.GK * (C >> 1); pix_w = C >> 1
    wget = lambda w, s_, v: bf((int(w[v * 8 + (s_ >> 1)]) >> 16) if (s_ & 1) else (int(w[v * 8 + (s_ >> 1)]) & 0xFFFF))
    for b in range(n):
        blk = logical_block(b, n, True); sl_ = blk % slices; chunk = blk // slices
        for ty in range(tl):
            for tx in range(bcg):
                c0 = (sl_ * bcg + tx) * V
                if c0 >= C: continue
                bwv = [bw16[(c0 * S) // 2 + k] for k in range(16)]
                awv = [aw16[(c0 * S) // 2 + k] for k in range(16)] if has_z else None
                m_begin = chunk * tpb; m_end = min(m_begin + tpb, M)
                for m in range(m_begin + ty, m_end, U * tl):
                    for u in range(U):
                        ok = m + u * tl < m_end; mu = m + u * tl if ok else m
                        p = cell_pixel0(mu, g, index) * C + c0; b0 = p >> 1; zwi = (mu * C + c0) >> 1
                        dr = int(dzw[zwi]); d = [bf(dr & 0xFFFF), bf(dr >> 16)]
                        zacc = [np.float32(0), np.float32(0)]
                        for s_ in range(S):
                            o = b0 + (s_ // K) * row_w + (s_ % K) * pix_w
                            xr = int(xw[o]); xv = [bf(xr & 0xFFFF), bf(xr >> 16)]
                            for v in range(V):
                                xv[v] = bf(bf16_bits(np.float32(float(wget(bwv, s_, v)) * float(d[v]) + float(xv[v]))))
                                if has_z: zacc[v] = np.float32(float(wget(awv, s_, v)) * float(xv[v]) + float(zacc[v]))
                            if ok:
                                bits = bf16_bits(np.array(xv, np.float32)); xo[o] = int(bits[0]) | (int(bits[1]) << 16)
                        if has_z and ok:
                            bits = bf16_bits(np.array(zacc, np.float32)); zo[2 * zwi] = bits[0]; zo[2 * zwi + 1] = bits[1]
    return xo.a, zo.a

def run_fwd16(B, G, C, index=False, seed=0):
    rng = np.random.default_rng(seed)
    g = Geo(B, G, 4, C)
    idx = np.array([(m % g.GG * 7 + 3) % g.GG for m in range(g.M)], np.int32) if index else None
    x = bf16_bits(rng.standard_normal(B * g.GK * g.GK * C)); dz = bf16_bits(rng.standard_normal(g.M * C))
    beta = bf16_bits(1 + 0.02 * rng.standard_normal(C * 16)); alpha = bf16_bits(0.25 + 0.02 * rng.standard_normal(C * 16))
    xo, zo = emu_event_fwd16(x, dz, beta, alpha, g, idx)
    X = bf(x).astype(np.float64); D = bf(dz).astype(np.float64).reshape(g.M, C)
    b = bf(beta).astype(np.float64).reshape(C, 16); a = bf(alpha).astype(np.float64).reshape(C, 16)
    rx = X.copy(); rz = np.zeros((g.M, C))
    for m in range(g.M):
        p0 = cell_pixel0(m, g, idx)
        for s in range(16):
            o = slot_offset(p0, s, g, 0)
            v = bf(bf16_bits((X[o:o + C] + b[:, s] * D[m]).astype(np.float32))).astype(np.float64)
            rx[o:o + C] = v; rz[m] += a[:, s] * v
    e1 = ulps_ok(xo.view(np.uint16), rx); e2 = ulps_ok(zo, rz.reshape(-1))
    assert e1 <= 1.0 and e2 <= 1.0, (e1, e2)
    print(f"event_fwd16 B={B} G={G} C={C} index={index}: bounds ok, x_out {e1:.2f} ulp, z_out {e2:.2f} ulp", flush=True)

def emu_read_w(xbits, abits, E, g, index, TT=32):
    K, S, C, M = 2, 4, g.C, g.M
    LX, V, BC, RY = 16, 8, 128, 4
    slices = -(-C // BC); chunks = -(-M // TT); n = slices * chunks
    X4 = xbits.view(np.uint32).reshape(-1, 4)
    aw = Arr(len(abits) // 2, "alpha", data=abits.view(np.uint32))
    outs = [Arr(M * C, f"out{e}", dtype=np.uint16) for e in range(E)]
    written = [np.zeros(M * C, bool) for _ in range(E)]
    for blk in range(n):
        sl_ = blk % slices; chunk = blk // slices; cs = sl_ * BC
        m0 = chunk * TT; tn = min(TT, M - m0)
        lds = Arr((TT + E) * 2 * BC, "lds"); xp0 = 0; ap0 = TT * 2 * BC
        for i in range(E * BC * 2):
            e = i // (BC * 2); r = i - e * BC * 2; cl, pr = r >> 1, r & 1; c = cs + cl
            lds[ap0 + (e * 2 + pr) * BC + cl] = aw[(e * C + c) * 2 + pr] if c < C else 0
        for u in range(TT * LX):
            t, j = u // LX, u % LX; c = cs + j * V
            if t < tn and c < C:
                p0 = cell_pixel0(m0 + t, g, index)
                v = []
                for s_ in range(4):
                    off = (p0 + (s_ // K) * g.GK + (s_ % K)) * C + c
                    assert off % 8 == 0
                    if not (0 <= off // 8 < len(X4)): raise IndexError("x vector")
                    v.append([int(q) for q in X4[off // 8]])
                for pr in range(2):
                    a, b = v[2 * pr], v[2 * pr + 1]
                    words = [pair_lo(a[0], b[0]), pair_hi(a[0], b[0]), pair_lo(a[1], b[1]), pair_hi(a[1], b[1]),
                             pair_lo(a[2], b[2]), pair_hi(a[2], b[2]), pair_lo(a[3], b[3]), pair_hi(a[3], b[3])]
                    base = xp0 + (t * 2 + pr) * BC + j * V
                    for k in range(8): lds[base + k] = words[k]
        for tid in range(256):
            wave, lane = tid // 64, tid % 64; lx, ly = lane % LX, lane // LX
            c0 = cs + lx * V
            if c0 >= C: continue
            for e in range(wave, E, 4):
                ae = ap0 + e * 2 * BC + lx * V
                w0 = [lds[ae + k] for k in range(8)]; w1 = [lds[ae + BC + k] for k in range(8)]
                for t in range(ly, tn, RY):
                    xt = xp0 + t * 2 * BC + lx * V
                    x0 = [lds[xt + k] for k in range(8)]; x1 = [lds[xt + BC + k] for k in range(8)]
                    acc = [dot2(x1[k], w1[k], dot2(x0[k], w0[k], np.float32(0))) for k in range(8)]
                    bits = bf16_bits(np.array(acc, np.float32))
                    o = (m0 + t) * C + c0
                    for k in range(8): outs[e][o + k] = bits[k]; written[e][o + k] = True
    return [o.a for o in outs], written

def run_read_w(B, G, C, E, index=False, seed=0):
    rng = np.random.default_rng(seed)
    g = Geo(B, G, 2, C)
    idx = np.array([(m % g.GG * 7 + 3) % g.GG for m in range(g.M)], np.int32) if index else None
    xbits = bf16_bits(rng.standard_normal(B * g.GK * g.GK * C))
    abits = bf16_bits(0.25 + 0.02 * rng.standard_normal(E * C * 4))
    outs, written = emu_read_w(xbits, abits, E, g, idx)
    x = bf(xbits).astype(np.float64); a = bf(abits).astype(np.float64).reshape(E, C, 4)
    worst = 0
    for m in range(g.M):
        p0 = cell_pixel0(m, g, idx)
        xs = np.stack([x[slot_offset(p0, s, g, 0, K=2):slot_offset(p0, s, g, 0, K=2) + C] for s in range(4)])
        ref = np.einsum('ecs,sc->ec', a, xs)
        for e in range(E):
            worst = max(worst, ulps_ok(outs[e][m * C:(m + 1) * C], ref[e]))
    assert all(w.all() for w in written), "unwritten outputs"
    assert worst <= 1.0, worst
    print(f"read_w B={B} G={G} C={C} E={E} index={index}: bounds ok, all written, worst {worst:.3f} ulp", flush=True)
