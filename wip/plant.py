import numpy as np, emu_d2 as m
# extra dispatch combinations of the host (E -> ep, nw, npq)
for E, ep, nw, npq in [(16, 4, 4, 2), (9, 4, 3, 3), (21, 4, 6, 2), (12, 3, 4, 2)]:
    m.run(dict(kind="wgrad", B=1, G=5, C=64, E=E, chunks=3, ep=ep, nw=nw, npq=npq))
# planted bug 1: the earlier (wrong) channel order of the packed token-pair words
def bad_put(lds, dst, a, b, second):
    lo = [0] * 4; hi = [0] * 4
    for q in range(2):
        b0 = b[2 * q] if second else 0; b1 = b[2 * q + 1] if second else 0
        lo[2 * q] = m.pair_lo(a[2 * q], b0); lo[2 * q + 1] = m.pair_hi(a[2 * q], b0)
        hi[2 * q] = m.pair_lo(a[2 * q + 1], b1); hi[2 * q + 1] = m.pair_hi(a[2 * q + 1], b1)
    for k in range(4): lds[dst + k] = lo[k]
    for k in range(4): lds[dst + 4 + k] = hi[k]
import inspect
src = inspect.getsource(m.emu_wgradz)
# swap in the bad packing by patching the nested function via source edit
bad_src = src.replace("for k in range(2):\n            bl = b[k] if second else 0; bh = b[k + 2] if second else 0\n            lo[2 * k] = pair_lo(a[k], bl); lo[2 * k + 1] = pair_hi(a[k], bl)\n            hi[2 * k] = pair_lo(a[k + 2], bh); hi[2 * k + 1] = pair_hi(a[k + 2], bh)",
  "for q in range(2):\n            b0 = b[2 * q] if second else 0; b1 = b[2 * q + 1] if second else 0\n            lo[2 * q] = pair_lo(a[2 * q], b0); lo[2 * q + 1] = pair_hi(a[2 * q], b0)\n            hi[2 * q] = pair_lo(a[2 * q + 1], b1); hi[2 * q + 1] = pair_hi(a[2 * q + 1], b1)")
assert bad_src != src
ns = dict(m.__dict__); exec(bad_src, ns); m.emu_wgradz = ns["emu_wgradz"]
try:
    m.run(dict(kind="wgrad", B=1, G=5, C=64, E=8, chunks=2, ep=4, nw=2, npq=4))
    print("PLANTED BUG NOT CAUGHT")
except AssertionError:
    print("planted channel-order bug caught")
