"""The range bookkeeping of the long-row merge in global memory (merge_global in
torchisotonic_amd/csrc/ti_merge.hip), restated in Python on integer points: children are
convex lower chains sharing their boundary points, each keeps a range of its vertices, pairwise
rounds bridge the concatenations of those ranges (with the kernel's bridge: a walk from the
junction, then binary searches) and only shorten the ranges. The survivors must be the lower
hull of all the points (equal slopes pool), for random child sets that keep most vertices,
lose most, tie, or mix. The GPU tests check the kernel itself on near-monotone rows."""

from __future__ import annotations

import numpy as np

def lower_hull(pts):
    h = []
    for p in pts:
        while len(h) >= 2 and cross(h[-2], h[-1], p) <= 0:  # pools: equal slopes merge
            h.pop()
        h.append(p)
    return h

def cross(a, b, c):  # > 0: b strictly below chord a-c (convex turn)
    return (b[0] - a[0]) * (c[1] - a[1]) - (b[1] - a[1]) * (c[0] - a[0])

def pools(a, b, c):  # vertex b dies between a and c: slope(a,b) >= slope(b,c)
    return cross(a, b, c) <= 0

def vtangent(p, getB, cB):
    lo, hi = 1, cB - 1
    while lo < hi:
        mid = (lo + hi) >> 1
        if not pools(p, getB(mid), getB(mid + 1)): hi = mid
        else: lo = mid + 1
    return lo

def vbridge(getA, cA, getB, cB):
    if cB <= 1: return cA, cB
    if cA <= 1: return 0, 0
    a, x, b = getA(cA - 2), getA(cA - 1), getB(1)
    if not pools(a, x, b): return cA, 1
    i, j = cA - 2, 1
    done = False
    ap = getA(i - 1) if i > 0 else a
    bn = getB(j + 1) if j + 1 < cB else b
    for _ in range(24):
        if i > 0 and pools(ap, a, b):
            i -= 1; a = ap
            if i > 0: ap = getA(i - 1)
        elif j + 1 < cB and pools(a, b, bn):
            j += 1; b = bn
            if j + 1 < cB: bn = getB(j + 1)
        else:
            done = True; break
    if not done:
        lo, hi = 0, cA - 2
        while lo < hi:
            mid = (lo + hi) >> 1
            am = getA(mid)
            t = vtangent(am, getB, cB)
            if pools(am, getA(mid + 1), getB(t)): hi = mid
            else: lo = mid + 1
        i = lo
        j = vtangent(getA(lo), getB, cB)
    return i + 1, j

def merge_ranges(children):
    nch = len(children)
    lo = [0 if c == 0 else 1 for c in range(nch)]
    hi = [len(ch) for ch in children]
    span = 1
    while span < nch:
        for pa in range(0, nch, 2 * span):
            pb = pa + span
            if pb >= nch: continue
            pe = min(pb + span, nch)
            pre = {}
            acc = 0
            for c in range(pa, pb): pre[c] = acc; acc += hi[c] - lo[c]
            nA = acc
            acc = 0
            for c in range(pb, pe): pre[c] = acc; acc += hi[c] - lo[c]
            nB = acc
            def vget(a, b, i):
                c = max(cc for cc in range(a, b) if pre[cc] <= i)
                return children[c][lo[c] + i - pre[c]]
            s = 1 if pa > 0 else 0  # A's start point in front (the previous segment keeps it)
            cA = s + nA
            getA = (lambda i: children[pa][0] if i == 0 else vget(pa, pb, i - 1)) if s else (lambda i: vget(pa, pb, i))
            cB = 1 + nB
            getB = lambda j: getA(cA - 1) if j == 0 else vget(pb, pe, j - 1)
            keep, frm = vbridge(getA, cA, getB, cB)
            a_keep = nA if frm == 0 else keep - s
            assert 0 <= a_keep <= nA
            b_drop = max(frm - 1, 0)
            assert b_drop <= nB
            left = a_keep
            for c in range(pa, pb):
                k = hi[c] - lo[c]
                if left >= k: left -= k
                else: hi[c] = lo[c] + left; left = 0
            d = b_drop
            for c in range(pb, pe):
                k = hi[c] - lo[c]
                if d >= k: lo[c] = hi[c]; d -= k
                else: lo[c] += d; d = 0
        span *= 2
    out = []
    for c in range(nch): out += children[c][lo[c]:hi[c]]
    return out



def test_range_merge_gives_the_lower_hull_of_all_points() -> None:
    rng = np.random.default_rng(0)
    for trial in range(1500):
        nch = int(rng.integers(1, 70))
        kind = trial % 5
        pts_all = [(0, 0)]
        children = []
        x, s = 0, 0
        for _ in range(nch):
            m = int(rng.integers(1, 40 if kind == 4 else 9))
            seg = [(x, s)]
            for _ in range(m):
                x += 1
                if kind == 0:
                    s += int(rng.integers(-3, 4))
                elif kind == 1:
                    s += x  # convex: every vertex survives
                elif kind == 2:
                    s += -x  # concave: almost every vertex dies
                elif kind == 3:
                    s += int(rng.integers(-1, 2)) * 2  # ties and collinear runs
                else:
                    s += int(rng.integers(-50, 51)) + (x * x) // 200
                seg.append((x, s))
            pts_all += seg[1:]
            children.append(lower_hull(seg))
        assert merge_ranges(children) == lower_hull(pts_all), (trial, kind)
