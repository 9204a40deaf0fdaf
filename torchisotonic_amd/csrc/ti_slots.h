// The in-LDS merge of neighbouring hulls: G <= 64 child hulls laid end to end -> their parent's
// hull, in log2(G) pairwise rounds. Shared by the merge kernel (children from a node array) and
// the span kernel (its lanes' own hulls).
//
// A round merges hull pairs (L, R) that share their boundary point q, L's last vertex and R's
// first; the parent keeps a prefix of L and a suffix of R (the bridge). Per pair, a group of S
// lanes tests q and, if it dies, walks outwards from it (reference src/torchisotonic/csrc/
// tiles.cuh:1524-1537 merges segment pairs through the same bridge): with L's end vertex a and
// R's first b, lane k tests L's k-th vertex from the end against b and R's k-th from the start
// against a, and each side drops its vertices up to the first that stays (along a convex chain
// the test holds for a run from the end and then fails), until a step drops nothing: then both
// ends are convex, the bridge. The arrays are compact, so a step is one round of reads at known
// addresses. A walk still going after kWalk steps hands over to every thread at once: each
// remaining vertex of L decides whether it stays (its slope in below its lowest slope out to R,
// whose contact point a binary search over R finds), likewise R's, and the pair's first dying
// slot of L and last of R fix the bridge. The survivors then move down in one ordered compaction.
#pragma once

#include "ti_tile.h"

namespace ti {

// `cap` slots: coordinates in the parent's frame (double-double for float64 data), the vertex
// index within the parent, and the child (0..63) that owns each slot. A boundary point between
// two children is stored once, as the last vertex of the child on its left; slot 0 is the
// parent's first point. Where the children are several rows (aligned groups of 2^row_lg
// children, each row in a frame of its own from its first point), a row's first child stores
// its first point too, in the slot after the previous row's last.
template <bool W, bool PR>
struct Slots {
  double *s, *sl, *w, *wl;
  int* idx;
  uint8_t* cid;
};

template <bool W, bool PR>
constexpr size_t slot_bytes() {
  return 8 + (PR ? 8 : 0) + (W ? 8 : 0) + (W && PR ? 8 : 0) + 4 + 1;
}

// (cap a multiple of 64: every array stays 8-byte aligned)
template <bool W, bool PR>
__device__ __forceinline__ Slots<W, PR> slots_carve(char* p, int cap) {
  Slots<W, PR> v;
  v.s = reinterpret_cast<double*>(p);
  p += cap * 8;
  v.sl = v.w = v.wl = nullptr;
  if constexpr (PR) {
    v.sl = reinterpret_cast<double*>(p);
    p += cap * 8;
  }
  if constexpr (W) {
    v.w = reinterpret_cast<double*>(p);
    p += cap * 8;
  }
  if constexpr (W && PR) {
    v.wl = reinterpret_cast<double*>(p);
    p += cap * 8;
  }
  v.idx = reinterpret_cast<int*>(p);
  p += cap * 4;
  v.cid = reinterpret_cast<uint8_t*>(p);
  return v;
}

template <bool W, bool PR>
__device__ __forceinline__ HPt sget(const Slots<W, PR>& v, int k) {
  HPt p;
  p.i = v.idx[k];
  p.s = v.s[k];
  p.sl = PR ? v.sl[k] : 0.0;
  p.w = W ? v.w[k] : 0.0;
  p.wl = (W && PR) ? v.wl[k] : 0.0;
  return p;
}

template <bool W, bool PR>
__device__ __forceinline__ void sput(const Slots<W, PR>& v, int k, const HPt& p) {
  v.idx[k] = p.i;
  v.s[k] = p.s;
  if constexpr (PR) v.sl[k] = p.sl;
  if constexpr (W) v.w[k] = p.w;
  if constexpr (W && PR) v.wl[k] = p.wl;
}

// Round state: the last slot of every segment (this round's and the next's), and per pair
// whether its junction dies, the first dying slot of its left part, the last dying slot of its
// right part, and the two edges at the junction (dS, dW into q from L, out of q into R).
struct MergeRounds {
  int seg[2][kGroup];
  int fdl[kGroup / 2];
  int ldr[kGroup / 2];
  int jdead[kGroup / 2];
  double edge[kGroup / 2][4];
  int walk[kGroup / 2][2];  // where a pair's walk stopped: L's and R's current end vertices
  int wflag[16];            // per wave: bit 0 some junction died, bit 1 some walk did not finish
  int wsum[4][16];
};

template <bool W, bool PR>
__device__ __forceinline__ void hdiff(const HPt& a, const HPt& b, double& dS, double& dW) {
  dS = b.s - a.s;
  if constexpr (PR) dS += b.sl - a.sl;
  if constexpr (W) {
    dW = b.w - a.w;
    if constexpr (PR) dW += b.wl - a.wl;
  } else {
    dW = static_cast<double>(b.i - a.i);
  }
}

// c ? a : b, field by field (a select of whole structs would keep them in memory)
__device__ __forceinline__ HPt hsel(bool c, const HPt& a, const HPt& b) {
  HPt r;
  r.i = c ? a.i : b.i;
  r.s = c ? a.s : b.s;
  r.sl = c ? a.sl : b.sl;
  r.w = c ? a.w : b.w;
  r.wl = c ? a.wl : b.wl;
  return r;
}

template <bool W, bool PR>
__device__ __forceinline__ bool hpools_nb(const HPt& a, const HPt& b, const HPt& c) {
  double dS1, dW1, dS2, dW2;
  hdiff<W, PR>(a, b, dS1, dW1);
  hdiff<W, PR>(b, c, dS2, dW2);
  return pools_nb(dS1, dW1, dS2, dW2);
}

// Merges the `nch` children in slots [0, total) into one hull in slots [0, result). On entry
// rs.seg[0][c] holds the last slot of child c and every thread has passed a barrier since the
// slots were written. row_lg: children in aligned groups of 2^row_lg are separate rows (then
// max_rounds <= row_lg), a row's first slot its first child's own (see Slots). NT >= 64 threads; the vertex tests take slots s = tid + k * NT, G of
// them at a time in lockstep (their LDS reads in flight together). After max_rounds rounds it
// stops: segment s (children [s * 2^R, (s + 1) * 2^R), R the rounds run) is then one hull, and
// rs.seg[R & 1][s] its last slot.
//
// Which vertices can die: L keeps every vertex whose slope in is below R's first edge (R lies
// above that edge's line, so no slope from the vertex to R is lower), R every vertex whose slope
// out is above L's last edge. By convexity those are all but a suffix of L and a prefix of R,
// the only vertices that search.
constexpr int kWalk = 8;

// The number of leading ones of the S-bit group g.
__device__ __forceinline__ int lead_ones(uint64_t g, uint64_t gmask, int S) {
  const uint64_t z = ~g & gmask;
  return z ? __builtin_ctzll(z) : S;
}

template <bool W, bool PR, int NT, int G>
__device__ int merge_rounds(const Slots<W, PR>& v, MergeRounds& rs, int total, int nch, int max_rounds = 6,
                            int row_lg = 30) {
  constexpr int NW = NT / kWave;
  const int row_mask = (1 << row_lg) - 1;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  int cur = 0;
#pragma unroll 1
  for (int r = 0; (1 << r) < nch && r < max_rounds; ++r) {
    const int nseg = (nch + (1 << r) - 1) >> r;
    const int npair = nseg >> 1;
    const int* se = rs.seg[cur];
    int* sn = rs.seg[cur ^ 1];
    // 1. per pair (a group of S lanes each, the at most 32 pairs spread over the waves): the
    // junction, and from a dying junction the walk outwards, for at most kWalk steps
    {
      const int per_wave = (npair + NW - 1) / NW;
      int lg_ppw = 0;
      while ((1 << lg_ppw) < per_wave) ++lg_ppw;
      const int lg_s = 6 - lg_ppw;  // S = 64 / (pairs per wave), at least 2
      const int S = 1 << lg_s;
      const int sub = lane >> lg_s, k = lane & (S - 1);
      const int p_raw = (wave << lg_ppw) + sub;
      const bool has = p_raw < npair;
      const int p = has ? p_raw : 0;
      const uint64_t gmask = S == 64 ? ~uint64_t{0} : ((uint64_t{1} << S) - 1);
      const int gshift = sub << lg_s;
      const int q = se[2 * p];
      // (L's first point: the previous segment's last, or its own slot after it at a row's start)
      const int lo_l = p > 0 ? se[max(2 * p - 1, 0)] + ((((2 * p) << r) & row_mask) == 0 ? 1 : 0) : 0;
      const int hi_r = se[2 * p + 1];
      double dSl, dWl, dSr, dWr;
      {
        const HPt A = sget(v, q - 1), Q = sget(v, q), B = sget(v, q + 1);
        hdiff<W, PR>(A, Q, dSl, dWl);
        hdiff<W, PR>(Q, B, dSr, dWr);
      }
      const bool dead = has & pools_nb(dSl, dWl, dSr, dWr);
      int ia = q - 1, ib = q + 1;
      bool walking = dead;
      for (int it = 0; it < kWalk; ++it) {
        if (!__any(walking)) break;
        // every read of the step first: both ends, lane k's L vertex (and the one before it)
        // and R vertex (and the one after it), indices clamped into the pair
        const int xl = ia - k, xr = ib + k;
        const HPt A = sget(v, ia), B = sget(v, ib);
        const HPt XL = sget(v, max(xl, lo_l)), XLP = sget(v, max(xl - 1, lo_l));
        const HPt XR = sget(v, min(xr, hi_r)), XRN = sget(v, min(xr + 1, hi_r));
        const bool dl = walking & (xl > lo_l) & hpools_nb<W, PR>(XLP, XL, B);
        const bool dr = walking & (xr < hi_r) & hpools_nb<W, PR>(A, XR, XRN);
        const int ml = lead_ones(__ballot(dl) >> gshift, gmask, S);
        const int mr = lead_ones(__ballot(dr) >> gshift, gmask, S);
        ia -= ml;
        ib += mr;
        walking = walking & ((ml | mr) != 0);
      }
      if (has && k == 0) {
        rs.jdead[p] = dead ? (walking ? 2 : 1) : 0;
        rs.fdl[p] = dead ? ia + 1 : 0x7FFFFFFF;
        rs.ldr[p] = dead ? ib - 1 : -1;
        rs.walk[p][0] = ia;
        rs.walk[p][1] = ib;
        rs.edge[p][0] = dSl;
        rs.edge[p][1] = dWl;
        rs.edge[p][2] = dSr;
        rs.edge[p][3] = dWr;
      }
      const bool anydead = __any(dead), more = __any(walking);
      if (lane == 0) rs.wflag[wave] = (anydead ? 1 : 0) | (more ? 2 : 0);
    }
    __syncthreads();
    int flags = 0;
#pragma unroll
    for (int w2 = 0; w2 < NW; ++w2) flags |= rs.wflag[w2];
    // 2. the vertices near a dying junction. Straight-line code: every read has a valid
    // (clamped) index and results are selected, so the G slots' LDS reads overlap instead of each
    // waiting behind its own branch.
    static_assert(G >= 1 && G <= 4, "lockstep group of 1..4 slots");
#pragma unroll 1
    for (int g0 = 0; (flags & 2) != 0 && g0 < total; g0 += NT * G) {
      int sk[G], lo[G], hi[G], pk[G];
      bool left[G], need[G];
      HPt P[G], N[G];
#pragma unroll
      for (int u = 0; u < G; ++u) {
        const int s_raw = g0 + u * NT + tid;
        const int s = min(s_raw, total - 1);
        const int c = v.cid[s] >> r;
        const int p = c >> 1;
        const int pc = p < npair ? p : 0;
        const int q = se[2 * pc];
        const int lo_l = pc > 0 ? se[max(2 * pc - 1, 0)] + ((((2 * pc) << r) & row_mask) == 0 ? 1 : 0) : 0;
        const int hi_r = se[2 * pc + 1];
        const int jd = rs.jdead[pc];
        const int wl = rs.walk[pc][0], wr = rs.walk[pc][1];
        const bool lf = (c & 1) == 0;
        sk[u] = s;
        pk[u] = pc;
        left[u] = lf;
        lo[u] = lf ? q : lo_l;
        hi[u] = lf ? hi_r : q;
        // (only pairs whose walk did not finish, and only what the walk has not removed)
        const bool lneed = (s > lo_l) & (s <= wl), rneed = (s >= wr) & (s < hi_r);
        need[u] = (s_raw < total) & (p < npair) & (jd == 2) & ((lf & lneed) | (!lf & rneed));
        P[u] = sget(v, s);
        N[u] = sget(v, lf ? max(s - 1, 0) : min(s + 1, total - 1));
      }
#pragma unroll
      for (int u = 0; u < G; ++u) {
        // L can lose a vertex only if its slope in is at least R's first edge's; R only if its
        // slope out is at most L's last edge's
        const bool lf = left[u];
        double dS, dW;
        hdiff<W, PR>(hsel(lf, N[u], P[u]), hsel(lf, P[u], N[u]), dS, dW);
        const double* e = rs.edge[pk[u]];
        const double e0 = e[0], e1 = e[1], e2 = e[2], e3 = e[3];
        need[u] = need[u] & pools_nb(lf ? dS : e0, lf ? dW : e1, lf ? e2 : dS, lf ? e3 : dW);
      }
      // contact points, all searches stepping together: on R, the first j where the slope from
      // P stops falling (pools(P, j, j+1) fails); on L, the first i where the slope to P stops
      // rising (pools(i, i+1, P) holds)
      for (;;) {
        bool any = false;
#pragma unroll
        for (int u = 0; u < G; ++u) any |= need[u] & (lo[u] < hi[u]);
        if (!__any(any)) break;
        // every slot's two reads first, then the tests
        int mid[G];
        HPt A[G], B[G];
#pragma unroll
        for (int u = 0; u < G; ++u) {
          mid[u] = (lo[u] + hi[u]) >> 1;
          A[u] = sget(v, mid[u]);
          B[u] = sget(v, min(mid[u] + 1, total - 1));
        }
#pragma unroll
        for (int u = 0; u < G; ++u) {
          const bool act = need[u] & (lo[u] < hi[u]);
          const bool lf = left[u];
          const bool t = hpools_nb<W, PR>(hsel(lf, P[u], A[u]), hsel(lf, A[u], B[u]), hsel(lf, B[u], P[u])) == lf;
          lo[u] = (act && t) ? mid[u] + 1 : lo[u];
          hi[u] = (act && !t) ? mid[u] : hi[u];
        }
      }
      bool dies[G];
      {
        HPt T[G];
#pragma unroll
        for (int u = 0; u < G; ++u) T[u] = sget(v, lo[u]);
#pragma unroll
        for (int u = 0; u < G; ++u) {
          const bool lf = left[u];
          dies[u] = need[u] & hpools_nb<W, PR>(hsel(lf, N[u], T[u]), P[u], hsel(lf, T[u], N[u]));
        }
      }
#pragma unroll
      for (int u = 0; u < G; ++u) {
        if (dies[u]) {
          if (left[u]) atomicMin(&rs.fdl[pk[u]], sk[u]);
          else atomicMax(&rs.ldr[pk[u]], sk[u]);
        }
      }
    }
    __syncthreads();
    if ((flags & 1) == 0) {
      // nothing died: nothing moves, and a merged pair ends where its right part did
      for (int k = tid; k < (nseg + 1) / 2; k += NT) sn[k] = se[min(2 * k + 1, nseg - 1)];
      __syncthreads();
      cur ^= 1;
      continue;
    }
    // 3. compaction, G batches of NT slots at a time: every slot of the group read, then the
    // survivors written in slot order (a slot only moves down, and never past the group's start
    // into a later group's slots)
    int base = 0;
#pragma unroll 1
    for (int g0 = 0; g0 < total; g0 += NT * G) {
      HPt x[G];
      uint8_t id[G];
      bool alive[G], isend[G];
      int cnt[G];
#pragma unroll
      for (int u = 0; u < G; ++u) {
        const int s_raw = g0 + u * NT + tid;
        const int s = min(s_raw, total - 1);
        id[u] = v.cid[s];
        const int c = id[u] >> r;
        const int p = c >> 1;
        const int pc = p < npair ? p : 0;
        const int ldr = rs.ldr[pc], fdl = rs.fdl[pc], end = se[c];
        const bool keep = (p >= npair) | ((c & 1) ? s > ldr : s < fdl);
        alive[u] = (s_raw < total) & keep;
        // the next round's segment ends: the right part's last slot, or an unpaired segment's
        isend[u] = (s == end) & (((c & 1) != 0) | (c == nseg - 1));
        x[u] = sget(v, s);
      }
      uint64_t m[G];
#pragma unroll
      for (int u = 0; u < G; ++u) {
        m[u] = __ballot(alive[u]);
        cnt[u] = __popcll(m[u]);
      }
      int before[G];
      if constexpr (NW == 1) {
        int b = base;
#pragma unroll
        for (int u = 0; u < G; ++u) {
          before[u] = b;
          b += cnt[u];
        }
        base = b;
      } else {
        if (lane == 0) {
#pragma unroll
          for (int u = 0; u < G; ++u) rs.wsum[u][wave] = cnt[u];
        }
        __syncthreads();
        int b = base;
#pragma unroll
        for (int u = 0; u < G; ++u) {
          int mine = 0, all = 0;
#pragma unroll
          for (int k = 0; k < NW; ++k) {
            const int c = rs.wsum[u][k];
            mine += k < wave ? c : 0;
            all += c;
          }
          before[u] = b + mine;
          b += all;
        }
        base = b;
        __syncthreads();  // all slots of the group read, wsum free again
      }
#pragma unroll
      for (int u = 0; u < G; ++u) {
        if (alive[u]) {
          const int s = g0 + u * NT + tid;
          const int np = before[u] + __popcll(m[u] & ((uint64_t{1} << lane) - 1));
          if (isend[u]) sn[(id[u] >> r) >> 1] = np;
          if (np != s) {
            sput(v, np, x[u]);
            v.cid[np] = id[u];
          }
        }
      }
    }
    total = base;
    __syncthreads();
    cur ^= 1;
  }
  return total;
}

}  // namespace ti
