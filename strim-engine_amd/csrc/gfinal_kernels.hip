// gfinal_kernels.hip — k_gfinal: the general rows, decided from the chunks' lattice
// histograms and candidates.
//
// A general row (top-p alone, a top-k above KLOC, a min-p below MINP_FAST, no filter with
// icdf noise) cannot bound its candidates by a chunk's own maximum. k_stream bins every
// general row's tokens on one absolute lattice of l, A(l) = floor(l * LBS): a chunk keeps
// the counts and masses of the NBW bins below its top bin A(m_c) (its window) and writes
// its window tokens in bin order, as many whole bins as fit LCAP slots (nfull bins). Since
// every chunk bins the same way, row bin rb = A(m) - A(l) below the row's maximum m
// collects chunk c's bin rb - d_c, d_c = A(m) - A(m_c): the chunks' histograms add up to
// the row's, and every decision of the row (the k-th token, the min-p bound, the top-p
// cut, the icdf draw) is found in two steps:
//   1. the row bin where the cumulative count or mass crosses the decision's threshold;
//   2. the bin's tokens (its zone), gathered from the chunks' slot regions (each chunk's
//      part of the bin is a contiguous run there) and resolved exactly in (l desc, id asc)
//      order, each token's mass taken from its own l.
// A zone in a bin that some chunk could not write whole is collected by one streaming
// pass of this workgroup over the row. A decision below a chunk's window (the lattice
// cannot place it), rank-indexed noise and rows whose lattice words were not written take
// the exact streaming resolution (exact.hpp).
//
// Masses are fixed point, 2^40 per unit of exp(l - m) (RFIX): integer sums make every
// cumulative mass independent of summation order. A chunk's bin masses (2^37 per unit of
// exp(l - m_c), from float exponentials) are scaled by exp(m_c - m) once per (chunk, bin);
// a zone token's mass is expf(l - m) 2^40. Both are within a few 1e-7 relative of the
// exact mass, inside the 1e-6 decision tolerance.
//
// One 512-thread workgroup per row. Its time is latency (one global round trip for the
// chunk statistics and lattice words, then one per zone), so the loads that do not depend
// on the row's parameters are issued first, and every wave keeps the row's cumulative
// histogram in its own registers (a decision's bin search needs no barrier).
#include "exact.hpp"

namespace strim {

constexpr int GT = 512;                          // threads of a k_gfinal workgroup
constexpr int GW = GT / WAVE;                    // its waves
constexpr int LPL = NBW / WAVE;                  // row bins per lane (bins LPL lane + q)
constexpr float RFIXF = 1099511627776.0f;        // 2^40: fixed-point unit of row mass
constexpr double RFIX = 1099511627776.0;
constexpr int ZCAP = 4096;                       // keys of one zone
constexpr int ZQ = ZCAP / GT;                    // zone positions per thread (radix picks)
constexpr int RADIX_MIN = 256;  // wider zones are picked by radix select, not all pairs
constexpr int PF = 160;                          // candidates of each chunk prefetched
// The lattice words and the prefetched candidates are loaded straight into LDS, 1 KB per
// wave instruction (16 bytes per lane): KW and KP instructions per wave.
constexpr int LWB = LWMAX * NBW * 8, PFB = LWMAX * PF * 8;  // their bytes
constexpr int DW = GW - 1;  // the waves that issue them: all but wave 0
constexpr int KW = (LWB / 1024 + DW - 1) / DW, KP = (PFB / 1024 + DW - 1) / DW;
static_assert(LWB % 1024 == 0 && PFB % 1024 == 0, "whole 1 KB blocks");
static_assert(PF <= LCAP && PF % 2 == 0, "prefetch layout");
constexpr int NOBIN = 1 << 20;                   // "no bin": beyond every window
static_assert(NBW % WAVE == 0 && LWMAX % GW == 0 && LWMAX <= WAVE, "lattice layout");
static_assert(LCAP <= SLOT && LCAP < 65536, "the candidates fit a chunk's slot region");

// LDS of one k_gfinal workgroup: the two large areas the lattice words and candidates are
// loaded into (objects of their own: the loads into them are then known not to touch the
// small state, so reading the chunk statistics does not wait for them), and the rest.
union GBig {
  uint64_t E[LWMAX * NBW];        // the chunks' lattice words (until they are merged)
  struct {                        // a zone: its keys and their masses
    uint64_t zkey[ZCAP];
    uint64_t zmass[ZCAP];
  } z;
  struct {                        // the exact streaming resolution
    uint64_t xkey[XB > XCOL ? XB : XCOL];
    uint32_t xhc[XB];
    uint32_t xcnt[GT * EPT];
    uint64_t xu2[2 * GT / WAVE];
    XState x;
  } x;
};
union GPf {
  Cand pfb[LWMAX * PF];           // each chunk's first PF candidates (prefetched)
  uint32_t ccnt[GT * EPT];        // a collect pass: history counts of one window (the
};                                // prefetched candidates are dropped by then)
// A step of the decision loop, as the leader wave posts it to the workgroup.
enum { GOP_PICK = 0, GOP_SUM = 1, GOP_SKIP = 2, GOP_BOUND = 3, GOP_FAIL = 4 };
struct GCmd {
  int op;           // GOP_*: pick a key, sum the zone's masses up to a bound, skip the
                    // step, only set the bound, or leave the row to the exact resolution
  int load;         // the zone to load first: 0 none (in LDS), 1 from the chunks' parts
                    // (zpo / zpc / zpz), 2 by a collect pass
  int bz, also;     // the step's bin; the bin loaded beside it (-1: none)
  int n0, n1;       // the loaded bins' key counts
  int by_mass, excl;
  double thr;
  uint64_t bnd, c0, m0, bmp;
};
struct GFinalShared {
  uint16_t pc[LWMAX][NBW];        // per chunk: inclusive count prefix of its window bins
  uint32_t rc[NBW];               // row bins: counts
  unsigned long long rm[NBW];     // row bins: masses (RFIX per unit of exp(l - m))
  int nbch[LWMAX];                // per chunk: window bins written
  int ncnt[LWMAX];                // per chunk: allowed tokens
  int dch[LWMAX];                 // per chunk: its top bin's distance below the row's
  double sch[LWMAX];              // per chunk: its mass sum relative to the row maximum
  int zoff[LWMAX + 1];            // the Gumbel walk: exclusive offsets of the chunks' parts
  float v[GW];
  int i[GW], f[GW];
  double d[GW];
  uint64_t u[GW], u2[2 * GW];
  int ii[GW];
  int misc[8];                    // 0 rowfull, 1 rowwin, 2 collect count, 3 some tail
  uint64_t res[2][4];             // a pick: key, count before, mass before, mass (two
  int32_t tag[2];                 // slots, alternating; tag = the pick's number)
  int zpo[2][LWMAX], zpc[2][LWMAX], zpz[2][LWMAX];  // a zone's parts per chunk: first
                                                    // slot, count, place in the zone
  GCmd cmd;                       // the decision loop's current step
  uint32_t prk[GT];               // a pick: each zone key's rank and the mass before it
  unsigned long long pmb[GT];
};

__device__ __forceinline__ float key_l(uint64_t k) { return fkey_desc_inv((uint32_t)(k >> 32)); }
// Fixed-point mass of a token relative to the row maximum m (l <= m).
__device__ __forceinline__ uint64_t rmass(float l, float m) {
  return (uint64_t)(expf(l - m) * RFIXF);
}
// Row bin of l: A(m) - A(l) (arow = A(m)); NOBIN past the row's window or for -inf.
__device__ __forceinline__ int row_bin(float arow, float l) {
  if (!(l > -INFINITY)) return NOBIN;
  const float d = arow - floorf(l * (float)LBS);
  return d < (float)NBW ? (int)d : NOBIN;
}

// A pick: the key (~0: none), the count and mass of the keys before it in the row's
// order, and its own mass.
struct GHit {
  uint64_t key, cnt_before, mass_before, mass;
};

// The row's cumulative histogram in a wave's registers: lane l holds bins LPL l + q.
// Three named members, not an array: a runtime-indexed array would be placed in scratch
// memory, a round trip to the cache for every read.
struct RowCum {
  uint32_t c0, c1, c2;
  uint64_t m0, m1, m2;
  __device__ __forceinline__ uint32_t& cq(int q) { return q == 0 ? c0 : (q == 1 ? c1 : c2); }
  __device__ __forceinline__ uint64_t& mq(int q) { return q == 0 ? m0 : (q == 1 ? m1 : m2); }
  // inclusive cumulative count / mass of bin b (wave-uniform; b < 0: 0, b past the row's
  // window: the window's total): the three bins of lane b / LPL read, one kept
  __device__ __forceinline__ uint64_t cnt(int b) const {
    b = uniform_copy(b);
    if (b < 0) return 0ull;
    if (b >= NBW) b = NBW - 1;
    const int L = b / LPL, q = b - LPL * L;
    const uint32_t v0 = (uint32_t)__builtin_amdgcn_readlane((int)c0, L);
    const uint32_t v1 = (uint32_t)__builtin_amdgcn_readlane((int)c1, L);
    const uint32_t v2 = (uint32_t)__builtin_amdgcn_readlane((int)c2, L);
    return (uint64_t)(q == 0 ? v0 : (q == 1 ? v1 : v2));
  }
  __device__ __forceinline__ uint64_t mass(int b) const {
    b = uniform_copy(b);
    if (b < 0) return 0ull;
    if (b >= NBW) b = NBW - 1;
    const int L = b / LPL, q = b - LPL * L;
    const uint64_t v0 = rl_u64(m0, L), v1 = rl_u64(m1, L), v2 = rl_u64(m2, L);
    return q == 0 ? v0 : (q == 1 ? v1 : v2);
  }
  // the first bin b < limit whose cumulative value (the mass less excl_w from bin excl_b
  // on) exceeds thr; limit when none does
  __device__ __forceinline__ int find(bool by_mass, double thr, int limit, uint64_t excl_w,
                                      int excl_b) const {
    const int lane = threadIdx.x & (WAVE - 1);
    const uint32_t cc[LPL] = {c0, c1, c2};
    const uint64_t mm[LPL] = {m0, m1, m2};
    int first = NOBIN;
#pragma unroll
    for (int q = LPL - 1; q >= 0; --q) {
      const int b = LPL * lane + q;
      const uint64_t val = by_mass ? mm[q] - (b >= excl_b ? excl_w : 0ull) : (uint64_t)cc[q];
      if (b < limit && (double)val > thr) first = b;
    }
    first = wave_min_i(first);
    return uniform_copy(first < limit ? first : limit);
  }
};
static_assert(LPL == 3, "RowCum holds three bins per lane");

// Pick number np over the zone zkey/zmass[z0, z0 + n) (unsorted, n <= GT): the first key in
// key order, key <= bound and id != excl, whose inclusive cumulative count (by_mass false:
// every key counts) or mass exceeds thr, from cnt0 / mass0 before the zone. Every thread
// compares one key with every R-th key of the zone (R = GT / n), so each key's rank and
// the mass before it are summed from R partial counts; the unique key whose interval
// contains thr writes its result to slot np & 1 (a slot is rewritten two picks later,
// after every thread has read it). Three barriers.
__device__ __forceinline__ GHit pick_rank(GFinalShared& S, GBig& G, int np, int z0, int n, bool by_mass,
                                          double thr, uint64_t bound, int excl, uint64_t cnt0,
                                          uint64_t mass0) {
  const int t = threadIdx.x;
  const int slot = np & 1;
  if (t < n) {
    S.prk[t] = 0u;
    S.pmb[t] = 0ull;
  }
  __syncthreads();
  const int R = n > 0 ? GT / n : 1;
  const int i = t / R, sg = t - i * R;
  if (i < n) {
    const uint64_t* zk = G.z.zkey + z0;
    const uint64_t* zm = G.z.zmass + z0;
    const uint64_t k = zk[i];
    uint32_t rank = 0u;
    uint64_t mb = 0ull;
    int jj = sg;
    for (; jj + 3 * R < n; jj += 4 * R) {
      uint64_t kj[4], mj[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        kj[u] = zk[jj + u * R];
        mj[u] = zm[jj + u * R];
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const bool lt = kj[u] < k;
        rank += lt ? 1u : 0u;
        mb += (lt && kj[u] <= bound && (int)(uint32_t)kj[u] != excl) ? mj[u] : 0ull;
      }
    }
    for (; jj < n; jj += R) {
      const uint64_t kj = zk[jj];
      const bool lt = kj < k;
      rank += lt ? 1u : 0u;
      mb += (lt && kj <= bound && (int)(uint32_t)kj != excl) ? zm[jj] : 0ull;
    }
    if (rank) atomicAdd(&S.prk[i], rank);
    if (mb) atomicAdd(&S.pmb[i], (unsigned long long)mb);
  }
  __syncthreads();
  if (t < n) {
    const uint64_t k = G.z.zkey[z0 + t];
    const uint64_t km = G.z.zmass[z0 + t];
    const bool in = k <= bound && (int)(uint32_t)k != excl;
    const uint32_t rank = S.prk[t];
    const uint64_t mb = S.pmb[t];
    const uint64_t before = by_mass ? mass0 + mb : cnt0 + rank;
    const uint64_t own = by_mass ? (in ? km : 0ull) : 1ull;
    if (own > 0ull && (double)before <= thr && (double)(before + own) > thr) {
      S.res[slot][0] = k;
      S.res[slot][1] = cnt0 + rank;
      S.res[slot][2] = mass0 + mb;
      S.res[slot][3] = km;
      S.tag[slot] = np;
    }
  }
  __syncthreads();
  if (S.tag[slot] != np) return GHit{~0ull, 0ull, 0ull, 0ull};
  return GHit{S.res[slot][0], S.res[slot][1], S.res[slot][2], S.res[slot][3]};
}

// The same pick over a zone of up to ZCAP keys at z0 (unsorted), for zones too wide for
// pick_rank's all-pairs count (more than RADIX_MIN keys):
// an MSD radix select over the keys' compact form (fkey << 20 | id, in the keys' order:
// ids are below 2^20), up to 8 bits a pass from the highest bit where the zone's keys
// differ. A pass histograms the candidates' digits (their count, and the kept mass: keys
// <= bound, id != excl), and wave 0 finds the digit d whose interval of cumulative weight
// (count, or kept mass), from cnt0 / mass0 and the weight below the candidates, holds thr:
// (double)before(d) <= thr < (double)(before(d) + weight(d)), as pick_rank's rule for one
// key. The candidates narrow to d until every bit is fixed: about five passes of three
// barriers for the keys of one lattice bin.
__device__ __forceinline__ GHit pick_sorted(GFinalShared& S, GBig& G, int np, int z0, int n,
                                            bool by_mass, double thr, uint64_t bound, int excl,
                                            uint64_t cnt0, uint64_t mass0) {
  const int t = threadIdx.x, lane = t & (WAVE - 1), w = wave_id();
  const int slot = np & 1;
  auto compact = [](uint64_t k) { return ((k >> 32) << 20) | (k & 0xFFFFFull); };
  uint64_t ck[ZQ], km[ZQ];
  bool in[ZQ];
  const uint64_t ref = compact(G.z.zkey[z0]);
  uint64_t diff = 0ull;
#pragma unroll
  for (int q = 0; q < ZQ; ++q) {
    const int pos = t + GT * q;
    const bool pr = pos < n;
    const uint64_t k = pr ? G.z.zkey[z0 + pos] : 0ull;
    ck[q] = pr ? compact(k) : ~0ull;
    km[q] = pr ? G.z.zmass[z0 + pos] : 0ull;
    in[q] = pr && k <= bound && (int)(uint32_t)k != excl;
    if (pr) diff |= ck[q] ^ ref;
  }
  diff = block_or_u64<GT>(diff, S.u);
  int hb = diff ? 63 - __clzll((long long)diff) : -1;
  uint64_t pmask = ~((2ull << (hb < 0 ? 0 : hb)) - 1ull);  // the bits every candidate shares
  if (hb < 0) pmask = ~0ull;
  uint64_t prefix = ref & pmask;
  uint64_t bc = cnt0, bm = mass0;  // weights below the candidates
  while (hb >= 0) {
    const int shift = hb >= 7 ? hb - 7 : 0;
    if (t < 256) {
      S.prk[t] = 0u;
      S.pmb[t] = 0ull;
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < ZQ; ++q)
      if ((ck[q] & pmask) == prefix) {
        const int d = (int)((ck[q] >> shift) & 255ull);
        atomicAdd(&S.prk[d], 1u);
        if (in[q]) atomicAdd(&S.pmb[d], (unsigned long long)km[q]);
      }
    __syncthreads();
    if (w == 0) {
      // lane l: digits 4 l .. 4 l + 3
      uint32_t c[4];
      uint64_t mm[4];
      uint32_t lc = 0u;
      uint64_t lm = 0ull;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        c[i] = S.prk[4 * lane + i];
        mm[i] = S.pmb[4 * lane + i];
        lc += c[i];
        lm += mm[i];
      }
      uint64_t Bc = bc + (uint64_t)(wave_incl_scan_u32(lc) - lc);
      uint64_t Bm = bm + (wave_incl_scan_u64(lm) - lm);
      int hit = -1;
      uint64_t hc = 0ull, hm = 0ull;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint64_t before = by_mass ? Bm : Bc;
        const uint64_t own = by_mass ? mm[i] : (uint64_t)c[i];
        if (hit < 0 && own > 0ull && (double)before <= thr && (double)(before + own) > thr) {
          hit = 4 * lane + i;
          hc = Bc;
          hm = Bm;
        }
        Bc += c[i];
        Bm += mm[i];
      }
      const uint64_t bal = __ballot(hit >= 0);
      if (lane == 0) S.ii[0] = -1;
      if (bal != 0ull) {
        const int hl = (int)__ffsll((long long)bal) - 1;
        if (lane == hl) {
          S.ii[0] = hit;
          S.u2[0] = hc;
          S.u2[1] = hm;
        }
      }
    }
    __syncthreads();
    const int d = S.ii[0];
    if (d < 0) return GHit{~0ull, 0ull, 0ull, 0ull};  // (uniform) no key crosses
    prefix |= (uint64_t)d << shift;
    pmask |= 255ull << shift;
    bc = S.u2[0];
    bm = S.u2[1];
    // the bits that still differ among the keys under the prefix (set in some, clear in
    // others): the next pass starts at the highest of them, and the bits above it that
    // every such key shares (a float's low bits that bf16 values leave zero, say) join
    // the prefix without a pass; none left ends the search
    uint64_t vo = 0ull, va = 0ull;  // OR of the keys, OR of their complements
#pragma unroll
    for (int q = 0; q < ZQ; ++q)
      if ((ck[q] & pmask) == prefix) {
        vo |= ck[q];
        va |= ~ck[q];
      }
    vo = wave_or_u64(vo);
    va = wave_or_u64(va);
    if (lane == 0) {
      S.u[w] = vo;
      S.u2[GW + w] = va;  // (S.u2[0..1] are read above, before the barrier)
    }
    __syncthreads();  // (also: S.ii and S.u2 are rewritten by the next pass)
    vo = 0ull;
    va = 0ull;
#pragma unroll
    for (int q = 0; q < GW; ++q) {
      vo |= S.u[q];
      va |= S.u2[GW + q];
    }
    const uint64_t vary = vo & va & ~pmask;
    hb = vary ? 63 - __clzll((long long)vary) : -1;
    const uint64_t above = hb >= 0 ? ~((2ull << hb) - 1ull) : ~0ull;
    prefix |= ~va & above & ~pmask;  // (~va: the bits every key under the prefix sets)
    pmask = above;
  }
  // the crossing key: the candidate whose compact key is the prefix
#pragma unroll
  for (int q = 0; q < ZQ; ++q)
    if (ck[q] == prefix) {
      const int pos = t + GT * q;
      S.res[slot][0] = G.z.zkey[z0 + pos];
      S.res[slot][1] = bc;
      S.res[slot][2] = bm;
      S.res[slot][3] = km[q];
      S.tag[slot] = np;
    }
  __syncthreads();
  if (S.tag[slot] != np) return GHit{~0ull, 0ull, 0ull, 0ull};
  return GHit{S.res[slot][0], S.res[slot][1], S.res[slot][2], S.res[slot][3]};
}

// Sum of the masses of the zone's keys <= bound, zone zkey/zmass[z0, z0 + n) (every
// thread; two barriers).
__device__ __forceinline__ uint64_t zone_mass_upto(GFinalShared& S, GBig& G, int z0, int n,
                                                  uint64_t bound) {
  const int t = threadIdx.x, lane = t & (WAVE - 1), w = wave_id();
  uint64_t s = 0ull;
  for (int i = t; i < n; i += GT) s += G.z.zkey[z0 + i] <= bound ? G.z.zmass[z0 + i] : 0ull;
  s = wave_sum_u64(s);
  if (lane == 0) S.u[w] = s;
  __syncthreads();
  uint64_t tot = 0ull;
#pragma unroll
  for (int q = 0; q < GW; ++q) tot += S.u[q];
  __syncthreads();
  return tot;
}

// Out-of-line forms of the rare paths (their code stays out of the common path's
// instruction stream; the LDS arrives as an address-space-typed pointer, and only the
// launch fields they read are passed: a reference to the argument block would copy it
// to private memory).
__device__ __noinline__ GHit pick_sorted_ool(lds_t<GFinalShared>* Sl, lds_t<GBig>* Gl, int np,
                                             int z0, int n, bool by_mass, double thr,
                                             uint64_t bound, int excl, uint64_t cnt0,
                                             uint64_t mass0) {
  GFinalShared& S = *(GFinalShared*)Sl;
  GBig& G = *(GBig*)Gl;
  return pick_sorted(S, G, np, z0, n, by_mass, thr, bound, excl, cnt0, mass0);
}
// The last key passing min-p, (double)l - (double)m >= lmp: the first fkey (descending l)
// that fails, less one.
__device__ __noinline__ uint32_t minp_last_fkey(float m, double lmp) {
  return x_first_fkey(fkey_desc(m), fkey_desc(-INFINITY), [&](float l) {
           return !((double)l - (double)m >= lmp);
         }) - 1u;
}
// Gumbel over every kept candidate of a row (key <= bound, not the draft): the chunks'
// candidate entries of bins up to the bound's bin bb, scored in fp64. Returns the token
// (-1: none kept but the draft).
__device__ __noinline__ int gumbel_kept(lds_t<GFinalShared>* Sl, const Cand* base,
                                        const float* noise, int W, int bb, uint64_t bound,
                                        int draft, const RowParams p, float m, uint64_t S1,
                                        bool cand_sorted) {
  GFinalShared& S = *(GFinalShared*)Sl;
  const int t = threadIdx.x, lane = t & (WAVE - 1), w = wave_id();
  if (w == 0) {
    // lane c: chunk c's entries up to its part of the bound's bin
    int lim = 0;
    if (lane < W) {
      const int lb = bb - S.dch[lane];
      if (lb >= 0 && S.nbch[lane] > 0) lim = S.pc[lane][lb < S.nbch[lane] ? lb : S.nbch[lane] - 1];
    }
    const int zof = (int)wave_incl_scan_u32((uint32_t)lim) - lim;
    if (lane < W) S.zoff[lane] = zof;
    if (lane == W - 1) S.zoff[W] = zof + lim;
  }
  __syncthreads();
  const int N = S.zoff[W];
  const bool no_lse = (p.flags & STRIM_FLAG_SCORE_NO_LSE) != 0;
  const double lse = log((double)S1 / RFIX);
  const uint64_t pkey = mix64(p.seed, p.position);
  double bsc = -INFINITY;
  uint64_t btk = ~0ull;
  int bid = -1;
  for (int i = t; i < N; i += GT) {
    // the chunk holding entry i: the last c with zoff[c] <= i
    int lo = 0, hi = W - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (S.zoff[mid] <= i) lo = mid;
      else hi = mid - 1;
    }
    const Cand x = base[(int64_t)lo * SLOT + (i - S.zoff[lo])];
    const uint64_t k = ckey(x.l, x.id);
    if (k > bound || x.id == draft) continue;
    const float u = noise ? noise[x.id] : philox_uniform(pkey, (uint64_t)x.id);
    const double bs = no_lse ? (double)x.l : ((double)x.l - (double)m) - lse;
    const double sc = bs + gumbel64(u);
    const uint64_t tk = cand_sorted ? k : (uint64_t)x.id;
    if (bid < 0 || sc > bsc || (sc == bsc && tk < btk)) {
      bsc = sc;
      btk = tk;
      bid = x.id;
    }
  }
  block_argmax_score<GT>(bsc, btk, bid, S.d, S.u, S.ii, &S.misc[4]);
  return S.misc[4];
}

// The LDS a collect pass writes (address-space-typed: see lds_t).
struct ZoneLds {
  lds_t<uint64_t>* key;
  lds_t<uint64_t>* mass;
  lds_t<uint32_t>* cnt;  // GT * EPT history counts of one window
  lds_t<int>* n;
};
// The collect pass of a row without penalties: streams the row's raw logits and
// allow-bits window by window, GT * EPT tokens a window, with the loads of D windows
// issued (from clamped indices, no branch between them) before any is consumed; selects
// the tokens with xa <= x < xb, reserves their places once per batch of D windows (one
// LDS atomic a wave, not one a window) and writes each lane's selected tokens,
// l = x / T (x for a greedy row). The window holding the row end goes through `tail`.
template <bool BF16, int D, typename Tail>
__device__ __forceinline__ void collect_nopen(const XArgs& a, int r, float xa, float xb,
                                              bool greedy, float T, float m, const ZoneLds& z,
                                              Tail&& tail) {
  constexpr int WINT = GT * EPT;
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const int t = threadIdx.x, lane = t & (WAVE - 1);
  const int64_t base = (int64_t)r * a.row_stride;
  const glb_t<const uint8_t>* lg = (const glb_t<const uint8_t>*)a.logits;
  const glb_t<const uint8_t>* mg =
      a.mask ? (const glb_t<const uint8_t>*)(a.mask + (int64_t)r * a.mask_stride) : nullptr;
  const int nwin = (a.V + WINT - 1) / WINT;
  // raw value e of a thread's window (its words w0..w3, and w4..w7 for fp32)
  auto raw = [&](const u32x4& v0, const u32x4& v1, int e) -> float {
    if constexpr (BF16) {
      const int q = e >> 1;
      const uint32_t wv = q == 0 ? v0.x : (q == 1 ? v0.y : (q == 2 ? v0.z : v0.w));
      return __uint_as_float((e & 1) ? (wv & 0xFFFF0000u) : (wv << 16));
    } else {
      const int q = e & 3;
      const u32x4 v = e < 4 ? v0 : v1;
      return __uint_as_float(q == 0 ? v.x : (q == 1 ? v.y : (q == 2 ? v.z : v.w)));
    }
  };
  for (int w0 = 0; w0 < nwin; w0 += D) {
    u32x4 x0[D], x1[D];
    uint32_t mb[D];
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int i0 = (w0 + d) * WINT + t * EPT;
      const int ii = i0 + EPT <= a.V ? i0 : 0;
      if constexpr (BF16) {
        x0[d] = *(const glb_t<const u32x4>*)(lg + 2 * (base + ii));
        x1[d] = x0[d];
      } else {
        x0[d] = *(const glb_t<const u32x4>*)(lg + 4 * (base + ii));
        x1[d] = *(const glb_t<const u32x4>*)(lg + 4 * (base + ii + 4));
      }
      mb[d] = mg ? (uint32_t)mg[ii >> 3] : 0xFFu;
    }
    // the selection bits of every whole window of the batch
    uint32_t sel[D];
    uint32_t cnt = 0u;
#pragma unroll
    for (int d = 0; d < D; ++d) {
      sel[d] = 0u;
      const int i0 = (w0 + d) * WINT + t * EPT;
      if (w0 + d < nwin && (w0 + d + 1) * WINT <= a.V) {
#pragma unroll
        for (int e = 0; e < EPT; ++e) {
          const float x = raw(x0[d], x1[d], e);
          sel[d] |= (((mb[d] >> e) & 1u) && x >= xa && x < xb) ? 1u << e : 0u;
        }
        cnt += (uint32_t)__popc(sel[d]);
      }
      (void)i0;
    }
    // one reservation a wave for the batch; each lane stages its tokens there as
    // (raw value bits, id) (a few instructions a token, in window order), then the
    // wave's lanes share the staged tokens evenly for the keys and masses (a division
    // and an exponential each), in place (the wave's LDS operations complete in order)
    const uint32_t inc = wave_incl_scan_u32(cnt);
    const int tot = __builtin_amdgcn_readlane((int)inc, WAVE - 1);
    if (tot > 0) {
      int b0 = 0;
      if (lane == 0) b0 = atomicAdd((int*)z.n, tot);
      b0 = __builtin_amdgcn_readfirstlane(b0);
      int pos = b0 + (int)(inc - cnt);
#pragma unroll
      for (int d = 0; d < D; ++d) {
        const int i0 = (w0 + d) * WINT + t * EPT;
        uint32_t sl = sel[d];
        while (sl) {
          const int e = __builtin_ctz(sl);
          sl &= sl - 1u;
          if (pos < ZCAP)
            z.key[pos] = ((uint64_t)__float_as_uint(raw(x0[d], x1[d], e)) << 32) | (uint32_t)(i0 + e);
          ++pos;
        }
      }
      __builtin_amdgcn_wave_barrier();
      const int end = min(b0 + tot, ZCAP);
      for (int i = b0 + lane; i < end; i += WAVE) {
        const uint64_t v = z.key[i];
        const float xe = __uint_as_float((uint32_t)(v >> 32));
        const float le = greedy ? xe : xe / T;
        z.key[i] = ckey(le, (int)(uint32_t)v);
        z.mass[i] = rmass(le, m);
      }
      __builtin_amdgcn_wave_barrier();
    }
    // a window holding the row end: element by element
#pragma unroll
    for (int d = 0; d < D; ++d)
      if (w0 + d < nwin && (w0 + d + 1) * WINT > a.V) tail(w0 + d);
  }
}

// The least float x with fl(x / T) >= A (T > 0; x / T rounded as the streaming passes
// divide): x -> fl(x / T) is monotone. Stepped in ulps from A T (a few ulps from the
// answer), or found by bisection over the floats in order where that does not settle.
__device__ __forceinline__ float least_x_for(float T, float A) {
  auto ord = [](float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  };
  auto unord = [](uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
  };
  const float x0 = A * T;
  if (x0 > -INFINITY && x0 < INFINITY) {
    uint32_t k = ord(x0);
    if (unord(k) / T >= A) {
      for (int it = 0; it < 16; ++it) {  // down while the float below still passes
        if (!(unord(k - 1u) / T >= A)) return unord(k);
        --k;
      }
    } else {
      for (int it = 0; it < 16; ++it) {  // up to the first float that passes
        ++k;
        if (unord(k) / T >= A) return unord(k);
      }
    }
  }
  uint32_t lo = ord(-INFINITY), hi = ord(INFINITY);  // pred(hi) holds (A is finite)
  while (lo < hi) {
    const uint32_t mid = lo + (hi - lo) / 2u;
    if (unord(mid) / T >= A) hi = mid;
    else lo = mid + 1u;
  }
  return unord(lo);
}

// Collect pass: every token of the row whose lattice bin A(l) is `at`, by one streaming
// pass of the workgroup over the row's logits (the chain recomputed per window), into
// key / mass. Returns their number, -1 past ZCAP. Out of line: the common path of
// k_gfinal keeps none of the pass's registers.
__device__ __noinline__ int collect_zone(const XArgs a_in, int r, int b, int j,
                                         const RowParams p_in, float at, float m,
                                         const ZoneLds z_in) {
  const XArgs a = uniform_copy(a_in);
  const RowParams p = uniform_copy(p_in);
  const ZoneLds z = uniform_copy(z_in);
  r = __builtin_amdgcn_readfirstlane(r);
  b = __builtin_amdgcn_readfirstlane(b);
  j = __builtin_amdgcn_readfirstlane(j);
  // (readfirstlane takes an int: floats go through their bits)
  at = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(at)));
  m = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(m)));
  const int lane = threadIdx.x & (WAVE - 1);
  if (threadIdx.x == 0) *z.n = 0;
  __syncthreads();
  // A(l) = at, l = x / T (x for a greedy row): at / LBS <= l < (at + 1) / LBS, both bounds
  // exact floats; for a row without penalties the same test on x is xa <= x < xb
  const float la = at * (1.0f / (float)LBS), lb = (at + 1.0f) * (1.0f / (float)LBS);
  const float xa = p.greedy ? la : least_x_for(p.T, la);
  const float xb = p.greedy ? lb : least_x_for(p.T, lb);
  // appends the thread's selected tokens (bits of sel), l = lof(e): a lane loops over its
  // own set bits only (a window selects few tokens, so most lanes none)
  auto append = [&](int i0, uint32_t sel, auto&& lof) {
    const int c = __popc(sel);
    int tot;
    const int ex = wave_excl_count(c, &tot);
    if (tot > 0) {
      int base = 0;
      if (lane == 0) base = atomicAdd((int*)z.n, tot);
      base = __builtin_amdgcn_readfirstlane(base);
      int pos = base + ex;
      while (sel) {
        const int e = __builtin_ctz(sel);
        sel &= sel - 1u;
        const float le = lof(e);
        if (pos < ZCAP) {
          z.key[pos] = ckey(le, i0 + e);
          z.mass[pos] = rmass(le, m);
        }
        ++pos;
      }
    }
  };
  if (!p.pen && a.vec_ok) {
    // the window holding the row end, token by token
    auto tail = [&](int wi) {
      const int i0 = wi * GT * EPT + (int)threadIdx.x * EPT;
      const int64_t base = (int64_t)r * a.row_stride;
      uint32_t bits = (a.mask && i0 < a.V) ? (uint32_t)((const uint8_t*)(a.mask + (int64_t)r * a.mask_stride))[i0 >> 3] : 0xFFu;
      bits &= i0 < a.V ? (i0 + EPT <= a.V ? 0xFFu : (1u << (a.V - i0)) - 1u) : 0u;
      float x[EPT];
#pragma unroll
      for (int e = 0; e < EPT; ++e) {
        const int id = i0 + e < a.V ? i0 + e : 0;
        x[e] = a.dtype == STRIM_DTYPE_BF16 ? bf16_to_f32(((const uint16_t*)a.logits)[base + id])
                                           : ((const float*)a.logits)[base + id];
      }
      uint32_t sel = 0u;
#pragma unroll
      for (int e = 0; e < EPT; ++e) sel |= (((bits >> e) & 1u) && x[e] >= xa && x[e] < xb) ? 1u << e : 0u;
      append(i0, sel, [&](int e) {
        const float xe = pick8(x, e);
        return p.greedy ? xe : xe / p.T;
      });
    };
    if (a.dtype == STRIM_DTYPE_BF16) collect_nopen<true, 16>(a, r, xa, xb, p.greedy, p.T, m, z, tail);
    else collect_nopen<false, 8>(a, r, xa, xb, p.greedy, p.T, m, z, tail);
  } else {
    x_pass<GT, false>(a, r, b, j, p, (uint32_t*)z.cnt,
                      [&](int i0, const float (&l)[EPT], const float (&)[EPT]) {
      uint32_t sel = 0u;
#pragma unroll
      for (int e = 0; e < EPT; ++e)
        sel |= (l[e] > -INFINITY && floorf(l[e] * (float)LBS) == at) ? 1u << e : 0u;
      append(i0, sel, [&](int e) { return pick8(l, e); });
    });
  }
  __syncthreads();
  const int n = *z.n;
  return n <= ZCAP ? n : -1;
}

// The leading arguments repeat fields of `a` (a.s.cstat, a.s.lat, a.s.slot, a.s.wmax,
// a.W): built with kernel-argument preloading, they arrive in SGPRs, so the chunk
// statistics' load is issued before any wait for the argument block.
__global__ __launch_bounds__(GT) void k_gfinal(const ChunkStat* pre_cstat,
                                                const unsigned long long* pre_lat,
                                                const Cand* pre_slot, int pre_wmax, int pre_W,
                                                Args a) {
  __shared__ GFinalShared S;
  __shared__ GBig G;
  __shared__ GPf P;
  // the chunk statistics first, their address from the preloaded arguments alone (a row
  // of at most 64 chunks: every wave loads all of them, lane c chunk c; wider rows:
  // thread t chunk t)
  const int ci = pre_W <= WAVE ? (int)(threadIdx.x & (WAVE - 1)) : (int)threadIdx.x;
  const ChunkStat cs = pre_cstat[(int64_t)blockIdx.x * pre_wmax + (ci < pre_W ? ci : 0)];
  // the launch fields of the first loads, read together (see k_stream)
  asm volatile("" ::"s"(a.s.rs), "s"(a.V), "s"(a.noise), "s"(a.noise_stride),
               "s"(a.noise_mode), "s"(a.verify), "s"(a.k), "s"(a.drafts));
  const int r = blockIdx.x;
  int b, j;
  row_bj(a, r, b, j);
  const int t = threadIdx.x, lane = t & (WAVE - 1), w = wave_id();
  const int V = a.V, W = pre_W;
  // ---- every load that does not depend on the row's parameters ------------------
  // the chunk statistics (above), the noise, the draft and the chunks' lattice words (no
  // branch between the loads: a missing optional input reads the row's own state and is
  // ignored; words past a chunk's written bins are dropped later)
  RowState* rsp = &a.s.rs[r];
  const bool gum = a.noise && a.noise_mode != STRIM_NOISE_ICDF;
  const float* nz = a.noise ? a.noise + (int64_t)r * a.noise_stride : (const float*)rsp;
  const float n0 = nz[gum ? V : 0], n1 = nz[gum ? V : 1];
  const bool vdr = a.verify && j < a.k;
  const int32_t* dp = vdr ? a.drafts + (int64_t)b * a.k + j : (const int32_t*)rsp;
  const int d_raw = *dp;
  const float ld_raw = rsp->l_draft;
  // the chunks' lattice words (E[c NBW + lb]) and each chunk's first PF candidates
  // (pfb[c PF + place]; places past what a chunk wrote are stale and never used),
  // straight into LDS by waves 1-7: wave w issues blocks w - 1, w - 1 + DW, ... of 1 KB
  // (16 bytes per lane; a fixed count per wave: blocks past the row's repeat its last
  // block, the same bytes to the same place). Wave 0 issues none, so its waits cover its
  // own loads alone while the others' land.
  const unsigned long long* lwp = pre_lat + (int64_t)r * pre_wmax * NBW;
  const Cand* slots = pre_slot + (int64_t)r * pre_wmax * SLOT;
  if (w > 0) {
    const int wl = W <= LWMAX ? W : 1;
    const int nwb = (wl * NBW * 8 + 1023) / 1024, npb = (wl * PF * 8 + 1023) / 1024;
#pragma unroll
    for (int q = 0; q < KW; ++q) {
      const int blk = min(w - 1 + DW * q, nwb - 1);
      const int e = blk * 128 + 2 * lane;  // its words e, e + 1
      const int ec = e < wl * NBW ? e : 0;
      __builtin_amdgcn_global_load_lds((const void*)(lwp + ec),
                                       (lds_t<void>*)((char*)G.E + blk * 1024), 16, 0, 0);
    }
#pragma unroll
    for (int q = 0; q < KP; ++q) {
      const int blk = min(w - 1 + DW * q, npb - 1);
      const int e = blk * 128 + 2 * lane;  // its candidates e, e + 1 (PF even)
      const int c = e / PF, pl = e - c * PF;
      const Cand* src = c < wl ? slots + (int64_t)c * SLOT + pl : slots;
      __builtin_amdgcn_global_load_lds((const void*)src,
                                       (lds_t<void>*)((char*)P.pfb + blk * 1024), 16, 0, 0);
    }
  }
  const RowParams p = load_params(a, b, j);
  // the row's own uniforms (rows without given noise), computed while the loads above
  // are in flight: they depend on the parameters alone
  float pu_draw = 0.0f, pu_acc = 0.0f;
  if (!a.noise) {
    const uint64_t pkey = mix64(p.seed, p.position);
    pu_draw = philox_uniform(pkey, 0);
    pu_acc = philox_uniform(pkey, a.noise_mode == STRIM_NOISE_GUMBEL ? (uint64_t)V : 1u);
  }
  if (!gfinal_row(a.p[b], V, a.noise_mode, a.dlog != nullptr && vdr)) {
    __builtin_amdgcn_s_waitcnt(0);  // (no LDS write may land after the workgroup ends)
    return;
  }
  const int draft = vdr ? d_raw : -1;
  const float l_draft = vdr ? ld_raw : -INFINITY;

  // ---- the chunk statistics ---------------------------------------------------------
  // A row of at most 64 chunks is reduced by every wave alone, with no LDS: an LDS access
  // after the loads into LDS above waits for all of them (the compiler cannot tell the
  // areas apart), so the first one is left to the lattice code, which needs them.
  // Wider rows merge the waves' results through LDS.
  const bool own = t < W;     // thread t holds chunk t (wave 0's lanes, W <= 64)
  const bool hold = ci < W;   // this lane holds chunk ci
  int ff = hold ? (cs.flags | (cs.n > 0 ? 4 : 0)) : 0;
  if (hold && cs.n > 0 && cs.ncand2 == LNONE) ff |= 8;  // a chunk without lattice words
  float m = hold ? cs.m : -INFINITY;
  int arg = hold ? cs.arg : -1;
  wave_argmax(m, arg);
  int flags = wave_or_i(ff);
  if (W > WAVE) {
    if (lane == 0) {
      S.v[w] = m;
      S.i[w] = arg;
      S.f[w] = flags;
    }
    __syncthreads();
    // lane q holds wave q's results
    m = lane < GW ? S.v[lane] : -INFINITY;
    arg = lane < GW ? S.i[lane] : -1;
    flags = lane < GW ? S.f[lane] : 0;
    wave_argmax(m, arg);
    flags = wave_or_i(flags);
  }
  auto finish = [&](int status, int token, int accept, double sig, uint64_t last_key) {
    if (t != 0) return;
    rsp->status = status;
    rsp->token = token;
    rsp->accept = accept;
    rsp->sum_kept = sig;
    rsp->m = m;
    rsp->last_key = last_key;
    rsp->phase = PH_DONE;
    if (!a.verify) {
      a.out_ids[r] = status == STRIM_OK ? token : -1;
      if (a.out_status) a.out_status[r] = status;
    }
  };
  int status = STRIM_OK;
  if (vdr && (draft < 0 || draft >= V)) status = STRIM_EINVAL;
  if (status == STRIM_OK && (flags & 1)) status = STRIM_ENONFINITE;
  if (status == STRIM_OK && !(flags & 4)) status = STRIM_EEMPTY;
  if (status != STRIM_OK) {
    __builtin_amdgcn_s_waitcnt(0);  // (no LDS write may land after the workgroup ends)
    finish(status, -1, 0, 0.0, 0ull);
    return;
  }
  float u_draw = 0.0f, u_acc = 0.0f;
  if (a.noise) {
    if (a.noise_mode == STRIM_NOISE_ICDF) u_draw = n0;
    u_acc = n1;
  } else {
    u_draw = pu_draw;
    u_acc = pu_acc;
  }
  // the streaming passes' view of the launch (collect passes and the exact resolution)
  XArgs xa;
  xa.logits = a.logits;
  xa.row_stride = a.row_stride;
  xa.dtype = a.dtype;
  xa.vec_ok = a.vec_ok;
  xa.V = a.V;
  xa.H = a.H;
  xa.verify = a.verify;
  xa.k = a.k;
  xa.noise_mode = a.noise_mode;
  xa.mask = a.mask;
  xa.mask_stride = a.mask_stride;
  xa.hist = a.hist;
  xa.hist_len = a.hist_len;
  xa.drafts = a.drafts;
  xa.noise = a.noise;
  xa.noise_stride = a.noise_stride;
  xa.has_q = 0;

  // ---- the row's lattice ---------------------------------------------------------
  const float arow = floorf(m * (float)LBS);
  const bool lat = W <= LWMAX && !(flags & 8) && fabsf(arow) < 0x1p+23f;
  auto decide = [&]() -> bool {
    // per chunk (the thread of chunk t): its distance below the row's top bin, its mass
    // sum relative to the row maximum, how far down its bins are whole; the chunks'
    // lattice words staged in LDS with their count prefixes (for the gathers)
    // (the chunks' threads are all in wave 0, W <= LWMAX: the row's limits are wave
    // reductions there, one store each; an LDS atomic from every lane to one word is
    // serialised lane by lane, about 2.5 us for 38 chunks)
    if (t < NBW) {
      S.rc[t] = 0u;
      S.rm[t] = 0ull;
    }
    if (t < 2) S.tag[t] = -1;
    if (w == 0) {
      int lwin = NBW, lfull = NBW, tail = 0;
      if (own) {
        S.nbch[t] = cs.n > 0 ? (int)cs.ncand2 : 0;
        S.ncnt[t] = cs.n;
        if (cs.n > 0) {
          const int d = (int)(arow - floorf(cs.m * (float)LBS));
          const int nb = (int)cs.ncand2, nf = (int)cs.ncand;
          S.dch[t] = d;
          S.sch[t] = cs.S * exp((double)cs.m - (double)m);
          if (nb == 0) {  // (no window words: nothing of the chunk is known)
            lwin = d;
            tail = 1;
          }
          if (nf < nb && d + nf < NBW) lfull = d + nf;
          if (d + nb > NBW) tail = 1;  // its window reaches past the row's
        } else {
          S.dch[t] = NOBIN;
          S.sch[t] = 0.0;
        }
      }
      lwin = wave_min_i(lwin);
      lfull = wave_min_i(lfull);
      tail = wave_or_i(tail);
      if (lane == 0) {
        S.misc[1] = lwin;
        S.misc[0] = lfull;
        S.misc[3] = tail;
      }
    }
    // the LDS loads have landed (every wave waits for its own, then the barrier)
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    // every row bin: the counts and masses of its chunks' bins. Wave w takes chunks w,
    // w + 8, ... (at most LWMAX / 8), lane l row bins 3 l .. 3 l + 2 of each (a chunk's
    // bins read with the one before them: four words for three bins, all requested
    // before any is used); a lattice bin's masses share their unit, so they add as
    // integers, and each row bin gets one LDS atomic per wave. Each chunk's inclusive
    // count prefixes are kept for the gathers.
    {
      static_assert(LPL == 3 && LWMAX % GW == 0, "three row bins a lane, whole chunk rounds");
      const int dreg = lane < W ? S.dch[lane] : NOBIN;
      const int nbreg = lane < W ? S.nbch[lane] : 0;
      uint32_t cq[LPL] = {0u, 0u, 0u};
      uint64_t mq[LPL] = {0ull, 0ull, 0ull};
#pragma unroll
      for (int k = 0; k < LWMAX / GW; ++k) {
        const int c = w + GW * k;
        if (c >= W) break;
        const int d = __builtin_amdgcn_readlane(dreg, c);
        const int nb = __builtin_amdgcn_readlane(nbreg, c);
        const int lb0 = LPL * lane - d;  // the chunk's bin of row bin 3 l
        uint64_t wv[LPL + 1];  // words of chunk bins lb0 - 1 .. lb0 + 2
        bool in[LPL + 1];
#pragma unroll
        for (int q = 0; q <= LPL; ++q) {
          const int lb = lb0 + q - 1;
          in[q] = lb >= 0 && lb < nb;
          wv[q] = G.E[in[q] ? c * NBW + lb : 0];
        }
#pragma unroll
        for (int q = 0; q < LPL; ++q)
          if (in[q + 1]) {
            const uint32_t incl = (uint32_t)(wv[q + 1] >> LCSH);
            const uint32_t prev = in[q] ? (uint32_t)(wv[q] >> LCSH) : 0u;
            S.pc[c][lb0 + q] = (uint16_t)incl;
            cq[q] += incl - prev;
            mq[q] += wv[q + 1] & LMMASK;
          }
      }
#pragma unroll
      for (int q = 0; q < LPL; ++q)
        if (cq[q]) {
          atomicAdd(&S.rc[LPL * lane + q], cq[q]);
          atomicAdd(&S.rm[LPL * lane + q], (unsigned long long)mq[q]);
        }
    }
    if (w == 0) {
      // tokens below a chunk's window (one store, not one a lane)
      const bool below = own && cs.n > 0 && cs.ncand2 > 0u && cs.ncand2 != LNONE &&
                         cs.n > (int)(uint32_t)(G.E[t * NBW + cs.ncand2 - 1] >> LCSH);
      if (__ballot(below) != 0ull && lane == 0) S.misc[3] = 1;
    }
    __syncthreads();
    // The leader wave (wave 0) keeps the row's cumulative histogram in its registers,
    // scaled from each bin's lattice unit to RFIX per unit of exp(l - m): scale(b) =
    // 8 exp(arow / LBS - m) 2^(-b log2(e) / LBS). Every wave takes the totals and limits.
    RowCum rcum;
    if (w == 0) {
      const float base = 8.0f * expf(arow * (1.0f / (float)LBS) - m);
      uint32_t lc = 0u;
      uint64_t lm = 0ull;
#pragma unroll
      for (int q = 0; q < LPL; ++q) {
        const int bq = LPL * lane + q;
        rcum.cq(q) = S.rc[bq];
        const float sc = base * __builtin_amdgcn_exp2f(-(float)bq * (1.44269504f / (float)LBS));
        rcum.mq(q) = (uint64_t)__double2ull_rn((double)S.rm[bq] * (double)sc);
        lc += rcum.cq(q);
        lm += rcum.mq(q);
      }
      uint32_t bc = wave_incl_scan_u32(lc) - lc;
      uint64_t bm = wave_incl_scan_u64(lm) - lm;
#pragma unroll
      for (int q = 0; q < LPL; ++q) {
        bc += rcum.cq(q);
        bm += rcum.mq(q);
        rcum.cq(q) = bc;
        rcum.mq(q) = bm;
      }
    }
    // (LDS values the same in every lane, kept in scalar registers: see uniform_copy)
    const int rowwin = uniform_copy(S.misc[1] < NBW ? S.misc[1] : NBW);
    const int rowfull = uniform_copy(S.misc[0] < rowwin ? S.misc[0] : rowwin);
    const bool anytail = uniform_copy(S.misc[3]) != 0;
    const int n_all = wave_sum(lane < W ? S.ncnt[lane] : 0);
    const double S_all = wave_sum(lane < W ? S.sch[lane] : 0.0);
    const uint64_t S0 = (uint64_t)__double2ull_rn(S_all * RFIX);

    const bool topk = p.top_k > 0 && p.top_k < V;
    const bool topp = p.top_p < 1.0f;
    const bool minp = p.min_p > 0.0f;
    const bool icdf = a.noise_mode == STRIM_NOISE_ICDF;
    // rank-indexed noise needs every kept token's rank
    if ((p.flags & STRIM_FLAG_NOISE_BY_RANK) && topp && !icdf) return false;

    // ---- the leader alone ------------------------------------------------------------
    // A row whose zones are small (the common case) is decided by wave 0 alone, with no
    // workgroup barrier: it lays out each zone from the prefetched candidates (each
    // place's source recorded by its chunk's lane, then the keys and masses built by all
    // lanes) and picks within the wave: up to 64 keys by ranks (one key a lane, the zone
    // read as LDS broadcasts), up to SOLO by a radix select in the wave. A zone that needs
    // a chunk's slot region or a collect pass, or holds more than SOLO keys, and Gumbel
    // draws, go to the cooperative loop below (every wave; it starts over). Both follow
    // the same decision rules.
    constexpr int SQ = 3, SOLO = SQ * WAVE;  // zone keys a lane holds, a zone's keys
    // (a zone of at most 64 keys starts below 2 SOLO; its rank loop reads up to 7 places
    // past its end)
    static_assert(2 * SOLO + WAVE + 8 <= ZCAP && WAVE + 8 <= GT, "rank loop reads in bounds");
    bool pfok = true;  // the prefetched candidates are in LDS
    auto solo = [&]() -> int {  // 0 decided, 1 cooperative, 2 exact resolution
      if (!icdf) return 1;
      int zb0 = -1, zb1 = -1, zn0 = 0, zn1 = 0;
      // lane c's chunk: its top bin's distance below the row's and its window bins
      // written, from its own statistics (the values decide() stores, without the reads)
      const int dme = own && cs.n > 0 ? (int)(arow - floorf(cs.m * (float)LBS)) : NOBIN;
      const int nbme = own && cs.n > 0 ? (int)cs.ncand2 : 0;
      // bins {bz, also} into the zone (bz at 0, also after it): 0 loaded, else a verdict
      auto load = [&](int bz, int also) -> int {
        if (bz >= rowwin) return 2;
        if (bz >= rowfull) return 1;
        const uint64_t cr = rcum.cnt(bz) - rcum.cnt(bz - 1);
        if (cr > (uint64_t)SOLO) return 1;
        const bool two = also >= 0 && also != bz && also < rowfull &&
                         cr + rcum.cnt(also) - rcum.cnt(also - 1) <= (uint64_t)SOLO;
        const int bins[2] = {bz, two ? also : -1};
        int off[2], cnt[2], zoo[2], n[2];
        bool ok = pfok;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          off[hh] = 0;
          cnt[hh] = 0;
          if (lane < W && bins[hh] >= 0) {
            const int lb = bins[hh] - dme;
            if (lb >= 0 && lb < nbme) {
              off[hh] = lb > 0 ? (int)S.pc[lane][lb - 1] : 0;
              cnt[hh] = (int)S.pc[lane][lb] - off[hh];
            }
          }
          zoo[hh] = (int)wave_incl_scan_u32((uint32_t)cnt[hh]) - cnt[hh];
          n[hh] = __builtin_amdgcn_readlane(zoo[hh] + cnt[hh], WAVE - 1);
          ok = ok && off[hh] + cnt[hh] <= PF;
        }
        if (__ballot(!ok) != 0ull || n[0] + n[1] > SOLO) return 1;
        zoo[1] += n[0];
        // each zone place's source in the prefetched candidates, c PF + its place in
        // chunk c's part: lane c writes its part's (a few stores each), then every lane
        // builds the keys and masses of places lane, lane + 64, ... (S.prk is idle here)
        lds_t<uint32_t>* src = (lds_t<uint32_t>*)S.prk;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
          for (int i = 0; i < cnt[hh]; ++i) src[zoo[hh] + i] = (uint32_t)(lane * PF + off[hh] + i);
        __builtin_amdgcn_wave_barrier();
        // (at most SOLO places: every lane's SQ sources read first, then their candidates)
        const int ntot = n[0] + n[1];
        uint32_t si[SQ];
#pragma unroll
        for (int q = 0; q < SQ; ++q) {
          const int i = lane + WAVE * q;
          si[q] = src[i < ntot ? i : 0];
        }
        Cand xc[SQ];
#pragma unroll
        for (int q = 0; q < SQ; ++q) xc[q] = P.pfb[lane + WAVE * q < ntot ? si[q] : 0u];
#pragma unroll
        for (int q = 0; q < SQ; ++q) {
          const int i = lane + WAVE * q;
          if (i < ntot) {
            G.z.zkey[i] = ckey(xc[q].l, xc[q].id);
            G.z.zmass[i] = rmass(xc[q].l, m);
          }
        }
        // (one wave's LDS operations complete in order: its later reads see these)
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        __builtin_amdgcn_wave_barrier();
        zb0 = bz;
        zn0 = n[0];
        zb1 = bins[1];
        zn1 = n[1];
        return 0;
      };
      // the zone of bin bz: its place and size (z0 < 0: not loaded)
      auto where = [&](int bz, int& z0, int& n) {
        z0 = -1;
        n = 0;
        if (bz == zb0) { z0 = 0; n = zn0; }
        else if (bz == zb1) { z0 = zn0; n = zn1; }
      };
      // pick_rank within the wave: lane l holds key z0 + l
      // wider zones (65..SOLO keys, SQ a lane): pick_sorted's radix select within the wave.
      // The wave's LDS operations complete in order, so its digit histogram (S.prk /
      // S.pmb, idle while the leader decides alone) needs no barrier.
      auto wradix = [&](int z0, int n, bool by_mass, double thr, uint64_t bnd, int excl,
                        uint64_t c0, uint64_t m0) -> GHit {
        auto compact = [](uint64_t k) { return ((k >> 32) << 20) | (k & 0xFFFFFull); };
        uint64_t ck[SQ], km[SQ];
        bool in[SQ];
        uint64_t diff = 0ull;
        const uint64_t ref = compact(G.z.zkey[z0]);
#pragma unroll
        for (int q = 0; q < SQ; ++q) {
          const int i = lane + WAVE * q;
          const bool pr = i < n;
          const uint64_t k = pr ? G.z.zkey[z0 + i] : 0ull;
          ck[q] = pr ? compact(k) : ~0ull;
          km[q] = pr ? G.z.zmass[z0 + i] : 0ull;
          in[q] = pr && k <= bnd && (int)(uint32_t)k != excl;
          if (pr) diff |= ck[q] ^ ref;
        }
        diff = wave_or_u64(diff);
        int hb = diff ? 63 - __clzll((long long)diff) : -1;
        uint64_t pmask = hb < 0 ? ~0ull : ~((2ull << hb) - 1ull);
        uint64_t prefix = ref & pmask;
        uint64_t bc = c0, bm = m0;
        while (hb >= 0) {
          const int shift = hb >= 7 ? hb - 7 : 0;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            S.prk[4 * lane + i] = 0u;
            S.pmb[4 * lane + i] = 0ull;
          }
          __builtin_amdgcn_wave_barrier();
#pragma unroll
          for (int q = 0; q < SQ; ++q)
            if ((ck[q] & pmask) == prefix) {
              const int d = (int)((ck[q] >> shift) & 255ull);
              atomicAdd(&S.prk[d], 1u);
              if (in[q]) atomicAdd(&S.pmb[d], (unsigned long long)km[q]);
            }
          __builtin_amdgcn_wave_barrier();
          uint32_t c[4];
          uint64_t mm[4];
          uint32_t lc = 0u;
          uint64_t lm = 0ull;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            c[i] = S.prk[4 * lane + i];
            mm[i] = S.pmb[4 * lane + i];
            lc += c[i];
            lm += mm[i];
          }
          uint64_t Bc = bc + (uint64_t)(wave_incl_scan_u32(lc) - lc);
          uint64_t Bm = bm + (wave_incl_scan_u64(lm) - lm);
          int hit = -1;
          uint64_t hc = 0ull, hm = 0ull;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint64_t before = by_mass ? Bm : Bc;
            const uint64_t own = by_mass ? mm[i] : (uint64_t)c[i];
            if (hit < 0 && own > 0ull && (double)before <= thr && (double)(before + own) > thr) {
              hit = 4 * lane + i;
              hc = Bc;
              hm = Bm;
            }
            Bc += c[i];
            Bm += mm[i];
          }
          const uint64_t bal = __ballot(hit >= 0);
          if (bal == 0ull) return GHit{~0ull, 0ull, 0ull, 0ull};
          const int hl = (int)__ffsll((long long)bal) - 1;
          const int d = __builtin_amdgcn_readlane(hit, hl);
          bc = rl_u64(hc, hl);
          bm = rl_u64(hm, hl);
          prefix |= (uint64_t)d << shift;
          pmask |= 255ull << shift;
          // the bits still differing among the keys under the prefix (as pick_sorted)
          uint64_t vo = 0ull, va = 0ull;
#pragma unroll
          for (int q = 0; q < SQ; ++q)
            if ((ck[q] & pmask) == prefix) {
              vo |= ck[q];
              va |= ~ck[q];
            }
          vo = wave_or_u64(vo);
          va = wave_or_u64(va);
          const uint64_t vary = vo & va & ~pmask;
          hb = vary ? 63 - __clzll((long long)vary) : -1;
          const uint64_t above = hb >= 0 ? ~((2ull << hb) - 1ull) : ~0ull;
          prefix |= ~va & above & ~pmask;
          pmask = above;
          __builtin_amdgcn_wave_barrier();  // (this pass's reads before the next clear)
        }
        // the crossing key: its holder's key and mass
        int hq = -1;
#pragma unroll
        for (int q = 0; q < SQ; ++q)
          if (ck[q] == prefix) hq = q;
        const uint64_t bal = __ballot(hq >= 0);
        if (bal == 0ull) return GHit{~0ull, 0ull, 0ull, 0ull};
        const int hl = (int)__ffsll((long long)bal) - 1;
        const int q = __builtin_amdgcn_readlane(hq, hl);
        const uint64_t key = G.z.zkey[z0 + hl + WAVE * q], kmass = G.z.zmass[z0 + hl + WAVE * q];
        return GHit{key, bc, bm, kmass};
      };
      auto wpick = [&](int z0, int n, bool by_mass, double thr, uint64_t bnd, int excl,
                       uint64_t c0, uint64_t m0) -> GHit {
        z0 = uniform_copy(z0);
        n = uniform_copy(n);
        if (n > WAVE) return wradix(z0, n, by_mass, thr, bnd, excl, c0, m0);
        const bool mine = lane < n;
        const uint64_t k = mine ? G.z.zkey[z0 + lane] : ~0ull;
        const uint64_t km = mine ? G.z.zmass[z0 + lane] : 0ull;
        const bool in = mine && k <= bnd && (int)(uint32_t)k != excl;
        const uint64_t kin = in ? km : 0ull;  // its mass where it is kept
        // every lane compares its key with each zone key, read from LDS as a broadcast
        // eight at a time (S.pmb, idle while the leader decides alone, holds the kept
        // masses; the wave's LDS operations complete in order)
        if (mine) S.pmb[lane] = kin;
        __builtin_amdgcn_wave_barrier();
        uint32_t rk = 0u;
        uint64_t mb = 0ull;
        // (places past n read stale entries inside the zone buffer and S.pmb, dropped by
        // the scalar test below: the reads take constant offsets from one base)
        const lds_t<uint64_t>* zk = (const lds_t<uint64_t>*)G.z.zkey + z0;
        const lds_t<unsigned long long>* zm = (const lds_t<unsigned long long>*)S.pmb;
        for (int j0 = 0; j0 < n; j0 += 8) {
          uint64_t kj[8], mj[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            kj[u] = zk[j0 + u];
            mj[u] = zm[j0 + u];
          }
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const bool lt = j0 + u < n && kj[u] < k;
            rk += lt ? 1u : 0u;
            mb += lt ? mj[u] : 0ull;
          }
        }
        __builtin_amdgcn_wave_barrier();  // (the reads before a later pick's stores)
        const uint64_t before = by_mass ? m0 + mb : c0 + rk;
        const uint64_t own = by_mass ? kin : 1ull;
        const bool hit = mine && own > 0ull && (double)before <= thr && (double)(before + own) > thr;
        const uint64_t bal = __ballot(hit);
        if (bal == 0ull) return GHit{~0ull, 0ull, 0ull, 0ull};
        const int hl = (int)__ffsll((long long)bal) - 1;
        return GHit{rl_u64(k, hl), c0 + (uint32_t)__builtin_amdgcn_readlane((int)rk, hl),
                    m0 + rl_u64(mb, hl), rl_u64(km, hl)};
      };
      // the zone's masses of keys <= bnd (n <= SOLO)
      auto wsum = [&](int z0, int n, uint64_t bnd) -> uint64_t {
        uint64_t sm = 0ull;
        for (int i = lane; i < n; i += WAVE) sm += G.z.zkey[z0 + i] <= bnd ? G.z.zmass[z0 + i] : 0ull;
        return wave_sum_u64(sm);
      };
      uint64_t bound = ~0ull, Sk = S0;
      int bbin = NOBIN;
      int z0, n, v;
      // top-k: the k-th key in order (every key counts)
      if (topk && n_all >= p.top_k) {
        const double thr = (double)(p.top_k - 1);
        const int bz = rcum.find(false, thr, rowwin, 0ull, NOBIN);
        if (bz >= rowwin) return 2;
        if ((v = load(bz, -1)) != 0) return v;
        const GHit g = wpick(0, zn0, false, thr, ~0ull, -1, rcum.cnt(bz - 1), rcum.mass(bz - 1));
        if (g.key == ~0ull) return 2;
        if (p.flags & STRIM_FLAG_TOPK_KEEP_TIES) {
          bound = g.key | 0xFFFFFFFFull;
          Sk = rcum.mass(bz - 1) + wsum(0, zn0, bound);
        } else {
          bound = g.key;
          Sk = g.mass_before + g.mass;
        }
        bbin = bz;
      }
      // min-p: every key whose l passes, (double)l - (double)m >= log(min_p)
      if (minp) {
        const uint32_t flast = minp_last_fkey(m, p.lmp);
        const uint64_t bmp = ((uint64_t)flast << 32) | 0xFFFFFFFFull;
        if (bmp < bound) {
          const int bz = row_bin(arow, fkey_desc_inv(flast));
          bound = bmp;
          if (bz >= rowwin) {
            if (anytail) return 2;
          } else {
            where(bz, z0, n);
            if (z0 < 0) {
              if ((v = load(bz, -1)) != 0) return v;
              z0 = 0;
              n = zn0;
            }
            Sk = rcum.mass(bz - 1) + wsum(z0, n, bound);
            bbin = bz;
          }
        }
      }
      // top-p (SpecSampling.swift:62-66)
      uint64_t bound1 = bound, S1 = Sk;
      int bb1 = bbin;
      if (topp) {
        const double thr = (double)p.top_p * (double)Sk;
        const int lim = bbin < rowwin ? bbin : rowwin;
        int bz = rcum.find(true, thr, lim, 0ull, NOBIN);
        if (bz >= lim) {
          if (bbin >= rowwin) return 2;
          bz = bbin;
        }
        where(bz, z0, n);
        if (z0 < 0) {
          int also = -1;
          if (!vdr) {
            const int blo = rcum.find(true, (double)u_draw * (double)rcum.mass(bz - 1), bz + 1, 0ull, NOBIN);
            const int bhi = rcum.find(true, (double)u_draw * (double)rcum.mass(bz), bz + 1, 0ull, NOBIN);
            if (blo == bhi && blo <= bz) also = blo;
          }
          if ((v = load(bz, also)) != 0) return v;
          z0 = 0;
          n = zn0;
        }
        const GHit g = wpick(z0, n, true, thr, bound, -1, rcum.cnt(bz - 1), rcum.mass(bz - 1));
        if (g.key != ~0ull) {
          bound1 = g.key;
          S1 = g.mass_before + g.mass;
          bb1 = bz;
        } else if (bz != bbin) {
          return 2;
        }
      }
      // the draft of a verify row: kept? its mass and bin
      uint64_t wd = 0ull;
      int xb = NOBIN;
      if (vdr && l_draft > -INFINITY && ckey(l_draft, draft) <= bound1) {
        wd = rmass(l_draft, m);
        xb = row_bin(arow, l_draft);
      }
      // the icdf draw over the kept keys without the draft
      int token;
      if (S1 <= wd) {
        token = arg;  // only the draft kept: the first kept token
      } else {
        const double thr = (double)u_draw * (double)(S1 - wd);
        const int lim = bb1 < rowwin ? bb1 : rowwin;
        int bz = rcum.find(true, thr, lim, wd, xb);
        if (bz >= lim) {
          if (bb1 >= rowwin) return 2;
          bz = bb1;
        }
        where(bz, z0, n);
        if (z0 < 0) {
          if ((v = load(bz, -1)) != 0) return v;
          z0 = 0;
          n = zn0;
        }
        const uint64_t m0 = rcum.mass(bz - 1) - (bz - 1 >= xb ? wd : 0ull);
        const GHit g = wpick(z0, n, true, thr, bound1, draft, rcum.cnt(bz - 1), m0);
        if (g.key == ~0ull) return 2;
        token = (int)(uint32_t)g.key;
      }
      const int acc = vdr && ((double)u_acc < (double)wd / (double)S1) ? 1 : 0;
      finish(STRIM_OK, token, acc, (double)S1 / RFIX, bound1);
      return 0;
    };
    if (w == 0) {
      const int verdict = solo();
      if (lane == 0) S.misc[5] = verdict;
    }
    __syncthreads();
    const int verdict = uniform_copy(S.misc[5]);
    if (verdict == 0) return true;
    if (verdict == 2) return false;

    // The zone in LDS: up to two bins, zb[h] at [zo[h], zo[h] + zn[h]). A chunk's part of a
    // bin comes from its prefetched candidates when it lies among them, else from its slot
    // region; a bin some chunk could not write whole is collected by a streaming pass.
    int zb[2] = {-1, -1}, zo[2] = {0, 0}, zn[2] = {0, 0}, npick = 0;
    lds_t<GFinalShared>* Sl = (lds_t<GFinalShared>*)&S;
    lds_t<GBig>* Gl = (lds_t<GBig>*)&G;

    // The decisions, in order, through one loop (its code is fetched once):
    //   0 top-k: the k-th key in order (every key counts);
    //   1 min-p: the kept mass of the keys whose l passes, (double)l - (double)m >= lmp;
    //   2 top-p: the last kept token is the first whose inclusive mass exceeds P Sk (a
    //     token is dropped iff the mass before it exceeds P, SpecSampling.swift:62-66);
    //   3 the icdf draw over the kept keys without the draft.
    // The leader finds each step's bin and lays out its zone; every wave then loads the
    // zone and takes part in the pick, and keeps the same state (all of it uniform).
    // The kept set before top-p: keys <= bound, mass Sk, the bound's bin bbin (NOBIN:
    // none inside the window); after it: bound1, S1, bb1.
    uint64_t bound = ~0ull, Sk = S0, bound1 = ~0ull, S1 = S0, wd = 0ull;
    int bbin = NOBIN, bb1 = NOBIN, xb = NOBIN, token = -1;
    for (int step = 0; step < 4; ++step) {
      if (step == 0 && !topk) continue;
      if (step == 1 && !minp) continue;
      if (step == 2) {
        bound1 = bound;
        S1 = Sk;
        bb1 = bbin;
        if (!topp) continue;
      }
      if (step == 3) {
        // the draft of a verify row: kept? its mass and bin
        if (vdr && l_draft > -INFINITY && ckey(l_draft, draft) <= bound1) {
          wd = rmass(l_draft, m);
          xb = row_bin(arow, l_draft);
        }
        if (!icdf) break;
        if (S1 <= wd) {
          token = arg;  // only the draft kept: the first kept token
          break;
        }
      }
      // ---- the leader: this step's bin and zone -------------------------------------
      if (w == 0) {
        GCmd cmd;
        cmd.op = GOP_PICK;
        cmd.load = 0;
        cmd.also = -1;
        cmd.by_mass = 1;
        cmd.excl = -1;
        cmd.thr = 0.0;
        cmd.bnd = ~0ull;
        cmd.bmp = ~0ull;
        int bz = -1, bfall = NOBIN;
        uint64_t xw = 0ull;
        int xbn = NOBIN;
        if (step == 0) {
          if (n_all < p.top_k) cmd.op = GOP_SKIP;  // every allowed token is kept
          cmd.by_mass = 0;
          cmd.thr = (double)(p.top_k - 1);
        } else if (step == 1) {
          const uint32_t flast = minp_last_fkey(m, p.lmp);
          cmd.bmp = ((uint64_t)flast << 32) | 0xFFFFFFFFull;
          cmd.op = GOP_SUM;
          if (cmd.bmp >= bound) {
            cmd.op = GOP_SKIP;
          } else {
            bz = row_bin(arow, fkey_desc_inv(flast));
            // below the window: with no token below some chunk's window every allowed
            // token passes (the bound alone is set), else the lattice cannot tell
            if (bz >= rowwin) cmd.op = anytail ? GOP_FAIL : GOP_BOUND;
          }
        } else if (step == 2) {
          cmd.thr = (double)p.top_p * (double)Sk;
          cmd.bnd = bound;
          bfall = bbin;  // the cut lies in the bound's bin when no bin above it crosses
        } else {
          cmd.thr = (double)u_draw * (double)(S1 - wd);
          cmd.bnd = bound1;
          cmd.excl = draft;
          xw = wd;
          xbn = xb;
          bfall = bb1;
        }
        if (cmd.op == GOP_PICK || cmd.op == GOP_SUM) {
          if (bz < 0) {
            const int lim = bfall < rowwin ? bfall : rowwin;
            bz = rcum.find(cmd.by_mass, cmd.thr, lim, xw, xbn);
            if (bz >= lim) bz = bfall < rowwin ? bfall : NOBIN;
            // top-p of a sample row: the icdf draw's bin, when it can be told now, is
            // loaded with the cut's (the kept mass lies between the masses before and
            // through the cut's bin, so the draw's threshold lies between u times each)
            if (bz < NOBIN && step == 2 && icdf && !vdr) {
              const int blo = rcum.find(true, (double)u_draw * (double)rcum.mass(bz - 1), bz + 1, 0ull, NOBIN);
              const int bhi = rcum.find(true, (double)u_draw * (double)rcum.mass(bz), bz + 1, 0ull, NOBIN);
              if (blo == bhi && blo <= bz) cmd.also = blo;
            }
          }
          if (bz >= rowwin) {
            cmd.op = GOP_FAIL;
          } else if (zb[0] != bz && zb[1] != bz) {
            if (bz >= rowfull) {
              cmd.load = 2;
              cmd.also = -1;
            } else {
              const uint64_t cr = rcum.cnt(bz) - rcum.cnt(bz - 1);
              const int also = cmd.also;
              const bool two = also >= 0 && also != bz && also < rowfull &&
                               cr + rcum.cnt(also) - rcum.cnt(also - 1) <= (uint64_t)GT;
              cmd.also = two ? also : -1;
              if (cr > (uint64_t)ZCAP) cmd.op = GOP_FAIL;
              // lane c: chunk c's parts of the bins and their places in the zone
              const int bins[2] = {bz, cmd.also};
              int n[2];
#pragma unroll
              for (int hh = 0; hh < 2; ++hh) {
                int cnt = 0, off = 0;
                if (lane < W && bins[hh] >= 0) {
                  const int lb = bins[hh] - S.dch[lane];
                  if (lb >= 0 && lb < S.nbch[lane]) {
                    off = lb > 0 ? (int)S.pc[lane][lb - 1] : 0;
                    cnt = (int)S.pc[lane][lb] - off;
                  }
                }
                const int zo_ = (int)wave_incl_scan_u32((uint32_t)cnt) - cnt;
                n[hh] = __builtin_amdgcn_readlane(zo_ + cnt, WAVE - 1);
                if (lane < W) {
                  S.zpo[hh][lane] = off;
                  S.zpc[hh][lane] = cnt;
                  S.zpz[hh][lane] = zo_ + (hh ? n[0] : 0);
                }
              }
              cmd.load = 1;
              cmd.n0 = n[0];
              cmd.n1 = n[1];
            }
          }
          cmd.c0 = rcum.cnt(bz - 1);
          cmd.m0 = rcum.mass(bz - 1) - (bz - 1 >= xbn ? xw : 0ull);
        }
        cmd.bz = bz;
        if (lane == 0) S.cmd = cmd;
      }
      __syncthreads();
      const GCmd cmd = uniform_copy(S.cmd);
      if (cmd.op == GOP_FAIL) return false;
      if (cmd.op == GOP_SKIP) continue;
      if (cmd.op == GOP_BOUND) {
        bound = cmd.bmp;
        continue;
      }
      const int bz = cmd.bz;
      // ---- every wave: the zone ------------------------------------------------------
      if (cmd.load == 1) {
        // wave w copies the parts of chunks w, w + GW, ...: from the prefetched
        // candidates where they lie among them, else from the chunk's slot region
        for (int cq = w; cq < W; cq += GW) {
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            const int o = S.zpo[hh][cq], cn = S.zpc[hh][cq], z0 = S.zpz[hh][cq];
            for (int i = lane; i < cn; i += WAVE) {
              const int e = o + i;
              const Cand x = (pfok && e < PF) ? P.pfb[cq * PF + e] : slots[(int64_t)cq * SLOT + e];
              if (z0 + i < ZCAP) {
                G.z.zkey[z0 + i] = ckey(x.l, x.id);
                G.z.zmass[z0 + i] = rmass(x.l, m);
              }
            }
          }
        }
        __syncthreads();
        zb[0] = bz;
        zo[0] = 0;
        zn[0] = cmd.n0;
        zb[1] = cmd.also;
        zo[1] = cmd.n0;
        zn[1] = cmd.n1;
      } else if (cmd.load == 2) {
        const int n = collect_zone(xa, r, b, j, p, arow - (float)bz, m,
                                   ZoneLds{(lds_t<uint64_t>*)G.z.zkey, (lds_t<uint64_t>*)G.z.zmass,
                                           (lds_t<uint32_t>*)P.ccnt, (lds_t<int>*)&S.misc[2]});
        pfok = false;  // (the pass's history counts took the prefetched candidates' LDS)
        if (n < 0) return false;
        zb[0] = bz;
        zo[0] = 0;
        zn[0] = n;
        zb[1] = -1;
      }
      const int h = zb[0] == bz ? 0 : 1;
      if (cmd.op == GOP_SUM) {
        // min-p: the kept mass is everything before the bound's bin and the zone's keys
        // up to the bound
        bound = cmd.bmp;
        Sk = cmd.m0 + zone_mass_upto(S, G, zo[h], zn[h], bound);
        bbin = bz;
        continue;
      }
      // ---- the pick: the key whose cumulative interval contains thr ------------------
      GHit g;
      {
        const int np = npick++;
        if (zn[h] <= RADIX_MIN)
          g = pick_rank(S, G, np, zo[h], zn[h], cmd.by_mass != 0, cmd.thr, cmd.bnd, cmd.excl,
                        cmd.c0, cmd.m0);
        else
          g = pick_sorted_ool(Sl, Gl, np, zo[h], zn[h], cmd.by_mass != 0, cmd.thr, cmd.bnd,
                              cmd.excl, cmd.c0, cmd.m0);
      }
      if (step == 0) {
        if (g.key == ~0ull) return false;
        if (p.flags & STRIM_FLAG_TOPK_KEEP_TIES) {
          // the keys tied with the k-th one are kept too (same value, same bin)
          bound = g.key | 0xFFFFFFFFull;
          Sk = cmd.m0 + zone_mass_upto(S, G, zo[h], zn[h], bound);
        } else {
          bound = g.key;
          Sk = g.mass_before + g.mass;
        }
        bbin = bz;
      } else if (step == 2) {
        if (g.key != ~0ull) {
          bound1 = g.key;
          S1 = g.mass_before + g.mass;
          bb1 = bz;
        } else if (bz != bbin) {
          return false;
        }
      } else {
        if (g.key == ~0ull) return false;
        token = (int)(uint32_t)g.key;
      }
    }
    if (!icdf) {
      // Gumbel: every kept candidate (key <= bound1, not the draft)
      if (bb1 >= rowfull) return false;  // every kept token must be a candidate
      const bool cand_sorted = (p.flags & STRIM_FLAG_SCORE_NO_LSE) ? topp : (topk || topp);
      token = gumbel_kept(Sl, slots, a.noise ? a.noise + (int64_t)r * a.noise_stride : nullptr,
                          W, bb1, bound1, draft, p, m, S1, cand_sorted);
      if (token < 0) token = arg;  // only the draft kept
    }
    const int acc = vdr && ((double)u_acc < (double)wd / (double)S1) ? 1 : 0;
    finish(STRIM_OK, token, acc, (double)S1 / RFIX, bound1);
    return true;
  };
  if (lat && decide()) return;

  // ---- the exact streaming resolution ----------------------------------------------
  const XScratch xs = xscratch(G.x.xkey, G.x.xhc, G.x.xcnt, G.x.xu2, S.d, S.u, S.ii);
  __builtin_amdgcn_s_waitcnt(0);  // (its LDS overlaps the lattice words' and candidates')
  __syncthreads();
  const XOut xo =
      exact_row<GT, false>(xa, r, b, j, p, m, arg, draft, vdr, l_draft, xs, *(lds_t<XState>*)&G.x.x);
  finish(xo.status, xo.token, xo.accept, xo.sig, xo.last_key);
}

hipError_t launch_gfinal(const Args& a, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
  const ChunkStat* c = a.s.cstat;
  const unsigned long long* l = a.s.lat;
  const Cand* sl = a.s.slot;
  int wm = a.s.wmax, W = a.W;
  void* args[] = {&c, &l, &sl, &wm, &W, const_cast<Args*>(&a)};
  const dim3 grid((unsigned)a.R), block(GT);
  const void* k = (const void*)k_gfinal;
  if (e0 || e1) return hipExtLaunchKernel(k, grid, block, args, 0, st, e0, e1, 0);
  return hipLaunchKernel(k, grid, block, args, 0, st);
}

}  // namespace strim
