// gfinal_kernels.hip — k_gfinal: the general rows, decided from the chunks' candidates.
//
// A general row (top-p alone, a top-k above KLOC, a min-p below MINP_FAST, no filter with
// icdf noise) cannot bound its candidates by a chunk's own maximum. k_stream keeps every
// token with l > cs.g of its chunk as a candidate (at most GCAP per chunk, in the chunk's
// slot region as (l, id)), so with G the largest cs.g of the row every token with l > G
// is a candidate: the order, the masses and the cumulative sums of the row above G are
// known exactly. When every decision of the row (the k-th token, the top-p cut, the draw)
// lies above G, one workgroup takes them from the candidates alone. Otherwise the row
// deepens once: k_stream also keeps a second tier of up to GCAP2 tokens per chunk below
// the first, with its own bound cs.g2, and the decisions run again over both tiers above
// G2 = max cs.g2. A row that still falls short (a nucleus wider than both tiers, a flat
// row) is resolved by the exact streaming resolution (exact.hpp) in the same workgroup.
// The first tier is kept small (GCAP = 32 per chunk decides the common rows: a nucleus up
// to a few hundred tokens) because every candidate of a round costs LDS atomics and
// stores on the one CU the row runs on.
//
// One 512-thread workgroup per row (eight waves: 1,024 threads measured 1.4 us slower on
// its merges and barriers, 256 slower on its per-thread loops); each thread holds up to
// GNE candidates in registers:
//   1. the chunk statistics and every candidate slot are loaded together (the slots of
//      a region past its count are read and dropped, so nothing waits for the counts);
//      the waves' maxima, flags, bounds and chunk mass sums are merged with one barrier;
//   2. the candidates above G are binned by d = m - l into GNB bins. A bin is one 64-bit
//      word, count << 49 | mass, so each candidate costs one LDS atomic (they run about
//      one lane per cycle, so their number sets this step's time), and the atomic's old
//      count is the candidate's place in its bin. Masses are fixed point,
//      round(2^35 * expf(l - m)): integer sums make every cumulative mass independent of
//      summation order, 8192 unit masses stay below 2^48, and the per-token error (the
//      float exp's 2^-23 relative plus 2^-36 absolute) keeps any cumulative mass within
//      5e-7 relative of the exact one, inside the 1e-6 decision tolerance. Each wave turns
//      its 64 bins into inclusive prefixes (a bin's cumulative count or mass is its
//      group's prefix plus the totals of the groups before it), and every candidate is
//      stored with its mass in bin order;
//   3. the decisions run in order (the k-th token, the top-p cut, the icdf draw) through
//      one loop, so their shared code is fetched once: each finds the bin where its
//      threshold is crossed from the prefixes, and each key of that bin counts the bin's
//      keys before it in order; the key whose interval contains the threshold is the
//      decision (one barrier per decision). A Gumbel draw scores every kept candidate.
// The kernel's time is latency (dependent steps, barriers and the first fetch of its
// code), so the code is kept short: loops that run once per decision are not repeated
// per decision.
#include "exact.hpp"

namespace strim {

constexpr int GT = 512;             // threads of a k_gfinal workgroup
constexpr int GW = GT / WAVE;       // its waves; wave w owns the histogram bins of group w
constexpr int GNE = 4;              // candidate slots per thread: W * GCAP <= GT * GNE
constexpr int GNE2 = 12;            // second-tier slots per thread: W * GCAP2 <= GT * GNE2
constexpr int GCAND = 8192;         // candidates of a row held in bin order (both tiers)
constexpr int GNB = GW * WAVE;      // histogram bins of d = m - l (64 per group)
constexpr int GZCAP = GT;           // keys of one bin a decision resolves (one per thread)
constexpr double GFIX = 34359738368.0;  // 2^35: the fixed-point unit of mass
constexpr int GCSH = 49;                // a bin word: count << GCSH | mass
constexpr uint64_t GMMASK = (1ull << GCSH) - 1ull;
constexpr int GSH = __builtin_ctz(GCAP), GSH2 = __builtin_ctz(GCAP2);  // region of entry e: e >> GSH
static_assert((1 << GSH) == GCAP && (1 << GSH2) == GCAP2, "tier sizes are powers of two");
static_assert(GT % GCAP == 0 && GT % GCAP2 == 0, "whole regions per pass of the workgroup");
static_assert(GT * GNE >= 64 * GCAP, "the first tier of 64 chunks fits the slots");
static_assert(GT * (GNE + GNE2) <= GCAND, "a second round fits the bin-order arrays");
static_assert(GNB == GT, "one bin per thread to clear");

// LDS of one k_gfinal workgroup.
struct GFinalShared {
  union {
    struct {                  // the decision from the candidates
      uint64_t bkey[GCAND + WAVE];   // the candidates above G in bin order (64 KB; the
                                     // last WAVE entries take the writes of empty slots)
      uint64_t bmass[GCAND + WAVE];  // their fixed-point masses
    };
    struct {                  // the exact streaming resolution (rows decided at or below G)
      uint64_t xkey[XB > XCOL ? XB : XCOL];
      uint32_t xhc[XB];
      uint32_t xcnt[GT * EPT];
      uint64_t xu2[2 * GT / WAVE];
      XState x;
    };
  };
  uint64_t hist[GNB];         // per bin count << GCSH | mass, then the group-local
                              // inclusive prefix
  uint64_t gt[GW];            // per group: its total
  uint32_t rcnt[GT];          // per chunk: its candidates
  uint32_t rcnt2[GT];         // per chunk: its second-tier candidates
  float v[GW], g[GW], g2[GW];
  int i[GW], f[GW];
  double sw[GW];              // per wave: its chunks' mass, relative to the row maximum
  double d[GW];
  uint64_t u[GW];
  int misc[8];
  uint64_t res[2][4];         // a decision: key, count before, mass before, mass (two slots,
  int32_t tag[2];             // alternating; tag = the decision's number when it holds one)
};

// Fixed-point mass of a token: round(2^35 * exp(l - m)), from the float exp of the
// float difference (l <= m).
__device__ __forceinline__ uint64_t gmass(float l, float m) {
  return (uint64_t)(expf(l - m) * 34359738368.0f + 0.5f);
}
__device__ __forceinline__ int gbin(float m, float l, float hscale) {
  return (int)fminf((m - l) * hscale, (float)(GNB - 1));
}
__device__ __forceinline__ float key_l(uint64_t k) { return fkey_desc_inv((uint32_t)(k >> 32)); }

// Cumulative bin word (count << GCSH | mass) of bins 0 .. b, from the group-local
// prefixes and `ginc`, lane g's inclusive prefix of the group totals (b is wave-uniform).
__device__ __forceinline__ uint64_t gcum(const GFinalShared& S, uint64_t ginc, int b) {
  if (b < 0) return 0ull;
  const int g = b / WAVE;
  const uint64_t before = g > 0 ? rl_u64(ginc, g - 1) : 0ull;
  return before + S.hist[b];
}
__device__ __forceinline__ uint64_t wcount(uint64_t x) { return x >> GCSH; }
__device__ __forceinline__ uint64_t wmass(uint64_t x) { return x & GMMASK; }

// The first bin whose cumulative count or mass, less excl_w from bin excl_b on, exceeds
// thr, among the bins before bb; bb when none does (every wave computes the same bin).
__device__ __forceinline__ int gfind_bin(const GFinalShared& S, bool mass, uint64_t ginc,
                                         double thr, int bb, uint64_t excl_w, int excl_b) {
  const int lane = threadIdx.x & (WAVE - 1);
  auto val = [&](uint64_t x, bool ex) -> uint64_t {
    return mass ? wmass(x) - (ex ? excl_w : 0ull) : wcount(x);
  };
  // the first group whose cumulative total (with the exclusion) exceeds thr
  const uint64_t gv = val(ginc, excl_b <= WAVE * lane + WAVE - 1);
  const uint64_t gh = __ballot(lane < GW && (double)gv > thr);
  if (gh == 0ull) return bb;
  const int g = (int)__ffsll((long long)gh) - 1;
  if (g * WAVE >= bb) return bb;
  // within the group: one bin per lane
  const int b = g * WAVE + lane;
  const uint64_t before = g > 0 ? rl_u64(ginc, g - 1) : 0ull;
  const uint64_t bv = val(before + S.hist[b], b >= excl_b);
  const uint64_t bh = __ballot((double)bv > thr);
  const int bz = bh ? g * WAVE + (int)__ffsll((long long)bh) - 1 : bb;
  return bz < bb ? bz : bb;
}

// A decision: the key (~0: none), the count and mass of the keys before it in the row's
// order, and its own mass.
struct GHit {
  uint64_t key, cnt_before, mass_before, mass;
};

// Decision number n over the zone bkey/bmass[z0, z0 + nz) (one bin in bin order; every
// thread, nz <= GT): the first zone key in key order, key <= bound and id != excl, whose
// inclusive cumulative count (mass == false) or mass exceeds thr, starting from cnt0 /
// mass0 before the zone. Thread t owns zone key t and counts the zone keys before it; the
// unique key whose interval contains thr writes its result with tag n to slot n & 1 (a
// slot is rewritten two decisions later, after every thread has read it). One barrier.
__device__ __forceinline__ GHit gresolve(GFinalShared& S, int n, int z0, int nz, bool mass,
                                         double thr, uint64_t bound, int excl, uint64_t cnt0,
                                         uint64_t mass0) {
  const int t = threadIdx.x;
  const int slot = n & 1;
  if (t < nz) {
    const uint64_t k = S.bkey[z0 + t];
    const uint64_t km = S.bmass[z0 + t];
    const bool in = k <= bound && (int)(uint32_t)k != excl;
    uint32_t rank = 0u;
    uint64_t mb = 0ull;
    for (int jj = 0; jj < nz; ++jj) {
      const uint64_t kj = S.bkey[z0 + jj];
      const uint64_t mj = S.bmass[z0 + jj];
      const bool lt = kj < k;
      rank += lt ? 1u : 0u;
      mb += (lt && kj <= bound && (int)(uint32_t)kj != excl) ? mj : 0ull;
    }
    // count mode counts every key (no bound, no exclusion)
    const uint64_t before = mass ? mass0 + mb : cnt0 + rank;
    const uint64_t own = mass ? (in ? km : 0ull) : 1ull;
    if (own > 0ull && (double)before <= thr && (double)(before + own) > thr) {
      S.res[slot][0] = k;
      S.res[slot][1] = cnt0 + rank;
      S.res[slot][2] = mass0 + mb;
      S.res[slot][3] = km;
      S.tag[slot] = n;
    }
  }
  __syncthreads();
  if (S.tag[slot] != n) return GHit{~0ull, 0ull, 0ull, 0ull};
  return GHit{S.res[slot][0], S.res[slot][1], S.res[slot][2], S.res[slot][3]};
}

__global__ __launch_bounds__(GT) void k_gfinal(Args a) {
  __shared__ GFinalShared S;
  // the launch fields of the first loads, read together (see k_stream)
  asm volatile("" ::"s"(a.s.cstat), "s"(a.s.wmax), "s"(a.s.rs), "s"(a.s.slot), "s"(a.W),
               "s"(a.V), "s"(a.noise), "s"(a.noise_stride), "s"(a.noise_mode), "s"(a.verify),
               "s"(a.k), "s"(a.drafts));
  const int r = blockIdx.x;
  int b, j;
  row_bj(a, r, b, j);
  const int t = threadIdx.x, lane = t & (WAVE - 1), w = t / WAVE;
  const int V = a.V, W = a.W;
  // ---- step 1: every load that does not depend on the row's parameters ------------
  // the chunk statistics (one chunk per thread), the noise, the draft and every candidate
  // slot of the row (no branch between the loads: a missing optional input reads the
  // row's own state and is ignored; slots past a region's count are dropped later)
  const ChunkStat cs = a.s.cstat[(int64_t)r * a.s.wmax + (t < W ? t : 0)];
  static_assert(sizeof(ChunkStat) == 48, "ChunkStat layout");
  RowState* rsp = &a.s.rs[r];
  const bool gum = a.noise && a.noise_mode != STRIM_NOISE_ICDF;
  const float* nz = a.noise ? a.noise + (int64_t)r * a.noise_stride : (const float*)rsp;
  const float n0 = nz[gum ? V : 0], n1 = nz[gum ? V : 1];
  const bool vdr = a.verify && j < a.k;
  const int32_t* dp = vdr ? a.drafts + (int64_t)b * a.k + j : (const int32_t*)rsp;
  const int d_raw = *dp;
  const float ld_raw = rsp->l_draft;
  const int ne = W * GCAP;  // candidate slots of the row
  const Cand* slots = a.s.slot + (int64_t)r * a.s.wmax * SLOT;
  // slots 0 .. GNE - 1: the first tier (entry e = q GT + t is region e / GCAP, offset
  // e % GCAP); slots GNE .. GNE + GNE2 - 1: the second tier, loaded only when a decision
  // falls at or below the first tier's bound (entry e is region e / GCAP2, offset GCAP +
  // e % GCAP2)
  Cand cd[GNE];
#pragma unroll
  for (int q = 0; q < GNE; ++q) {
    const int e = q * GT + t;
    cd[q] = slots[e < ne ? (int64_t)(e >> GSH) * SLOT + (e & (GCAP - 1)) : 0];
  }
  const RowParams p = load_params(a, b, j);
  if (!gfinal_row(a.p[b], V, a.noise_mode, a.dlog != nullptr && vdr)) return;
  const int draft = vdr ? d_raw : -1;
  const float l_draft = vdr ? ld_raw : -INFINITY;

  // ---- the chunk statistics: per wave, then every wave merges the waves' results --
  const bool own = t < W;
  int ff = own ? (cs.flags | (cs.n > 0 ? 4 : 0)) : 0;
  float mv = own ? cs.m : -INFINITY, gv = own ? cs.g : -INFINITY;
  float gv2 = own ? cs.g2 : -INFINITY;
  int mi = own ? cs.arg : -1;
  S.rcnt[t] = own ? cs.ncand : 0u;
  S.rcnt2[t] = own ? cs.ncand2 : 0u;
  wave_argmax(mv, mi);
  ff = wave_or_i(ff);
  gv = wave_max_f(gv);
  gv2 = wave_max_f(gv2);
  if (lane == 0) {
    S.v[w] = mv;
    S.i[w] = mi;
    S.f[w] = ff;
    S.g[w] = gv;
    S.g2[w] = gv2;
  }
  S.hist[t] = 0ull;
  if (t < 2) S.tag[t] = -1;
  __syncthreads();
  // lane q holds wave q's results
  float m = lane < GW ? S.v[lane] : -INFINITY, G = lane < GW ? S.g[lane] : -INFINITY;
  float G2 = lane < GW ? S.g2[lane] : -INFINITY;
  int arg = lane < GW ? S.i[lane] : -1, flags = lane < GW ? S.f[lane] : 0;
  wave_argmax(m, arg);
  flags = wave_or_i(flags);
  G = wave_max_f(G);
  G2 = wave_max_f(G2);
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
    finish(status, -1, 0, 0.0, 0ull);
    return;
  }
  const uint64_t pkey = mix64(p.seed, p.position);
  float u_draw = 0.0f, u_acc = 0.0f;
  if (a.noise) {
    if (a.noise_mode == STRIM_NOISE_ICDF) u_draw = n0;
    u_acc = n1;
  } else {
    u_draw = philox_uniform(pkey, 0);
    u_acc = philox_uniform(pkey, a.noise_mode == STRIM_NOISE_GUMBEL ? (uint64_t)V : 1u);
  }

  // ---- steps 2 and 3: the decision from the candidates ---------------------------
  // Round 0 uses the first tier and the bound G, round 1 (when a decision of round 0
  // fell at or below G) both tiers and the bound G2. The verdict: 0 decided, 1 a
  // decision lies at or below the round's bound, 2 the candidates cannot decide the row
  // (both lead to the exact resolution when no round is left). Every condition is uniform
  // over the workgroup.
  // (one instantiation per round: the first round's code and registers carry nothing
  // of the second tier)
  enum { DECIDED = 0, BELOW = 1, OTHER = 2 };
  const int ne2 = W * GCAP2;  // second-tier slots of the row
  auto decide = [&](auto round_c, const Cand (&cd2)[GNE2]) -> int {
    constexpr int round = decltype(round_c)::value;
    constexpr int NS = round == 0 ? GNE : GNE + GNE2;  // slots of this round
    auto cand = [&](int q) -> const Cand& { return q < GNE ? cd[q] : cd2[q - GNE]; };
    const bool topk = p.top_k > 0 && p.top_k < V;
    const bool topp = p.top_p < 1.0f;
    const bool minp = p.min_p > 0.0f;
    const bool icdf = a.noise_mode == STRIM_NOISE_ICDF;
    // rank-indexed noise needs every kept token's rank
    if ((p.flags & STRIM_FLAG_NOISE_BY_RANK) && topp && !icdf) return OTHER;
    if (ne > GT * GNE) return OTHER;
    const float Gr = round == 0 ? G : G2;
    const bool all_in = !(Gr > -INFINITY);  // every allowed token is a candidate
    // min-p keeps a set that lies above the bound only if the bound itself fails it
    if (minp && !all_in && ((double)Gr - (double)m) >= p.lmp) return BELOW;
    const float span = all_in ? 64.0f : fminf(fmaxf(m - Gr, 1.0f / 64.0f), 64.0f);
    const float hscale = (float)GNB / span;
    // which of this thread's slots hold a candidate: first-tier entry e = q GT + t lies
    // in region e / GCAP at offset e % GCAP, second-tier entry e = q GT + t in region
    // e / GCAP2 at offset GCAP + e % GCAP2
    uint32_t vmask = 0u;
    {
      uint32_t rc[NS];
#pragma unroll
      for (int q = 0; q < GNE; ++q) rc[q] = S.rcnt[min(q * (GT / GCAP) + (t >> GSH), GT - 1)];
#pragma unroll
      for (int q = GNE; q < NS; ++q)
        rc[q] = S.rcnt2[min((q - GNE) * (GT / GCAP2) + (t >> GSH2), GT - 1)];
#pragma unroll
      for (int q = 0; q < GNE; ++q)
        vmask |= (((q * GT + t < ne) & ((uint32_t)(t & (GCAP - 1)) < rc[q])) ? 1u : 0u) << q;
#pragma unroll
      for (int q = GNE; q < NS; ++q)
        vmask |= ((((q - GNE) * GT + t < ne2) & ((uint32_t)(t & (GCAP2 - 1)) < rc[q])) ? 1u : 0u)
                 << q;
    }
    // bin every candidate above the bound (passing min-p); the atomic's old count is its place in
    // the bin. A lane without a candidate leaves old[q] unset and never reads it; the
    // empty asm statements after the loop keep the compiler from reading any result
    // before every atomic is issued (it would otherwise wait for each in turn).
    uint64_t old[NS], cm[NS];
    int bn[NS];
#pragma unroll
    for (int q = 0; q < NS; ++q) {
      const float l = cand(q).l;
      const bool k = ((vmask >> q) & 1u) && l > Gr && l > -INFINITY &&
                     (!minp || ((double)l - (double)m) >= p.lmp);
      bn[q] = k ? gbin(m, l, hscale) : -1;
      if (k) {
        cm[q] = gmass(l, m);
        old[q] = atomicAdd(&S.hist[bn[q]], (unsigned long long)((1ull << GCSH) | cm[q]));
      }
    }
#pragma unroll
    for (int q = 0; q < NS; ++q) asm volatile("" : "+v"(old[q]));
    // the whole row's mass relative to m, from the chunk sums (used while the kept set
    // reaches below the bound), while the atomics complete
    {
      const double sw = wave_sum((own && cs.n > 0) ? cs.S * exp((double)cs.m - (double)m) : 0.0);
      if (lane == 0) S.sw[w] = sw;
    }
    __syncthreads();
    // group-local inclusive prefixes: wave w over bins 64 w .. 64 w + 63
    {
      const int bb = w * WAVE + lane;
      const uint64_t ci = wave_incl_scan_u64(S.hist[bb]);
      S.hist[bb] = ci;
      if (lane == WAVE - 1) S.gt[w] = ci;
    }
    double S_all = 0.0;
#pragma unroll
    for (int q = 0; q < GW; ++q) S_all += S.sw[q];
    __syncthreads();
    // lane g: inclusive prefix of the group totals
    const uint64_t gl = lane < GW ? S.gt[lane] : 0ull;
    const uint64_t ginc = wave_incl_scan_u64(gl);
    const uint64_t tot = rl_u64(ginc, GW - 1);
    const uint64_t n_all = wcount(tot), m_all = wmass(tot);
    if (n_all == 0ull) return BELOW;
    // every candidate with its mass into bin order: bin b starts at the cumulative count
    // of the bins before it (the group's exclusive prefix from lane g, plus the bins
    // before b in the group); a slot without a candidate writes past the row's entries
    {
      const int gce = (int)wcount(ginc - gl);
      // every read first (the empty asm statements keep them ahead of their uses), then
      // every write
      int at[NS];
      uint32_t hb[NS];
      int gb[NS];
#pragma unroll
      for (int q = 0; q < NS; ++q) {
        const int bq = bn[q] < 0 ? 0 : bn[q];
        hb[q] = (uint32_t)(S.hist[bq > 0 ? bq - 1 : 0] >> 32);
        gb[q] = __shfl(gce, bq / WAVE);
      }
#pragma unroll
      for (int q = 0; q < NS; ++q) asm volatile("" : "+v"(hb[q]), "+v"(gb[q]));
#pragma unroll
      for (int q = 0; q < NS; ++q) {
        const int before = gb[q] + ((bn[q] & (WAVE - 1)) ? (int)(hb[q] >> (GCSH - 32)) : 0);
        at[q] = bn[q] >= 0 ? before + (int)wcount(old[q]) : GCAND + lane;
      }
#pragma unroll
      for (int q = 0; q < NS; ++q) {
        S.bkey[at[q]] = ckey(cand(q).l, cand(q).id);
        S.bmass[at[q]] = cm[q];
      }
    }
    __syncthreads();

    // ---- the decisions, in order: 0 the k-th token (count), 1 the top-p cut (mass), 2
    // the icdf draw (mass, without the draft) -----------------------------------------
    bool known0 = all_in || minp;  // every token of the set is a candidate
    uint64_t bound0 = ~0ull, S0 = known0 ? m_all : (uint64_t)__double2ull_rn(S_all * GFIX);
    uint64_t bound1 = ~0ull, S1 = S0, wd = 0ull;
    bool known1 = known0;
    int token = -1;
    int nres = 0;  // decisions resolved so far (consecutive ones alternate result slots)
    for (int step = 0; step < 3; ++step) {
      bool mass = true;
      double thr;
      uint64_t bound, xw = 0ull;
      int excl = -1, xb = GNB;
      if (step == 0) {
        if (!topk) continue;
        if (n_all < (uint64_t)p.top_k) {
          if (!all_in) return BELOW;  // the k-th token lies at or below the bound
          continue;                   // every allowed token is kept
        }
        mass = false;
        thr = (double)(p.top_k - 1);
        bound = ~0ull;
      } else if (step == 1) {
        bound1 = bound0;
        S1 = S0;
        known1 = known0;
        if (!topp) continue;
        // the last kept token is the first whose inclusive mass exceeds P S0 (a token is
        // dropped iff the mass before it exceeds P, SpecSampling.swift:62-66)
        thr = (double)p.top_p * (double)S0;
        bound = bound0;
      } else {
        if (!icdf && !known1) return BELOW;
        // the draft of a verify row: kept? its mass, and its bin when a candidate
        if (vdr && l_draft > -INFINITY && ckey(l_draft, draft) <= bound1) {
          wd = gmass(l_draft, m);
          if (l_draft > Gr && (!minp || ((double)l_draft - (double)m) >= p.lmp)) {
            xb = gbin(m, l_draft, hscale);
            xw = wd;
          }
        }
        if (!icdf) break;
        thr = (double)u_draw * (double)(S1 - wd);
        bound = bound1;
        excl = draft;
      }
      const int bb = bound == ~0ull ? GNB - 1 : gbin(m, key_l(bound), hscale);
      const int bz = gfind_bin(S, mass, ginc, thr, bb, xw, xb);
      const uint64_t w0 = gcum(S, ginc, bz - 1);
      const uint64_t c0 = wcount(w0);
      const int nzc = (int)(wcount(gcum(S, ginc, bz)) - c0);
      if (nzc > GZCAP) return OTHER;
      const uint64_t m0 = wmass(w0) - (bz - 1 >= xb ? xw : 0ull);
      const GHit h = gresolve(S, nres++, (int)c0, nzc, mass, thr, bound, excl, c0, m0);
      if (step == 0) {
        if (h.key == ~0ull) return OTHER;
        known0 = true;
        if (!(p.flags & STRIM_FLAG_TOPK_KEEP_TIES)) {
          bound0 = h.key;
          S0 = h.mass_before + h.mass;
        } else {
          // the keys tied with the k-th one are kept too (same value, same bin)
          bound0 = h.key | 0xFFFFFFFFull;
          uint64_t loc = (t < nzc && S.bkey[c0 + t] <= bound0) ? S.bmass[c0 + t] : 0ull;
          loc = wave_sum_u64(loc);
          if (lane == 0) S.u[w] = loc;
          __syncthreads();
          uint64_t s = 0ull;
#pragma unroll
          for (int q = 0; q < GW; ++q) s += S.u[q];
          S0 = wmass(w0) + s;
        }
      } else if (step == 1) {
        if (h.key != ~0ull) {
          bound1 = h.key;
          S1 = h.mass_before + h.mass;
          known1 = true;
        } else if (!known0) {
          return BELOW;  // the cut lies at or below the bound
        }
      } else {
        if (h.key != ~0ull) token = (int)(uint32_t)h.key;
        else if (!known1) return BELOW;  // the draw lies at or below the bound
        else token = arg;                // only the draft kept: the first kept
      }
    }
    if (!icdf) {
      // ---- Gumbel: every kept candidate (key <= bound1, not the draft) ----------------
      const bool no_lse = (p.flags & STRIM_FLAG_SCORE_NO_LSE) != 0;
      const bool cand_sorted = no_lse ? topp : (topk || topp);
      const double lse = log((double)S1 / GFIX);
      double bsc = -INFINITY;
      uint64_t btk = ~0ull;
      int bid = -1;
      for (int i = t; i < (int)n_all; i += GT) {
        const uint64_t k = S.bkey[i];
        const int id = (int)(uint32_t)k;
        if (k > bound1 || id == draft) continue;
        const float l = key_l(k);
        const float u = a.noise ? a.noise[(int64_t)r * a.noise_stride + id]
                                : philox_uniform(pkey, (uint64_t)id);
        const double base = no_lse ? (double)l : ((double)l - (double)m) - lse;
        const double sc = base + gumbel64(u);
        const uint64_t tk = cand_sorted ? k : (uint64_t)id;
        if (bid < 0 || sc > bsc || (sc == bsc && tk < btk)) { bsc = sc; btk = tk; bid = id; }
      }
      block_argmax_score<GT>(bsc, btk, bid, S.d, S.u, S.i, &S.misc[3]);
      token = S.misc[3];
      if (token < 0) token = arg;  // only the draft kept
    }
    const int acc = vdr && ((double)u_acc < (double)wd / (double)S1) ? 1 : 0;
    finish(STRIM_OK, token, acc, (double)S1 / GFIX, bound1);
    return DECIDED;
  };
  // the second round needs room for both tiers and a lower bound than the first
  const bool deepen_ok = W * (GCAP + GCAP2) <= GCAND && ne2 <= GT * GNE2 && G2 < G;
  {
    const Cand none[GNE2] = {};
    const int verdict = decide(std::integral_constant<int, 0>{}, none);
    if (verdict == DECIDED) return;
    if (verdict == BELOW && deepen_ok) {
      // the second tier (its loads are the only wait of this step), and the histogram
      // and result slots cleared for the second round
      Cand cd2[GNE2];
#pragma unroll
      for (int q = 0; q < GNE2; ++q) {
        const int e = q * GT + t;
        cd2[q] = slots[e < ne2 ? (int64_t)(e >> GSH2) * SLOT + GCAP + (e & (GCAP2 - 1)) : 0];
      }
      __syncthreads();  // every read of the first round's histogram is done
      S.hist[t] = 0ull;
      if (t < 2) S.tag[t] = -1;
      __syncthreads();
      if (decide(std::integral_constant<int, 1>{}, cd2) == DECIDED) return;
    }
  }

  // ---- a decision at or below G: the exact streaming resolution --------------------
  const XScratch xs = xscratch(S.xkey, S.xhc, S.xcnt, S.xu2, S.d, S.u, S.i);
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
  __syncthreads();
  const XOut xo =
      exact_row<GT, false>(xa, r, b, j, p, m, arg, draft, vdr, l_draft, xs, *(lds_t<XState>*)&S.x);
  finish(xo.status, xo.token, xo.accept, xo.sig, xo.last_key);
}

hipError_t launch_gfinal(const Args& a, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
  return launch_args((const void*)k_gfinal, dim3((unsigned)a.R), dim3(GT), a, st, e0, e1);
}

}  // namespace strim
