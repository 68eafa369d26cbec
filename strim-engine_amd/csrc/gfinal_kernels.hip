// gfinal_kernels.hip — k_gfinal: the general rows, decided from the chunks' candidates.
//
// A general row (top-p alone, a top-k above KLOC, a min-p below MINP_FAST, no filter with
// icdf noise) cannot bound its candidates by a chunk's own maximum. k_stream keeps every
// token with l > cs.g of its chunk as a candidate (at most GCAP per chunk, in the chunk's
// slot region as (l, id)), so with G the largest cs.g of the row every token with l > G
// is a candidate: the order, the masses and the cumulative sums of the row above G are
// known exactly. When every decision of the row (the k-th token, the top-p cut, the draw)
// lies above G, one workgroup takes them from the candidates alone; otherwise the row is
// resolved by the exact streaming resolution (exact.hpp) in the same workgroup.
//
// One workgroup per row, in three steps:
//   1. the chunk statistics and every candidate slot are loaded together (the slots of
//      a region past its count are read and dropped, so nothing waits for the counts);
//   2. the candidates above G are binned by d = m - l into a 256-bin histogram of counts
//      and fixed-point masses, round(2^50 * expf(l - m)) (integer sums: every cumulative
//      mass is independent of summation order, and 8192 unit masses stay below 2^63; the
//      float exp keeps each mass within 2^-23 relative, far inside the 1e-6 decision and
//      probability tolerances), and scattered with their masses into bin order (each
//      candidate's place in its bin comes from the count atomic). The atomics are issued
//      without branches: a lane without a candidate adds to a slot of its own;
//   3. wave 0 alone finds the k-th token, the top-p cut and the icdf draw: the bin where
//      a cumulative count or mass first exceeds the threshold comes from the histogram's
//      prefix, and only that bin's keys are put in order and scanned. A Gumbel draw scores
//      every kept candidate on all waves.
#include "exact.hpp"

namespace strim {

constexpr int GNE = 32;        // candidate slots per thread: W * GCAP <= FTPB * GNE
constexpr int GZCAP = 1024;    // keys of one bin put in order
constexpr double GFIX = 1125899906842624.0;  // 2^50: the fixed-point unit of mass
static_assert(GCAP == 128, "candidate slot of an entry: e >> 7, e & 127");
static_assert(FCAP >= FTPB * GNE, "every candidate fits the bin-ordered array");

// LDS of one k_gfinal workgroup.
struct GFinalShared {
  uint64_t bkey[FCAP];   // the candidates above G in bin order (64 KB)
  union {
    uint64_t bmass[FCAP];  // their fixed-point masses (64 KB)
    struct {               // the exact streaming resolution (rows decided at or below G)
      uint32_t xhc[XB];
      uint32_t xcnt[FTPB * EPT];
      uint64_t xu2[2 * FTPB / WAVE];
      XState x;
    };
  };
  uint64_t zone[GZCAP];  // one bin's keys (with their zone index), in order
  uint64_t zmass[GZCAP]; // their masses, by zone index
  uint64_t hmass[256];   // fixed-point mass per bin, then the inclusive prefix
  uint64_t dmass[FTPB];  // per thread: where a lane without a candidate adds its mass
  uint32_t hist[256];    // count per bin, then the inclusive prefix
  uint32_t dcnt[FTPB];   // per thread: where a lane without a candidate adds its count
  uint32_t rcnt[256];    // per chunk: its candidates
  float v[FTPB / WAVE], g[FTPB / WAVE];
  int i[FTPB / WAVE], f[FTPB / WAVE];
  double d[FTPB / WAVE];
  uint64_t u[FTPB / WAVE];
  int misc[8];
  uint64_t res[8];       // wave 0's decisions, for the other waves
};
static_assert(FCAP >= XB && FCAP >= XCOL, "the exact path reuses the candidate keys");
static_assert(GZCAP == 1024, "zone index: the low 10 bits of a zone key");

// Fixed-point mass of a token: round(2^50 * exp(l - m)), from the float exp of the
// float difference (l <= m).
__device__ __forceinline__ uint64_t gmass(float l, float m) {
  return (uint64_t)(expf(l - m) * 1125899906842624.0f);
}
// A zone key: the order key with the id moved up by 10 bits and the zone index below it
// (ids < 2^22), so sorting zone keys orders the tokens and keeps each one's index.
__device__ __forceinline__ uint64_t zkey(uint64_t k, int idx) {
  return (k & 0xFFFFFFFF00000000ull) | ((k & 0x3FFFFFull) << 10) | (uint64_t)idx;
}
__device__ __forceinline__ uint64_t zkey_key(uint64_t z) {
  return (z & 0xFFFFFFFF00000000ull) | ((z >> 10) & 0x3FFFFFull);
}
__device__ __forceinline__ int gbin256(float m, float l, float hscale) {
  return (int)fminf((m - l) * hscale, 255.0f);
}
__device__ __forceinline__ float key_l(uint64_t k) { return fkey_desc_inv((uint32_t)(k >> 32)); }

// Result of a search: the key found (~0: none), the prefix count and mass of the keys
// before it and its own mass.
struct GHit {
  uint64_t key, cnt_before, mass_before, mass;
};

// Wave 0 only: the first candidate in key order with key <= bound and id != excl whose
// inclusive cumulative count (mass == false) or mass exceeds thr. hist / hmass hold the
// inclusive bin prefixes of all candidates; excl_w and excl_b are the excluded key's mass
// and bin when it is a candidate (0 and 256 otherwise). False when the bin to scan holds
// more than GZCAP keys.
__device__ __forceinline__ bool gsearch(GFinalShared& S, float m, float hscale, bool mass,
                                        double thr, uint64_t bound, int excl, uint64_t excl_w,
                                        int excl_b, GHit& hit) {
  const int lane = threadIdx.x & (WAVE - 1);
  // (memory accesses are kept out of branches throughout: a load inside a branch is
  // waited for at the branch's end, which would serialise them)
  auto cumv = [&](int bq) -> uint64_t {  // uniform bq
    if (bq < 0) return 0ull;
    if (!mass) return (uint64_t)S.hist[bq];
    return S.hmass[bq] - (bq >= excl_b ? excl_w : 0ull);
  };
  const int bb = bound == ~0ull ? 255 : gbin256(m, key_l(bound), hscale);
  // the first bin below the bound's whose prefix exceeds thr, else the bound's bin
  uint64_t c4[4];
#pragma unroll
  for (int q = 0; q < 4; ++q)
    c4[q] = mass ? S.hmass[4 * lane + q] : (uint64_t)S.hist[4 * lane + q];
  int bz = 256;
#pragma unroll
  for (int q = 3; q >= 0; --q) {
    const int bq = 4 * lane + q;
    const uint64_t v = c4[q] - ((mass && bq >= excl_b) ? excl_w : 0ull);
    bz = ((bq < bb) & ((double)v > thr)) ? bq : bz;
  }
  bz = wave_min_i(bz);
  if (bz > bb) bz = bb;
  const uint32_t z0 = bz > 0 ? S.hist[bz - 1] : 0u, z1 = S.hist[bz];
  const int nz = (int)(z1 - z0);
  if (nz > GZCAP) return false;
  for (int i = lane; i < nz; i += WAVE) {
    S.zone[i] = zkey(S.bkey[z0 + i], i);
    S.zmass[i] = S.bmass[z0 + i];
  }
  wave_sync();
  if (nz <= WAVE) wave_rank_sort(S.zone, nz);
  else wave_sort_lds(S.zone, nz);
  // scan in order: a pass of 64 lanes x 4 keys at a time, each key counting 1 or its
  // mass unless it lies past the bound or is the excluded one
  uint64_t run = mass ? cumv(bz - 1) : (uint64_t)z0;
  hit.key = ~0ull;
  for (int p0 = 0; p0 < nz; p0 += 4 * WAVE) {
    uint64_t val[4], own = 0ull;
    uint64_t zz[4], zm[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) zz[q] = S.zone[min(p0 + 4 * lane + q, GZCAP - 1)];
#pragma unroll
    for (int q = 0; q < 4; ++q) zm[q] = S.zmass[zz[q] & 1023u];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint64_t k = zkey_key(zz[q]);
      const bool in = (p0 + 4 * lane + q < nz) & (k <= bound) & ((int)(uint32_t)k != excl);
      val[q] = in ? (mass ? zm[q] : 1ull) : 0ull;
      own += val[q];
    }
    const uint64_t incl = wave_incl_scan_u64(own);
    uint64_t r0 = run + incl - own;
    int fq = 4;
    uint64_t fb = 0ull;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (fq == 4 && val[q] > 0ull && (double)(r0 + val[q]) > thr) {
        fq = q;
        fb = r0;
      }
      r0 += val[q];
    }
    const uint64_t hitm = __ballot(fq < 4);
    if (hitm) {
      const int fl = (int)__ffsll((long long)hitm) - 1;
      const int i = p0 + 4 * fl + rl_i(fq, fl);
      const uint64_t z = S.zone[i];
      hit.key = zkey_key(z);
      hit.cnt_before = (uint64_t)z0 + (uint64_t)i;
      hit.mass_before = rl_u64(fb, fl);
      hit.mass = mass ? S.zmass[z & 1023u] : 1ull;
      break;
    }
    run += rl_u64(incl, WAVE - 1);
  }
  return true;
}

// The mass of the candidates with key <= bound (wave 0 only): the bins before the
// bound's, plus that bin's keys up to the bound.
__device__ __forceinline__ uint64_t gmass_upto(GFinalShared& S, float m, float hscale,
                                               uint64_t bound) {
  const int lane = threadIdx.x & (WAVE - 1);
  const int bb = gbin256(m, key_l(bound), hscale);
  const uint32_t z0 = bb > 0 ? S.hist[bb - 1] : 0u, z1 = S.hist[bb];
  uint64_t loc = 0ull;
  for (uint32_t i = z0 + (uint32_t)lane; i < z1; i += WAVE)
    if (S.bkey[i] <= bound) loc += S.bmass[i];
  return (bb > 0 ? S.hmass[bb - 1] : 0ull) + wave_sum_u64(loc);
}

__global__ __launch_bounds__(FTPB) void k_gfinal(Args a) {
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
  RowState* rsp = &a.s.rs[r];
  const bool gum = a.noise && a.noise_mode != STRIM_NOISE_ICDF;
  const float* nz = a.noise ? a.noise + (int64_t)r * a.noise_stride : (const float*)rsp;
  const float n0 = nz[gum ? V : 0], n1 = nz[gum ? V : 1];
  const bool vdr = a.verify && j < a.k;
  const int32_t* dp = vdr ? a.drafts + (int64_t)b * a.k + j : (const int32_t*)rsp;
  const int d_raw = *dp;
  const float ld_raw = rsp->l_draft;
  const int ne = W * GCAP;  // candidate slots of the row (<= FTPB * GNE)
  const Cand* slots = a.s.slot + (int64_t)r * a.s.wmax * SLOT;
  Cand cd[GNE];
#pragma unroll
  for (int q = 0; q < GNE; ++q) {
    const int e = q * FTPB + t;
    cd[q] = slots[e < ne ? (int64_t)(e >> 7) * SLOT + (e & (GCAP - 1)) : 0];
  }
  const RowParams p = load_params(a, b, j);
  if (!gfinal_row(a.p[b], V, a.noise_mode, a.dlog != nullptr && vdr)) return;
  const int draft = vdr ? d_raw : -1;
  const float l_draft = vdr ? ld_raw : -INFINITY;

  // ---- the chunk statistics ------------------------------------------------------
  const bool own = t < W;
  int ff = own ? (cs.flags | (cs.n > 0 ? 4 : 0)) : 0;
  float mv = own ? cs.m : -INFINITY, gv = own ? cs.g : -INFINITY;
  int mi = own ? cs.arg : -1;
  if (own) S.rcnt[t] = cs.ncand;
  const double wS = (own && cs.n > 0) ? cs.S : 0.0;
  const float wm = own ? cs.m : 0.0f;
  wave_argmax(mv, mi);
  ff = wave_or_i(ff);
  gv = wave_max_f(gv);
  if (lane == 0) {
    S.v[w] = mv;
    S.i[w] = mi;
    S.f[w] = ff;
    S.g[w] = gv;
  }
  for (int q = t; q < 256; q += FTPB) {
    S.hist[q] = 0u;
    S.hmass[q] = 0ull;
  }
  __syncthreads();
  float m = S.v[0], G = S.g[0];
  int arg = S.i[0], flags = S.f[0];
#pragma unroll
  for (int q = 1; q < FTPB / WAVE; ++q) {
    argmax_merge(m, arg, S.v[q], S.i[q]);
    flags |= S.f[q];
    G = fmaxf(G, S.g[q]);
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
  // (a lambda so that every "not above G" exit leads to the one exact-resolution call;
  // its conditions are uniform over the workgroup)
  auto decide = [&]() -> bool {
    const bool topk = p.top_k > 0 && p.top_k < V;
    const bool topp = p.top_p < 1.0f;
    const bool minp = p.min_p > 0.0f;
    const bool icdf = a.noise_mode == STRIM_NOISE_ICDF;
    // rank-indexed noise needs every kept token's rank
    if ((p.flags & STRIM_FLAG_NOISE_BY_RANK) && topp && !icdf) return false;
    if (ne > FTPB * GNE) return false;
    const bool all_in = !(G > -INFINITY);  // every allowed token is a candidate
    // min-p keeps a set that lies above G only if G itself fails it
    if (minp && !all_in && ((double)G - (double)m) >= p.lmp) return false;
    const float span = all_in ? 64.0f : fminf(fmaxf(m - G, 1.0f / 64.0f), 64.0f);
    const float hscale = 256.0f / span;
    // which of this thread's slots hold a candidate: entry e = q FTPB + t lies in region
    // 2 q + (t >> 7) (FTPB = 2 GCAP), at offset t & 127
    static_assert(FTPB == 2 * GCAP, "two regions per pass of the workgroup");
    uint32_t vmask = 0u;
    {
      uint32_t rc[GNE];
#pragma unroll
      for (int q = 0; q < GNE; ++q) rc[q] = S.rcnt[min(2 * q + (t >> 7), 255)];
#pragma unroll
      for (int q = 0; q < GNE; ++q)
        vmask |= ((q * FTPB + t < ne) & ((uint32_t)(t & (GCAP - 1)) < rc[q]) ? 1u : 0u) << q;
    }
    // bin every candidate above G (passing min-p); its count atomic returns its place in
    // the bin. No branch around the atomics: a lane without a candidate adds to its own
    // slot.
    // (a wave skips the slots where none of its lanes has a candidate: LDS atomics are
    // this step's cost)
    uint32_t place[GNE];
#pragma unroll
    for (int q = 0; q < GNE; ++q) {
      const float l = cd[q].l;
      const bool k = ((vmask >> q) & 1u) & (l > G) & (l > -INFINITY) &
                     (!minp | (((double)l - (double)m) >= p.lmp));
      place[q] = 0xFFFFFFFFu;
      if (__ballot(k)) {
        const int bn = k ? gbin256(m, l, hscale) : 0;
        const uint64_t cm = k ? gmass(l, m) : 0ull;
        const uint32_t o = atomicAdd(k ? &S.hist[bn] : &S.dcnt[t], 1u);
        atomicAdd(k ? &S.hmass[bn] : &S.dmass[t], (unsigned long long)cm);
        place[q] = k ? (((uint32_t)bn << 24) | o) : 0xFFFFFFFFu;
      }
    }
    // the whole row's mass from the chunk sums (used while the kept set reaches below
    // G), folded with the barrier the histogram needs
    const double S_all = block_sum_f64<FTPB>(wS * exp((double)wm - (double)m), S.d);
    // inclusive bin prefixes (wave 0; a lane owns bins 4 lane .. 4 lane + 3), the counts'
    // exclusive prefix kept for the scatter
    if (w == 0) {
      uint32_t c4[4], cs4 = 0u;
      uint64_t m4[4], ms4 = 0ull;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        c4[q] = S.hist[4 * lane + q];
        m4[q] = S.hmass[4 * lane + q];
        cs4 += c4[q];
        ms4 += m4[q];
      }
      uint32_t rc = wave_incl_scan_u32(cs4) - cs4;
      uint64_t rm = wave_incl_scan_u64(ms4) - ms4;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        rc += c4[q];
        rm += m4[q];
        S.hist[4 * lane + q] = rc;
        S.hmass[4 * lane + q] = rm;
      }
    }
    __syncthreads();
    // scatter into bin order (bin bn starts at hist[bn - 1]); a lane without a candidate
    // writes to its own slot
    uint32_t start[GNE];
#pragma unroll
    for (int q = 0; q < GNE; ++q) {
      const int bn = (int)(place[q] >> 24);
      start[q] = S.hist[bn > 0 && bn < 256 ? bn - 1 : 0];
    }
#pragma unroll
    for (int q = 0; q < GNE; ++q) {
      const bool k = place[q] != 0xFFFFFFFFu;
      if (__ballot(k)) {
        const int bn = (int)(place[q] >> 24);
        const uint32_t o = (bn > 0 ? start[q] : 0u) + (place[q] & 0xFFFFFFu);
        uint64_t* kd = k ? &S.bkey[o] : &S.dmass[t];
        uint64_t* md = k ? &S.bmass[o] : &S.dmass[t];
        *kd = ckey(cd[q].l, cd[q].id);
        *md = k ? gmass(cd[q].l, m) : 0ull;
      }
    }
    __syncthreads();
    const uint32_t n_all = S.hist[255];
    const uint64_t m_all = S.hmass[255];
    if (n_all == 0u) return false;

    // ---- wave 0: the k-th token, the top-p cut and the icdf draw ----------------
    // res: [0] ok, [1] bound1 (last kept key), [2] S1 (kept mass), [3] token (icdf),
    // [4] the draft's mass when kept
    if (w == 0) {
      uint64_t ok = 1ull, bound0 = ~0ull, bound1 = ~0ull, S0 = 0ull, S1 = 0ull, wd = 0ull;
      int token = -1;
      GHit hit;
      bool known0 = all_in || minp;  // every token of the set is a candidate
      do {
        // top-k (after min-p)
        if (topk) {
          if (n_all >= (uint32_t)p.top_k) {
            if (!gsearch(S, m, hscale, false, (double)(p.top_k - 1), ~0ull, -1, 0ull, 256, hit)) {
              ok = 0ull;
              break;
            }
            bound0 = (p.flags & STRIM_FLAG_TOPK_KEEP_TIES) ? (hit.key | 0xFFFFFFFFull) : hit.key;
            known0 = true;
          } else if (!all_in) {
            ok = 0ull;  // the k-th token lies at or below G
            break;
          }
        }
        // the kept mass before top-p: candidates up to bound0, or the chunk sums
        if (!known0) S0 = (uint64_t)__double2ull_rn(S_all * GFIX);
        else if (bound0 == ~0ull) S0 = m_all;
        else S0 = gmass_upto(S, m, hscale, bound0);
        // top-p: the last kept token is the first whose inclusive mass exceeds P S0 (a
        // token is dropped iff the mass before it exceeds P, SpecSampling.swift:62-66)
        bound1 = bound0;
        S1 = S0;
        bool known1 = known0;
        if (topp) {
          if (!gsearch(S, m, hscale, true, (double)p.top_p * (double)S0, bound0, -1, 0ull, 256,
                       hit)) {
            ok = 0ull;
            break;
          }
          if (hit.key != ~0ull) {
            bound1 = hit.key;
            S1 = hit.mass_before + hit.mass;
            known1 = true;
          } else if (!known0) {
            ok = 0ull;  // the cut lies at or below G
            break;
          }
        }
        if (!icdf && !known1) {
          ok = 0ull;
          break;
        }
        // the draft of a verify row
        int db = 256;
        if (vdr && l_draft > -INFINITY && ckey(l_draft, draft) <= bound1) {
          wd = gmass(l_draft, m);
          if (l_draft > G && (!minp || ((double)l_draft - (double)m) >= p.lmp))
            db = gbin256(m, l_draft, hscale);
        }
        if (icdf) {
          const double thr = (double)u_draw * (double)(S1 - wd);
          if (!gsearch(S, m, hscale, true, thr, bound1, vdr ? draft : -1, db < 256 ? wd : 0ull,
                       db, hit)) {
            ok = 0ull;
            break;
          }
          if (hit.key != ~0ull) token = (int)(uint32_t)hit.key;
          else if (!known1) { ok = 0ull; break; }  // the draw lies at or below G
          else token = arg;                        // only the draft kept: the first kept
        }
      } while (false);
      if (lane == 0) {
        S.res[0] = ok;
        S.res[1] = bound1;
        S.res[2] = S1;
        S.res[3] = (uint64_t)(int64_t)token;
        S.res[4] = wd;
      }
    }
    __syncthreads();
    if (S.res[0] == 0ull) return false;
    const uint64_t bound1 = S.res[1], S1 = S.res[2], wd = S.res[4];
    int token = (int)(int64_t)S.res[3];
    if (!icdf) {
      // Gumbel: every kept candidate (key <= bound1, not the draft) scored on all waves
      const bool no_lse = (p.flags & STRIM_FLAG_SCORE_NO_LSE) != 0;
      const bool cand_sorted = no_lse ? topp : (topk || topp);
      const int excl = vdr ? draft : -1;
      const double lse = log((double)S1 / GFIX);
      double bsc = -INFINITY;
      uint64_t btk = ~0ull;
      int bid = -1;
      for (uint32_t i = t; i < n_all; i += FTPB) {
        const uint64_t k = S.bkey[i];
        const int id = (int)(uint32_t)k;
        if (k > bound1 || id == excl) continue;
        const float l = key_l(k);
        const float u = a.noise ? a.noise[(int64_t)r * a.noise_stride + id]
                                : philox_uniform(pkey, (uint64_t)id);
        const double base = no_lse ? (double)l : ((double)l - (double)m) - lse;
        const double sc = base + gumbel64(u);
        const uint64_t tk = cand_sorted ? k : (uint64_t)id;
        if (bid < 0 || sc > bsc || (sc == bsc && tk < btk)) { bsc = sc; btk = tk; bid = id; }
      }
      block_argmax_score<FTPB>(bsc, btk, bid, S.d, S.u, S.i, &S.misc[3]);
      token = S.misc[3];
      if (token < 0) token = arg;  // only the draft kept
    }
    const int acc = vdr && ((double)u_acc < (double)wd / (double)S1) ? 1 : 0;
    finish(STRIM_OK, token, acc, (double)S1 / GFIX, bound1);
    return true;
  };
  if (decide()) return;

  // ---- a decision at or below G: the exact streaming resolution --------------------
  XScratch xs;
  xs.key = S.bkey;
  xs.hc = S.xhc;
  xs.cnt = S.xcnt;
  xs.u2 = S.xu2;
  xs.dred = S.d;
  xs.ured = S.u;
  xs.ired = S.i;
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
  const XOut xo = exact_row<FTPB>(xa, r, b, j, p, m, arg, draft, vdr, l_draft, xs, S.x);
  finish(xo.status, xo.token, xo.accept, xo.sig, xo.last_key);
}

}  // namespace strim
