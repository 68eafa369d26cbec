// stream.hpp — k_stream: the single streaming pass over the logits.
//
// A workgroup owns one (row, chunk of 4096 tokens): 512 threads with one 8-token segment
// each for small batches, 128 threads with four segments each for large ones; every
// wave-wide load is 1 KB (bf16) of contiguous logits. All global loads of a workgroup
// (logits, allow-bits, history ids) are issued before its first barrier. The workgroup
// writes its chunk statistics and its candidates: (v, id) above a bound for fast rows,
// the tokens of the chunk's first coarse bins as (l, id) for general rows. k_finalize
// (finalize_kernels.hip) then decides the greedy, fast and unfiltered Gumbel rows,
// k_gfinal (gfinal_kernels.hip) the general rows.
//
// The kernel is a template over the logits dtype, 16-byte alignment, penalties and the
// allow-mask, so each launch runs straight-line per-token code, and over the segments
// per thread (workgroup size). stream_kernels.hip is built once per (dtype, penalties,
// segments) triple, each object holding that triple's launcher.
#pragma once

#include "qprep.hpp"

namespace strim {

// threads of a k_stream workgroup with SSEG 8-token segments per thread
template <int SSEG>
constexpr int stpb() { return CHUNK / (EPT * SSEG); }

// LDS of one k_stream workgroup of NW waves (the history table only in the penalties
// variants and the lattice histogram only in the variants with general rows, so the
// narrow workgroups of large launches fit many to a CU).
template <int PEN, int NW, bool GEN>
struct StreamShared {
  // history counts of the chunk's tokens: 32 bits each (16 KB), or 16 bits (8 KB) when
  // the host knows no count reaches 65,536
  uint32_t cnt[PEN == 1 ? CHUNK : PEN == 2 ? CHUNK / 2 : 4];
  // general rows: the window's lattice bins (count << LCSH | mass), then each bin's
  // exclusive count prefix (its first entry in the chunk's slot region)
  unsigned long long lat[GEN ? NBW : 1];
  uint32_t lpre[GEN ? NBW : 1];
  uint32_t lad[2 * WAVE];
  float v[SMAXW];
  int i[SMAXW], n[SMAXW], f[SMAXW];
  uint32_t off[SMAXW], off2[SMAXW];
  double d[SMAXW];
  float tf[5 * SMAXW];
  int ti[2 * SMAXW];
  float wov[SMAXW];  // unfiltered Gumbel rows: a near-tie wave's largest own third score
  int near_n;        // unfiltered Gumbel rows: near-tie candidates written
};

// ---------------------------------------------------------------------------------
// k_stream
// ---------------------------------------------------------------------------------
// Ladder rung of dv = vmax - v >= 0 read from the float's bits: exponent and the top
// three mantissa bits, so consecutive rungs differ by 2^(1/8) in dv. Rung 0 holds
// dv < 2^-10, the last rung everything from 2^5.875 on. Monotone in dv.
constexpr int VRUNG = 128;
constexpr uint32_t VRUNG0 = (127u - 10u) << 3;
__device__ __forceinline__ int dv_rung(float dv) {
  const int r = (int)(__float_as_uint(dv) >> 20) - (int)VRUNG0;
  return r < 0 ? 0 : (r > VRUNG - 1 ? VRUNG - 1 : r);
}
// Smallest dv above rung r (r < VRUNG - 1).
__device__ __forceinline__ float dv_rung_end(int r) {
  return __uint_as_float(((uint32_t)r + 1u + VRUNG0) << 20);
}

// The raw values of this thread's SSEG 8-token segments as float32 (bf16 widens
// exactly). Every load is issued with no control flow between them: a divergent branch
// around a load makes the compiler wait for the load at the join, which would serialise
// the memory round trips. Aligned full chunks take 16-byte loads; otherwise each token
// is loaded from a clamped index and out-of-row tokens become -inf.
// The launch fields k_stream's first loads need, from its preloaded leading arguments
// (the same values as the argument block's): with them in SGPRs at wave start, the
// history, mask and logits loads are issued before any wait for the argument block.
struct StreamPre {
  const void* logits;
  int64_t row_stride;
  const int32_t* hist;
  const uint32_t* mask;
  int64_t mask_stride;
  int H, V, W, R, xmap;
};
// their packed flags (host): xmap | verify << 1 | wide strides << 2 | k << 3 (strides past
// 32 bits are read from the argument block)
inline bool pre_wide(const Args& a) {
  return a.row_stride > INT32_MAX || a.mask_stride > INT32_MAX;
}
inline int pre_bits(const Args& a) {
  return a.xmap | (a.verify << 1) | (pre_wide(a) ? 4 : 0) | (a.k << 3);
}

template <int DT, bool VEC, int SSEG, typename A>
__device__ __forceinline__ void load_chunk(const A& a, int r, const int (&i0)[SSEG], bool full,
                                           float (&x)[SSEG][EPT]) {
  const int64_t base = (int64_t)r * a.row_stride;
  if constexpr (DT == STRIM_DTYPE_BF16) {
    const uint16_t* xb = (const uint16_t*)a.logits + base;
    if (VEC && full) {
      uint4 q[SSEG];
#pragma unroll
      for (int s = 0; s < SSEG; ++s) q[s] = *(const uint4*)(xb + i0[s]);
#pragma unroll
      for (int s = 0; s < SSEG; ++s) {
        const uint32_t w[4] = {q[s].x, q[s].y, q[s].z, q[s].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          x[s][2 * e] = __uint_as_float(w[e] << 16);
          x[s][2 * e + 1] = __uint_as_float(w[e] & 0xFFFF0000u);
        }
      }
    } else {
      uint16_t h[SSEG][EPT];
#pragma unroll
      for (int s = 0; s < SSEG; ++s)
#pragma unroll
        for (int e = 0; e < EPT; ++e) h[s][e] = xb[i0[s] + e < a.V ? i0[s] + e : 0];
#pragma unroll
      for (int s = 0; s < SSEG; ++s)
#pragma unroll
        for (int e = 0; e < EPT; ++e)
          x[s][e] = i0[s] + e < a.V ? bf16_to_f32(h[s][e]) : -INFINITY;
    }
  } else {
    const float* xf = (const float*)a.logits + base;
    if (VEC && full) {
      float4 q[SSEG][2];
#pragma unroll
      for (int s = 0; s < SSEG; ++s) {
        q[s][0] = *(const float4*)(xf + i0[s]);
        q[s][1] = *(const float4*)(xf + i0[s] + 4);
      }
#pragma unroll
      for (int s = 0; s < SSEG; ++s) {
        x[s][0] = q[s][0].x; x[s][1] = q[s][0].y; x[s][2] = q[s][0].z; x[s][3] = q[s][0].w;
        x[s][4] = q[s][1].x; x[s][5] = q[s][1].y; x[s][6] = q[s][1].z; x[s][7] = q[s][1].w;
      }
    } else {
      float h[SSEG][EPT];
#pragma unroll
      for (int s = 0; s < SSEG; ++s)
#pragma unroll
        for (int e = 0; e < EPT; ++e) h[s][e] = xf[i0[s] + e < a.V ? i0[s] + e : 0];
#pragma unroll
      for (int s = 0; s < SSEG; ++s)
#pragma unroll
        for (int e = 0; e < EPT; ++e) x[s][e] = i0[s] + e < a.V ? h[s][e] : -INFINITY;
    }
  }
}

// DT: logits dtype; VEC: rows are 16-byte aligned; PEN: some row of the launch has
// penalties (1: 32-bit history counts, 2: 16-bit counts, for histories shorter than
// 65,536 ids with the draft prefix); MASK: allow-bits are given; GEN: some row of the
// launch is general (without it the general rows' code is left out, which at SSEG = 4
// halves the registers: 60 against 115 VGPRs, no SGPR spills). The host picks the
// instantiation, so each launch runs straight-line per-token code.
//
// Wave w owns the 1024 tokens [c0 + 1024 w, +1024) of the chunk; lane l holds the two
// 8-token segments at +8 l and +512 + 8 l, so each wave-wide load is 1 KB contiguous
// and the first maximum of the chunk lies in the lowest wave that holds the maximum.
// The chunk statistics are written without a closing barrier (see ChunkStat).
// The leading arguments repeat fields of `a` (StreamPre with 32-bit strides, and the flags
// of pre_bits); built with kernel-argument preloading, the 13 dwords arrive in SGPRs.
template <int DT, bool VEC, int PEN, bool MASK, int SSEG, bool GEN>
__global__ __launch_bounds__(stpb<SSEG>()) void k_stream(const void* pre_logits, int pre_rs,
                                                         const int32_t* pre_hist,
                                                         const uint32_t* pre_mask, int pre_ms,
                                                         int pre_H, int pre_V, int pre_W,
                                                         int pre_R, int pre_f, Args a) {
  constexpr int STPB = stpb<SSEG>();       // threads
  constexpr int NW = STPB / WAVE;          // waves
  __shared__ StreamShared<PEN, NW, GEN> S;
  const bool wide = (pre_f & 4) != 0;
  const StreamPre P{pre_logits, wide ? a.row_stride : (int64_t)pre_rs, pre_hist, pre_mask,
                    wide ? a.mask_stride : (int64_t)pre_ms, pre_H, pre_V, pre_W, pre_R,
                    pre_f & 1};
  // general-q verify: the workgroups past row R carry the draft distributions' work
  // (qprep.hpp), independent of the chunks'
  if (blockIdx.y >= (unsigned)P.R) {
    const int blk = (int)((blockIdx.y - (unsigned)P.R) * gridDim.x + blockIdx.x);
    if (blk < a.nqprep) qprep_block<STPB>(a, blk);
    return;
  }
  int r, c;
  map_block(P, r, c);
  int b = r, j = 0;  // (row_bj from the packed flags)
  if (pre_f & 2) {
    const int k1 = (pre_f >> 3) + 1;
    b = r / k1;
    j = r - b * k1;
  }
  const int t = threadIdx.x, lane = t & (WAVE - 1), w = wave_id();
  const int c0 = c * CHUNK;
  const bool full = VEC && c0 + CHUNK <= P.V;

  // history ids first: the counts are built while the logits are still in flight (the
  // ids are requested before the row's parameters are known, so no load waits for them)
  int hid[hpt<STPB>()];
  if constexpr (PEN != 0) hist_load<STPB>(P, b, hid);
  int i0[SSEG];
#pragma unroll
  for (int s = 0; s < SSEG; ++s)
    i0[s] = c0 + w * (SSEG * WAVE * EPT) + s * (WAVE * EPT) + lane * EPT;
  // allow-bits byte of each segment (a segment starts on a multiple of 8), from a
  // clamped index (tokens past the row end are -inf already); requested before the
  // logits so that unpacking the logits does not wait for it separately
  // (no branch around the loads: without a mask the unaligned variant reads a byte of
  // the logits instead and ignores it)
  uint32_t bits[SSEG];
#pragma unroll
  for (int s = 0; s < SSEG; ++s) bits[s] = 0xFFu;
  if constexpr (MASK) {
    const uint8_t* mb = P.mask ? (const uint8_t*)(P.mask + (int64_t)r * P.mask_stride)
                               : (const uint8_t*)P.logits;
#pragma unroll
    for (int s = 0; s < SSEG; ++s) bits[s] = mb[P.mask && i0[s] < P.V ? (i0[s] >> 3) : 0];
  }
  float v[SSEG][EPT];
  load_chunk<DT, VEC, SSEG>(P, r, i0, full, v);
  // the launch fields used next, read together: a field first read inside a branch would
  // be its own scalar-load round trip
  asm volatile("" ::"s"(a.verify), "s"(a.k), "s"(a.hist_len), "s"(a.s.cstat), "s"(a.s.wmax));
  ChunkStat* csp = &a.s.cstat[(int64_t)r * a.s.wmax + c];
  // the row's parameters only now: a scalar-load wait for them before this point would
  // also hold back the loads above
  const RowParams p = load_params(a, b, j);
  const bool pen = PEN != 0 && p.pen;
  const int hl = PEN != 0 ? hist_len(a, b) : 0;
  if constexpr (MASK) {
    if (!P.mask) {
#pragma unroll
      for (int s = 0; s < SSEG; ++s) bits[s] = 0xFFu;
    }
  }
  const bool fast = p.cls == CLS_FAST;
  const bool topk = p.top_k > 0 && p.top_k < a.V;
  if (fast && topk)
    for (int q = t; q < VRUNG; q += STPB) S.lad[q] = 0u;
  if (GEN && p.cls == CLS_GENERAL)
    for (int q = t; q < NBW; q += STPB) S.lat[q] = 0ull;
  if (pen) hist_count<STPB, CHUNK, Args, PEN == 2>(a, b, j, c0, hid, hl, S.cnt);

  // ---- penalties and mask, before temperature ("v space") ------------------------
  // Dividing by T > 0 is monotone, so maxima and candidate bounds are found on v; only
  // the chunk maximum and (in k_finalize) the candidates are divided. Tokens past the
  // row end load as -inf (not allowed).
  // The uniform tests (penalties at all, a repetition penalty of 1) are taken once, each
  // case a straight-line pass over the tokens: tested inside the unrolled token loop they
  // cost scalar branches and moves per token.
  auto seg_counts = [&](int s, uint32_t (&cnt)[EPT]) {
    if constexpr (PEN == 2) {
      const uint4 c4 = *(const uint4*)(S.cnt + ((i0[s] - c0) >> 1));
      const uint32_t cw[4] = {c4.x, c4.y, c4.z, c4.w};
#pragma unroll
      for (int e = 0; e < EPT; ++e) cnt[e] = (cw[e >> 1] >> ((e & 1) << 4)) & 0xFFFFu;
    } else {
      const uint4 c4a = *(const uint4*)(S.cnt + (i0[s] - c0));
      const uint4 c4b = *(const uint4*)(S.cnt + (i0[s] - c0) + 4);
      cnt[0] = c4a.x; cnt[1] = c4a.y; cnt[2] = c4a.z; cnt[3] = c4a.w;
      cnt[4] = c4b.x; cnt[5] = c4b.y; cnt[6] = c4b.z; cnt[7] = c4b.w;
    }
  };
  if constexpr (PEN != 0) {
    if (pen && p.rep == 1.0f) {
      // a repetition penalty of 1 is exact identity (x / 1 = x * 1 = x): branch-free
#pragma unroll
      for (int s = 0; s < SSEG; ++s) {
        uint32_t cnt[EPT];
        seg_counts(s, cnt);
#pragma unroll
        for (int e = 0; e < EPT; ++e) {
          float yp = v[s][e] - p.freq * (float)cnt[e];
          yp = yp - p.pres;
          v[s][e] = cnt[e] > 0u ? yp : v[s][e];
        }
      }
    } else if (pen) {
      // otherwise only tokens in the history divide
#pragma unroll
      for (int s = 0; s < SSEG; ++s) {
        uint32_t cnt[EPT];
        seg_counts(s, cnt);
#pragma unroll
        for (int e = 0; e < EPT; ++e) {
          float y = v[s][e];
          if (cnt[e] > 0u) {
            y = y > 0.0f ? y / p.rep : y * p.rep;
            y = y - p.freq * (float)cnt[e];
            y = y - p.pres;
          }
          v[s][e] = y;
        }
      }
    }
  }
  float vmax = -INFINITY;
#pragma unroll
  for (int s = 0; s < SSEG; ++s) {
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      float y = v[s][e];
      if constexpr (MASK) {
        // all ones where the token is allowed: y or -inf by a bit merge, no compare
        const uint32_t keep = (uint32_t)((int32_t)(bits[s] << (31 - e)) >> 31);
        y = __uint_as_float((__float_as_uint(y) & keep) | (0xFF800000u & ~keep));
      }
      v[s][e] = y;
      vmax = __builtin_elementwise_maximum(vmax, y);  // NaN-propagating
    }
  }
  // NaN or +inf in an allowed position (the maximum above keeps a NaN)
  const bool nf = !(vmax < INFINITY);
  if (a.verify && j < a.k) {
    const int d = a.drafts[(int64_t)b * a.k + j];
#pragma unroll
    for (int s = 0; s < SSEG; ++s) {
      const int o = d - i0[s];
      if (o >= 0 && o < EPT) {
        float ld = -INFINITY;
#pragma unroll
        for (int e = 0; e < EPT; ++e)
          if (e == o) ld = v[s][e];
        a.s.rs[r].l_draft = (ld > -INFINITY && !p.greedy) ? ld / p.T : ld;
      }
    }
  }
  if (c == 0 && t == 0) a.s.ncand[r] = 0u;
  if (t == 0) S.near_n = 0;  // (read after the barriers below)

  // ---- wave maxima ----------------------------------------------------------------
  const float wmv = wave_max_f(vmax);
  const int fw = __any(nf) ? 1 : 0;
  if (lane == 0) {
    S.v[w] = wmv;
    S.f[w] = fw;
  }
  __syncthreads();
  float vm = S.v[0];
  int f_w = S.f[0];
#pragma unroll
  for (int q = 1; q < NW; ++q) {
    vm = fmaxf(vm, S.v[q]);
    f_w |= S.f[q];
  }
  // the first maximum: the lowest wave holding it finds its first token and records it
  {
    int wfirst = -1;
#pragma unroll
    for (int q = NW - 1; q >= 0; --q)
      if (vm > -INFINITY && S.v[q] == vm) wfirst = q;
    if (w == (wfirst < 0 ? 0 : wfirst)) {
      int fid = 0x7FFFFFFF;
      if (wfirst >= 0) {
#pragma unroll
        for (int s = SSEG - 1; s >= 0; --s)
#pragma unroll
          for (int e = EPT - 1; e >= 0; --e)
            if (v[s][e] == vm) fid = i0[s] + e;
      }
      fid = wave_min_i(fid);
      if (lane == 0) csp->arg = wfirst < 0 ? -1 : fid;
    }
  }
  int n_w = vm > -INFINITY ? 1 : 0;  // "some token allowed"; general rows count below
  // chunk max after temperature; an overflow to +inf is a non-finite logit, one to -inf
  // leaves nothing allowed
  const float m_w = (p.greedy || !(vm > -INFINITY)) ? vm : vm / p.T;
  if (m_w == INFINITY) f_w = 1;
  if (!(m_w > -INFINITY)) n_w = 0;
  ChunkStat cs{m_w, n_w, f_w, -INFINITY, 0.0, -1, 0u, -INFINITY, 0u, 0u};
  uint32_t cs_ncand = 0u, cs_ncand2 = 0u;
  const bool live = n_w > 0 && !f_w;

  if (fast && live) {
    // Local candidates, in v space: every token that can pass min-p (on the row maximum
    // m >= m_w) and the chunk's top-k, written as (v, id) to the chunk's slot region.
    // A lower bound of -FLT_MAX keeps the -inf of disallowed tokens out in one compare.
    float vlo = p.min_p > 0.0f ? fmaxf(minp_vlo(m_w, p), -__FLT_MAX__) : -__FLT_MAX__;
    uint32_t sel[SSEG];  // bit e of sel[s]: token i0[s] + e is a candidate
    int wtot, wex;
    auto select = [&]() {
      int mycnt = 0;
#pragma unroll
      for (int s = 0; s < SSEG; ++s) {
        sel[s] = 0u;
#pragma unroll
        for (int e = 0; e < EPT; ++e) sel[s] |= (v[s][e] >= vlo ? 1u : 0u) << e;
        mycnt += __popc(sel[s]);
      }
      wex = wave_excl_count_bits<(SSEG == 1 ? 4 : SSEG == 2 ? 5 : SSEG == 4 ? 6 : 7)>(mycnt, &wtot);
    };
    // every wave publishes its count; a wave's candidates follow those of the waves
    // before it (the conditions below are uniform over the workgroup)
    int tot, before;
    auto place = [&]() {
      if (lane == 0) S.n[w] = wtot;
      __syncthreads();
      tot = 0;
      before = 0;
#pragma unroll
      for (int q = 0; q < NW; ++q) {
        before += q < w ? S.n[q] : 0;
        tot += S.n[q];
      }
    };
    select();
    place();
    // the ladder bounds the chunk's top-k when the min-p band alone holds more than 2k
    // tokens or overflows the region
    if (topk && (tot > SLOT || tot > max(2 * p.top_k, 128))) {
#pragma unroll
      for (int s = 0; s < SSEG; ++s)
#pragma unroll
        for (int e = 0; e < EPT; ++e)
          if ((sel[s] >> e) & 1u) atomicAdd(&S.lad[dv_rung(vm - v[s][e])], 1u);
      __syncthreads();  // (also orders every read of S.n above before its rewrite)
      // every wave finds the first rung whose cumulative count reaches k (lane owns
      // rungs 2 lane and 2 lane + 1)
      const uint32_t h0 = S.lad[2 * lane], h1 = S.lad[2 * lane + 1];
      const uint32_t cum = wave_incl_scan_u32(h0 + h1);
      const uint64_t reach = __ballot(cum >= (uint32_t)p.top_k);
      if (reach) {
        const int ln = (int)__ffsll((long long)reach) - 1;
        const uint32_t bef = (uint32_t)rl_i((int)(cum - h0 - h1), ln);
        const uint32_t hl0 = (uint32_t)rl_i((int)h0, ln);
        const int rstar = 2 * ln + (bef + hl0 >= (uint32_t)p.top_k ? 0 : 1);
        if (rstar < VRUNG - 1) {
          // v > vm - end(rstar) holds the rung; the margin (a few ulps of the values
          // involved) keeps tokens whose l = v / T ties with one inside it
          const float bnd = dv_rung_end(rstar);
          const float thr = vm - bnd;
          const float margin = (fabsf(vm) + fabsf(thr)) * 1e-6f + bnd * 1.6e-5f + 1e-30f;
          // the rungs up to rstar hold >= k tokens of the window, all with v >= g
          cs.g = thr - margin;
          if (cs.g > vlo) {
            vlo = cs.g;
            select();
          }
        }
      }
      place();
    }
    // a lane loops over its set bits only, so waves without candidates skip the writes
    if (tot <= SLOT) {
      Cand* dst = a.s.slot + ((int64_t)r * a.s.wmax + c) * SLOT + before;
      int pos = wex;
#pragma unroll
      for (int s = 0; s < SSEG; ++s) {
        uint32_t m = sel[s];
        while (m) {
          const int e = __builtin_ctz(m);
          m &= m - 1u;
          dst[pos++] = Cand{pick8(v[s], e), i0[s] + e};
        }
      }
    }
    cs_ncand = tot <= SLOT ? (uint32_t)tot : 0xFFFFFFFFu;
  } else if (GEN && p.cls == CLS_GENERAL && live) {
    // Chunk mass sum exp(l - m_w) and, for the rows k_gfinal decides, the chunk's lattice
    // histogram and its window tokens in bin order. The mass needs l to its float
    // rounding (a term's relative error is that of its exponent, which is |l| times the
    // rounding), so l is formed as v / T by one FMA correction of v * RN(1/T), correctly
    // rounded but for rare last-bit cases that move a term by an ulp of l; the
    // exponential is 2^((l - m_w) log2(e)), a sum of positive terms good to a few 1e-7
    // relative. A token's lattice bin A(l) = floor(l * LBS) needs the exact quotient (an
    // ulp off at a bin edge would put it in the neighbouring bin, out of order), which is
    // formed for the tokens near or inside the window only. General-q draft rows keep the
    // sum alone (the residual draw takes the row's mass from the chunks' sums and makes
    // its own passes, qres_kernels.hip), and unfiltered Gumbel rows are decided from the
    // chunks' two best tokens and the sum.
    const bool qdraft = a.dlog && a.verify && j < a.k;
    const bool gum_nf = !qdraft && a.noise_mode == STRIM_NOISE_GUMBEL && row_nofilter(p, a.V);
    const float yT = 1.0f / p.T;
    // the FMA quotient needs 1/T and its products far from the float range's ends
    const bool fq = p.T > 0x1p-100f && p.T < 0x1p+100f;
    // the window: lattice bins atop - NBW + 1 .. atop (every bin index an exact float)
    const float atop = floorf(m_w * (float)LBS);
    const bool latr = !qdraft && !gum_nf && fabsf(atop) < 0x1p+23f;
    const float lwin = (atop - (float)(NBW - 1)) * (1.0f / (float)LBS);
    // the FMA quotient is within an ulp of l: tokens whose quotient reaches this bound
    // get the exact one
    const float lwin_lo = lwin - (fabsf(lwin) * 1e-6f + 1e-30f);
    double ssum = 0.0;
    int na = 0;
    // window tokens: lb = atop - A(l) in [0, NBW), -1 otherwise; the fixed-point mass word
    int lbw[SSEG][EPT];
    uint64_t wword[SSEG][EPT];
#pragma unroll
    for (int s = 0; s < SSEG; ++s) {
      float es = 0.0f, eh = 0.0f;  // two float partial sums of four terms, each <= 1
#pragma unroll
      for (int e = 0; e < EPT; ++e) {
        const float ve = v[s][e];
        float le;
        if (fq) {
          const float q0 = ve * yT;
          le = __builtin_fmaf(__builtin_fmaf(-p.T, q0, ve), yT, q0);
        } else {
          le = ve / p.T;
        }
        // a NaN (from -inf, or l overflowing to -inf) gives the floor: a zero term
        const float ex = __builtin_amdgcn_exp2f(fmaxf((le - m_w) * 1.44269504f, -200.0f));
        if (e < EPT / 2) es += ex; else eh += ex;
        na += ve > -INFINITY ? 1 : 0;
        lbw[s][e] = -1;
        wword[s][e] = 0ull;
        if (latr && le >= lwin_lo && ve > -INFINITY) {
          const float l = ve / p.T;  // exact
          const float d = atop - floorf(l * (float)LBS);
          if (d < (float)NBW) {
            lbw[s][e] = (int)d;
            v[s][e] = l;  // the value written with the candidate
            // the term relative to its bin's base, exp(l - A(l) / LBS) in [1, e^(1/LBS)):
            // every chunk's bin at A has the same unit, so the chunks' bins add as
            // integers and are scaled to the row's maximum once per row bin
            const float lbase = (atop - d) * (1.0f / (float)LBS);
            const float ew = __builtin_amdgcn_exp2f((l - lbase) * 1.44269504f);
            wword[s][e] = (1ull << LCSH) | (uint64_t)(ew * 0x1p37f);
          }
        }
      }
      ssum += (double)es + (double)eh;
    }
    // the window tokens into the histogram; the atomic's old count is the token's place
    // in its bin (every atomic is issued before any result is read)
    uint32_t lrank[SSEG][EPT];
    if (latr) {
      uint64_t old[SSEG][EPT];
#pragma unroll
      for (int s = 0; s < SSEG; ++s)
#pragma unroll
        for (int e = 0; e < EPT; ++e)
          if (lbw[s][e] >= 0) old[s][e] = atomicAdd(&S.lat[lbw[s][e]], (unsigned long long)wword[s][e]);
#pragma unroll
      for (int s = 0; s < SSEG; ++s)
#pragma unroll
        for (int e = 0; e < EPT; ++e) asm volatile("" : "+v"(old[s][e]));
#pragma unroll
      for (int s = 0; s < SSEG; ++s)
#pragma unroll
        for (int e = 0; e < EPT; ++e) lrank[s][e] = (uint32_t)(old[s][e] >> LCSH);
    }
    // the sums of the waves, one barrier (the histogram's atomics are complete after it)
    ssum = wave_sum(ssum);
    na = wave_sum(na);
    if (lane == 0) {
      S.d[w] = ssum;
      S.n[w] = na;
    }
    __syncthreads();
    cs.S = 0.0;
    cs.n = 0;
#pragma unroll
    for (int q = 0; q < NW; ++q) {
      cs.S += S.d[q];
      cs.n += S.n[q];
    }
    if (latr) {
      // wave 0: the bins' exclusive count prefixes, the bins written whole (nfull: the
      // bins whose inclusive prefix stays within LCAP) and the last non-empty bin; the
      // lattice words (inclusive prefix << LCSH | mass) of bins 0 .. nb - 1 to scratch
      constexpr int LPL = NBW / WAVE;  // bins per lane
      static_assert(NBW % WAVE == 0, "whole bins per lane");
      if (w == 0) {
        uint64_t hw[LPL];
        uint32_t hc[LPL], tot = 0u;
#pragma unroll
        for (int q = 0; q < LPL; ++q) {
          hw[q] = S.lat[LPL * lane + q];
          hc[q] = (uint32_t)(hw[q] >> LCSH);
          tot += hc[q];
        }
        uint32_t run = wave_incl_scan_u32(tot) - tot;
        int nfull = 0, nbl = 0;
        unsigned long long* lw = a.s.lat + ((int64_t)r * a.s.wmax + c) * NBW;
#pragma unroll
        for (int q = 0; q < LPL; ++q) {
          const int bq = LPL * lane + q;
          S.lpre[bq] = run;
          run += hc[q];
          nfull += run <= (uint32_t)LCAP ? 1 : 0;
          nbl = hc[q] > 0u ? bq + 1 : nbl;
          hw[q] = ((uint64_t)run << LCSH) | (hw[q] & LMMASK);
        }
        nfull = wave_sum(nfull);
        nbl = wave_max_i(nbl);
#pragma unroll
        for (int q = 0; q < LPL; ++q)
          if (LPL * lane + q < nbl) lw[LPL * lane + q] = hw[q];
        if (lane == 0) {
          S.i[0] = nfull < nbl ? nfull : nbl;
          S.i[1] = nbl;
        }
      }
      __syncthreads();
      const int nfull = S.i[0];
      // the window tokens of bins 0 .. nfull - 1 as (l, id), at their bin's prefix plus
      // their place in it
      Cand* dst = a.s.slot + ((int64_t)r * a.s.wmax + c) * SLOT;
#pragma unroll
      for (int s = 0; s < SSEG; ++s)
#pragma unroll
        for (int e = 0; e < EPT; ++e)
          if (lbw[s][e] >= 0 && lbw[s][e] < nfull)
            dst[S.lpre[lbw[s][e]] + lrank[s][e]] = Cand{v[s][e], i0[s] + e};
      cs_ncand = (uint32_t)nfull;
      cs_ncand2 = (uint32_t)S.i[1];
    } else if (!qdraft && !gum_nf) {
      cs_ncand2 = LNONE;  // the lattice cannot hold the row: k_gfinal resolves it exactly
    }
    if (qdraft || !gum_nf) {
      // the sum alone (qdraft), or the lattice above
    } else {
      // the fp32 proxy scores take l to its float rounding (the FMA-corrected quotient);
      // the tokens the chunk keeps are divided exactly when they are written
      auto lq = [&](float ve) -> float {
        float le;
        if (fq) {
          const float q0 = ve * yT;
          le = __builtin_fmaf(__builtin_fmaf(-p.T, q0, ve), yT, q0);
        } else {
          le = ve / p.T;
        }
        return ve > -INFINITY ? le : -INFINITY;
      };
      const uint64_t key = mix64(p.seed, p.position);
      // the segment's 8 uniforms: two Philox blocks (a segment starts on a multiple of 8)
      auto uniforms = [&](int s, float* u) {
        if (a.noise) {
#pragma unroll
          for (int e = 0; e < EPT; ++e) {
            const int id = i0[s] + e < a.V ? i0[s] + e : 0;
            u[e] = a.noise[(int64_t)r * a.noise_stride + id];
          }
        } else {
#pragma unroll
          for (int hb = 0; hb < 2; ++hb) {
            const uint4 wb = philox_block(key, (uint64_t)((i0[s] >> 2) + hb));
            u[4 * hb] = u01(wb.x); u[4 * hb + 1] = u01(wb.y);
            u[4 * hb + 2] = u01(wb.z); u[4 * hb + 3] = u01(wb.w);
          }
        }
      };
      auto proxy = [&](float ve, float u) -> float {
        const float le = lq(ve);
        return le > -INFINITY ? le + gumbel32(u) : -INFINITY;
      };
      // each thread keeps its two best tokens (score, v, id)
      float s0 = -INFINITY, s1 = -INFINITY, s2 = -INFINITY, l0 = 0.f, l1 = 0.f;
      int id0 = -1, id1 = -1;
#pragma unroll
      for (int s = 0; s < SSEG; ++s) {
        float u[EPT];
        uniforms(s, u);
        // ids rise along the thread's tokens: a strict compare keeps the first of ties
#pragma unroll
        for (int e = 0; e < EPT; ++e) {
          const float sc = proxy(v[s][e], u[e]);
          const int id = i0[s] + e;
          if (sc > s0) {
            s1 = s0; l1 = l0; id1 = id0;
            s0 = sc; l0 = v[s][e]; id0 = id;
          } else if (sc > s1) {
            s1 = sc; l1 = v[s][e]; id1 = id;
          }
        }
      }
      // The fp64 decision rescores the tokens the chunk keeps; a token left out can win
      // only if its proxy score is within twice the proxy's error of a kept one. The error
      // is at most 2e-6 for the transform plus the float roundings of l (one ulp at worst)
      // and of l + g, below 1e-5 + 5e-7 |s| in all; tol(s) = 2e-5 + 1e-6 |s| is twice it.
      // Every token other than the chunk's two best whose score reaches s1 - tol(s1) (s1:
      // the chunk's second score) is kept as well, as one of the chunk's candidates (slot
      // entries 0 ..). Since the chunk's s1 is at least its wave's second score w1, such a
      // token reaches w1 - tol(w1) too: each wave whose third comes that close collects
      // its lanes' kept tokens above that bound (before the barrier, so nothing of a lane
      // stays live across it), and thread 0 adds the waves' own pairs. A lane's third
      // (a token it did not keep) reaching the chunk's bound sends the row to the exact
      // resolution (STRIM flag 8).
      auto tol = [](float x) { return 2e-5f + 1e-6f * fabsf(x); };
      // A lane's third is not tracked in the token loop: its second score stands in as
      // the bound. When one lane holds both of the wave's winners, that bound opens the
      // near-tie gate and the lanes' exact thirds are recomputed below, so w2 is always
      // at least the best score the wave leaves out.
      float w0 = s0, wl0 = l0, w1 = s1, wl1 = l1, w2 = s1;
      int wi0 = id0, wi1 = id1;
      wave_top2(w0, wl0, wi0, w1, wl1, wi1, &w2);
      float wov = -INFINITY;
      const float wthr = w1 - tol(w1);
      if (wi1 >= 0 && w2 >= wthr) {
        const bool n0 = id0 >= 0 && s0 >= wthr && id0 != wi0 && id0 != wi1;
        const bool n1 = id1 >= 0 && s1 >= wthr && id1 != wi0 && id1 != wi1;
        float t3 = -INFINITY;
#pragma unroll
        for (int s = 0; s < SSEG; ++s) {
          float u[EPT];
          uniforms(s, u);
#pragma unroll
          for (int e = 0; e < EPT; ++e) {
            const int id = i0[s] + e;
            if (id != id0 && id != id1) t3 = fmaxf(t3, proxy(v[s][e], u[e]));
          }
        }
        wov = wave_max_f(t3);
        const uint64_t b0 = __ballot(n0), b1 = __ballot(n1);
        int base = 0;
        if (lane == 0) base = atomicAdd(&S.near_n, __popcll(b0) + __popcll(b1));
        base = __builtin_amdgcn_readfirstlane(base);
        Cand* dst = a.s.slot + ((int64_t)r * a.s.wmax + c) * SLOT;
        const int p0 = base + lanes_below(b0), p1 = base + __popcll(b0) + lanes_below(b1);
        if (n0 && p0 < SLOT) dst[p0] = Cand{l0 / p.T, id0};
        if (n1 && p1 < SLOT) dst[p1] = Cand{l1 / p.T, id1};
      }
      // the block's two best and third: wave 0 over the waves' pairs
      constexpr int NWV = STPB / WAVE;
      if (lane == 0) {
        S.tf[4 * w + 0] = w0; S.tf[4 * w + 1] = wl0; S.tf[4 * w + 2] = w1; S.tf[4 * w + 3] = wl1;
        S.tf[4 * NWV + w] = w2;
        S.ti[2 * w + 0] = wi0; S.ti[2 * w + 1] = wi1;
        S.wov[w] = wov;
      }
      __syncthreads();
      if (w == 0) {
        const bool own = lane < NWV;
        const int q = own ? lane : 0;
        s0 = S.tf[4 * q]; l0 = S.tf[4 * q + 1]; s1 = S.tf[4 * q + 2]; l1 = S.tf[4 * q + 3];
        s2 = own ? S.tf[4 * NWV + q] : -INFINITY;
        id0 = own ? S.ti[2 * q] : -1;
        id1 = own ? S.ti[2 * q + 1] : -1;
        wave_top2(s0, l0, id0, s1, l1, id1, &s2);
      }
      if (t == 0) {
        const float thr = s1 - tol(s1);
        if (id1 >= 0 && s2 >= thr) {
          Cand* dst = a.s.slot + ((int64_t)r * a.s.wmax + c) * SLOT;
          int n = S.near_n;
          bool over = false;
#pragma unroll 1
          for (int q = 0; q < NWV; ++q) {
            over = over || S.wov[q] >= thr;
            for (int h = 0; h < 2; ++h) {
              const float sc = S.tf[4 * q + 2 * h];
              const int id = S.ti[2 * q + h];
              if (id >= 0 && sc >= thr && id != id0 && id != id1) {
                if (n < SLOT) dst[n] = Cand{S.tf[4 * q + 2 * h + 1] / p.T, id};
                ++n;
              }
            }
          }
          if (over || n > SLOT) cs.flags |= 8;
          cs_ncand = (over || n > SLOT) ? 0u : (uint32_t)n;
        }
        ChunkPart& pt = a.s.part[(int64_t)r * a.s.wmax + c];
        pt.l0 = id0 >= 0 ? l0 / p.T : -INFINITY;
        pt.id0 = id0;
        pt.l1 = id1 >= 0 ? l1 / p.T : -INFINITY;
        pt.id1 = id1;
      }
    }
  }
  if (t == 0) {
    *(float4*)csp = make_float4(cs.m, __int_as_float(cs.n), __int_as_float(cs.flags), cs.g);
    csp->S = cs.S;
    csp->ncand = cs_ncand;
    csp->g2 = cs.g2;
    csp->ncand2 = cs_ncand2;
  }
}

// Launches the k_stream variant of one (dtype, penalties, segments) triple that matches
// the call's alignment and mask. Defined in stream_kernels.hip, one object per triple;
// unaligned calls always take the penalties object.
template <int DT, int PEN, int SSEG>
hipError_t launch_stream_group(const Args& a, dim3 grid, hipStream_t st, hipEvent_t e0,
                               hipEvent_t e1);

}  // namespace strim
