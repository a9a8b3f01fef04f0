// Frozen-stats SDPA JVP for gfx950.
//
// Replaces the eager sdpa_jvp of the reference (theria/attention/triton_sdpa_backward.py:465-503),
// which materialises several (B,H,T,M) float32 tensors. Contract (docs/phase9.md:30-39): P is rebuilt
// from the saved row statistics and held fixed, and with tangents (tq, tk, tv)
//   G = scale (tq K^T + Q tk^T),  c_i = sum_j P_ij G_ij,
//   tO = P o (G - c) V + P tv = (P o G) V - c o O + P tv,
// where O = P V (the saved forward output, or rebuilt in the same pass when it is not supplied).
// The same kernel yields the G_dO output of the double backward (tangents = cotangents of dQ, dK, dV).
//
// 16-bit inputs: the two large terms (P o G) V and c o O of tO cancel, so operand rounding in them is
// amplified (a bfloat16-rounded P o G gave 0.03 absolute error on a row with four visible keys). Both
// products are therefore formed from two-term 16-bit splits (hi + lo) of P o G and of P, and O is always
// rebuilt in the pass from the same P (the saved O, rounded to 16 bits, is not used). The key-split kernel
// (jvp_ksplit_kernel, below) takes the split only in waves holding a row flagged peaked in lse: elsewhere the
// rounding of P o G and P spreads over many keys and one 16-bit term each suffices.
// p.normalize divides P by its own row sum (every dtype): the JVP of the exact softmax for an lse this
// library's forward wrote (a 16-bit forward's lse comes from rounded probabilities, so P rebuilt from it
// sums to 1 only within ~2^-9). Without it P = exp(S - lse) is held exactly as given, which is the
// reference's frozen-stats contract for caller-supplied (m, l).
//
// Work decomposition as in the forward: one workgroup = 4 waves = 128 query rows, lane per query in
// the transposed score tiles S^T = K Q^T and G^T = K tq^T + tk Q^T (Q and tq stay in registers as B
// operands); per 64-key tile, K, tk, V, tv are staged in LDS and the three output products
// (P o G) V, P tv and (if needed) P V accumulate lane-per-query as V^T (.)^T, with V^T / tv^T
// fragments from the LDS transpose read. A single pass: c_i is folded in at the end.
#include <initializer_list>
#include <type_traits>

#include "dispatch.hpp"
#include "sdpa_common.hpp"
#include "sdpa_lds.hpp"

namespace theria {

// DMA: 16-bit inputs with head dim exactly 64 or 128 and 16-byte-aligned rows. The K, tK, V, tV tiles are
// then filled by LDS DMA into two sets of unpadded, XOR-swizzled buffers (sdpa_lds.hpp), one barrier per
// tile with the next tile's copies in flight; otherwise they pass through registers into padded LDS rows.
template <typename T, int DP, bool CAUSAL, bool HAS_O, bool DMA>
__global__ __launch_bounds__(256) void jvp_kernel(const JvpParams p) {
  using MM = Mfma<T>;
  using F = typename MM::frag_t;
  constexpr int KC = MM::KC;
  constexpr int NW = 4, BM = 32 * NW, NT = 64 * NW;
  constexpr int BN = (DP == 128 || sizeof(T) == 4) ? 32 : 64;  // keys per tile (register budget)
  constexpr int PITCH = DP + 16 / (int)sizeof(T);
  constexpr int NDT = DP / 32, NKC = DP / KC, NPC = 32 / KC, NST = BN / 32;
  constexpr int TB = DMA ? BN * DP * 2 : BN * PITCH * (int)sizeof(T);  // bytes per tile
  constexpr int TB2 = DMA ? TB : 16;                                    // second set (DMA only)
  __shared__ __attribute__((aligned(1024))) char sK0[TB];
  __shared__ __attribute__((aligned(1024))) char sV0[TB];
  __shared__ __attribute__((aligned(1024))) char stK0[TB];
  __shared__ __attribute__((aligned(1024))) char stV0[TB];
  __shared__ __attribute__((aligned(1024))) char sK1[TB2];
  __shared__ __attribute__((aligned(1024))) char sV1[TB2];
  __shared__ __attribute__((aligned(1024))) char stK1[TB2];
  __shared__ __attribute__((aligned(1024))) char stV1[TB2];

  const Shape& s = p.s;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, li = lane & 31, g = lane >> 5;
  const int nqb = (s.T + BM - 1) / BM;
  const int bid = xcd_remap(blockIdx.x, gridDim.x);
  const int bh = bid / nqb;
  int qb = bid - bh * nqb;
  if (CAUSAL) qb = nqb - 1 - qb;
  const int b = bh / s.H, h = bh - b * s.H;
  const T* Q = (const T*)p.q.p + b * p.q.sb + h * p.q.sh;
  const T* K = (const T*)p.k.p + b * p.k.sb + h * p.k.sh;
  const T* V = (const T*)p.v.p + b * p.v.sb + h * p.v.sh;
  const bool has_tq = p.tq.p != nullptr, has_tk = p.tk.p != nullptr, has_tv = p.tv.p != nullptr;
  const T* TQ = has_tq ? (const T*)p.tq.p + b * p.tq.sb + h * p.tq.sh : nullptr;
  const T* TK = has_tk ? (const T*)p.tk.p + b * p.tk.sb + h * p.tk.sh : nullptr;
  const T* TV = has_tv ? (const T*)p.tv.p + b * p.tv.sb + h * p.tv.sh : nullptr;
  const int q0w = qb * BM + wave * 32;
  const int myq = q0w + li;
  const bool qvalid = myq < s.T;
  const int64_t row_id = (int64_t)bh * s.T + myq;

  F qf[NKC], tqf[NKC];
#pragma unroll
  for (int c = 0; c < NKC; ++c) {
    qf[c] = gload_frag<T>(Q, p.q.sr, myq, s.T, c, s.D, s.vec);
    tqf[c] = has_tq ? gload_frag<T>(TQ, p.tq.sr, myq, s.T, c, s.D, s.vec) : F{};
  }
  f32x16_t accA[NDT], accC[NDT], accO[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
    accA[dt] = zero16();
    accC[dt] = zero16();
    accO[dt] = zero16();
  }
  const float c2 = s.scale * kLog2e;
  const float lse2 = qvalid ? p.lse[row_id] * kLog2e : THERIA_INF;
  const float moff = lse2 == -THERIA_INF ? THERIA_INF : lse2;  // a row without visible keys has P = 0
  constexpr bool SPLIT = sizeof(T) == 2;     // hi/lo operands, renormalised P (see the header)
  constexpr bool REBUILD = SPLIT || !HAS_O;  // O = P V formed in this pass
  float cpart = 0.f, lpart = 0.f;

  int kend = s.M;
  if (CAUSAL) kend = min(s.M, qb * BM + BM);
  const int nkt = (kend + BN - 1) / BN;
  auto colsf = [&](const char* t, int row, int c) -> F {
    if constexpr (DMA)
      return swz_cols<T, DP>(t, row, c);
    else
      return lds_cols<T, KLIN>((const T*)t, PITCH, row, 0, c);
  };
  auto rowsf = [&](const char* t, int kbase, int c, int col0) -> F {
    if constexpr (DMA)
      return swz_rows<T, DP>(t, kbase, c, col0);
    else
      return lds_rows<T, KACC>((const T*)t, PITCH, kbase, c, col0);
  };

  // The key tile kt held in (tK, tV, ttK, ttV).
  auto compute = [&](int kt, const char* tK, const char* tV, const char* ttK, const char* ttV) {
    const int k0 = kt * BN;
    if (CAUSAL && k0 > q0w + 31) return;

    f32x16_t sc[NST], gm[NST];
#pragma unroll
    for (int t = 0; t < NST; ++t) {
      sc[t] = zero16();
      gm[t] = zero16();
#pragma unroll
      for (int c = 0; c < NKC; ++c) {
        const F kfr = colsf(tK, t * 32 + li, c);
        sc[t] = MM::mma(kfr, qf[c], sc[t]);
        if (has_tq) gm[t] = MM::mma(kfr, tqf[c], gm[t]);
        if (has_tk) gm[t] = MM::mma(colsf(ttK, t * 32 + li, c), qf[c], gm[t]);
      }
    }
    const bool need_mask = (k0 + BN > s.M) || (CAUSAL && k0 + BN - 1 > q0w);
#pragma unroll
    for (int t = 0; t < NST; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float pv = fast_exp2(fmaf(sc[t][r], c2, -moff));
        if (need_mask) {
          const int key = k0 + t * 32 + acc_row(r, g);
          if (key >= s.M || (CAUSAL && key > myq)) pv = 0.f;
        }
        sc[t][r] = pv;
        lpart += pv;
        const float pg = pv * gm[t][r];
        gm[t][r] = pg;
        cpart += pg;
      }
#pragma unroll
    for (int t = 0; t < NST; ++t)
#pragma unroll
      for (int cc = 0; cc < NPC; ++cc) {
        F pf, pgf, pf_lo{}, pgf_lo{};
        if constexpr (SPLIT) {
          split_frag<T>(sc[t], cc, pf, pf_lo);
          split_frag<T>(gm[t], cc, pgf, pgf_lo);
        } else {
          pf = acc_frag<T>(sc[t], cc);
          pgf = acc_frag<T>(gm[t], cc);
        }
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
          const F vfr = rowsf(tV, t * 32, cc, dt * 32);
          accA[dt] = MM::mma(vfr, pgf, accA[dt]);
          if (SPLIT) accA[dt] = MM::mma(vfr, pgf_lo, accA[dt]);
          if (REBUILD) accO[dt] = MM::mma(vfr, pf, accO[dt]);
          if (REBUILD && SPLIT) accO[dt] = MM::mma(vfr, pf_lo, accO[dt]);
          if (has_tv) accC[dt] = MM::mma(rowsf(ttV, t * 32, cc, dt * 32), pf, accC[dt]);
        }
      }
  };

  if constexpr (DMA) {
    using Dma = SwzDma<NW, DP>;
    constexpr int NSLAB = BN / Dma::SLAB_ROWS;
    static_assert(NSLAB * Dma::SLAB_ROWS == BN, "key tiles must be whole DMA slabs");
    const Dma dma(__builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane);
    // Byte offsets fit in 32 bits: the host only selects this path when each (batch, head) slab of K, V,
    // tK and tV spans less than 2^31 bytes.
    const uint32_t krs = (uint32_t)p.k.sr * 2, vrs = (uint32_t)p.v.sr * 2;
    const uint32_t tkrs = has_tk ? (uint32_t)p.tk.sr * 2 : 0u, tvrs = has_tv ? (uint32_t)p.tv.sr * 2 : 0u;
    const rsrc_t krsrc = make_rsrc(K, (uint32_t)slab_span(s.M, krs, 2 * DP)),
                  vrsrc = make_rsrc(V, (uint32_t)slab_span(s.M, vrs, 2 * DP));
    const rsrc_t tkrsrc = make_rsrc(has_tk ? (const void*)TK : (const void*)K, (uint32_t)slab_span(s.M, tkrs, 2 * DP));
    const rsrc_t tvrsrc = make_rsrc(has_tv ? (const void*)TV : (const void*)V, (uint32_t)slab_span(s.M, tvrs, 2 * DP));
    auto issue = [&](int kt, char* tK, char* tV, char* ttK, char* ttV) {
      const int k0 = kt * BN;
      dma.template issue_clamped<NSLAB>(krsrc, krs, k0, s.M, tK);
      dma.template issue_clamped<NSLAB>(vrsrc, vrs, k0, s.M, tV);
      if (has_tk) dma.template issue_clamped<NSLAB>(tkrsrc, tkrs, k0, s.M, ttK);
      if (has_tv) dma.template issue_clamped<NSLAB>(tvrsrc, tvrs, k0, s.M, ttV);
    };
    // Tile kt from the set c*; the next tile's copies go to the set n* (read in the previous step, which
    // every wave has finished at the barrier).
    auto step = [&](int kt, const char* cK, const char* cV, const char* ctK, const char* ctV, char* nK, char* nV,
                    char* ntK, char* ntV) {
      wait_vm_all();
      __syncthreads();
      if (kt + 1 < nkt) issue(kt + 1, nK, nV, ntK, ntV);
      compute(kt, cK, cV, ctK, ctV);
      __builtin_amdgcn_sched_barrier(0);  // keep the two unrolled steps apart (register pressure)
    };
    if (nkt > 0) {
      issue(0, sK0, sV0, stK0, stV0);
      int kt = 0;
      for (; kt + 1 < nkt; kt += 2) {
        step(kt, sK0, sV0, stK0, stV0, sK1, sV1, stK1, stV1);
        step(kt + 1, sK1, sV1, stK1, stV1, sK0, sV0, stK0, stV0);
      }
      if (kt < nkt) step(kt, sK0, sV0, stK0, stV0, sK1, sV1, stK1, stV1);
    }
  } else {
    TileStage<T, BN, DP, NT> gK, gV, gtK, gtV;
    auto prefetch = [&](int k0) {
      gK.load(K, p.k.sr, k0, s.M, s.D, s.vec);
      gV.load(V, p.v.sr, k0, s.M, s.D, s.vec);
      if (has_tk) gtK.load(TK, p.tk.sr, k0, s.M, s.D, s.vec);
      if (has_tv) gtV.load(TV, p.tv.sr, k0, s.M, s.D, s.vec);
    };
    if (nkt > 0) prefetch(0);
    for (int kt = 0; kt < nkt; ++kt) {
      __syncthreads();
      gK.store((T*)sK0, PITCH);
      gV.store((T*)sV0, PITCH);
      if (has_tk) gtK.store((T*)stK0, PITCH);
      if (has_tv) gtV.store((T*)stV0, PITCH);
      __syncthreads();
      if (kt + 1 < nkt) prefetch((kt + 1) * BN);
      compute(kt, sK0, sV0, stK0, stV0);
    }
  }

  // normalize: P / L with L = sum_j P_j, i.e. every term below is divided by L (and a rebuilt O as well)
  float inv = 1.f;
  if (p.normalize) {
    const float L = pair_sum(lpart);
    inv = L > 0.f ? 1.f / L : 0.f;
  }
  const float cval = pair_sum(cpart) * s.scale * inv;
  if (qvalid) {
    const T* O = (HAS_O && !REBUILD) ? (const T*)p.o.p + b * p.o.sb + h * p.o.sh : nullptr;
    T* TO = (T*)p.tout.p + b * p.tout.sb + h * p.tout.sh;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        const int d0 = dt * 32 + 8 * qd + 4 * g;
        if (d0 < s.D) {
          f32x4_t ov;
          if (!REBUILD) {
            ov = load4<T>(O, p.o.sr, myq, d0, s.D, s.vec);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) ov[e] = accO[dt][4 * qd + e] * inv;
          }
          float r4[4];
#pragma unroll
          for (int e = 0; e < 4; ++e)
            r4[e] = inv * (s.scale * accA[dt][4 * qd + e] + accC[dt][4 * qd + e]) - cval * ov[e];
          store4<T>(TO, p.tout.sr, myq, d0, s.D, r4[0], r4[1], r4[2], r4[3], s.vec);
        }
      }
  }
}

// 16-bit inputs at head dims up to 64 (a multiple of 8, computed at 64 with the tile columns past D zero) with
// LDS-DMA tiles: the same JVP with the keys of a query block split between two groups of four waves
// (eight-wave workgroups), so that a SIMD holds two waves at 256 registers each
// where jvp_kernel holds one at ~380 (config 4: B H T / 32 = 1024 query waves for 1024 SIMDs; 27.1 -> 23.0 us
// there, same box). Each group streams its own half of the key tiles (64 keys per tile, 128 KB of LDS in
// all) through its own double-buffered tiles; both groups meet at the same barrier every step (a group
// whose half is shorter idles through the last step). The float32 partial sums of group 1 (accumulators,
// row sums) pass to group 0 through LDS at the end. ALL: every tangent is given (the presence tests are then
// constants, and the loop body has no branches between its products).
template <typename T, bool CAUSAL, bool HAS_O, bool ALL, bool FD>
__global__ __launch_bounds__(512, 2) void jvp_ksplit_kernel(const JvpParams p) {
  using MM = Mfma<T>;
  using F = typename MM::frag_t;
  static_assert(sizeof(T) == 2, "16-bit inputs only");
  constexpr int DP = 64, NW = 4, BM = 32 * NW, BN = 64, NST = BN / 32;
  constexpr int NDT = DP / 32, NKC = DP / MM::KC, NPC = 32 / MM::KC;
  constexpr int TB = BN * DP * 2;  // bytes per tile
  using Dma = SwzDma<NW, DP>;
  constexpr int NSLAB = BN / Dma::SLAB_ROWS;
  static_assert(NSLAB * Dma::SLAB_ROWS == BN, "key tiles must be whole DMA slabs");
  // [group][set][K, V, tK, tV]; reused for the partial sums after the key loop
  __shared__ __attribute__((aligned(1024))) char smem[2 * 2 * 4 * TB];
  static_assert(sizeof(smem) >= (2 * 3 * 16 + 4) * 256 * 4, "the partial sums fit in the tile memory");

  const Shape& s = p.s;
  const int lane = threadIdx.x & 63, li = lane & 31, g = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = wave >> 2, wig = wave & 3;  // key group, wave in group
  const int nqb = (s.T + BM - 1) / BM;
  const int bid = xcd_remap(blockIdx.x, gridDim.x);
  const int bh = bid / nqb;
  int qb = bid - bh * nqb;
  if (CAUSAL) qb = nqb - 1 - qb;
  const int b = bh / s.H, h = bh - b * s.H;
  const T* Q = (const T*)p.q.p + b * p.q.sb + h * p.q.sh;
  const T* K = (const T*)p.k.p + b * p.k.sb + h * p.k.sh;
  const T* V = (const T*)p.v.p + b * p.v.sb + h * p.v.sh;
  const bool has_tq = ALL || p.tq.p != nullptr, has_tk = ALL || p.tk.p != nullptr, has_tv = ALL || p.tv.p != nullptr;
  const T* TQ = has_tq ? (const T*)p.tq.p + b * p.tq.sb + h * p.tq.sh : nullptr;
  const T* TK = has_tk ? (const T*)p.tk.p + b * p.tk.sb + h * p.tk.sh : nullptr;
  const T* TV = has_tv ? (const T*)p.tv.p + b * p.tv.sb + h * p.tv.sh : nullptr;
  const int q0w = qb * BM + wig * 32;
  const int myq = q0w + li;
  const bool qvalid = myq < s.T;
  const int64_t row_id = (int64_t)bh * s.T + myq;

  F qf[NKC], tqf[NKC];
#pragma unroll
  for (int c = 0; c < NKC; ++c) {
    qf[c] = gload_frag<T>(Q, p.q.sr, myq, s.T, c, s.D, s.vec);
    tqf[c] = has_tq ? gload_frag<T>(TQ, p.tq.sr, myq, s.T, c, s.D, s.vec) : F{};
  }
  f32x16_t accA[NDT], accC[NDT], accO[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
    accA[dt] = zero16();
    accC[dt] = zero16();
    accO[dt] = zero16();
  }
  const float c2 = s.scale * kLog2e;
  const float lse_raw = qvalid ? p.lse[row_id] : THERIA_INF;
  const float lse2 = lse_raw * kLog2e;
  const float moff = lse2 == -THERIA_INF ? THERIA_INF : lse2;  // a row without visible keys has P = 0
  float cpart = 0.f, lpart = 0.f;
  // The two-term products only in waves holding a row flagged peaked in lse (a dominant probability, which
  // rows with few visible keys have): there (P o G) V and c o O cancel. Elsewhere the rounding of P o G and
  // P spreads over many keys and one 16-bit term each suffices (uniform per wave).
  const bool split = __any(lse_peaked(lse_raw));

  int kend = s.M;
  if (CAUSAL) kend = min(s.M, qb * BM + BM);
  const int nkt = (kend + BN - 1) / BN;
  const int half = (nkt + 1) / 2;
  const int kt0 = grp * half, kt1 = min(nkt, kt0 + half);  // this group's tiles [kt0, kt1)

  // The key tile kt held in (tK, tV, ttK, ttV): as jvp_kernel, 32-key subtiles one after the other. MASK: the
  // tile reaches past the last key or (causal) past this wave's first query.
  auto compute = [&](auto split_tag, auto mask_tag, int kt, const char* tK, const char* tV, const char* ttK,
                     const char* ttV) __attribute__((always_inline)) {
    constexpr bool SPLIT = decltype(split_tag)::value;
    constexpr bool MASK = decltype(mask_tag)::value;
#pragma unroll
    for (int st = 0; st < NST; ++st) {
      const int k0 = kt * BN + 32 * st;
      if (CAUSAL && k0 > q0w + 31) continue;
      f32x16_t sc = zero16(), gm = zero16();
#pragma unroll
      for (int c = 0; c < NKC; ++c) {
        const F kfr = swz_cols<T, DP>(tK, 32 * st + li, c);
        sc = MM::mma(kfr, qf[c], sc);
        if (has_tq) gm = MM::mma(kfr, tqf[c], gm);
        if (has_tk) gm = MM::mma(swz_cols<T, DP>(ttK, 32 * st + li, c), qf[c], gm);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float pv = fast_exp2(fmaf(sc[r], c2, -moff));
        if constexpr (MASK) {
          const int key = k0 + acc_row(r, g);
          if (key >= s.M || (CAUSAL && key > myq)) pv = 0.f;
        }
        sc[r] = pv;
        lpart += pv;
        const float pg = pv * gm[r];
        gm[r] = pg;
        cpart += pg;
      }
      if constexpr (SPLIT) {
#pragma unroll
        for (int cc = 0; cc < NPC; ++cc) {
          F pf, pf_lo, pgf, pgf_lo;
          split_frag<T>(sc, cc, pf, pf_lo);
          split_frag<T>(gm, cc, pgf, pgf_lo);
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) {
            const F vfr = swz_rows<T, DP>(tV, 32 * st, cc, dt * 32);
            accA[dt] = MM::mma(vfr, pgf, accA[dt]);
            accA[dt] = MM::mma(vfr, pgf_lo, accA[dt]);
            accO[dt] = MM::mma(vfr, pf, accO[dt]);
            accO[dt] = MM::mma(vfr, pf_lo, accO[dt]);
            if (has_tv) accC[dt] = MM::mma(swz_rows<T, DP>(ttV, 32 * st, cc, dt * 32), pf, accC[dt]);
          }
        }
      } else {
#pragma unroll
        for (int cc = 0; cc < NPC; ++cc) {
          const F pf = acc_frag<T>(sc, cc), pgf = acc_frag<T>(gm, cc);
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) {
            const F vfr = swz_rows<T, DP>(tV, 32 * st, cc, dt * 32);
            accA[dt] = MM::mma(vfr, pgf, accA[dt]);
            accO[dt] = MM::mma(vfr, pf, accO[dt]);
            if (has_tv) accC[dt] = MM::mma(swz_rows<T, DP>(ttV, 32 * st, cc, dt * 32), pf, accC[dt]);
          }
        }
      }
    }
  };

  // Head dims below 64 (a multiple of 8): the tiles' columns D .. 63 are filled with zeros by the DMA.
  const Dma dma(wig, lane, FD ? 8 : s.D / 8);  // FD: head dim 64
  // Byte offsets fit in 32 bits: the host only selects this path when each (batch, head) slab of K, V, tK
  // and tV spans less than 2^31 bytes.
  const uint32_t krs = (uint32_t)p.k.sr * 2, vrs = (uint32_t)p.v.sr * 2;
  const uint32_t tkrs = has_tk ? (uint32_t)p.tk.sr * 2 : 0u, tvrs = has_tv ? (uint32_t)p.tv.sr * 2 : 0u;
  const int64_t rb = 2 * (FD ? 64 : s.D);  // bytes of a row the DMA reads
  const rsrc_t krsrc = make_rsrc(K, (uint32_t)slab_span(s.M, krs, rb)),
               vrsrc = make_rsrc(V, (uint32_t)slab_span(s.M, vrs, rb));
  const rsrc_t tkrsrc = make_rsrc(has_tk ? (const void*)TK : (const void*)K, (uint32_t)slab_span(s.M, tkrs, rb));
  const rsrc_t tvrsrc = make_rsrc(has_tv ? (const void*)TV : (const void*)V, (uint32_t)slab_span(s.M, tvrs, rb));
  auto tile = [&](int set, int a) { return smem + ((grp * 2 + set) * 4 + a) * TB; };  // a: K, V, tK, tV
  auto issue = [&](int kt, int set) {
    const int k0 = kt * BN;
    dma.template issue_clamped<NSLAB>(krsrc, krs, k0, s.M, tile(set, 0));
    dma.template issue_clamped<NSLAB>(vrsrc, vrs, k0, s.M, tile(set, 1));
    if (has_tk) dma.template issue_clamped<NSLAB>(tkrsrc, tkrs, k0, s.M, tile(set, 2));
    if (has_tv) dma.template issue_clamped<NSLAB>(tvrsrc, tvrs, k0, s.M, tile(set, 3));
  };
  // Step i: tile kt0 + i of this group (if it has one) from set i & 1; the next one's copies go to the other
  // set, read in step i - 1, which every wave has finished at the barrier. The tiles from mask_from on may
  // reach past the last key or (causal) past the block's first query and take the masked copy of the loop;
  // the groups may be in different copies at a step, but both meet the same barriers.
  const int mask_from = min(kend % BN ? nkt - 1 : nkt, CAUSAL ? qb * BM / BN : nkt);
  auto sweep = [&](auto split_tag) __attribute__((always_inline)) {
    auto step = [&](auto mask_tag, int i) __attribute__((always_inline)) {
      const int kt = kt0 + i;
      wait_vm_all();
      __syncthreads();
      if (kt + 1 < kt1) issue(kt + 1, (i + 1) & 1);
      if (kt < kt1) compute(split_tag, mask_tag, kt, tile(i & 1, 0), tile(i & 1, 1), tile(i & 1, 2), tile(i & 1, 3));
    };
    const int isplit = min(half, max(0, mask_from - kt0));
    int i = 0;
    for (; i < isplit; ++i) step(std::false_type{}, i);
    for (; i < half; ++i) step(std::true_type{}, i);
  };
  if (kt0 < kt1) issue(kt0, 0);
  // The waves of a workgroup may take different copies of the loop: both meet the same barriers.
  if (split)
    sweep(std::integral_constant<bool, true>{});
  else
    sweep(std::integral_constant<bool, false>{});

  // The groups finish one column tile each (group g the tile dt = g): each hands the other tile's partial sums
  // and its row sums to the other group in one round, 16 bytes per lane per store (elements 4c .. 4c + 3 of
  // accumulator a of lane l of wave w of group g at words (((g * 3 + a) * 4 + c) * 256 + w * 64 + l) * 4, so one
  // store instruction covers 1 KiB of consecutive words), then stores its half of the output.
  static_assert(NDT == 2, "one column tile per group");
  float* buf = reinterpret_cast<float*>(smem);
  f32x4_t* buf4 = reinterpret_cast<f32x4_t*>(smem);
  constexpr int RS = 2 * 3 * 4 * 256 * 4;  // the row sums, [group][l, c]
  __syncthreads();  // every wave is done with the last tile
  auto finish = [&](auto keep_tag) __attribute__((always_inline)) {
    constexpr int KEEP = decltype(keep_tag)::value, GIVE = 1 - KEEP;
    const int mine = KEEP * 3 * 4 * 256, theirs = GIVE * 3 * 4 * 256;  // group KEEP writes at `mine`
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int i = c * 256 + wig * 64 + lane;
      buf4[mine + i] = f32x4_t{accA[GIVE][4 * c], accA[GIVE][4 * c + 1], accA[GIVE][4 * c + 2], accA[GIVE][4 * c + 3]};
      buf4[mine + 4 * 256 + i] =
          f32x4_t{accO[GIVE][4 * c], accO[GIVE][4 * c + 1], accO[GIVE][4 * c + 2], accO[GIVE][4 * c + 3]};
      if (has_tv)
        buf4[mine + 8 * 256 + i] =
            f32x4_t{accC[GIVE][4 * c], accC[GIVE][4 * c + 1], accC[GIVE][4 * c + 2], accC[GIVE][4 * c + 3]};
    }
    buf[RS + KEEP * 512 + wig * 64 + lane] = lpart;
    buf[RS + KEEP * 512 + 256 + wig * 64 + lane] = cpart;
    __syncthreads();
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int i = c * 256 + wig * 64 + lane;
      const f32x4_t a = buf4[theirs + i], o4 = buf4[theirs + 4 * 256 + i];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        accA[KEEP][4 * c + e] += a[e];
        accO[KEEP][4 * c + e] += o4[e];
      }
      if (has_tv) {
        const f32x4_t c4 = buf4[theirs + 8 * 256 + i];
#pragma unroll
        for (int e = 0; e < 4; ++e) accC[KEEP][4 * c + e] += c4[e];
      }
    }
    lpart += buf[RS + GIVE * 512 + wig * 64 + lane];
    cpart += buf[RS + GIVE * 512 + 256 + wig * 64 + lane];

    // Epilogue as jvp_kernel's (O rebuilt from the same P; normalize: P divided by its own row sum), for the
    // columns of tile KEEP.
    float inv = 1.f;
    if (p.normalize) {
      const float L = pair_sum(lpart);
      inv = L > 0.f ? 1.f / L : 0.f;
    }
    const float cval = pair_sum(cpart) * s.scale * inv;
    if (qvalid) {
      T* TO = (T*)p.tout.p + b * p.tout.sb + h * p.tout.sh;
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        const int d0 = KEEP * 32 + 8 * qd + 4 * g;
        float r4[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float ov = accO[KEEP][4 * qd + e] * inv;
          r4[e] = inv * (s.scale * accA[KEEP][4 * qd + e] + accC[KEEP][4 * qd + e]) - cval * ov;
        }
        store4<T>(TO, p.tout.sr, myq, d0, s.D, r4[0], r4[1], r4[2], r4[3], s.vec);
      }
    }
  };
  // both branches meet the one barrier inside finish
  if (grp == 0)
    finish(std::integral_constant<int, 0>{});
  else
    finish(std::integral_constant<int, 1>{});
}

template <bool HAS_O>
struct JvpLauncher {
  template <typename T, int DP, bool CAUSAL>
  static hipError_t run(const JvpParams& p, hipStream_t st) {
    const int nqb = (p.s.T + 127) / 128;
    const int64_t nblk = (int64_t)nqb * p.s.B * p.s.H;
    if (nblk == 0) return hipSuccess;
    if constexpr (sizeof(T) == 2) {
      // LDS-DMA tiles: 16-byte-aligned views, each streamed (batch, head) slab < 2^31 bytes, and a head dim that
      // is a multiple of 8 up to 64 (the key-split kernel, columns past D zero-filled) or exactly 128
      bool ok = p.s.vec && (DP <= 64 ? p.s.D % 8 == 0 : p.s.D == DP);
      for (const View* v : {&p.k, &p.v, &p.tk, &p.tv})
        if (v->p && !slab_fits_dma(p.s.M, v->sr, p.s.D)) ok = false;
      if (ok) {
        if constexpr (DP <= 64) {
          const bool all = p.tq.p && p.tk.p && p.tv.p, fd = p.s.D == 64;
          const dim3 grid((unsigned)nblk), block(512);
          if (all && fd)
            hipLaunchKernelGGL((jvp_ksplit_kernel<T, CAUSAL, HAS_O, true, true>), grid, block, 0, st, p);
          else if (all)
            hipLaunchKernelGGL((jvp_ksplit_kernel<T, CAUSAL, HAS_O, true, false>), grid, block, 0, st, p);
          else if (fd)
            hipLaunchKernelGGL((jvp_ksplit_kernel<T, CAUSAL, HAS_O, false, true>), grid, block, 0, st, p);
          else
            hipLaunchKernelGGL((jvp_ksplit_kernel<T, CAUSAL, HAS_O, false, false>), grid, block, 0, st, p);
        } else
          hipLaunchKernelGGL((jvp_kernel<T, DP, CAUSAL, HAS_O, true>), dim3((unsigned)nblk), dim3(256), 0, st, p);
        return hipGetLastError();
      }
    }
    hipLaunchKernelGGL((jvp_kernel<T, DP, CAUSAL, HAS_O, false>), dim3((unsigned)nblk), dim3(256), 0, st, p);
    return hipGetLastError();
  }
};

hipError_t launch_jvp(const JvpParams& p, hipStream_t st) {
  return p.o.p ? dispatch_all<JvpLauncher<true>>(p, st) : dispatch_all<JvpLauncher<false>>(p, st);
}

}  // namespace theria
