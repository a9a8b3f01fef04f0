// SDPA double backward for gfx950: the vector-Jacobian product of the backward map
// (Q, K, V, dO) -> (dQ, dK, dV) with cotangents (gQ, gK, gV).
//
// The reference has no kernel for this (docs/STATUS.md:265-271; its HVP is finite differences of the
// VJP, theria/attention/hvp_utils.py:30-49, or autograd through eager PyTorch,
// theria/autograd/sdpa_custom_function.py:32-53). With s = scale, P from the saved lse,
// dP = dO V^T, z = delta (row term of the backward), dS = P o (dP - z):
//   Gam = s (gQ K^T + Q gK^T),  r_i = sum_j P_ij Gam_ij,   W = dO gV^T,
//   E1  = Gam o (dP - z) + W,   t_i = sum_j P_ij E1_ij,
//   Gbar_dP = P o (Gam - r),    Gbar_S = P o E1 - r o dS - t o P,
//   G_dO = Gbar_dP V + P gV     (the frozen-stats JVP with tangents (gQ, gK, gV): jvp kernel)
//   G_V  = Gbar_dP^T dO
//   G_Q  = s (Gbar_S K + dS gK) = s (sum_j (P o E1)_ij K_j - r_i (dS K)_i - t_i (P K)_i + (dS gK)_i)
//   G_K  = s (Gbar_S^T Q + dS^T gQ)
// (Gbar_S = P o (Gbar_P - s_row) with Gbar_P = E1 - r o dP and s_row = t - r z, rearranged so that a
// single pass over the keys suffices for G_Q.)
//
// rows kernel: lane per query (transposed score tiles, as in the forward). One pass over key tiles (64
//   keys as two 32-key subtiles for 16-bit inputs at head dim <= 64, else 32) accumulates the four D-wide
//   products of the G_Q expression plus r and t, writes G_Q, r, t.
//   16-bit workgroups holding a row flagged peaked in lse are redone after it (as extra workgroups of the
//   cols kernel's grid): with the exact r and t the first launch wrote, Gbar_S = P o ((Gam - r)(dP - z) + W - t)
//   is formed in float32 and, with dS, entered as two 16-bit terms (hi + lo), so that
//   G_Q = s (Gbar_S K + dS gK) is no longer a small difference of large products.
// cols kernel: lane per key (as in the backward). One pass over query tiles (64 queries as two 32-query
//   subtiles for 16-bit inputs at head dim <= 64, else 32) with r, t, z, lse per row staged in LDS
//   accumulates G_V and G_K in registers. 16-bit query tiles holding a row flagged peaked are skipped by
//   that pass and run after it with Gbar_dP, Gbar_S and dS entered as two 16-bit terms each (their sums over
//   many queries are small there).
// 16-bit inputs at head dims up to 64 (a multiple of 8, computed at 64 with the tile columns past D zero-filled by
// the DMA) take two split kernels instead, eight-wave workgroups of two
// four-wave groups (two waves per SIMD at 256 registers): the key-split row kernel (bwdbwd_rows_ks_kernel) forms
// the exact row terms, G_Q and G_dO in one launch (the groups split each query block's key tiles and combine
// through LDS), and the query-split column kernel (bwdbwd_cols_qs_kernel) G_K and G_V (the groups split each
// key block's query tiles).
#include <initializer_list>
#include <type_traits>

#include "dispatch.hpp"
#include "sdpa_common.hpp"
#include "sdpa_lds.hpp"

namespace theria {

// DMA: 16-bit inputs with head dim exactly 64 or 128 and 16-byte-aligned rows. The K, V, gK, gV tiles are
// then filled by LDS DMA into two sets of unpadded, XOR-swizzled buffers (sdpa_lds.hpp), one barrier per
// tile with the next tile's copies in flight; otherwise they pass through registers into padded LDS rows
// (two barriers per tile).
// EXACT: the second pass of 16-bit problems, which redoes only the workgroups holding a row flagged peaked in
// lse in the exact form (overwriting G_Q; r and t are the first launch's); apart, the first launch keeps its
// registers and schedule.
template <typename T, int DP, bool CAUSAL, bool DMA, bool EXACT>
__device__ __attribute__((always_inline)) inline void rows_block(const BwdBwdParams& p, const int blk, const int nblk) {
  using MM = Mfma<T>;
  using F = typename MM::frag_t;
  constexpr int KC = MM::KC;
  constexpr int NW = 4, BM = 32 * NW, NT = 64 * NW;
  // keys per tile: two 32-key subtiles per tile where the registers allow (one wave per SIMD)
  constexpr int BN = (DP == 128 || sizeof(T) == 4 || DMA) ? 32 : 64;
  constexpr int PITCH = DP + 16 / (int)sizeof(T);
  constexpr int NDT = DP / 32, NKC = DP / KC, NPC = 32 / KC, NST = BN / 32;
  constexpr int TB = DMA ? BN * DP * 2 : BN * PITCH * (int)sizeof(T);  // bytes per tile
  constexpr int TB2 = DMA ? TB : 16;                                    // second set (DMA only)
  __shared__ __attribute__((aligned(1024))) char sK0[TB];
  __shared__ __attribute__((aligned(1024))) char sV0[TB];
  __shared__ __attribute__((aligned(1024))) char sgK0[TB];
  __shared__ __attribute__((aligned(1024))) char sgV0[TB];
  __shared__ __attribute__((aligned(1024))) char sK1[TB2];
  __shared__ __attribute__((aligned(1024))) char sV1[TB2];
  __shared__ __attribute__((aligned(1024))) char sgK1[TB2];
  __shared__ __attribute__((aligned(1024))) char sgV1[TB2];

  const Shape& s = p.s;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, li = lane & 31, g = lane >> 5;
  const int nqb = (s.T + BM - 1) / BM;
  const int bid = xcd_remap(blk, nblk);
  const int bh = bid / nqb;
  int qb = bid - bh * nqb;
  if (CAUSAL && !EXACT) qb = nqb - 1 - qb;  // longest first (the exact pass: query order, see the cols grid)
  const int b = bh / s.H, h = bh - b * s.H;
  const T* Q = (const T*)p.q.p + b * p.q.sb + h * p.q.sh;
  const T* K = (const T*)p.k.p + b * p.k.sb + h * p.k.sh;
  const T* V = (const T*)p.v.p + b * p.v.sb + h * p.v.sh;
  const T* dO = (const T*)p.dout.p + b * p.dout.sb + h * p.dout.sh;
  const bool has_gq = p.gq.p != nullptr, has_gk = p.gk.p != nullptr, has_gv = p.gv.p != nullptr;
  const T* GQ = has_gq ? (const T*)p.gq.p + b * p.gq.sb + h * p.gq.sh : nullptr;
  const T* GK = has_gk ? (const T*)p.gk.p + b * p.gk.sb + h * p.gk.sh : nullptr;
  const T* GV = has_gv ? (const T*)p.gv.p + b * p.gv.sb + h * p.gv.sh : nullptr;
  const int q0w = qb * BM + wave * 32;
  const int myq = q0w + li;
  const bool qvalid = myq < s.T;
  const int64_t row_id = (int64_t)bh * s.T + myq;
  int kend = s.M;
  if (CAUSAL) kend = min(s.M, qb * BM + BM);
  const int nkt = (kend + BN - 1) / BN;
  // 16-bit workgroups holding a row flagged peaked in lse take the exact form (uniform). Causal ones with at
  // most half the longest workgroup's key tiles run both of its passes in the first launch, inside that
  // launch's slack (every head's first query block holds such rows); the others are the second pass's.
  static_assert(!EXACT || sizeof(T) == 2, "the exact form is for 16-bit inputs");
  constexpr bool LIGHT_OK = CAUSAL && sizeof(T) == 2 && DP <= 64;  // at 128 the second sweep spills
  const bool light = LIGHT_OK && 2 * nkt <= (s.M + BN - 1) / BN;
  bool flagged = false;
  if (EXACT || (LIGHT_OK && light)) flagged = __syncthreads_or(qvalid && lse_peaked(p.lse[row_id]));
  const bool exact = EXACT && flagged && !light;
  const bool two_pass = !EXACT && LIGHT_OK && flagged && light;
  if (EXACT && !exact) return;

  F qf[NKC], dof[NKC], gqf[NKC];
#pragma unroll
  for (int c = 0; c < NKC; ++c) {
    qf[c] = gload_frag<T>(Q, p.q.sr, myq, s.T, c, s.D, s.vec);
    dof[c] = gload_frag<T>(dO, p.dout.sr, myq, s.T, c, s.D, s.vec);
    gqf[c] = has_gq ? gload_frag<T>(GQ, p.gq.sr, myq, s.T, c, s.D, s.vec) : F{};
  }
  f32x16_t x13[NDT], x2[NDT], x4[NDT], yk[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
    x13[dt] = zero16();
    x2[dt] = zero16();
    x4[dt] = zero16();
    yk[dt] = zero16();
  }
  const float c2 = s.scale * kLog2e;
  const float lse2 = qvalid ? p.lse[row_id] * kLog2e : THERIA_INF;
  const float moff = lse2 == -THERIA_INF ? THERIA_INF : lse2;
  // float32: P = exp2((fl(S c2) - m2) - L2) from the row's own statistics, and dP formed from zero, both as in
  // the row-term pass that wrote m2, L2 and z (so the largest score gives exactly 2^-L2, and dP - z keeps only
  // z's own rounding)
  constexpr bool OWN = sizeof(T) == 4;
  const float m2 = OWN && qvalid ? p.lse[row_id] : THERIA_INF;
  const float l2 = OWN && qvalid ? p.row_l2[row_id] : 0.f;
  const float z = qvalid ? p.delta[row_id] : 0.f;
  float r_part = 0.f, t_part = 0.f;
  // 16-bit inputs: Gbar_S = P o ((Gam - r)(dP - z) + W - t), and for any row constants cr, ct
  //   Gbar_S = P o E1c - (r - cr) dS - (t - ct) P  with  E1c = (Gam - cr)(dP - z) + W - ct,
  // so x13 takes P o E1c and G_Q = s (x13 - (r - cr) x2 - t_c x4 + yk), t_c = sum_j of the rounded P o E1c
  // operands (= t - ct in exact arithmetic). The centres are r and t over the first key tile (a pre-pass),
  // used when that tile holds more than half of the row's probability (else cr = ct = 0):
  // on rows with few visible keys, where G_Q is a small difference of large terms, the products then carry
  // small centred values instead (one visible key gives G_Q = 0 exactly).
  float t_frag = 0.f, cr = 0.f, ct = 0.f;
  float rx = 0.f, tx = 0.f;  // exact row terms of the exact form
  float c_p = 0.f, c_pg = 0.f, c_pgd = 0.f, c_pd = 0.f, c_pw = 0.f;

  // Fragment reads: "cols" (k along a tile row, KLIN) and "rows" (k down the tile rows, KACC).
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

  // The key tile kt held in (tK, tV, tgK, tgV), as 32-key subtiles.
  // PASS: 0 the pre-pass (sums only: for the centres over the first tile, or for r and t over every tile),
  // 1 the common pass, 3 the exact pass (Gbar_S from exact row terms r, t; 16-bit only).
  auto compute = [&](auto pass_tag, int kt, const char* tK, const char* tV, const char* tgK,
                     const char* tgV) __attribute__((always_inline)) {
    constexpr int PASS = decltype(pass_tag)::value;
    constexpr bool PRE = PASS == 0;
    const int k0 = kt * BN;
#pragma unroll
    for (int st = 0; st < NST; ++st) {
      const int k0s = k0 + 32 * st;  // this 32-key subtile
      if (CAUSAL && k0s > q0w + 31) continue;

      f32x16_t sc = zero16(), gm = zero16(), w = zero16(), dpz;
#pragma unroll
      for (int r = 0; r < 16; ++r) dpz[r] = OWN ? 0.f : -z;
#pragma unroll
      for (int c = 0; c < NKC; ++c) {
        const F kfr = colsf(tK, 32 * st + li, c);
        sc = MM::mma(kfr, qf[c], sc);
        dpz = MM::mma(colsf(tV, 32 * st + li, c), dof[c], dpz);
        if (has_gq) gm = MM::mma(kfr, gqf[c], gm);
        if (has_gk) gm = MM::mma(colsf(tgK, 32 * st + li, c), qf[c], gm);
        if (has_gv) w = MM::mma(colsf(tgV, 32 * st + li, c), dof[c], w);
      }
      const bool need_mask = (k0s + 32 > s.M) || (CAUSAL && k0s + 31 > q0w);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        if constexpr (OWN) dpz[r] -= z;
        float pv = OWN ? own_prob(sc[r], c2, m2, l2) : fast_exp2(fmaf(sc[r], c2, -moff));
        if (need_mask) {
          const int key = k0s + acc_row(r, g);
          if (key >= s.M || (CAUSAL && key > myq)) pv = 0.f;
        }
        const float gam = s.scale * gm[r];
        const float e1 = fmaf(gam, dpz[r], w[r]);
        const float pe1 = pv * e1;
        if constexpr (PRE) {
          c_p += pv;
          c_pg = fmaf(pv, gam, c_pg);
          c_pd = fmaf(pv, dpz[r], c_pd);
          c_pgd = fmaf(pv * gam, dpz[r], c_pgd);
          c_pw = fmaf(pv, w[r], c_pw);
        } else if constexpr (PASS == 3) {
          gm[r] = pv * (fmaf(gam - rx, dpz[r], w[r]) - tx);  // Gbar_S
          dpz[r] = pv * dpz[r];                              // dS
        } else {
          r_part = fmaf(pv, gam, r_part);
          t_part += pe1;
          sc[r] = pv;
          gm[r] = sizeof(T) == 2 ? pv * (fmaf(gam - cr, dpz[r], w[r]) - ct) : pe1;
          dpz[r] = pv * dpz[r];  // dS
        }
      }
      if constexpr (PRE) continue;
      if constexpr (PASS == 3 && sizeof(T) == 2) {
#pragma unroll
        for (int cc = 0; cc < NPC; ++cc) {
          F gh, gl, dh, dl;
          split_frag<T>(gm, cc, gh, gl);
          split_frag<T>(dpz, cc, dh, dl);
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) {
            const F kr = rowsf(tK, 32 * st, cc, dt * 32);
            x13[dt] = MM::mma(kr, gh, x13[dt]);
            x13[dt] = MM::mma(kr, gl, x13[dt]);
            if (has_gk) {
              const F gkr = rowsf(tgK, 32 * st, cc, dt * 32);
              yk[dt] = MM::mma(gkr, dh, yk[dt]);
              yk[dt] = MM::mma(gkr, dl, yk[dt]);
            }
          }
        }
        continue;
      }
#pragma unroll
      for (int cc = 0; cc < NPC; ++cc) {
        const F pf = acc_frag<T>(sc, cc);
        const F pe1f = acc_frag<T>(gm, cc);
        const F dsf = acc_frag<T>(dpz, cc);
        if constexpr (sizeof(T) == 2) t_frag = frag_sum<T>(pe1f, t_frag);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
          const F kr = rowsf(tK, 32 * st, cc, dt * 32);
          x13[dt] = MM::mma(kr, pe1f, x13[dt]);
          x2[dt] = MM::mma(kr, dsf, x2[dt]);
          x4[dt] = MM::mma(kr, pf, x4[dt]);
          if (has_gk) yk[dt] = MM::mma(rowsf(tgK, 32 * st, cc, dt * 32), dsf, yk[dt]);
        }
      }
    }
  };

  const std::integral_constant<int, 0> pre_pass;
  const std::integral_constant<int, 1> full_pass;
  const std::integral_constant<int, 3> exact_pass;
  if (exact) {  // the first launch's exact float32 row terms (same stream, so already written)
    rx = qvalid ? p.r_row[row_id] : 0.f;
    tx = qvalid ? p.t_row[row_id] : 0.f;
  }
  // r = sum_j P Gam, t = sum_j P (Gam (dP - z) + W) from the pre-pass sums over all keys
  auto set_exact_terms = [&]() {
    rx = pair_sum(c_pg);
    tx = pair_sum(c_pgd) + pair_sum(c_pw);
  };
  auto set_centre = [&]() {
    const float sp = pair_sum(c_p), spg = pair_sum(c_pg), spd = pair_sum(c_pd), spgd = pair_sum(c_pgd),
                spw = pair_sum(c_pw);
    // only where the first tile holds most of the row's probability (its means then stand for the row)
    if (sp > 0.5f) {
      cr = spg / sp;
      ct = (spgd - cr * spd + spw) / sp;
    }
  };

  if constexpr (DMA) {
    using Dma = SwzDma<NW, DP>;
    constexpr int NSLAB = BN / Dma::SLAB_ROWS;
    static_assert(NSLAB * Dma::SLAB_ROWS == BN, "key tiles must be whole DMA slabs");
    const Dma dma(__builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane);
    // Byte offsets fit in 32 bits: the host only selects this path when each (batch, head) slab of K, V,
    // gK and gV spans less than 2^31 bytes.
    const uint32_t krs = (uint32_t)p.k.sr * 2, vrs = (uint32_t)p.v.sr * 2;
    const uint32_t gkrs = has_gk ? (uint32_t)p.gk.sr * 2 : 0u, gvrs = has_gv ? (uint32_t)p.gv.sr * 2 : 0u;
    const rsrc_t krsrc = make_rsrc(K, (uint32_t)slab_span(s.M, krs, 2 * DP)),
                  vrsrc = make_rsrc(V, (uint32_t)slab_span(s.M, vrs, 2 * DP));
    const rsrc_t gkrsrc = make_rsrc(has_gk ? (const void*)GK : (const void*)K, (uint32_t)slab_span(s.M, gkrs, 2 * DP));
    const rsrc_t gvrsrc = make_rsrc(has_gv ? (const void*)GV : (const void*)V, (uint32_t)slab_span(s.M, gvrs, 2 * DP));
    auto issue = [&](int kt, char* tK, char* tV, char* tgK, char* tgV) {
      const int k0 = kt * BN;
      dma.template issue_clamped<NSLAB>(krsrc, krs, k0, s.M, tK);
      dma.template issue_clamped<NSLAB>(vrsrc, vrs, k0, s.M, tV);
      if (has_gk) dma.template issue_clamped<NSLAB>(gkrsrc, gkrs, k0, s.M, tgK);
      if (has_gv) dma.template issue_clamped<NSLAB>(gvrsrc, gvrs, k0, s.M, tgV);
    };
    // Tile kt from the set c*; the next tile's copies go to the set n* (read in the previous step, which
    // every wave has finished at the barrier).
    auto step = [&](auto pass_tag, int kt, const char* cK, const char* cV, const char* cgK, const char* cgV, char* nK,
                    char* nV, char* ngK, char* ngV) __attribute__((always_inline)) {
      wait_vm_all();
      __syncthreads();
      if (kt + 1 < nkt) issue(kt + 1, nK, nV, ngK, ngV);
      compute(pass_tag, kt, cK, cV, cgK, cgV);
      __builtin_amdgcn_sched_barrier(0);  // keep the two unrolled steps apart (register pressure)
    };
    // every key tile once, from tile 0 already issued
    auto sweep = [&](auto pass_tag) __attribute__((always_inline)) {
      int kt = 0;
      for (; kt + 1 < nkt; kt += 2) {
        step(pass_tag, kt, sK0, sV0, sgK0, sgV0, sK1, sV1, sgK1, sgV1);
        step(pass_tag, kt + 1, sK1, sV1, sgK1, sgV1, sK0, sV0, sgK0, sgV0);
      }
      if (kt < nkt) step(pass_tag, kt, sK0, sV0, sgK0, sgV0, sK1, sV1, sgK1, sgV1);
    };
    if (nkt > 0) {
      issue(0, sK0, sV0, sgK0, sgV0);
      if (exact) {
        sweep(exact_pass);
      } else if (two_pass) {
        sweep(pre_pass);  // r and t of every row from all its keys
        set_exact_terms();
        __syncthreads();  // every wave is done with the last tile's buffers
        issue(0, sK0, sV0, sgK0, sgV0);
        sweep(exact_pass);
      } else {
        if constexpr (sizeof(T) == 2) {
          wait_vm_all();
          __syncthreads();
          compute(pre_pass, 0, sK0, sV0, sgK0, sgV0);
          set_centre();
        }
        sweep(full_pass);
      }
    }
  } else {
    TileStage<T, BN, DP, NT> gsK, gsV, gsgK, gsgV;
    auto prefetch = [&](int k0) {
      gsK.load(K, p.k.sr, k0, s.M, s.D, s.vec);
      gsV.load(V, p.v.sr, k0, s.M, s.D, s.vec);
      if (has_gk) gsgK.load(GK, p.gk.sr, k0, s.M, s.D, s.vec);
      if (has_gv) gsgV.load(GV, p.gv.sr, k0, s.M, s.D, s.vec);
    };
    // every key tile once, from tile 0 already prefetched
    auto sweep = [&](auto pass_tag) __attribute__((always_inline)) {
      for (int kt = 0; kt < nkt; ++kt) {
        __syncthreads();
        gsK.store((T*)sK0, PITCH);
        gsV.store((T*)sV0, PITCH);
        if (has_gk) gsgK.store((T*)sgK0, PITCH);
        if (has_gv) gsgV.store((T*)sgV0, PITCH);
        __syncthreads();
        if (kt + 1 < nkt) prefetch((kt + 1) * BN);
        compute(pass_tag, kt, sK0, sV0, sgK0, sgV0);
      }
    };
    if (nkt > 0) prefetch(0);
    if (exact) {
      if (nkt > 0) sweep(exact_pass);
    } else if (two_pass) {
      if (nkt > 0) {
        sweep(pre_pass);  // r and t of every row from all its keys
        set_exact_terms();
        prefetch(0);
        sweep(exact_pass);
      }
    } else {
      if (sizeof(T) == 2 && nkt > 0) {
        // centre pre-pass over tile 0 (the loop stages the same registers again)
        gsK.store((T*)sK0, PITCH);
        gsV.store((T*)sV0, PITCH);
        if (has_gk) gsgK.store((T*)sgK0, PITCH);
        if (has_gv) gsgV.store((T*)sgV0, PITCH);
        __syncthreads();
        compute(pre_pass, 0, sK0, sV0, sgK0, sgV0);
        set_centre();
      }
      sweep(full_pass);
    }
  }

  const float rr = two_pass ? rx : pair_sum(r_part), tt = two_pass ? tx : pair_sum(t_part);
  const float tg = sizeof(T) == 2 ? pair_sum(t_frag) : tt;  // t_c as G_Q uses it; the cols kernel takes tt
  const float rg = rr - cr;                                   // r - cr (cr = 0 for float32)
  if (qvalid) {
    T* OG = (T*)p.out_gq.p + b * p.out_gq.sb + h * p.out_gq.sh;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        const int d0 = dt * 32 + 8 * qd + 4 * g;
        if (d0 < s.D) {
          float r4[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int i = 4 * qd + e;
            r4[e] = s.scale * (x13[dt][i] - rg * x2[dt][i] - tg * x4[dt][i] + yk[dt][i]);
          }
          store4<T>(OG, p.out_gq.sr, myq, d0, s.D, r4[0], r4[1], r4[2], r4[3], s.vec);
        }
      }
    if (g == 0 && !EXACT) {
      p.r_row[row_id] = rr;
      p.t_row[row_id] = tt;
    }
  }
}

template <typename T, int DP, bool CAUSAL, bool DMA, bool EXACT>
__global__ __launch_bounds__(256) void bwdbwd_rows_kernel(const BwdBwdParams p) {
  rows_block<T, DP, CAUSAL, DMA, EXACT>(p, blockIdx.x, gridDim.x);
}

// DMA: as in the rows kernel, for the Q, dO, gQ tiles (the row terms are loaded two tiles ahead by the
// first BM threads and written beside them one tile ahead).
template <typename T, int DP, bool CAUSAL, bool DMA>
__device__ __attribute__((always_inline)) inline void cols_block(const BwdBwdParams& p, const int blk, const int nblk) {
  using MM = Mfma<T>;
  using F = typename MM::frag_t;
  constexpr int KC = MM::KC;
  constexpr int NW = 4, BN = 32 * NW, NT = 64 * NW;
  // queries per tile: two 32-query subtiles per tile where the registers allow
  constexpr int BM = (DP == 128 || sizeof(T) == 4 || DMA) ? 32 : 64;
  constexpr int PITCH = DP + 16 / (int)sizeof(T);
  constexpr int NDT = DP / 32, NKC = DP / KC, NPC = 32 / KC, NSQ = BM / 32;
  constexpr int TB = DMA ? BM * DP * 2 : BM * PITCH * (int)sizeof(T);  // bytes per tile
  constexpr int TB2 = DMA ? TB : 16;                                    // second set (DMA only)
  // float32 (OWN): P = exp2((fl(S c2) - m2) - L2) with the rows' own m2 (in lse) and L2 (row_l2), and dP formed
  // from zero, as in the row-term pass that wrote them
  constexpr bool OWN = sizeof(T) == 4;
  constexpr int FLAG = OWN ? 5 * BM : 4 * BM;  // row terms, then whether the tile holds a row flagged peaked
  constexpr int RB = FLAG + 4;
  constexpr int RB2 = DMA ? RB : 4;
  __shared__ __attribute__((aligned(1024))) char sQ0[TB];
  __shared__ __attribute__((aligned(1024))) char sdO0[TB];
  __shared__ __attribute__((aligned(1024))) char sgQ0[TB];
  __shared__ __attribute__((aligned(1024))) char sQ1[TB2];
  __shared__ __attribute__((aligned(1024))) char sdO1[TB2];
  __shared__ __attribute__((aligned(1024))) char sgQ1[TB2];
  // row terms [lse * log2(e) (float32: m2) | delta | r | t | (float32: L2) | peaked] of a tile
  __shared__ __attribute__((aligned(16))) float sRow0[RB];
  __shared__ __attribute__((aligned(16))) float sRow1[RB2];

  const Shape& s = p.s;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6, li = lane & 31, g = lane >> 5;
  const int nkb = (s.M + BN - 1) / BN;
  const int bid = xcd_remap(blk, nblk);
  const int bh = bid / nkb;
  const int kb = bid - bh * nkb;
  const int b = bh / s.H, h = bh - b * s.H;
  const T* Q = (const T*)p.q.p + b * p.q.sb + h * p.q.sh;
  const T* K = (const T*)p.k.p + b * p.k.sb + h * p.k.sh;
  const T* V = (const T*)p.v.p + b * p.v.sb + h * p.v.sh;
  const T* dO = (const T*)p.dout.p + b * p.dout.sb + h * p.dout.sh;
  const bool has_gq = p.gq.p != nullptr, has_gk = p.gk.p != nullptr, has_gv = p.gv.p != nullptr;
  const T* GQ = has_gq ? (const T*)p.gq.p + b * p.gq.sb + h * p.gq.sh : nullptr;
  const T* GK = has_gk ? (const T*)p.gk.p + b * p.gk.sb + h * p.gk.sh : nullptr;
  const T* GV = has_gv ? (const T*)p.gv.p + b * p.gv.sb + h * p.gv.sh : nullptr;
  const int key0 = kb * BN;
  const int kw0 = key0 + wave * 32;
  const int mykey = kw0 + li;
  const bool kvalid = mykey < s.M;

  F kf[NKC], vf[NKC], gkf[NKC], gvf[NKC];
#pragma unroll
  for (int c = 0; c < NKC; ++c) {
    kf[c] = gload_frag<T>(K, p.k.sr, mykey, s.M, c, s.D, s.vec);
    vf[c] = gload_frag<T>(V, p.v.sr, mykey, s.M, c, s.D, s.vec);
    gkf[c] = has_gk ? gload_frag<T>(GK, p.gk.sr, mykey, s.M, c, s.D, s.vec) : F{};
    gvf[c] = has_gv ? gload_frag<T>(GV, p.gv.sr, mykey, s.M, c, s.D, s.vec) : F{};
  }
  f32x16_t accV[NDT], accK[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
    accV[dt] = zero16();
    accK[dt] = zero16();
  }
  const float c2 = s.scale * kLog2e;
  const int qbeg = CAUSAL ? (key0 / BM) * BM : 0;
  const int nqt = s.T > qbeg ? (s.T - qbeg + BM - 1) / BM : 0;
  const int64_t rowbase = (int64_t)bh * s.T;

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

  // Row terms of a tile for thread tid < BM, held raw (rows past the end: lse = +inf) and converted when
  // stored: lse * log2(e) (+inf for rows past the end or without visible keys, so P = 0), delta, r, t.
  float r_lse = THERIA_INF, r_z = 0.f, r_r = 0.f, r_t = 0.f, r_l2 = 0.f;
  auto load_rows = [&](int it) {
    if (tid < BM && it < nqt) {
      const int qq = qbeg + it * BM + tid;
      const bool ok = qq < s.T;
      r_lse = ok ? p.lse[rowbase + qq] : THERIA_INF;
      r_z = ok ? p.delta[rowbase + qq] : 0.f;
      r_r = ok ? p.r_row[rowbase + qq] : 0.f;
      r_t = ok ? p.t_row[rowbase + qq] : 0.f;
      if constexpr (OWN) r_l2 = ok ? p.row_l2[rowbase + qq] : 0.f;
    }
  };
  auto store_rows = [&](float* sr) {
    if (tid < BM) {
      // float32: m2 as it is (+inf for a row without visible keys or past the end, so P = 0)
      sr[tid] = OWN ? r_lse : (__builtin_isinf(r_lse) ? THERIA_INF : r_lse * kLog2e);
      sr[BM + tid] = r_z;
      sr[2 * BM + tid] = r_r;
      sr[3 * BM + tid] = r_t;
      if constexpr (OWN) sr[4 * BM + tid] = r_l2;
      const bool pk = !OWN && __any(lse_peaked(r_lse));  // the tile's rows are the lanes of wave 0
      if (tid == 0) sr[FLAG] = pk ? 1.f : 0.f;
    }
  };

  // The query tile it held in (tQ, tO, tgQ) with its row terms in sr, as 32-query subtiles. SPLIT: Gbar_dP,
  // Gbar_S and dS enter the products as two 16-bit terms each.
  auto tile = [&](auto split_tag, int it, const char* tQ, const char* tO, const char* tgQ,
                  const float* sr) __attribute__((always_inline)) {
    constexpr bool SPLIT = decltype(split_tag)::value;
    const int q0 = qbeg + it * BM;
    if (CAUSAL && kw0 > q0 + BM - 1) return;
#pragma unroll
    for (int sq = 0; sq < NSQ; ++sq) {
      const int q0s = q0 + 32 * sq;  // this 32-query subtile
      if (CAUSAL && kw0 > q0s + 31) continue;

      f32x16_t sc = zero16(), gm = zero16(), w = zero16(), dpz;
      f32x4_t l4[4], z4[4], r4[4], t4[4], lo4[4];
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        const int o = 32 * sq + 8 * qd + 4 * g;
        l4[qd] = *reinterpret_cast<const f32x4_t*>(sr + o);
        z4[qd] = *reinterpret_cast<const f32x4_t*>(sr + BM + o);
        r4[qd] = *reinterpret_cast<const f32x4_t*>(sr + 2 * BM + o);
        t4[qd] = *reinterpret_cast<const f32x4_t*>(sr + 3 * BM + o);
        if constexpr (OWN) lo4[qd] = *reinterpret_cast<const f32x4_t*>(sr + 4 * BM + o);
#pragma unroll
        for (int e = 0; e < 4; ++e) dpz[4 * qd + e] = OWN ? 0.f : -z4[qd][e];
      }
#pragma unroll
      for (int c = 0; c < NKC; ++c) {
        const F qfr = colsf(tQ, 32 * sq + li, c);
        const F ofr = colsf(tO, 32 * sq + li, c);
        sc = MM::mma(qfr, kf[c], sc);
        dpz = MM::mma(ofr, vf[c], dpz);
        if (has_gq) gm = MM::mma(colsf(tgQ, 32 * sq + li, c), kf[c], gm);
        if (has_gk) gm = MM::mma(qfr, gkf[c], gm);
        if (has_gv) w = MM::mma(ofr, gvf[c], w);
      }
      const bool diag = CAUSAL && (kw0 + 31 > q0s);
      f32x16_t gdp, gs;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int qd = r >> 2, e = r & 3;
        if constexpr (OWN) dpz[r] -= z4[qd][e];
        float pv = OWN ? own_prob(sc[r], c2, l4[qd][e], lo4[qd][e]) : fast_exp2(fmaf(sc[r], c2, -l4[qd][e]));
        if (!kvalid) pv = 0.f;
        if (diag && mykey > q0s + acc_row(r, g)) pv = 0.f;
        const float gam = s.scale * gm[r];
        const float ds = pv * dpz[r];
        const float e1 = fmaf(gam, dpz[r], w[r]);
        gdp[r] = pv * (gam - r4[qd][e]);
        gs[r] = pv * e1 - r4[qd][e] * ds - t4[qd][e] * pv;
        dpz[r] = ds;
      }
      if constexpr (SPLIT && sizeof(T) == 2) {
#pragma unroll
        for (int cc = 0; cc < NPC; ++cc) {
          F gdph, gdpl, gsh, gsl, dsh, dsl;
          split_frag<T>(gdp, cc, gdph, gdpl);
          split_frag<T>(gs, cc, gsh, gsl);
          split_frag<T>(dpz, cc, dsh, dsl);
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) {
            const F ro = rowsf(tO, 32 * sq, cc, dt * 32);
            accV[dt] = MM::mma(gdph, ro, accV[dt]);
            accV[dt] = MM::mma(gdpl, ro, accV[dt]);
            const F rq = rowsf(tQ, 32 * sq, cc, dt * 32);
            accK[dt] = MM::mma(gsh, rq, accK[dt]);
            accK[dt] = MM::mma(gsl, rq, accK[dt]);
            if (has_gq) {
              const F rg = rowsf(tgQ, 32 * sq, cc, dt * 32);
              accK[dt] = MM::mma(dsh, rg, accK[dt]);
              accK[dt] = MM::mma(dsl, rg, accK[dt]);
            }
          }
        }
      } else {
#pragma unroll
        for (int cc = 0; cc < NPC; ++cc) {
          const F gdpf = acc_frag<T>(gdp, cc);
          const F gsf = acc_frag<T>(gs, cc);
          const F dsf = acc_frag<T>(dpz, cc);
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) {
            accV[dt] = MM::mma(gdpf, rowsf(tO, 32 * sq, cc, dt * 32), accV[dt]);
            accK[dt] = MM::mma(gsf, rowsf(tQ, 32 * sq, cc, dt * 32), accK[dt]);
            if (has_gq) accK[dt] = MM::mma(dsf, rowsf(tgQ, 32 * sq, cc, dt * 32), accK[dt]);
          }
        }
      }
    }
  };
  const std::integral_constant<bool, true> with_split;
  const std::integral_constant<bool, false> no_split;
  bool pk_any = false;  // uniform: a tile holding a peaked row was skipped (16-bit)
  auto compute = [&](int it, const char* tQ, const char* tO, const char* tgQ,
                     const float* sr) __attribute__((always_inline)) {
    // uniform: every thread reads the same flag
    const bool pk = sizeof(T) == 2 && __builtin_amdgcn_readfirstlane(__float_as_uint(sr[FLAG])) != 0u;
    pk_any |= pk;  // run after the loop, so the loop's schedule holds only the one-term products
    if (!pk) tile(no_split, it, tQ, tO, tgQ, sr);
  };
  // The tiles holding a peaked row, found 64 at a time from the lse flags and run one after the other with
  // the split products, from stage(it) (loads tile it into sQ0, sdO0, sgQ0 and its row terms into sRow0).
  auto peaked_tiles = [&](auto stage) __attribute__((always_inline)) {
    __shared__ int sPk[64];
    for (int t0 = 0; t0 < nqt; t0 += 64) {
      const int nt = min(64, nqt - t0);
      __syncthreads();  // every thread is done with the previous flags and tile buffers
      if (tid < 64) sPk[tid] = 0;
      __syncthreads();
      constexpr int RPT = (64 * BM + NT - 1) / NT;
      const int r0 = qbeg + t0 * BM, r1 = min(s.T, qbeg + (t0 + nt) * BM);
      float lv[RPT];
#pragma unroll
      for (int j = 0; j < RPT; ++j) {
        const int r = r0 + tid + NT * j;
        lv[j] = r < r1 ? p.lse[rowbase + r] : THERIA_INF;  // rows past the end: no flag
      }
#pragma unroll
      for (int j = 0; j < RPT; ++j)
        if (lse_peaked(lv[j])) sPk[(tid + NT * j) / BM] = 1;
      __syncthreads();
      for (int i = 0; i < nt; ++i) {
        if (!sPk[i]) continue;  // uniform: every thread reads the same flag
        stage(t0 + i);
        __syncthreads();
        tile(with_split, t0 + i, sQ0, sdO0, sgQ0, sRow0);
        __syncthreads();  // the tile buffers are free again
      }
    }
  };

  if constexpr (DMA) {
    using Dma = SwzDma<NW, DP>;
    constexpr int NSLAB = BM / Dma::SLAB_ROWS;
    static_assert(NSLAB * Dma::SLAB_ROWS == BM, "query tiles must be whole DMA slabs");
    const Dma dma(__builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane);
    // Byte offsets fit in 32 bits: the host only selects this path when each (batch, head) slab of Q, dO
    // and gQ spans less than 2^31 bytes.
    const uint32_t qrs = (uint32_t)p.q.sr * 2, ors = (uint32_t)p.dout.sr * 2;
    const uint32_t gqrs = has_gq ? (uint32_t)p.gq.sr * 2 : 0u;
    const rsrc_t qrsrc = make_rsrc(Q, (uint32_t)slab_span(s.T, qrs, 2 * DP)),
                  orsrc = make_rsrc(dO, (uint32_t)slab_span(s.T, ors, 2 * DP));
    const rsrc_t gqrsrc = make_rsrc(has_gq ? (const void*)GQ : (const void*)Q, (uint32_t)slab_span(s.T, gqrs, 2 * DP));
    auto issue = [&](int it, char* tQ, char* tO, char* tgQ) {
      const int q0 = qbeg + it * BM;
      dma.template issue_clamped<NSLAB>(qrsrc, qrs, q0, s.T, tQ);
      dma.template issue_clamped<NSLAB>(orsrc, ors, q0, s.T, tO);
      if (has_gq) dma.template issue_clamped<NSLAB>(gqrsrc, gqrs, q0, s.T, tgQ);
    };
    auto step = [&](int it, const char* cQ, const char* cO, const char* cgQ, const float* cR, char* nQ, char* nO,
                    char* ngQ, float* nR) {
      wait_vm_all();
      __syncthreads();  // tile it (and its row terms) visible; the other set (tile it-1) is free
      if (it + 1 < nqt) {
        issue(it + 1, nQ, nO, ngQ);
        store_rows(nR);
        load_rows(it + 2);
      }
      compute(it, cQ, cO, cgQ, cR);
      __builtin_amdgcn_sched_barrier(0);  // keep the two unrolled steps apart (register pressure)
    };
    if (nqt > 0) {
      issue(0, sQ0, sdO0, sgQ0);
      load_rows(0);
      wait_vm_all();
      store_rows(sRow0);
      load_rows(1);
      int it = 0;
      for (; it + 1 < nqt; it += 2) {
        step(it, sQ0, sdO0, sgQ0, sRow0, sQ1, sdO1, sgQ1, sRow1);
        step(it + 1, sQ1, sdO1, sgQ1, sRow1, sQ0, sdO0, sgQ0, sRow0);
      }
      if (it < nqt) step(it, sQ0, sdO0, sgQ0, sRow0, sQ1, sdO1, sgQ1, sRow1);
    }
    if (pk_any)
      peaked_tiles([&](int it) __attribute__((always_inline)) {
        issue(it, sQ0, sdO0, sgQ0);
        load_rows(it);
        wait_vm_all();
        store_rows(sRow0);
      });
  } else {
    TileStage<T, BM, DP, NT> gsQ, gsO, gsgQ;
    auto prefetch = [&](int it) {
      const int q0 = qbeg + it * BM;
      gsQ.load(Q, p.q.sr, q0, s.T, s.D, s.vec);
      gsO.load(dO, p.dout.sr, q0, s.T, s.D, s.vec);
      if (has_gq) gsgQ.load(GQ, p.gq.sr, q0, s.T, s.D, s.vec);
      load_rows(it);
    };
    if (nqt > 0) prefetch(0);
    for (int it = 0; it < nqt; ++it) {
      __syncthreads();
      gsQ.store((T*)sQ0, PITCH);
      gsO.store((T*)sdO0, PITCH);
      if (has_gq) gsgQ.store((T*)sgQ0, PITCH);
      store_rows(sRow0);
      __syncthreads();
      if (it + 1 < nqt) prefetch(it + 1);
      compute(it, sQ0, sdO0, sgQ0, sRow0);
    }
    if (pk_any)
      peaked_tiles([&](int it) __attribute__((always_inline)) {
        prefetch(it);
        gsQ.store((T*)sQ0, PITCH);
        gsO.store((T*)sdO0, PITCH);
        if (has_gq) gsgQ.store((T*)sgQ0, PITCH);
        store_rows(sRow0);
      });
  }

  T* OV = (T*)p.out_gv.p + b * p.out_gv.sb + h * p.out_gv.sh;
  T* OK = (T*)p.out_gk.p + b * p.out_gk.sb + h * p.out_gk.sh;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
    const int d = dt * 32 + li;
    if (d < s.D) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kw0 + acc_row(r, g);
        if (key < s.M) {
          OV[(int64_t)key * p.out_gv.sr + d] = (T)accV[dt][r];
          OK[(int64_t)key * p.out_gk.sr + d] = (T)(accK[dt][r] * s.scale);
        }
      }
    }
  }
}

template <typename T, int DP, bool CAUSAL, bool DMA>
__global__ __launch_bounds__(256) void bwdbwd_cols_kernel(const BwdBwdParams p) {
  cols_block<T, DP, CAUSAL, DMA>(p, blockIdx.x, gridDim.x);
}

// 16-bit: the rows kernel's second (exact) launch and the column blocks as one grid. The exact row blocks
// read only what the first rows launch wrote (r, t) and write only G_Q, so they are independent of the
// column blocks; in one grid they run beside them, instead of as a launch of their own whose few busy
// workgroups would leave the GPU idle.
template <typename T, int DP, bool CAUSAL, bool DMA>
__global__ __launch_bounds__(256) void bwdbwd_cols_exact_kernel(const BwdBwdParams p) {
  const int ncols = ((p.s.M + 127) / 128) * p.s.B * p.s.H;
  const int nrows = (int)gridDim.x - ncols;
  const int bid = blockIdx.x;  // uniform
  // Row blocks first: most exit at once (no flagged row), and the few heavy ones (a single peaked row makes
  // its block sweep every key) start at once. A workgroup waits for the CU of its own place in the grid,
  // so the column block placed like a heavy row block starts when that one ends; for causal problems the
  // row blocks run in query order (no heavy-first reversal), which pairs query block i with key block i,
  // whose lengths (i + 1 and n - i key tiles) add up to about the longest column block's.
  if (bid < nrows)
    rows_block<T, DP, CAUSAL, DMA, true>(p, bid, nrows);
  else
    cols_block<T, DP, CAUSAL, DMA>(p, bid - nrows, ncols);
}

// The LDS-DMA tile path applies: 16-bit inputs, head dim exactly DP (64 or 128), 16-byte-aligned views,
// and every (batch, head) slab of the streamed tensors (rows x row stride) below 2^31 bytes.
template <typename T, int DP>
static bool dma_tiles_ok(const BwdBwdParams& p, int64_t rows, std::initializer_list<const View*> streamed) {
  if (!(sizeof(T) == 2 && (DP == 64 || DP == 128) && p.s.D == DP && p.s.vec)) return false;
  for (const View* v : streamed)
    if (v->p && !slab_fits_dma(rows, v->sr, p.s.D)) return false;
  return true;
}

template <typename T, int DP>
static bool rows_dma(const BwdBwdParams& p) {
  return dma_tiles_ok<T, DP>(p, p.s.M, {&p.k, &p.v, &p.gk, &p.gv});
}
template <typename T, int DP>
static bool cols_dma(const BwdBwdParams& p) {
  return dma_tiles_ok<T, DP>(p, p.s.T, {&p.q, &p.dout, &p.gq});
}
// The split kernels' LDS-DMA tiles: 16-bit inputs, a head dim that is a multiple of 8 up to 64 (computed at 64,
// the tile columns past D zero-filled by the DMA), 16-byte-aligned views, and every (batch, head) slab of the
// streamed tensors below 2^31 bytes.
template <typename T>
static bool split_tiles_ok(const BwdBwdParams& p, int64_t rows, std::initializer_list<const View*> streamed) {
  if (!(sizeof(T) == 2 && p.s.dp <= 64 && p.s.D % 8 == 0 && p.s.vec)) return false;
  for (const View* v : streamed)
    if (v->p && !slab_fits_dma(rows, v->sr, p.s.D)) return false;
  return true;
}

// The key-split row kernel takes 16-bit problems at head dims up to 64 whose K, V, gK, gV slabs allow LDS DMA.
template <typename T, int DP>
static bool rows_ks_ok(const BwdBwdParams& p) {
  return (DP == 32 || DP == 64) && split_tiles_ok<T>(p, p.s.M, {&p.k, &p.v, &p.gk, &p.gv});
}

// 16-bit: the rows kernel's exact launch rides in the column grid when both take the same tile path.
template <typename T, int DP>
static bool exact_in_cols(const BwdBwdParams& p) {
  return sizeof(T) == 2 && !rows_ks_ok<T, DP>(p) && rows_dma<T, DP>(p) == cols_dma<T, DP>(p);
}

// The row pass for 16-bit inputs at head dims up to 64 with LDS-DMA tiles (FD: exactly 64; otherwise a multiple of
// 8, the tile columns past D zero-filled), as two key groups of four waves (eight-wave workgroups, two waves per
// SIMD): the keys of each query block are split between the groups, whose partial sums meet in LDS. Each group makes two passes over its key tiles:
//   1. with P from the forward's lse: L = sum_j P, sum_j P Gam and the largest P, and the D-wide products
//      A = sum_j (P o Gam) V + sum_j P gV and O = sum_j P V, partial per group, then exchanged. Then
//      sum_j P dP = dO . O and sum_j P (Gam dP + W) = dO . A, which give the row's exact normaliser (P_c = P / L:
//      a 16-bit forward's lse comes from rounded probabilities, so P sums to one only within ~2^-9), the row
//      term z = sum_j P dP / L and the second-order row terms r = sum_j P_c Gam and t = sum_j P_c E1 with
//      E1 = Gam (dP - z) + W, i.e. t = (dO . A - z sum_j P Gam) / L; and G_dO = (A - r O) / L, the JVP of O;
//   2. G_Q = s sum_j (Gbar_S K + dS gK) with Gbar_S = P_c o ((Gam - r)(dP - z) + W - t), the exact form, in two
//      D-wide accumulators.
// Waves holding a row flagged peaked in the forward's lse enter P, P o Gam, Gbar_S and dS as two 16-bit terms.
// Every row takes the exact form (no centring, no second launch for flagged rows, no separate row-term or JVP
// pass); the gQ fragments sit in LDS, so that each pass's two accumulators, the per-wave Q and dO fragments and
// the products fit 256 registers. Writes G_Q and G_dO, and r, t, z and lse + ln L (flagged peaked when the
// row's largest P_c exceeds 1/4) for the column kernel. ALL: gQ, gK and gV are all given (the presence tests are
// then constants, and the loop bodies have no branches between their products).
template <typename T, bool CAUSAL, bool ALL, bool FD>
__global__ __launch_bounds__(512, 2) void bwdbwd_rows_ks_kernel(const BwdBwdParams p) {
  using MM = Mfma<T>;
  using F = typename MM::frag_t;
  static_assert(sizeof(T) == 2, "16-bit inputs only");
  constexpr int DP = 64, NW = 4, BM = 32 * NW, BN = 64, NST = BN / 32;
  constexpr int NDT = DP / 32, NKC = DP / MM::KC, NPC = 32 / MM::KC;
  constexpr int TB = BN * DP * 2;  // bytes per tile
  using Dma = SwzDma<NW, DP>;
  constexpr int NSLAB = BN / Dma::SLAB_ROWS;
  static_assert(NSLAB * Dma::SLAB_ROWS == BN, "key tiles must be whole DMA slabs");
  // [group][set][K, V, gK, gV]; reused for the exchanges between the passes and after the second
  __shared__ __attribute__((aligned(1024))) char smem[2 * 2 * 4 * TB];
  static_assert(sizeof(smem) >= 4 * (4096 + 2 * NDT * 16 * 256), "the exchanges fit in the tile memory");
  // the gQ fragments of the four query slices (both key groups read them; kept here rather than in registers,
  // which the two passes' accumulators fill): fragment c of lane l of slice w at (w * NKC + c) * 64 + l
  __shared__ __attribute__((aligned(16))) F sGQ[NW * NKC * 64];

  const Shape& s = p.s;
  const int lane = threadIdx.x & 63, li = lane & 31, g = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = wave >> 2, wig = wave & 3;  // key group, wave in group
  const int nqb = (s.T + BM - 1) / BM;
  const int bid = xcd_remap(blockIdx.x, gridDim.x);
  const int bh = bid / nqb;
  int qb = bid - bh * nqb;
  if (CAUSAL) qb = nqb - 1 - qb;  // longest first
  const int b = bh / s.H, h = bh - b * s.H;
  const T* Q = (const T*)p.q.p + b * p.q.sb + h * p.q.sh;
  const T* K = (const T*)p.k.p + b * p.k.sb + h * p.k.sh;
  const T* V = (const T*)p.v.p + b * p.v.sb + h * p.v.sh;
  const T* dO = (const T*)p.dout.p + b * p.dout.sb + h * p.dout.sh;
  const bool has_gq = ALL || p.gq.p != nullptr, has_gk = ALL || p.gk.p != nullptr, has_gv = ALL || p.gv.p != nullptr;
  const T* GQ = has_gq ? (const T*)p.gq.p + b * p.gq.sb + h * p.gq.sh : nullptr;
  const T* GK = has_gk ? (const T*)p.gk.p + b * p.gk.sb + h * p.gk.sh : nullptr;
  const T* GV = has_gv ? (const T*)p.gv.p + b * p.gv.sb + h * p.gv.sh : nullptr;
  const int q0w = qb * BM + wig * 32;
  const int myq = q0w + li;
  const bool qvalid = myq < s.T;
  const int64_t row_id = (int64_t)bh * s.T + myq;

  F qf[NKC], dof[NKC];
#pragma unroll
  for (int c = 0; c < NKC; ++c) {
    qf[c] = gload_frag<T>(Q, p.q.sr, myq, s.T, c, s.D, s.vec);
    dof[c] = gload_frag<T>(dO, p.dout.sr, myq, s.T, c, s.D, s.vec);
    // read after the first barrier of the first sweep
    if (has_gq && grp == 0) sGQ[(wig * NKC + c) * 64 + lane] = gload_frag<T>(GQ, p.gq.sr, myq, s.T, c, s.D, s.vec);
  }
  const float c2 = s.scale * kLog2e;
  const float lse_raw = qvalid ? p.lse_fwd[row_id] : THERIA_INF;
  const float lse2 = lse_raw * kLog2e;
  float moff = lse2 == -THERIA_INF ? THERIA_INF : lse2;  // a row without visible keys has P = 0; pass 2: P_c
  float z = 0.f;                                          // pass 2: the row term (pass 1 forms dP itself)
  const bool split = __any(lse_peaked(lse_raw));  // uniform per wave (the forward's bound: a superset)

  int kend = s.M;
  if (CAUSAL) kend = min(s.M, qb * BM + BM);
  const int nkt = (kend + BN - 1) / BN;
  const int half = (nkt + 1) / 2;
  const int kt0 = grp * half, kt1 = min(nkt, kt0 + half);  // this group's tiles [kt0, kt1)

  // S^T, Gam^T / s and (FULL) W^T and dP^T - z of 32-key subtile st of the tile in (tK, tV, tgK, tgV); P from S.
  // MASK: the tile reaches past the last key or (causal) past this wave's first query.
  auto products = [&](auto full_tag, auto mask_tag, int k0s, const char* tK, const char* tV, const char* tgK,
                      const char* tgV, int st, f32x16_t& pv, f32x16_t& gm, f32x16_t& w,
                      f32x16_t& dpz) __attribute__((always_inline)) {
    constexpr bool FULL = decltype(full_tag)::value;
    constexpr bool MASK = decltype(mask_tag)::value;
    f32x16_t sc = zero16();
    gm = zero16();
    if constexpr (FULL) {
      w = zero16();
#pragma unroll
      for (int r = 0; r < 16; ++r) dpz[r] = -z;
    }
#pragma unroll
    for (int c = 0; c < NKC; ++c) {
      const F kfr = swz_cols<T, DP>(tK, 32 * st + li, c);
      sc = MM::mma(kfr, qf[c], sc);
      if constexpr (FULL) dpz = MM::mma(swz_cols<T, DP>(tV, 32 * st + li, c), dof[c], dpz);
      if (has_gq) gm = MM::mma(kfr, sGQ[(wig * NKC + c) * 64 + lane], gm);
      if (has_gk) gm = MM::mma(swz_cols<T, DP>(tgK, 32 * st + li, c), qf[c], gm);
      if constexpr (FULL)
        if (has_gv) w = MM::mma(swz_cols<T, DP>(tgV, 32 * st + li, c), dof[c], w);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float x = fast_exp2(fmaf(sc[r], c2, -moff));
      if constexpr (MASK) {
        const int key = k0s + acc_row(r, g);
        if (key >= s.M || (CAUSAL && key > myq)) x = 0.f;
      }
      pv[r] = x;
    }
  };

  // pass 1: sum_j of P and P Gam, and max_j P (this lane's keys); sum_j P dP and sum_j P (Gam dP + W) follow from
  // the G_dO products as dO . sum_j P V and dO . (sum_j (P o Gam) V + sum_j P gV)
  float l_part = 0.f, r_part = 0.f, p_max = 0.f;
  float rx = 0.f, tx = 0.f;  // r, t of the row after the exchange
  f32x16_t acc[NDT], accy[NDT];  // pass 2: sum_j Gbar_S K and sum_j dS gK (transposed, lane per query)

  // G_dO (the JVP of O along (gQ, gK, gV)) from pass 1, as the JVP kernel forms it with normalised P:
  // G_dO = (sum_j (P o Gam) V + sum_j P gV) / L - r (sum_j P V) / L (jvp_kernel's epilogue). The first two sums
  // share one accumulator (their products chain into it).
  f32x16_t acc_a[NDT], acc_o[NDT];  // sum_j (P o Gam) V + sum_j P gV, and sum_j P V (transposed)
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) acc_a[dt] = acc_o[dt] = zero16();

  // PASS 1: the row sums and the G_dO products over this group's keys (SPLIT: P o Gam and P as two 16-bit terms).
  auto compute_sums = [&](auto split_tag, auto mask_tag, int kt, const char* tK, const char* tV, const char* tgK,
                          const char* tgV) __attribute__((always_inline)) {
    constexpr bool SPLIT = decltype(split_tag)::value;
#pragma unroll
    for (int st = 0; st < NST; ++st) {
      const int k0s = kt * BN + 32 * st;
      if (CAUSAL && k0s > q0w + 31) continue;
      f32x16_t pv, gm, w, dpz;
      products(std::false_type{}, mask_tag, k0s, tK, tV, tgK, tgV, st, pv, gm, w, dpz);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float pg = pv[r] * (s.scale * gm[r]);  // P o Gam
        l_part += pv[r];
        r_part += pg;
        p_max = fmaxf(p_max, pv[r]);
        gm[r] = pg;
      }
#pragma unroll
      for (int cc = 0; cc < NPC; ++cc) {
        if constexpr (SPLIT) {
          F ph, pl, gh, gl;
          split_frag<T>(pv, cc, ph, pl);
          split_frag<T>(gm, cc, gh, gl);
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) {
            const F vr = swz_rows<T, DP>(tV, 32 * st, cc, dt * 32);
            acc_a[dt] = MM::mma(vr, gh, acc_a[dt]);
            acc_a[dt] = MM::mma(vr, gl, acc_a[dt]);
            if (has_gv) {
              const F gvr = swz_rows<T, DP>(tgV, 32 * st, cc, dt * 32);
              acc_a[dt] = MM::mma(gvr, ph, acc_a[dt]);
              acc_a[dt] = MM::mma(gvr, pl, acc_a[dt]);
            }
            acc_o[dt] = MM::mma(vr, ph, acc_o[dt]);
            acc_o[dt] = MM::mma(vr, pl, acc_o[dt]);
          }
        } else {
          const F pf = acc_frag<T>(pv, cc), gf = acc_frag<T>(gm, cc);
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) {
            const F vr = swz_rows<T, DP>(tV, 32 * st, cc, dt * 32);
            acc_a[dt] = MM::mma(vr, gf, acc_a[dt]);
            if (has_gv) acc_a[dt] = MM::mma(swz_rows<T, DP>(tgV, 32 * st, cc, dt * 32), pf, acc_a[dt]);
            acc_o[dt] = MM::mma(vr, pf, acc_o[dt]);
          }
        }
      }
    }
  };
  // PASS 2: Gbar_S and dS products (SPLIT: two 16-bit terms each).
  auto compute_exact = [&](auto split_tag, auto mask_tag, int kt, const char* tK, const char* tV, const char* tgK,
                           const char* tgV) __attribute__((always_inline)) {
    constexpr bool SPLIT = decltype(split_tag)::value;
#pragma unroll
    for (int st = 0; st < NST; ++st) {
      const int k0s = kt * BN + 32 * st;
      if (CAUSAL && k0s > q0w + 31) continue;
      f32x16_t pv, gm, w, dpz;
      products(std::true_type{}, mask_tag, k0s, tK, tV, tgK, tgV, st, pv, gm, w, dpz);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float gam = s.scale * gm[r];
        gm[r] = pv[r] * (fmaf(gam - rx, dpz[r], w[r]) - tx);  // Gbar_S
        dpz[r] = pv[r] * dpz[r];                              // dS
      }
#pragma unroll
      for (int cc = 0; cc < NPC; ++cc) {
        if constexpr (SPLIT) {
          F gh, gl, dh, dl;
          split_frag<T>(gm, cc, gh, gl);
          split_frag<T>(dpz, cc, dh, dl);
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) {
            const F kr = swz_rows<T, DP>(tK, 32 * st, cc, dt * 32);
            acc[dt] = MM::mma(kr, gh, acc[dt]);
            acc[dt] = MM::mma(kr, gl, acc[dt]);
            if (has_gk) {
              const F gkr = swz_rows<T, DP>(tgK, 32 * st, cc, dt * 32);
              accy[dt] = MM::mma(gkr, dh, accy[dt]);
              accy[dt] = MM::mma(gkr, dl, accy[dt]);
            }
          }
        } else {
          const F gf = acc_frag<T>(gm, cc), df = acc_frag<T>(dpz, cc);
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) {
            acc[dt] = MM::mma(swz_rows<T, DP>(tK, 32 * st, cc, dt * 32), gf, acc[dt]);
            if (has_gk) accy[dt] = MM::mma(swz_rows<T, DP>(tgK, 32 * st, cc, dt * 32), df, accy[dt]);
          }
        }
      }
    }
  };

  const Dma dma(wig, lane, FD ? 8 : s.D / 8);  // FD: head dim 64; else tile columns D .. 63 zero-filled
  // Byte offsets fit in 32 bits: the host only selects this kernel when each (batch, head) slab of K, V, gK and
  // gV spans less than 2^31 bytes.
  const uint32_t krs = (uint32_t)p.k.sr * 2, vrs = (uint32_t)p.v.sr * 2;
  const uint32_t gkrs = has_gk ? (uint32_t)p.gk.sr * 2 : 0u, gvrs = has_gv ? (uint32_t)p.gv.sr * 2 : 0u;
  const int64_t rb = 2 * (FD ? 64 : s.D);  // bytes of a row the DMA reads
  const rsrc_t krsrc = make_rsrc(K, (uint32_t)slab_span(s.M, krs, rb)),
               vrsrc = make_rsrc(V, (uint32_t)slab_span(s.M, vrs, rb));
  const rsrc_t gkrsrc = make_rsrc(has_gk ? (const void*)GK : (const void*)K, (uint32_t)slab_span(s.M, gkrs, rb));
  const rsrc_t gvrsrc = make_rsrc(has_gv ? (const void*)GV : (const void*)V, (uint32_t)slab_span(s.M, gvrs, rb));
  auto tile = [&](int set, int a) { return smem + ((grp * 2 + set) * 4 + a) * TB; };  // a: K, V, gK, gV
  auto issue = [&](int kt, int set) {
    const int k0 = kt * BN;
    dma.template issue_clamped<NSLAB>(krsrc, krs, k0, s.M, tile(set, 0));
    dma.template issue_clamped<NSLAB>(vrsrc, vrs, k0, s.M, tile(set, 1));
    if (has_gk) dma.template issue_clamped<NSLAB>(gkrsrc, gkrs, k0, s.M, tile(set, 2));
    if (has_gv) dma.template issue_clamped<NSLAB>(gvrsrc, gvrs, k0, s.M, tile(set, 3));
  };
  // Step i: tile kt0 + i of this group (if it has one) from set i & 1; the next one's copies go to the other set,
  // read in step i - 1, which every wave has finished at the barrier. Both groups run `half` steps (the same
  // barriers); a group with fewer tiles idles through its last one. The tiles from mask_from on may reach past
  // the last key or (causal) past the block's first query and take the masked copy of the loop; the groups may
  // be in different copies at a step, but both meet the same barriers.
  const int mask_from = min(kend % BN ? nkt - 1 : nkt, CAUSAL ? qb * BM / BN : nkt);
  auto sweep = [&](auto body) __attribute__((always_inline)) {
    auto step = [&](auto mask_tag, int i) __attribute__((always_inline)) {
      const int kt = kt0 + i;
      wait_vm_all();
      __syncthreads();
      if (kt + 1 < kt1) issue(kt + 1, (i + 1) & 1);
      if (kt < kt1) body(mask_tag, kt, tile(i & 1, 0), tile(i & 1, 1), tile(i & 1, 2), tile(i & 1, 3));
    };
    if (kt0 < kt1) issue(kt0, 0);
    const int isplit = min(half, max(0, mask_from - kt0));
    int i = 0;
    for (; i < isplit; ++i) step(std::false_type{}, i);
    for (; i < half; ++i) step(std::true_type{}, i);
    __syncthreads();  // every wave is done with the tiles
  };
  float* buf = reinterpret_cast<float*>(smem);

  if (split)
    sweep([&](auto mask_tag, int kt, const char* a, const char* b_, const char* c, const char* d)
              __attribute__((always_inline)) { compute_sums(std::true_type{}, mask_tag, kt, a, b_, c, d); });
  else
    sweep([&](auto mask_tag, int kt, const char* a, const char* b_, const char* c, const char* d)
              __attribute__((always_inline)) { compute_sums(std::false_type{}, mask_tag, kt, a, b_, c, d); });
  // dO . sum_j P V and dO . (sum_j (P o Gam) V + sum_j P gV) over this lane's columns of the accumulators
  float a_dot = 0.f, uw_dot = 0.f;
  if (qvalid) {
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        const f32x4_t d4 = load4<T>(dO, p.dout.sr, myq, dt * 32 + 8 * qd + 4 * g, s.D, s.vec);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          a_dot = fmaf(d4[e], acc_o[dt][4 * qd + e], a_dot);
          uw_dot = fmaf(d4[e], acc_a[dt][4 * qd + e], uw_dot);
        }
      }
  }
  // the sums of the row: both lane halves of a query, then both key groups; group 1's G_dO accumulators to group 0
  // (sums at [0, 2560) floats, accumulator element e of lane l of wave w at 4096 + e * 256 + w * 64 + l):
  // sum_j P, sum_j P dP, sum_j P Gam, sum_j P (Gam dP + W), max_j P
  float sums[5] = {pair_sum(l_part), pair_sum(a_dot), pair_sum(r_part), pair_sum(uw_dot), pair_max(p_max)};
#pragma unroll
  for (int i = 0; i < 5; ++i) buf[(i * 8 + grp * 4 + wig) * 64 + lane] = sums[i];
  if (grp == 1) {
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        buf[4096 + ((0 * NDT + dt) * 16 + r) * 256 + wig * 64 + lane] = acc_a[dt][r];
        buf[4096 + ((1 * NDT + dt) * 16 + r) * 256 + wig * 64 + lane] = acc_o[dt][r];
      }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; ++i) sums[i] += buf[(i * 8 + (1 - grp) * 4 + wig) * 64 + lane];
  sums[4] = fmaxf(sums[4], buf[(4 * 8 + (1 - grp) * 4 + wig) * 64 + lane]);
  const float L = sums[0];
  if (grp == 0 && qvalid) {
    // G_dO = inv (A + C) - (r inv) (O inv) with the normalised P (inv = 1 / L)
    const float inv = L > 0.f ? 1.f / L : 0.f;
    const float cval = sums[2] * inv;
    T* OD = (T*)p.out_gdo.p + b * p.out_gdo.sb + h * p.out_gdo.sh;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        const int d0 = dt * 32 + 8 * qd + 4 * g;
        float r4[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = 4 * qd + e;
          const float a = acc_a[dt][i] + buf[4096 + ((0 * NDT + dt) * 16 + i) * 256 + wig * 64 + lane];
          const float o = acc_o[dt][i] + buf[4096 + ((1 * NDT + dt) * 16 + i) * 256 + wig * 64 + lane];
          r4[e] = inv * a - cval * (o * inv);
        }
        store4<T>(OD, p.out_gdo.sr, myq, d0, s.D, r4[0], r4[1], r4[2], r4[3], s.vec);
      }
  }
  __syncthreads();  // the exchange is read before the tiles are refilled
  float lse_c = lse_raw;
  if (L > 0.f) {
    const float inv = 1.f / L;
    z = sums[1] * inv;
    rx = sums[2] * inv;
    tx = (sums[3] - z * sums[2]) * inv;
    moff += __builtin_log2f(L);
    lse_c = lse_with_flag(lse_raw + __builtin_log2f(L) * kLn2, sums[4] > kPeakedFrac * L);
  }
  if (grp == 0 && qvalid && g == 0) {
    p.r_row[row_id] = rx;
    p.t_row[row_id] = tx;
    p.z_out[row_id] = z;
    p.lse_out[row_id] = lse_c;
  }
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) acc[dt] = accy[dt] = zero16();
  if (split)
    sweep([&](auto mask_tag, int kt, const char* a, const char* b_, const char* c, const char* d)
              __attribute__((always_inline)) { compute_exact(std::true_type{}, mask_tag, kt, a, b_, c, d); });
  else
    sweep([&](auto mask_tag, int kt, const char* a, const char* b_, const char* c, const char* d)
              __attribute__((always_inline)) { compute_exact(std::false_type{}, mask_tag, kt, a, b_, c, d); });

  // group 1's accumulators to group 0 (element e of lane l of wave w at e * 256 + w * 64 + l)
  if (grp == 1) {
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        buf[(dt * 16 + r) * 256 + wig * 64 + lane] = acc[dt][r];
        buf[((NDT + dt) * 16 + r) * 256 + wig * 64 + lane] = accy[dt][r];
      }
  }
  __syncthreads();
  if (grp == 1) return;
  if (qvalid) {
    T* OG = (T*)p.out_gq.p + b * p.out_gq.sb + h * p.out_gq.sh;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        const int d0 = dt * 32 + 8 * qd + 4 * g;
        float r4[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = 4 * qd + e;
          const float x = acc[dt][i] + buf[(dt * 16 + i) * 256 + wig * 64 + lane];
          const float y = accy[dt][i] + buf[((NDT + dt) * 16 + i) * 256 + wig * 64 + lane];
          r4[e] = s.scale * (x + y);
        }
        store4<T>(OG, p.out_gq.sr, myq, d0, s.D, r4[0], r4[1], r4[2], r4[3], s.vec);
      }
  }
}


// The column pass for 16-bit inputs at head dims up to 64 with LDS-DMA tiles (FD as in the row pass), as two
// query groups of four waves (eight-wave workgroups, two waves per SIMD). A workgroup owns 128 keys (32 per wave,
// lane per key, as in cols_block); the groups sweep the two halves of its 32-query tiles and sum G_V and G_K in
// registers, and group 1's sums reach group 0 through LDS at the end. Query tiles holding a row flagged peaked in lse are
// skipped by the sweep and run after it, shared out between the groups, with Gbar_dP, Gbar_S and dS entered as
// two 16-bit terms. The gK and gV fragments sit in LDS, so that the K and V fragments, the two accumulators and
// the products fit 256 registers. ALL as in the key-split row kernel.
template <typename T, bool CAUSAL, bool ALL, bool FD>
__global__ __launch_bounds__(512, 2) void bwdbwd_cols_qs_kernel(const BwdBwdParams p) {
  using MM = Mfma<T>;
  using F = typename MM::frag_t;
  static_assert(sizeof(T) == 2, "16-bit inputs only");
  constexpr int DP = 64, NW = 4, BN = 32 * NW, BM = 32;
  constexpr int NDT = DP / 32, NKC = DP / MM::KC, NPC = 32 / MM::KC;
  constexpr int TB = BM * DP * 2;  // bytes per tile
  using Dma = SwzDma<NW, DP>;
  constexpr int NSLAB = BM / Dma::SLAB_ROWS;
  static_assert(NSLAB * Dma::SLAB_ROWS == BM, "query tiles must be whole DMA slabs");
  constexpr int FLAG = 4 * BM, RB = FLAG + 4;  // row terms [lse * log2(e) | z | r | t] of a tile, then its flag
  constexpr int TILES = 2 * 2 * 3 * TB;        // [group][set][Q, dO, gQ]
  constexpr int NFR = NW * NKC * 64;           // fragments per operand
  // the tiles, then the gK and gV fragments (fragment c of lane l of key slice w at (w * NKC + c) * 64 + l);
  // group 1's accumulators reach group 0 through the same memory at the end
  __shared__ __attribute__((aligned(1024))) char smem[TILES + 2 * NFR * sizeof(F)];
  static_assert(sizeof(smem) >= 2 * NDT * 16 * 256 * sizeof(float), "the exchange fits in the tile memory");
  __shared__ __attribute__((aligned(16))) float sRow[2][2][RB];  // [group][set]
  __shared__ int sPk[64];
  __shared__ int sAny;

  const Shape& s = p.s;
  const int tid = threadIdx.x, lane = tid & 63, li = lane & 31, g = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2, wig = wave & 3;  // query group, wave in group
  const int ltid = tid & 255;                 // thread in group
  const int nkb = (s.M + BN - 1) / BN;
  const int bid = xcd_remap(blockIdx.x, gridDim.x);
  const int bh = bid / nkb;
  const int kb = bid - bh * nkb;
  const int b = bh / s.H, h = bh - b * s.H;
  const T* Q = (const T*)p.q.p + b * p.q.sb + h * p.q.sh;
  const T* K = (const T*)p.k.p + b * p.k.sb + h * p.k.sh;
  const T* V = (const T*)p.v.p + b * p.v.sb + h * p.v.sh;
  const T* dO = (const T*)p.dout.p + b * p.dout.sb + h * p.dout.sh;
  const bool has_gq = ALL || p.gq.p != nullptr, has_gk = ALL || p.gk.p != nullptr, has_gv = ALL || p.gv.p != nullptr;
  const T* GQ = has_gq ? (const T*)p.gq.p + b * p.gq.sb + h * p.gq.sh : nullptr;
  const T* GK = has_gk ? (const T*)p.gk.p + b * p.gk.sb + h * p.gk.sh : nullptr;
  const T* GV = has_gv ? (const T*)p.gv.p + b * p.gv.sb + h * p.gv.sh : nullptr;
  const int key0 = kb * BN;
  const int kw0 = key0 + wig * 32;
  const int mykey = kw0 + li;
  const bool kvalid = mykey < s.M;

  F* sFr = reinterpret_cast<F*>(smem + TILES);
  F kf[NKC], vf[NKC];
#pragma unroll
  for (int c = 0; c < NKC; ++c) {
    kf[c] = gload_frag<T>(K, p.k.sr, mykey, s.M, c, s.D, s.vec);
    vf[c] = gload_frag<T>(V, p.v.sr, mykey, s.M, c, s.D, s.vec);
    // read after the sweep's first barrier
    if (grp == 0) {
      if (has_gk) sFr[(wig * NKC + c) * 64 + lane] = gload_frag<T>(GK, p.gk.sr, mykey, s.M, c, s.D, s.vec);
      if (has_gv) sFr[NFR + (wig * NKC + c) * 64 + lane] = gload_frag<T>(GV, p.gv.sr, mykey, s.M, c, s.D, s.vec);
    }
  }
  if (tid == 0) sAny = 0;
  f32x16_t accV[NDT], accK[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) accV[dt] = accK[dt] = zero16();
  const float c2 = s.scale * kLog2e;
  const int qbeg = CAUSAL ? (key0 / BM) * BM : 0;
  const int nqt = s.T > qbeg ? (s.T - qbeg + BM - 1) / BM : 0;
  const int half = (nqt + 1) / 2;
  const int it0 = grp * half, it1 = min(nqt, it0 + half);  // this group's tiles [it0, it1) of the sweep
  const int64_t rowbase = (int64_t)bh * s.T;

  // Row terms of a tile for group thread ltid < BM, held raw (rows past the end: lse = +inf) and converted when
  // stored: lse * log2(e) (+inf for rows past the end or without visible keys, so P = 0), z, r, t.
  float r_lse = THERIA_INF, r_z = 0.f, r_r = 0.f, r_t = 0.f;
  auto load_rows = [&](int it, int lim) {
    if (ltid < BM && it < lim) {
      const int qq = qbeg + it * BM + ltid;
      const bool ok = qq < s.T;
      r_lse = ok ? p.lse[rowbase + qq] : THERIA_INF;
      r_z = ok ? p.delta[rowbase + qq] : 0.f;
      r_r = ok ? p.r_row[rowbase + qq] : 0.f;
      r_t = ok ? p.t_row[rowbase + qq] : 0.f;
    }
  };
  auto store_rows = [&](float* sr) {
    if (ltid < BM) {
      sr[ltid] = __builtin_isinf(r_lse) ? THERIA_INF : r_lse * kLog2e;
      sr[BM + ltid] = r_z;
      sr[2 * BM + ltid] = r_r;
      sr[3 * BM + ltid] = r_t;
      const bool pk = __any(lse_peaked(r_lse));  // the tile's rows are the lanes of the group's first wave
      if (ltid == 0) sr[FLAG] = pk ? 1.f : 0.f;
    }
  };

  // Query tile it held in (tQ, tO, tgQ) with its row terms in sr. SPLIT: Gbar_dP, Gbar_S and dS enter the
  // products as two 16-bit terms each.
  auto tile = [&](auto split_tag, int it, const char* tQ, const char* tO, const char* tgQ,
                  const float* sr) __attribute__((always_inline)) {
    constexpr bool SPLIT = decltype(split_tag)::value;
    const int q0 = qbeg + it * BM;
    if (CAUSAL && kw0 > q0 + BM - 1) return;
    f32x16_t sc = zero16(), gm = zero16(), w = zero16(), dpz;
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) {
      const f32x4_t z4 = *reinterpret_cast<const f32x4_t*>(sr + BM + 8 * qd + 4 * g);
#pragma unroll
      for (int e = 0; e < 4; ++e) dpz[4 * qd + e] = -z4[e];
    }
#pragma unroll
    for (int c = 0; c < NKC; ++c) {
      const F qfr = swz_cols<T, DP>(tQ, li, c);
      const F ofr = swz_cols<T, DP>(tO, li, c);
      sc = MM::mma(qfr, kf[c], sc);
      dpz = MM::mma(ofr, vf[c], dpz);
      if (has_gq) gm = MM::mma(swz_cols<T, DP>(tgQ, li, c), kf[c], gm);
      if (has_gk) gm = MM::mma(qfr, sFr[(wig * NKC + c) * 64 + lane], gm);
      if (has_gv) w = MM::mma(ofr, sFr[NFR + (wig * NKC + c) * 64 + lane], w);
    }
    const bool diag = CAUSAL && (kw0 + 31 > q0);
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) {
      const int o = 8 * qd + 4 * g;
      const f32x4_t l4 = *reinterpret_cast<const f32x4_t*>(sr + o);
      const f32x4_t r4 = *reinterpret_cast<const f32x4_t*>(sr + 2 * BM + o);
      const f32x4_t t4 = *reinterpret_cast<const f32x4_t*>(sr + 3 * BM + o);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = 4 * qd + e;
        float pv = fast_exp2(fmaf(sc[r], c2, -l4[e]));
        if (!kvalid) pv = 0.f;
        if (diag && mykey > q0 + acc_row(r, g)) pv = 0.f;
        const float gam = s.scale * gm[r];
        const float ds = pv * dpz[r];
        const float e1 = fmaf(gam, dpz[r], w[r]);
        gm[r] = pv * (gam - r4[e]);                        // Gbar_dP
        w[r] = pv * e1 - r4[e] * ds - t4[e] * pv;          // Gbar_S
        dpz[r] = ds;                                       // dS
      }
    }
#pragma unroll
    for (int cc = 0; cc < NPC; ++cc) {
      if constexpr (SPLIT) {
        F gdph, gdpl, gsh, gsl, dsh, dsl;
        split_frag<T>(gm, cc, gdph, gdpl);
        split_frag<T>(w, cc, gsh, gsl);
        split_frag<T>(dpz, cc, dsh, dsl);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
          const F ro = swz_rows<T, DP>(tO, 0, cc, dt * 32);
          accV[dt] = MM::mma(gdph, ro, accV[dt]);
          accV[dt] = MM::mma(gdpl, ro, accV[dt]);
          const F rq = swz_rows<T, DP>(tQ, 0, cc, dt * 32);
          accK[dt] = MM::mma(gsh, rq, accK[dt]);
          accK[dt] = MM::mma(gsl, rq, accK[dt]);
          if (has_gq) {
            const F rg = swz_rows<T, DP>(tgQ, 0, cc, dt * 32);
            accK[dt] = MM::mma(dsh, rg, accK[dt]);
            accK[dt] = MM::mma(dsl, rg, accK[dt]);
          }
        }
      } else {
        const F gdpf = acc_frag<T>(gm, cc), gsf = acc_frag<T>(w, cc), dsf = acc_frag<T>(dpz, cc);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
          accV[dt] = MM::mma(gdpf, swz_rows<T, DP>(tO, 0, cc, dt * 32), accV[dt]);
          accK[dt] = MM::mma(gsf, swz_rows<T, DP>(tQ, 0, cc, dt * 32), accK[dt]);
          if (has_gq) accK[dt] = MM::mma(dsf, swz_rows<T, DP>(tgQ, 0, cc, dt * 32), accK[dt]);
        }
      }
    }
  };

  const Dma dma(wig, lane, FD ? 8 : s.D / 8);  // FD: head dim 64; else tile columns D .. 63 zero-filled
  // Byte offsets fit in 32 bits: the host only selects this kernel when each (batch, head) slab of Q, dO and gQ
  // spans less than 2^31 bytes.
  const uint32_t qrs = (uint32_t)p.q.sr * 2, ors = (uint32_t)p.dout.sr * 2;
  const uint32_t gqrs = has_gq ? (uint32_t)p.gq.sr * 2 : 0u;
  const int64_t rb = 2 * (FD ? 64 : s.D);  // bytes of a row the DMA reads
  const rsrc_t qrsrc = make_rsrc(Q, (uint32_t)slab_span(s.T, qrs, rb)),
               orsrc = make_rsrc(dO, (uint32_t)slab_span(s.T, ors, rb));
  const rsrc_t gqrsrc = make_rsrc(has_gq ? (const void*)GQ : (const void*)Q, (uint32_t)slab_span(s.T, gqrs, rb));
  auto tiles = [&](int set) { return smem + (grp * 2 + set) * 3 * TB; };  // Q, dO, gQ at 0, TB, 2 TB
  auto issue = [&](int it, int set) {
    const int q0 = qbeg + it * BM;
    char* t = tiles(set);
    dma.template issue_clamped<NSLAB>(qrsrc, qrs, q0, s.T, t);
    dma.template issue_clamped<NSLAB>(orsrc, ors, q0, s.T, t + TB);
    if (has_gq) dma.template issue_clamped<NSLAB>(gqrsrc, gqrs, q0, s.T, t + 2 * TB);
  };

  // The sweep. Step i: tile it0 + i of this group (if it has one) from set i & 1; the next one's copies and row
  // terms go to the other set, read in step i - 1, which every wave has finished at the barrier. Both groups run
  // `half` steps (the same barriers); a group with fewer tiles idles through its last one.
  bool pk_any = false;  // a tile holding a peaked row was skipped
  if (it0 < it1) {
    issue(it0, 0);
    load_rows(it0, it1);
    store_rows(sRow[grp][0]);
    load_rows(it0 + 1, it1);
  }
  for (int i = 0; i < half; ++i) {
    const int it = it0 + i;
    wait_vm_all();
    __syncthreads();
    if (it + 1 < it1) {
      issue(it + 1, (i + 1) & 1);
      store_rows(sRow[grp][(i + 1) & 1]);
      load_rows(it + 2, it1);
    }
    if (it < it1) {
      const float* sr = sRow[grp][i & 1];
      const bool pk = __builtin_amdgcn_readfirstlane(__float_as_uint(sr[FLAG])) != 0u;  // uniform
      pk_any |= pk;
      const char* t = tiles(i & 1);
      if (!pk) tile(std::false_type{}, it, t, t + TB, t + 2 * TB, sr);
    }
  }
  if (pk_any && lane == 0) sAny = 1;
  __syncthreads();  // every wave is done with the tiles; sAny is final

  // The tiles holding a peaked row, found 64 at a time from the lse flags; the groups take alternate ones.
  if (sAny) {
    for (int t0 = 0; t0 < nqt; t0 += 64) {
      const int nt = min(64, nqt - t0);
      __syncthreads();  // every thread is done with the previous flags and tiles
      if (tid < 64) sPk[tid] = 0;
      __syncthreads();
      constexpr int RPT = 64 * BM / 512;
      const int r0 = qbeg + t0 * BM, r1 = min(s.T, qbeg + (t0 + nt) * BM);
#pragma unroll
      for (int j = 0; j < RPT; ++j) {
        const int r = r0 + tid + 512 * j;
        if (r < r1 && lse_peaked(p.lse[rowbase + r])) sPk[(tid + 512 * j) / BM] = 1;
      }
      __syncthreads();
      const uint64_t mask = __ballot(sPk[lane] != 0);  // the same in every wave
      const int npk = __builtin_popcountll(mask);
      for (int j = 0; j < npk; j += 2) {
        int ti = -1;  // this group's tile: the (j + grp)-th flagged one
        if (j + grp < npk) {
          uint64_t m = mask;
          for (int x = 0; x < j + grp; ++x) m &= m - 1;
          ti = t0 + __builtin_ctzll(m);
        }
        __syncthreads();  // the tile buffers are free
        if (ti >= 0) {
          issue(ti, 0);
          load_rows(ti, nqt);
          store_rows(sRow[grp][0]);
        }
        wait_vm_all();
        __syncthreads();
        if (ti >= 0) {
          const char* t = tiles(0);
          tile(std::true_type{}, ti, t, t + TB, t + 2 * TB, sRow[grp][0]);
        }
      }
    }
    __syncthreads();  // every wave is done with the tiles
  }

  // The groups finish one column tile each (group g the tile dt = g): each hands the other tile's G_V and G_K
  // partial sums to the other group (element e of accumulator a (V, K) of lane l of wave w of group g at
  // ((g * 2 + a) * 16 + e) * 256 + w * 64 + l), then stores its half of the columns.
  static_assert(NDT == 2, "one column tile per group");
  float* xb = reinterpret_cast<float*>(smem);
  T* OV = (T*)p.out_gv.p + b * p.out_gv.sb + h * p.out_gv.sh;
  T* OK = (T*)p.out_gk.p + b * p.out_gk.sb + h * p.out_gk.sh;
  auto finish = [&](auto keep_tag) __attribute__((always_inline)) {
    constexpr int KEEP = decltype(keep_tag)::value, GIVE = 1 - KEEP;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      xb[((KEEP * 2 + 0) * 16 + r) * 256 + wig * 64 + lane] = accV[GIVE][r];
      xb[((KEEP * 2 + 1) * 16 + r) * 256 + wig * 64 + lane] = accK[GIVE][r];
    }
    __syncthreads();
    const int d = KEEP * 32 + li;
    if (d < s.D) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kw0 + acc_row(r, g);
        if (key < s.M) {
          const float v = accV[KEEP][r] + xb[((GIVE * 2 + 0) * 16 + r) * 256 + wig * 64 + lane];
          const float k = accK[KEEP][r] + xb[((GIVE * 2 + 1) * 16 + r) * 256 + wig * 64 + lane];
          OV[(int64_t)key * p.out_gv.sr + d] = (T)v;
          OK[(int64_t)key * p.out_gk.sr + d] = (T)(k * s.scale);
        }
      }
    }
  };
  // both branches meet the one barrier inside finish
  if (grp == 0)
    finish(std::integral_constant<int, 0>{});
  else
    finish(std::integral_constant<int, 1>{});
}

// The query-split column kernel takes 16-bit problems at head dim 64 whose Q, dO, gQ slabs allow LDS DMA and
// whose rows kernel runs its exact row blocks on its own (no row blocks in the column grid).
template <typename T, int DP>
static bool cols_qs_ok(const BwdBwdParams& p) {
  return (DP == 32 || DP == 64) && split_tiles_ok<T>(p, p.s.T, {&p.q, &p.dout, &p.gq}) && !exact_in_cols<T, DP>(p);
}

struct RowsLauncher {
  template <typename T, int DP, bool CAUSAL>
  static hipError_t run(const BwdBwdParams& p, hipStream_t st) {
    const int nqb = (p.s.T + 127) / 128;
    const int64_t nblk = (int64_t)nqb * p.s.B * p.s.H;
    if (nblk == 0) return hipSuccess;
    if constexpr (sizeof(T) == 2 && (DP == 32 || DP == 64)) {
      if (rows_ks_ok<T, DP>(p)) {  // every row block exact in one launch (the column grid has no row blocks)
        const bool all = p.gq.p && p.gk.p && p.gv.p, fd = p.s.D == 64;
        const dim3 grid((unsigned)nblk), block(512);
        if (all && fd)
          hipLaunchKernelGGL((bwdbwd_rows_ks_kernel<T, CAUSAL, true, true>), grid, block, 0, st, p);
        else if (all)
          hipLaunchKernelGGL((bwdbwd_rows_ks_kernel<T, CAUSAL, true, false>), grid, block, 0, st, p);
        else if (fd)
          hipLaunchKernelGGL((bwdbwd_rows_ks_kernel<T, CAUSAL, false, true>), grid, block, 0, st, p);
        else
          hipLaunchKernelGGL((bwdbwd_rows_ks_kernel<T, CAUSAL, false, false>), grid, block, 0, st, p);
        return hipGetLastError();
      }
    }
    const bool with_cols = exact_in_cols<T, DP>(p);
    if constexpr (sizeof(T) == 2 && (DP == 64 || DP == 128)) {
      if (rows_dma<T, DP>(p)) {
        hipLaunchKernelGGL((bwdbwd_rows_kernel<T, DP, CAUSAL, true, false>), dim3((unsigned)nblk), dim3(256), 0, st, p);
        if (!with_cols)
          hipLaunchKernelGGL((bwdbwd_rows_kernel<T, DP, CAUSAL, true, true>), dim3((unsigned)nblk), dim3(256), 0, st, p);
        return hipGetLastError();
      }
    }
    hipLaunchKernelGGL((bwdbwd_rows_kernel<T, DP, CAUSAL, false, false>), dim3((unsigned)nblk), dim3(256), 0, st, p);
    if constexpr (sizeof(T) == 2)
      if (!with_cols)
        hipLaunchKernelGGL((bwdbwd_rows_kernel<T, DP, CAUSAL, false, true>), dim3((unsigned)nblk), dim3(256), 0, st, p);
    return hipGetLastError();
  }
};

// Runs after RowsLauncher on the same stream (the exact row blocks read the first rows launch's r and t).
struct ColsLauncher {
  template <typename T, int DP, bool CAUSAL>
  static hipError_t run(const BwdBwdParams& p, hipStream_t st) {
    const int64_t nblk = (int64_t)((p.s.M + 127) / 128) * p.s.B * p.s.H;
    const int64_t nrow = (int64_t)((p.s.T + 127) / 128) * p.s.B * p.s.H;
    const bool dma = (sizeof(T) == 2 && (DP == 64 || DP == 128)) && cols_dma<T, DP>(p);
    if constexpr (sizeof(T) == 2 && (DP == 32 || DP == 64)) {
      if (cols_qs_ok<T, DP>(p)) {
        if (nblk == 0) return hipSuccess;
        const bool all = p.gq.p && p.gk.p && p.gv.p, fd = p.s.D == 64;
        const dim3 grid((unsigned)nblk), block(512);
        if (all && fd)
          hipLaunchKernelGGL((bwdbwd_cols_qs_kernel<T, CAUSAL, true, true>), grid, block, 0, st, p);
        else if (all)
          hipLaunchKernelGGL((bwdbwd_cols_qs_kernel<T, CAUSAL, true, false>), grid, block, 0, st, p);
        else if (fd)
          hipLaunchKernelGGL((bwdbwd_cols_qs_kernel<T, CAUSAL, false, true>), grid, block, 0, st, p);
        else
          hipLaunchKernelGGL((bwdbwd_cols_qs_kernel<T, CAUSAL, false, false>), grid, block, 0, st, p);
        return hipGetLastError();
      }
    }
    if constexpr (sizeof(T) == 2) {
      if (exact_in_cols<T, DP>(p)) {
        if (nblk + nrow == 0) return hipSuccess;
        const dim3 grid((unsigned)(nblk + nrow));
        if constexpr (DP == 64 || DP == 128)
          if (dma) {
            hipLaunchKernelGGL((bwdbwd_cols_exact_kernel<T, DP, CAUSAL, true>), grid, dim3(256), 0, st, p);
            return hipGetLastError();
          }
        hipLaunchKernelGGL((bwdbwd_cols_exact_kernel<T, DP, CAUSAL, false>), grid, dim3(256), 0, st, p);
        return hipGetLastError();
      }
    }
    if (nblk == 0) return hipSuccess;
    if constexpr (sizeof(T) == 2 && (DP == 64 || DP == 128))
      if (dma) {
        hipLaunchKernelGGL((bwdbwd_cols_kernel<T, DP, CAUSAL, true>), dim3((unsigned)nblk), dim3(256), 0, st, p);
        return hipGetLastError();
      }
    hipLaunchKernelGGL((bwdbwd_cols_kernel<T, DP, CAUSAL, false>), dim3((unsigned)nblk), dim3(256), 0, st, p);
    return hipGetLastError();
  }
};

hipError_t launch_bwdbwd_rows(const BwdBwdParams& p, hipStream_t st) { return dispatch_all<RowsLauncher>(p, st); }

bool bwdbwd_rows_make_row_terms(const BwdBwdParams& p) {
  if (p.s.dp > 64) return false;
  if (p.s.dtype == 1) return rows_ks_ok<_Float16, 64>(p);
  if (p.s.dtype == 2) return rows_ks_ok<__bf16, 64>(p);
  return false;
}
hipError_t launch_bwdbwd_cols(const BwdBwdParams& p, hipStream_t st) { return dispatch_all<ColsLauncher>(p, st); }

}  // namespace theria
