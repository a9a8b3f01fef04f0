// Explicit SDPA backward (dQ, dK, dV) for gfx950: two deterministic kernels.
//
// Replaces the reference's three kernels _sdpa_bwd_dv_kernel, _sdpa_bwd_dk_kernel and
// _sdpa_bwd_dq_kernel (theria/attention/triton_sdpa_backward.py:106-191, 269-398, 505-632). Math
// (docs/phase9.md:19-26 of the reference): P from the saved lse, dV = P^T dO, dP = dO V^T,
// dS = P o (dP - delta), dQ = scale dS K, dK = scale dS^T Q, where delta_i = dO_i . O_i equals the
// reference's z_i = sum_j dP_ij P_ij and is computed once per row (the reference recomputes it per
// key tile inside its dK kernel, an O(S^3) pass).
//
// dq_kernel (first): lane per query, like the forward. Per 32-key tile it forms S^T = K Q^T and
// dP^T = V dO^T with Q and dO in registers as B operands and K / V rows from LDS, seeds dP with
// -delta so the MFMA yields dP - delta directly, rebuilds P = exp2(S scale log2e - lse log2e), and
// accumulates dQ^T += K^T dS^T with K^T from the LDS transpose read and dS^T straight from the
// accumulator tile. It also computes delta (16-bit: from O and dO at the start; float32, and 16-bit blocks
// holding a peaked row: sum_j P dP / sum_j P in a pass over the keys) and writes it for dkdv_kernel.
// dkdv_kernel (second): lane per key. Each wave owns KT tiles of 32 keys (K and V fragments in
// registers as B operands) and walks the query rows in tiles of 64 staged in LDS; S = Q K^T and
// dP = dO V^T land with one key per lane, so P and dS are directly the A operands of
// dV += P^T dO and dK += dS^T Q (dO^T / Q^T by LDS transpose read), accumulated in registers.
// Every LDS fragment feeds QT (dq) or KT (dkdv) MFMAs. No atomics, no float32 dQ workspace: the
// result is deterministic. The split costs two extra score products (S and dP are formed in both
// kernels) but removes the LDS round trip of dS, the atomics and the accumulator conversion.
// Causal: key tiles above a query block (dq) and query tiles before a key block (dkdv) are never
// visited, fully masked wave tiles skip their MFMAs, and only diagonal tiles are masked element-wise.
#include <type_traits>

#include "dispatch.hpp"
#include "sdpa_common.hpp"

// Tile choices (compile-time knobs; the defaults are the measured best on MI355X).
#ifndef DKDV_MINW
#define DKDV_MINW 2
#endif
#ifndef DQ_MINW
#define DQ_MINW 2
#endif
#ifndef DQ_QT_MAX
#define DQ_QT_MAX 2
#endif
#ifndef DKDV_KT_MAX
#define DKDV_KT_MAX 1
#endif

namespace theria {

template <typename T, int DP, bool CAUSAL, int QT>
__global__ __launch_bounds__(256, (DP <= 64 ? DQ_MINW : 1)) void dq_kernel(const DqParams p) {
  using MM = Mfma<T>;
  using F = typename MM::frag_t;
  constexpr int KC = MM::KC;
  constexpr int NW = 4, BM = 32 * NW * QT, BN = 32, NT = 64 * NW;
  constexpr int PITCH = DP + 16 / (int)sizeof(T);
  constexpr int NDT = DP / 32, NKC = DP / KC, NPC = 32 / KC;
  __shared__ __attribute__((aligned(16))) T sK[BN * PITCH];
  __shared__ __attribute__((aligned(16))) T sV[BN * PITCH];

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
  const T* dO = (const T*)p.dout.p + b * p.dout.sb + h * p.dout.sh;
  const int q0w = qb * BM + wave * 32 * QT;
  const int64_t rowbase = (int64_t)bh * s.T;

  F qf[QT][NKC], of[QT][NKC];
  float lse2[QT], del[QT];
  bool peaked = false;  // a row of this wave is flagged peaked in its lse
#pragma unroll
  for (int j = 0; j < QT; ++j) {
    const int myq = q0w + 32 * j + li;
    const bool qvalid = myq < s.T;
#pragma unroll
    for (int c = 0; c < NKC; ++c) {
      qf[j][c] = gload_frag<T>(Q, p.q.sr, myq, s.T, c, s.D, s.vec);
      of[j][c] = gload_frag<T>(dO, p.dout.sr, myq, s.T, c, s.D, s.vec);
    }
    const float lse = qvalid ? p.lse[rowbase + myq] : THERIA_INF;
    lse2[j] = lse == -THERIA_INF ? THERIA_INF : lse * kLog2e;  // a row without visible keys has P = 0
    peaked |= qvalid && lse_peaked(lse);
    del[j] = 0.f;
    if (sizeof(T) == 2 && p.row_term == kRowFromO) {
      // delta = dO . O over this lane's half of the head dim (the dO fragment's columns), then the pair
      float part = 0.f;
      if (qvalid) {
#pragma unroll
        for (int c = 0; c < NKC; ++c) {
          const F od = of[j][c];
          if constexpr (sizeof(T) == 2) {  // (float32 forms the row term in the pass below)
            const int col = c * 16 + 8 * g;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              if (col + e < s.D) {
                const int64_t off = (int64_t)myq * p.o.sr + col + e;
                const float ov = p.o_f32 ? ((const float*)p.o.p + b * p.o.sb + h * p.o.sh)[off]
                                         : (float)((const T*)p.o.p + b * p.o.sb + h * p.o.sh)[off];
                part += ov * (float)od[e];
              }
            }
          }
        }
      }
      del[j] = pair_sum(part);
      if (qvalid && g == 0) p.delta[rowbase + myq] = del[j];
    } else if (p.row_term == kRowGiven) {
      del[j] = qvalid ? p.delta[rowbase + myq] : 0.f;
    }
  }
  const float c2 = s.scale * kLog2e;

  int kend = s.M;
  if (CAUSAL) kend = min(s.M, qb * BM + BM);
  const int nkt = (kend + BN - 1) / BN;

  // The row term from a pass over the key tiles: always for the frozen / normalised forms, and (16-bit) for a
  // workgroup holding a peaked row in place of dO . O, whose 16-bit P rounding in the forward's PV product
  // a peaked row does not average out. The dK/dV kernel reads the same delta, so this pass runs whether or
  // not dQ is wanted.
  // Float32 always takes the pass in place of dO . O (the reference's own row term, z = sum_j dP_ij P_ij,
  // theria/attention/triton_sdpa_backward.py:312-353): on a row whose probability sits on one key dP - z ~ 0
  // there, and z from the forward's O would leave the roundings of O and of dP against it (~2e-5 in dQ where
  // the bar is 1e-5); from the same P and dP the difference keeps only z's own rounding.
  bool exact_row_term = p.row_term >= kRowFrozen || (sizeof(T) == 4 && p.row_term == kRowFromO);
  if (sizeof(T) == 2 && p.row_term == kRowFromO) exact_row_term = __syncthreads_or(__any(peaked));
  if (!p.dq.p && !exact_row_term) return;  // only dO . O or the given row term was needed (uniform)
  if (exact_row_term) {
    // own: float32 row statistics from these scores alone (kRowOwnStats), with a running max m_run of
    // fl(S c2) over this lane's keys (the partial sums are rescaled when it grows)
    const bool own = sizeof(T) == 4 && p.row_term == kRowOwnStats;
    float a_part[QT], l_part[QT], p_mx[QT], m_run[QT];
#pragma unroll
    for (int j = 0; j < QT; ++j) {
      a_part[j] = l_part[j] = p_mx[j] = 0.f;
      m_run[j] = -THERIA_INF;
    }
    TileStage<T, BN, DP, NT> pK, pV;
    for (int kt = 0; kt < nkt; ++kt) {
      const int k0 = kt * BN;
      pK.load(K, p.k.sr, k0, s.M, s.D, s.vec);
      pV.load(V, p.v.sr, k0, s.M, s.D, s.vec);
      __syncthreads();
      pK.store(sK, PITCH);
      pV.store(sV, PITCH);
      __syncthreads();
      if (CAUSAL && k0 > q0w + 32 * QT - 1) continue;
      f32x16_t sc[QT], dpp[QT];
#pragma unroll
      for (int j = 0; j < QT; ++j) sc[j] = dpp[j] = zero16();
#pragma unroll
      for (int c = 0; c < NKC; ++c) {
        const F kfr = lds_cols<T, KLIN>(sK, PITCH, li, 0, c);
        const F vfr = lds_cols<T, KLIN>(sV, PITCH, li, 0, c);
#pragma unroll
        for (int j = 0; j < QT; ++j) {
          sc[j] = MM::mma(kfr, qf[j][c], sc[j]);
          dpp[j] = MM::mma(vfr, of[j][c], dpp[j]);
        }
      }
#pragma unroll
      for (int j = 0; j < QT; ++j) {
        const int lim = CAUSAL ? min(s.M, q0w + 32 * j + li + 1) : s.M;  // first key this query cannot see
        if (own) {
          float t[16];
          float mt = m_run[j];
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            t[r] = k0 + acc_row(r, g) < lim ? mul_rn(sc[j][r], c2) : -THERIA_INF;
            mt = fmaxf(mt, t[r]);
          }
          if (mt > m_run[j]) {  // m_run = -inf: the partial sums are still 0
            const float f = fast_exp2(m_run[j] - mt);
            a_part[j] *= f;
            l_part[j] *= f;
            m_run[j] = mt;
          }
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const float pv = t[r] > -THERIA_INF ? fast_exp2(t[r] - m_run[j]) : 0.f;  // (m_run finite then)
            a_part[j] = fmaf(pv, dpp[j][r], a_part[j]);
            l_part[j] += pv;
          }
          continue;
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float pv = k0 + acc_row(r, g) < lim ? fast_exp2(fmaf(sc[j][r], c2, -lse2[j])) : 0.f;
          a_part[j] = fmaf(pv, dpp[j][r], a_part[j]);
          l_part[j] += pv;
          p_mx[j] = fmaxf(p_mx[j], pv);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < QT; ++j) {
      float mm = -THERIA_INF;
      if (own) {  // both halves of the row onto the common max
        mm = pair_max(m_run[j]);
        const float f = m_run[j] > -THERIA_INF ? fast_exp2(m_run[j] - mm) : 0.f;
        a_part[j] *= f;
        l_part[j] *= f;
      }
      const float a = pair_sum(a_part[j]), l = pair_sum(l_part[j]), pm = pair_max(p_mx[j]);
      del[j] = p.row_term == kRowFrozen ? a : (l > 0.f ? a / l : 0.f);
      const int myq = q0w + 32 * j + li;
      if (myq < s.T && g == 0) {
        p.delta[rowbase + myq] = del[j];
        if (own) {
          p.lse_out[rowbase + myq] = l > 0.f ? mm : THERIA_INF;
          p.l2_out[rowbase + myq] = l > 0.f ? __builtin_log2f(l) : 0.f;
        } else if (p.lse_out) {  // flagged from the exact largest probability
          const float lin = p.lse[rowbase + myq];
          p.lse_out[rowbase + myq] = l > 0.f ? lse_with_flag(lin + __builtin_log2f(l) * kLn2, pm > kPeakedFrac * l) : lin;
        }
      }
    }
  }
  if (!p.dq.p) return;  // only the row term was requested

  f32x16_t acc[QT][NDT];
#pragma unroll
  for (int j = 0; j < QT; ++j)
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) acc[j][dt] = zero16();

  // 16-bit: a wave holding a peaked row forms dS as two 16-bit terms (hi + lo) in every product. Both forms
  // of the loop are inlined (a call that is not would take the register arrays it captures by address).
  auto run = [&](auto split_tag) __attribute__((always_inline)) {
  constexpr bool SPLIT = decltype(split_tag)::value;
  TileStage<T, BN, DP, NT> stK, stV;
  if (nkt > 0) {
    stK.load(K, p.k.sr, 0, s.M, s.D, s.vec);
    stV.load(V, p.v.sr, 0, s.M, s.D, s.vec);
  }
  for (int kt = 0; kt < nkt; ++kt) {
    const int k0 = kt * BN;
    __syncthreads();
    stK.store(sK, PITCH);
    stV.store(sV, PITCH);
    __syncthreads();
    if (kt + 1 < nkt) {
      stK.load(K, p.k.sr, k0 + BN, s.M, s.D, s.vec);
      stV.load(V, p.v.sr, k0 + BN, s.M, s.D, s.vec);
    }
    if (CAUSAL && k0 > q0w + 32 * QT - 1) continue;

    // dP starts from -delta, so the MFMA yields dP - delta; float32 forms dP from zero and subtracts after, so
    // that dP rounds exactly as in the row-term pass and dP - delta keeps only delta's own rounding (a row whose
    // probability sits on one key has dP - delta ~ 0 there, and independent roundings of dP would remain).
    constexpr bool SEED = sizeof(T) == 2;
    f32x16_t sc[QT], dp[QT];
#pragma unroll
    for (int j = 0; j < QT; ++j) {
      sc[j] = zero16();
#pragma unroll
      for (int r = 0; r < 16; ++r) dp[j][r] = SEED ? -del[j] : 0.f;
    }
#pragma unroll
    for (int c = 0; c < NKC; ++c) {
      const F kfr = lds_cols<T, KLIN>(sK, PITCH, li, 0, c);
      const F vfr = lds_cols<T, KLIN>(sV, PITCH, li, 0, c);
#pragma unroll
      for (int j = 0; j < QT; ++j) {
        sc[j] = MM::mma(kfr, qf[j][c], sc[j]);
        dp[j] = MM::mma(vfr, of[j][c], dp[j]);
      }
    }
    // Boundary tiles only (a uniform branch): masked scores become -inf, so P = 0 there.
    if ((k0 + BN > s.M) || (CAUSAL && k0 + BN - 1 > q0w)) {
#pragma unroll
      for (int j = 0; j < QT; ++j) {
        const int lim = CAUSAL ? min(s.M, q0w + 32 * j + li + 1) : s.M;  // first key this query cannot see
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (k0 + acc_row(r, g) >= lim) sc[j][r] = -THERIA_INF;
      }
    }
#pragma unroll
    for (int j = 0; j < QT; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        sc[j][r] = fast_exp2(fmaf(sc[j][r], c2, -lse2[j])) * (SEED ? dp[j][r] : dp[j][r] - del[j]);  // dS^T
#pragma unroll
    for (int cc = 0; cc < NPC; ++cc) {
      F dsf[QT], dsl[QT];
#pragma unroll
      for (int j = 0; j < QT; ++j) {
        if constexpr (SPLIT) {
          split_frag<T>(sc[j], cc, dsf[j], dsl[j]);
        } else {
          dsf[j] = acc_frag<T>(sc[j], cc);
        }
      }
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const F ktf = lds_rows<T, KACC>(sK, PITCH, 0, cc, dt * 32);
#pragma unroll
        for (int j = 0; j < QT; ++j) {
          acc[j][dt] = MM::mma(ktf, dsf[j], acc[j][dt]);
          if constexpr (SPLIT) acc[j][dt] = MM::mma(ktf, dsl[j], acc[j][dt]);
        }
      }
    }
  }

  };
  if (sizeof(T) == 2 && __any(peaked))
    run(std::integral_constant<bool, sizeof(T) == 2>{});
  else
    run(std::integral_constant<bool, false>{});

  T* DQ = (T*)p.dq.p + b * p.dq.sb + h * p.dq.sh;
#pragma unroll
  for (int j = 0; j < QT; ++j) {
    const int myq = q0w + 32 * j + li;
    if (myq >= s.T) continue;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        const int d0 = dt * 32 + 8 * qd + 4 * g;
        if (d0 < s.D) {
          const f32x16_t& a = acc[j][dt];
          store4<T>(DQ, p.dq.sr, myq, d0, s.D, a[4 * qd] * s.scale, a[4 * qd + 1] * s.scale, a[4 * qd + 2] * s.scale,
                    a[4 * qd + 3] * s.scale, s.vec);
        }
      }
  }
}

template <typename T, int DP, bool CAUSAL, int KT, bool DV_ONLY>
__global__ __launch_bounds__(256, (DP <= 64 ? DKDV_MINW : 1)) void dkdv_kernel(const DkdvParams p) {
  using MM = Mfma<T>;
  using F = typename MM::frag_t;
  constexpr int KC = MM::KC;
  constexpr int NW = 4, BN = 32 * NW * KT, NT = 64 * NW;
  constexpr int BM = sizeof(T) == 2 ? 64 : 32;
  constexpr int PITCH = DP + 16 / (int)sizeof(T);
  constexpr int NDT = DP / 32, NKC = DP / KC, NPC = 32 / KC, NQT = BM / 32;
  __shared__ __attribute__((aligned(16))) T sQ[BM * PITCH];
  __shared__ __attribute__((aligned(16))) T sdO[BM * PITCH];
  __shared__ __attribute__((aligned(16))) float sLse[BM];
  __shared__ __attribute__((aligned(16))) float sDel[BM];
  __shared__ int sPk[1];  // 16-bit: the staged tile holds a peaked row

  const Shape& s = p.s;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6, li = lane & 31, g = lane >> 5;
  const int nkb = (s.M + BN - 1) / BN;
  const int bid = xcd_remap(blockIdx.x, gridDim.x);
  const int bh = bid / nkb;
  const int kb = bid - bh * nkb;  // causal: ascending key blocks = longest query ranges first
  const int b = bh / s.H, h = bh - b * s.H;
  const T* Q = (const T*)p.q.p + b * p.q.sb + h * p.q.sh;
  const T* K = (const T*)p.k.p + b * p.k.sb + h * p.k.sh;
  const T* dO = (const T*)p.dout.p + b * p.dout.sb + h * p.dout.sh;
  constexpr bool dv_only = DV_ONLY;
  const int key0 = kb * BN;
  const int kw0 = key0 + wave * 32 * KT;  // key tile t of this wave starts at kw0 + 32 t

  F kf[KT][NKC], vf[KT][NKC];
#pragma unroll
  for (int t = 0; t < KT; ++t)
#pragma unroll
    for (int c = 0; c < NKC; ++c) {
      kf[t][c] = gload_frag<T>(K, p.k.sr, kw0 + 32 * t + li, s.M, c, s.D, s.vec);
      vf[t][c] = F{};
    }
  if constexpr (!DV_ONLY) {
    const T* V = (const T*)p.v.p + b * p.v.sb + h * p.v.sh;
#pragma unroll
    for (int t = 0; t < KT; ++t)
#pragma unroll
      for (int c = 0; c < NKC; ++c) vf[t][c] = gload_frag<T>(V, p.v.sr, kw0 + 32 * t + li, s.M, c, s.D, s.vec);
  }
  f32x16_t dv[KT][NDT], dk[KT][NDT];
#pragma unroll
  for (int t = 0; t < KT; ++t)
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      dv[t][dt] = zero16();
      dk[t][dt] = zero16();
    }
  const float c2 = s.scale * kLog2e;
  const int qbeg = CAUSAL ? (key0 / BM) * BM : 0;
  const int nqt = s.T > qbeg ? (s.T - qbeg + BM - 1) / BM : 0;
  const int64_t rowbase = (int64_t)bh * s.T;

  TileStage<T, BM, DP, NT> stQ, stO;
  float pre_lse = THERIA_INF, pre_del = 0.f;
  bool pre_pk = false;  // 16-bit: this row is flagged peaked in its lse
  auto prefetch = [&](int q0) {
    stQ.load(Q, p.q.sr, q0, s.T, s.D, s.vec);
    stO.load(dO, p.dout.sr, q0, s.T, s.D, s.vec);
    if (tid < BM) {
      const int qq = q0 + tid;
      const float lse = qq < s.T ? p.lse[rowbase + qq] : THERIA_INF;
      pre_lse = lse == -THERIA_INF ? THERIA_INF : lse * kLog2e;
      pre_del = (qq < s.T && !dv_only) ? -p.delta[rowbase + qq] : 0.f;  // staged negated: dP starts at -delta
      if constexpr (sizeof(T) == 2) pre_pk = qq < s.T && lse_peaked(lse);
    }
  };
  if (nqt > 0) prefetch(qbeg);

  // S = Q K^T and dP = dO V^T - delta for the 32-row subtile qr0 of the staged tile (masked scores -inf).
  auto scores = [&](int qr0, int q0t, f32x16_t (&sc)[KT], f32x16_t (&dp)[KT]) {
    f32x4_t del4[4];
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) del4[qd] = *reinterpret_cast<const f32x4_t*>(sDel + qr0 + 8 * qd + 4 * g);
#pragma unroll
    for (int t = 0; t < KT; ++t) {
      sc[t] = zero16();
#pragma unroll
      for (int r = 0; r < 16; ++r) dp[t][r] = del4[r >> 2][r & 3];
    }
#pragma unroll
    for (int c = 0; c < NKC; ++c) {
      const F qfr = lds_cols<T, KLIN>(sQ, PITCH, qr0 + li, 0, c);
#pragma unroll
      for (int t = 0; t < KT; ++t) sc[t] = MM::mma(qfr, kf[t][c], sc[t]);
      if constexpr (!DV_ONLY) {
        const F ofr = lds_cols<T, KLIN>(sdO, PITCH, qr0 + li, 0, c);
#pragma unroll
        for (int t = 0; t < KT; ++t) dp[t] = MM::mma(ofr, vf[t][c], dp[t]);
      }
    }
    // Boundary sub-tiles only (a uniform branch): masked scores become -inf, so P = 0 there.
    if ((kw0 + 32 * KT > s.M) || (CAUSAL && kw0 + 32 * KT - 1 > q0t)) {
#pragma unroll
      for (int t = 0; t < KT; ++t) {
        const int mykey = kw0 + 32 * t + li;
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (mykey >= s.M || (CAUSAL && mykey > q0t + acc_row(r, g))) sc[t][r] = -THERIA_INF;
      }
    }
  };

  for (int it = 0; it < nqt; ++it) {
    const int q0 = qbeg + it * BM;
    __syncthreads();
    stQ.store(sQ, PITCH);
    stO.store(sdO, PITCH);
    if (tid < BM) {
      sLse[tid] = pre_lse;
      sDel[tid] = pre_del;
    }
    if constexpr (sizeof(T) == 2) {
      if (wave == 0) {  // BM = 64 rows: wave 0 staged them
        const bool pk = __any(pre_pk);
        if (lane == 0) sPk[0] = pk;
      }
    }
    __syncthreads();
    if (it + 1 < nqt) prefetch(q0 + BM);

#pragma unroll
    for (int qt = 0; qt < NQT; ++qt) {
      const int qr0 = qt * 32;
      const int q0t = q0 + qr0;
      if (q0t >= s.T || (CAUSAL && kw0 > q0t + 31)) continue;  // wave-uniform
      f32x4_t lse4[4];
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) lse4[qd] = *reinterpret_cast<const f32x4_t*>(sLse + qr0 + 8 * qd + 4 * g);
      f32x16_t sc[KT], dp[KT];
      scores(qr0, q0t, sc, dp);
#pragma unroll
      for (int t = 0; t < KT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float pv = fast_exp2(fmaf(sc[t][r], c2, -lse4[r >> 2][r & 3]));
          sc[t][r] = pv;
          if constexpr (!DV_ONLY) dp[t][r] *= pv;  // dS
        }
#pragma unroll
      for (int cc = 0; cc < NPC; ++cc) {
        F ot[NDT], qtr[NDT];
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) ot[dt] = lds_rows<T, KACC>(sdO, PITCH, qr0, cc, dt * 32);
#pragma unroll
        for (int t = 0; t < KT; ++t) {
          const F pa = acc_frag<T>(sc[t], cc);
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) dv[t][dt] = MM::mma(pa, ot[dt], dv[t][dt]);
        }
        if constexpr (!DV_ONLY) {
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) qtr[dt] = lds_rows<T, KACC>(sQ, PITCH, qr0, cc, dt * 32);
#pragma unroll
          for (int t = 0; t < KT; ++t) {
            const F da = acc_frag<T>(dp[t], cc);
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) dk[t][dt] = MM::mma(da, qtr[dt], dk[t][dt]);
          }
        }
      }
    }

    // 16-bit, a tile holding a peaked row: the residual products, with S and dP formed again, so that P and
    // dS enter as two 16-bit terms (hi + lo) in total.
    if constexpr (sizeof(T) == 2) {
      if (__builtin_amdgcn_readfirstlane(sPk[0])) {
#pragma unroll
        for (int qt = 0; qt < NQT; ++qt) {
          const int qr0 = qt * 32;
          const int q0t = q0 + qr0;
          if (q0t >= s.T || (CAUSAL && kw0 > q0t + 31)) continue;  // wave-uniform
          f32x4_t lse4[4];
#pragma unroll
          for (int qd = 0; qd < 4; ++qd) lse4[qd] = *reinterpret_cast<const f32x4_t*>(sLse + qr0 + 8 * qd + 4 * g);
          f32x16_t sc[KT], dp[KT];
          scores(qr0, q0t, sc, dp);
#pragma unroll
          for (int cc = 0; cc < NPC; ++cc) {
#pragma unroll
            for (int t = 0; t < KT; ++t) {
              F pl, dl;
#pragma unroll
              for (int e = 0; e < 8; ++e) {
                const float pv = fast_exp2(fmaf(sc[t][8 * cc + e], c2, -lse4[(8 * cc + e) >> 2][e & 3]));
                const float ds = pv * dp[t][8 * cc + e];
                pl[e] = (T)(pv - (float)(T)pv);
                dl[e] = (T)(ds - (float)(T)ds);
              }
#pragma unroll
              for (int dt = 0; dt < NDT; ++dt) {
                dv[t][dt] = MM::mma(pl, lds_rows<T, KACC>(sdO, PITCH, qr0, cc, dt * 32), dv[t][dt]);
                if constexpr (!DV_ONLY) dk[t][dt] = MM::mma(dl, lds_rows<T, KACC>(sQ, PITCH, qr0, cc, dt * 32), dk[t][dt]);
              }
            }
          }
        }
      }
    }
  }

  // Epilogue: lane holds column d = dt*32 + li of rows (keys) kw0 + 32 t + acc_row(r, g).
  T* DV = (T*)p.dv.p + b * p.dv.sb + h * p.dv.sh;
  T* DK = p.dk.p ? (T*)p.dk.p + b * p.dk.sb + h * p.dk.sh : nullptr;
#pragma unroll
  for (int t = 0; t < KT; ++t)
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const int d = dt * 32 + li;
      if (d < s.D) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kw0 + 32 * t + acc_row(r, g);
          if (key < s.M) {
            DV[(int64_t)key * p.dv.sr + d] = (T)dv[t][dt][r];
            if (!DV_ONLY && DK) DK[(int64_t)key * p.dk.sr + d] = (T)(dk[t][dt][r] * s.scale);
          }
        }
      }
    }
}

// Pipelined 16-bit dQ (sdpa_bwd_pipe.hip); false when it does not cover the problem.
template <typename T, bool CAUSAL>
bool launch_dq_pipe(const DqParams& p, hipStream_t st, hipError_t* err);

struct DqLauncher {
  template <typename T, int DP, bool CAUSAL>
  static hipError_t run(const DqParams& p, hipStream_t st) {
    if constexpr (sizeof(T) == 2) {
      hipError_t err;
      if (launch_dq_pipe<T, CAUSAL>(p, st, &err)) return err;
    }
    // Two query tiles per wave only for 16-bit inputs (float32 fragments would spill ~160 VGPRs).
    const int qt = (DQ_QT_MAX >= 2 && sizeof(T) == 2 && DP <= 64 && p.s.T > 128) ? 2 : 1;
    const int bm = 128 * qt;
    const int64_t nblk = (int64_t)((p.s.T + bm - 1) / bm) * p.s.B * p.s.H;
    if (nblk == 0) return hipSuccess;
    if constexpr (DP <= 64 && sizeof(T) == 2) {
      if (qt == 2) {
        hipLaunchKernelGGL((dq_kernel<T, DP, CAUSAL, 2>), dim3((unsigned)nblk), dim3(256), 0, st, p);
        return hipGetLastError();
      }
    }
    hipLaunchKernelGGL((dq_kernel<T, DP, CAUSAL, 1>), dim3((unsigned)nblk), dim3(256), 0, st, p);
    return hipGetLastError();
  }
};

// Pipelined 16-bit dK/dV (sdpa_bwd_pipe.hip); false when it does not cover the problem.
template <typename T, bool CAUSAL>
bool launch_dkdv_pipe(const DkdvParams& p, hipStream_t st, hipError_t* err);

struct DkdvLauncher {
  template <typename T, int DP, bool CAUSAL, int KT>
  static void go(const DkdvParams& p, unsigned nblk, hipStream_t st) {
    if (p.dv_only)
      hipLaunchKernelGGL((dkdv_kernel<T, DP, CAUSAL, KT, true>), dim3(nblk), dim3(256), 0, st, p);
    else
      hipLaunchKernelGGL((dkdv_kernel<T, DP, CAUSAL, KT, false>), dim3(nblk), dim3(256), 0, st, p);
  }
  template <typename T, int DP, bool CAUSAL>
  static hipError_t run(const DkdvParams& p, hipStream_t st) {
    if constexpr (sizeof(T) == 2) {
      hipError_t err;
      if (launch_dkdv_pipe<T, CAUSAL>(p, st, &err)) return err;
    }
    const int kt = (DKDV_KT_MAX >= 2 && DP <= 64 && p.s.M > 128) ? 2 : 1;
    const int bn = 128 * kt;
    const int64_t nblk = (int64_t)((p.s.M + bn - 1) / bn) * p.s.B * p.s.H;
    if (nblk == 0) return hipSuccess;
    if constexpr (DP <= 64 && DKDV_KT_MAX >= 2) {
      if (kt == 2) {
        go<T, DP, CAUSAL, 2>(p, (unsigned)nblk, st);
        return hipGetLastError();
      }
    }
    go<T, DP, CAUSAL, 1>(p, (unsigned)nblk, st);
    return hipGetLastError();
  }
};

hipError_t launch_bwd_dq(const DqParams& p, hipStream_t st) { return dispatch_all<DqLauncher>(p, st); }
hipError_t launch_bwd_dkdv(const DkdvParams& p, hipStream_t st) { return dispatch_all<DkdvLauncher>(p, st); }

}  // namespace theria
