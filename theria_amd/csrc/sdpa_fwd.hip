// Fused SDPA forward for gfx950.
//
// Replaces _fused_sdpa_kernel (reference theria/attention/triton_qk.py:242-304):
// O = softmax(scale * Q K^T) V with an online softmax, saving lse (and the reference's m, l).
//
// Work decomposition: one workgroup = 4 waves; each wave owns QT tiles of 32 query rows of one
// (batch, head) for the whole kernel. The score tile is computed transposed, S^T = K Q^T, so that in
// the accumulator layout each lane owns one query (column li) and 16 keys: the row max and row sum
// are in-lane reductions plus one permlane32 swap, and the output accumulator O^T = V^T P^T is also
// lane-per-query, so the online-softmax rescale is a per-lane scalar multiply. Q stays in registers
// as the B operand; K/V tiles of 64 keys are staged in LDS (register-prefetched one tile ahead), and
// every K fragment and every V^T fragment (LDS transpose read) read from LDS feeds QT MFMAs: with
// one MFMA per fragment the 32x32x16 MFMA rate equals the CU's LDS bandwidth, so QT = 2 halves the
// LDS traffic per FLOP. exp is evaluated as exp2 with scale*log2(e) folded into one FMA. The running
// max used for P is only moved when a row's max grows by more than 2^8 (P <= 256 stays exact in
// float32 and representable in bf16/fp16), so the O rescale is skipped on almost every tile.
#include "dispatch.hpp"
#include "sdpa_common.hpp"

#ifndef FWD_MINW
#define FWD_MINW 2
#endif

namespace theria {

template <typename T, int DP, bool CAUSAL, int QT, int BN>
__global__ __launch_bounds__(256, (DP <= 64 ? FWD_MINW : 1)) void fwd_kernel(const FwdParams p) {
  using MM = Mfma<T>;
  using F = typename MM::frag_t;
  constexpr int KC = MM::KC;
  constexpr int NW = 4, BM = 32 * NW * QT, NT = 64 * NW;
  constexpr int PITCH = DP + 16 / (int)sizeof(T);
  constexpr int NDT = DP / 32, NKC = DP / KC, NPC = 32 / KC, NST = BN / 32;
  __shared__ __attribute__((aligned(16))) T sK[BN * PITCH];
  __shared__ __attribute__((aligned(16))) T sV[BN * PITCH];

  const Shape& s = p.s;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, li = lane & 31, g = lane >> 5;
  const int nqb = (s.T + BM - 1) / BM;
  const int bid = xcd_remap(blockIdx.x, gridDim.x);
  const int bh = bid / nqb;
  int qb = bid - bh * nqb;
  if (CAUSAL) qb = nqb - 1 - qb;  // longest rows first
  const int b = bh / s.H, h = bh - b * s.H;
  const T* Q = (const T*)p.q.p + b * p.q.sb + h * p.q.sh;
  const T* K = (const T*)p.k.p + b * p.k.sb + h * p.k.sh;
  const T* V = (const T*)p.v.p + b * p.v.sb + h * p.v.sh;
  const int q0w = qb * BM + wave * 32 * QT;  // query tile j of this wave starts at q0w + 32 j
  const int64_t rowbase = (int64_t)bh * s.T;

  F qf[QT][NKC];
  f32x16_t o[QT][NDT];
  float m_use[QT], m_max[QT], l_part[QT];
#pragma unroll
  for (int j = 0; j < QT; ++j) {
    const int myq = q0w + 32 * j + li;
#pragma unroll
    for (int c = 0; c < NKC; ++c) qf[j][c] = gload_frag<T>(Q, p.q.sr, myq, s.T, c, s.D, s.vec);
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) o[j][dt] = zero16();
    m_use[j] = -THERIA_INF;  // offset of P in the log2 domain
    m_max[j] = -THERIA_INF;  // exact running row max (log2 domain)
    l_part[j] = 0.f;         // this lane's share of the row sum
  }
  const float c2 = s.scale * kLog2e;

  int kend = s.M;
  if (CAUSAL) kend = min(s.M, qb * BM + BM);
  const int nkt = (kend + BN - 1) / BN;
  TileStage<T, BN, DP, NT> stK, stV;
  if (nkt > 0) {
    stK.load_any(K, p.k.sr, 0, s.M, s.D, s.vec);
    stV.load_any(V, p.v.sr, 0, s.M, s.D, s.vec);
  }
  for (int kt = 0; kt < nkt; ++kt) {
    const int k0 = kt * BN;
    __syncthreads();
    stK.store(sK, PITCH);
    stV.store(sV, PITCH);
    __syncthreads();
    if (kt + 1 < nkt) {
      stK.load_any(K, p.k.sr, k0 + BN, s.M, s.D, s.vec);
      stV.load_any(V, p.v.sr, k0 + BN, s.M, s.D, s.vec);
    }
    if (CAUSAL && k0 > q0w + 32 * QT - 1) continue;  // tile entirely above this wave's diagonal

    f32x16_t sc[QT][NST];
#pragma unroll
    for (int t = 0; t < NST; ++t) {
#pragma unroll
      for (int j = 0; j < QT; ++j) sc[j][t] = zero16();
#pragma unroll
      for (int c = 0; c < NKC; ++c) {
        const F kfr = lds_cols<T, KLIN>(sK, PITCH, t * 32 + li, 0, c);
#pragma unroll
        for (int j = 0; j < QT; ++j) sc[j][t] = MM::mma(kfr, qf[j][c], sc[j][t]);
      }
    }
    // Boundary tiles only (a uniform branch): masked scores become -inf, so P = 0 there. Interior
    // tiles run the same code below with no per-element test.
    if ((k0 + BN > s.M) || (CAUSAL && k0 + BN - 1 > q0w)) {
#pragma unroll
      for (int j = 0; j < QT; ++j) {
        const int lim = CAUSAL ? min(s.M, q0w + 32 * j + li + 1) : s.M;  // first key this query cannot see
#pragma unroll
        for (int t = 0; t < NST; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (k0 + t * 32 + acc_row(r, g) >= lim) sc[j][t][r] = -THERIA_INF;
      }
    }
#pragma unroll
    for (int j = 0; j < QT; ++j) {
      {
        float mx = -THERIA_INF;
#pragma unroll
        for (int t = 0; t < NST; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sc[j][t][r]);
        mx = pair_max(mx) * c2;
        m_max[j] = fmaxf(m_max[j], mx);
        const bool resc = mx > m_use[j] + 8.f;
        if (__any(resc)) {
          const float alpha = resc ? fast_exp2(m_use[j] - mx) : 1.f;
          m_use[j] = resc ? mx : m_use[j];
          l_part[j] *= alpha;
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[j][dt][r] *= alpha;
        }
      }
      // m_use is -inf only while every key seen so far is masked (then every score is -inf and P = 0)
      const float moff = m_use[j] == -THERIA_INF ? 0.f : m_use[j];
      float ls = 0.f;
#pragma unroll
      for (int t = 0; t < NST; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float e = fast_exp2(fmaf(sc[j][t][r], c2, -moff));
          sc[j][t][r] = e;
          ls += e;
        }
      l_part[j] += ls;
    }
#pragma unroll
    for (int t = 0; t < NST; ++t)
#pragma unroll
      for (int cc = 0; cc < NPC; ++cc) {
        F pf[QT];
#pragma unroll
        for (int j = 0; j < QT; ++j) pf[j] = acc_frag<T>(sc[j][t], cc);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
          const F vfr = lds_rows<T, KACC>(sV, PITCH, t * 32, cc, dt * 32);
#pragma unroll
          for (int j = 0; j < QT; ++j) o[j][dt] = MM::mma(vfr, pf[j], o[j][dt]);
        }
      }
  }

#pragma unroll
  for (int j = 0; j < QT; ++j) {
    const int myq = q0w + 32 * j + li;
    const bool qvalid = myq < s.T;
    const int64_t row_id = rowbase + myq;
    {
      const float l = pair_sum(l_part[j]);
      const float inv = l > 0.f ? 1.f / l : 0.f;
      if (qvalid) {
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
          for (int qd = 0; qd < 4; ++qd) {
            const int d0 = dt * 32 + 8 * qd + 4 * g;
            if (d0 < s.D) {
              const float a0 = o[j][dt][4 * qd] * inv, a1 = o[j][dt][4 * qd + 1] * inv;
              const float a2 = o[j][dt][4 * qd + 2] * inv, a3 = o[j][dt][4 * qd + 3] * inv;
              if (p.o_f32) {
                float* O = (float*)p.o.p + b * p.o.sb + h * p.o.sh;
                store4<float>(O, p.o.sr, myq, d0, s.D, a0, a1, a2, a3, s.vec);
              } else {
                T* O = (T*)p.o.p + b * p.o.sb + h * p.o.sh;
                store4<T>(O, p.o.sr, myq, d0, s.D, a0, a1, a2, a3, s.vec);
              }
            }
          }
        if (g == 0) {
          // 16-bit: flag a peaked row, largest probability exp2(m_max - m_use) / l above 1/4 (log2: -2)
          const float lse2 = m_use[j] + __builtin_log2f(l);
          const bool peaked = sizeof(T) == 2 && m_max[j] - lse2 > -2.f;
          p.lse[row_id] = l > 0.f ? (sizeof(T) == 2 ? lse_with_flag(lse2 * kLn2, peaked) : lse2 * kLn2) : -THERIA_INF;
          if (p.row_max) p.row_max[row_id] = m_max[j] * kLn2;
          if (p.row_sum) p.row_sum[row_id] = l > 0.f ? l * fast_exp2(m_use[j] - m_max[j]) : 0.f;
        }
      }
    }
  }
}

// Tile choices (compile-time knobs; the defaults are the measured best on MI355X).
#ifndef FWD_BN_QT2
#define FWD_BN_QT2 64
#endif
#ifndef FWD_QT_MAX
#define FWD_QT_MAX 2
#endif
// Query tiles per wave: 2 where the registers allow it and the sequence fills the block.
template <int DP> constexpr int fwd_qt(int T) { return (FWD_QT_MAX >= 2 && DP <= 64 && T > 128) ? 2 : 1; }

// Pipelined 16-bit forward (sdpa_fwd_pipe.hip); false when it does not cover the problem.
template <typename T, bool CAUSAL>
bool launch_fwd_pipe(const FwdParams& p, hipStream_t st, hipError_t* err);

struct FwdLauncher {
  template <typename T, int DP, bool CAUSAL>
  static hipError_t run(const FwdParams& p, hipStream_t st) {
    if constexpr (sizeof(T) == 2) {
      hipError_t err;
      if (launch_fwd_pipe<T, CAUSAL>(p, st, &err)) return err;
    }
    // Two query tiles per wave only for 16-bit inputs: with float32 fragments (twice the registers)
    // that variant spills ~150 VGPRs and runs at half the one-tile rate.
    const int qt = sizeof(T) == 2 ? fwd_qt<DP>(p.s.T) : 1;
    const int bm = 128 * qt;
    const int64_t nblk = (int64_t)((p.s.T + bm - 1) / bm) * p.s.B * p.s.H;
    if (nblk == 0) return hipSuccess;
    if constexpr (DP <= 64 && sizeof(T) == 2) {
      if (qt == 2) {
        hipLaunchKernelGGL((fwd_kernel<T, DP, CAUSAL, 2, FWD_BN_QT2>), dim3((unsigned)nblk), dim3(256), 0, st, p);
        return hipGetLastError();
      }
    }
    hipLaunchKernelGGL((fwd_kernel<T, DP, CAUSAL, 1, 64>), dim3((unsigned)nblk), dim3(256), 0, st, p);
    return hipGetLastError();
  }
};

hipError_t launch_fwd(const FwdParams& p, hipStream_t st) { return dispatch_all<FwdLauncher>(p, st); }

}  // namespace theria
