// Fused SDPA forward for gfx950, plus the small row kernels around the backward.
//
// Forward (mode 0) replaces _fused_sdpa_kernel (reference theria/attention/triton_qk.py:242-304):
// O = softmax(scale * Q K^T) V with an online softmax, saving lse (and the reference's m, l).
// Mode 1 rebuilds O_i = sum_j P_ij V_j from a given lse and writes the backward row term
// delta_i = dO_i . O_i, for the reference's sdpa_bwd_* entry points that receive (m, l) but no O
// (triton_sdpa_backward.py:312-353 recomputes that term inside its dK kernel).
//
// Work decomposition: one workgroup = 4 waves = 128 query rows of one (batch, head); each wave owns
// 32 query rows for the whole kernel. The score tile is computed transposed, S^T = K Q^T, so that in
// the accumulator layout each lane owns one query (column li) and 16 keys: the row max and row sum
// are in-lane reductions plus one permlane32 swap, and the output accumulator O^T = V^T P^T is also
// lane-per-query, so the online-softmax rescale is a per-lane scalar multiply. Q stays in registers
// as the B operand; K/V tiles of 64 keys are staged in LDS (register-prefetched one tile ahead) and
// V^T fragments come from the LDS transpose read. exp is evaluated as exp2 with scale*log2(e) folded
// into one FMA. The running max used for P is only moved when a row's max grows by more than 2^8
// (P <= 256 stays exact in float32 and representable in bf16/fp16), so the O rescale is skipped on
// almost every tile.
#include "dispatch.hpp"
#include "sdpa_common.hpp"

namespace theria {

template <typename T, int DP, bool CAUSAL, int MODE>
__global__ __launch_bounds__(256) void fwd_kernel(const FwdParams p) {
  using MM = Mfma<T>;
  using F = typename MM::frag_t;
  constexpr int KC = MM::KC;
  constexpr int NW = 4, BM = 32 * NW, BN = 64, NT = 64 * NW;
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
  const int q0w = qb * BM + wave * 32;
  const int myq = q0w + li;
  const bool qvalid = myq < s.T;
  const int64_t row_id = (int64_t)bh * s.T + myq;

  F qf[NKC];
#pragma unroll
  for (int c = 0; c < NKC; ++c) qf[c] = gload_frag<T>(Q, p.q.sr, myq, s.T, c, s.D, s.vec);

  f32x16_t o[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) o[dt] = zero16();

  const float c2 = s.scale * kLog2e;
  float m_use = -THERIA_INF;  // offset of P in the log2 domain
  float m_max = -THERIA_INF;  // exact running row max (log2 domain)
  float l_part = 0.f;         // this lane's share of the row sum
  if (MODE == 1) m_use = qvalid ? p.lse[row_id] * kLog2e : THERIA_INF;

  int kend = s.M;
  if (CAUSAL) kend = min(s.M, qb * BM + BM);
  const int nkt = (kend + BN - 1) / BN;
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
    if (CAUSAL && k0 > q0w + 31) continue;  // tile entirely above this wave's diagonal

    f32x16_t sc[NST];
#pragma unroll
    for (int t = 0; t < NST; ++t) {
      sc[t] = zero16();
#pragma unroll
      for (int c = 0; c < NKC; ++c) sc[t] = MM::mma(lds_cols<T, KLIN>(sK, PITCH, t * 32 + li, 0, c), qf[c], sc[t]);
    }
    const bool need_mask = (k0 + BN > s.M) || (CAUSAL && k0 + BN - 1 > q0w);
    if (need_mask) {
#pragma unroll
      for (int t = 0; t < NST; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = k0 + t * 32 + acc_row(r, g);
          if (key >= s.M || (CAUSAL && key > myq)) sc[t][r] = -THERIA_INF;
        }
    }
    if (MODE == 0) {
      float mx = -THERIA_INF;
#pragma unroll
      for (int t = 0; t < NST; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sc[t][r]);
      mx = pair_max(mx) * c2;
      m_max = fmaxf(m_max, mx);
      const bool resc = mx > m_use + 8.f;
      if (__any(resc)) {
        const float alpha = resc ? fast_exp2(m_use - mx) : 1.f;
        m_use = resc ? mx : m_use;
        l_part *= alpha;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
          for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;
      }
    }
    // m_use is -inf only while every key seen so far is masked (then every score is -inf and P = 0);
    // in mode 1 a row without visible keys has lse = -inf and P must be 0 as well.
    const float moff = (m_use == -THERIA_INF) ? (MODE == 0 ? 0.f : THERIA_INF) : m_use;
    float ls = 0.f;
#pragma unroll
    for (int t = 0; t < NST; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float e = fast_exp2(fmaf(sc[t][r], c2, -moff));
        sc[t][r] = e;
        ls += e;
      }
    l_part += ls;
#pragma unroll
    for (int t = 0; t < NST; ++t)
#pragma unroll
      for (int cc = 0; cc < NPC; ++cc) {
        const F pf = acc_frag<T>(sc[t], cc);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
          o[dt] = MM::mma(lds_rows<T, KACC>(sV, PITCH, t * 32, cc, dt * 32), pf, o[dt]);
      }
  }

  if (MODE == 0) {
    const float l = pair_sum(l_part);
    const float inv = l > 0.f ? 1.f / l : 0.f;
    if (qvalid) {
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
          const int d0 = dt * 32 + 8 * qd + 4 * g;
          if (d0 < s.D) {
            const float a0 = o[dt][4 * qd] * inv, a1 = o[dt][4 * qd + 1] * inv;
            const float a2 = o[dt][4 * qd + 2] * inv, a3 = o[dt][4 * qd + 3] * inv;
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
        p.lse[row_id] = l > 0.f ? (m_use + __builtin_log2f(l)) * kLn2 : -THERIA_INF;
        if (p.row_max) p.row_max[row_id] = m_max * kLn2;
        if (p.row_sum) p.row_sum[row_id] = l > 0.f ? l * fast_exp2(m_use - m_max) : 0.f;
      }
    }
  } else {
    if (qvalid) {
      const T* dO = (const T*)p.dout.p + b * p.dout.sb + h * p.dout.sh;
      float* acc = p.dq_accum ? p.dq_accum + row_id * s.D : nullptr;
      float part = 0.f;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
          const int d0 = dt * 32 + 8 * qd + 4 * g;
          if (d0 < s.D) {
            const f32x4_t go = load4<T>(dO, p.dout.sr, myq, d0, s.D, s.vec);
#pragma unroll
            for (int e = 0; e < 4; ++e) part += go[e] * o[dt][4 * qd + e];
            if (acc) {
#pragma unroll
              for (int e = 0; e < 4; ++e)
                if (d0 + e < s.D) acc[d0 + e] = 0.f;
            }
          }
        }
      part = pair_sum(part);
      if (g == 0) p.delta[row_id] = part;
    }
  }
}

// delta_i = dO_i . O_i (the backward's row term), and zero the dQ accumulator rows.
template <typename TO, typename T, int DP>
__global__ __launch_bounds__(256) void pre_kernel(const PreParams p) {
  constexpr int LPR = DP / 8;  // lanes per row, 8 elements each
  constexpr int RPB = 256 / LPR;
  const Shape& s = p.s;
  const int64_t nrows = (int64_t)s.B * s.H * s.T;
  const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / LPR;
  const int part = threadIdx.x % LPR;
  const int col = part * 8;
  float acc = 0.f;
  if (row < nrows) {
    const int64_t bh = row / s.T;
    const int t = (int)(row - bh * s.T);
    const int b = (int)(bh / s.H), h = (int)(bh - (int64_t)b * s.H);
    const TO* O = (const TO*)p.o.p + b * p.o.sb + h * p.o.sh + (int64_t)t * p.o.sr;
    const T* G = (const T*)p.dout.p + b * p.dout.sb + h * p.dout.sh + (int64_t)t * p.dout.sr;
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (col + e < s.D) acc += (float)O[col + e] * (float)G[col + e];
    if (p.dq_accum) {
      float* z = p.dq_accum + row * s.D;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (col + e < s.D) z[col + e] = 0.f;
    }
  }
#pragma unroll
  for (int off = LPR / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (row < nrows && part == 0) p.delta[row] = acc;
}

// dQ (input dtype) from the float32 accumulator (which already carries the softmax scale).
template <typename T>
__global__ __launch_bounds__(256) void dq_convert_kernel(const DqParams p) {
  const Shape& s = p.s;
  const int64_t total = (int64_t)s.B * s.H * s.T * s.D;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int d = (int)(i % s.D);
    const int64_t row = i / s.D;
    const int64_t bh = row / s.T;
    const int t = (int)(row - bh * s.T);
    const int b = (int)(bh / s.H), h = (int)(bh - (int64_t)b * s.H);
    T* dq = (T*)p.dq.p + b * p.dq.sb + h * p.dq.sh + (int64_t)t * p.dq.sr;
    dq[d] = (T)p.dq_accum[i];
  }
}

template <int MODE>
struct FwdLauncher {
  template <typename T, int DP, bool CAUSAL>
  static hipError_t run(const FwdParams& p, hipStream_t st) {
    const int nqb = (p.s.T + 127) / 128;
    const int64_t nblk = (int64_t)nqb * p.s.B * p.s.H;
    if (nblk == 0) return hipSuccess;
    hipLaunchKernelGGL((fwd_kernel<T, DP, CAUSAL, MODE>), dim3((unsigned)nblk), dim3(256), 0, st, p);
    return hipGetLastError();
  }
};

hipError_t launch_fwd(const FwdParams& p, int mode, hipStream_t st) {
  return mode == 0 ? dispatch_all<FwdLauncher<0>>(p, st) : dispatch_all<FwdLauncher<1>>(p, st);
}

template <typename TO, typename T>
static hipError_t launch_pre_t(const PreParams& p, hipStream_t st) {
  const int64_t nrows = (int64_t)p.s.B * p.s.H * p.s.T;
  if (nrows == 0) return hipSuccess;
  const int lpr = p.s.dp / 8, rpb = 256 / lpr;
  const unsigned nblk = (unsigned)((nrows + rpb - 1) / rpb);
  switch (p.s.dp) {
    case 32: hipLaunchKernelGGL((pre_kernel<TO, T, 32>), dim3(nblk), dim3(256), 0, st, p); break;
    case 64: hipLaunchKernelGGL((pre_kernel<TO, T, 64>), dim3(nblk), dim3(256), 0, st, p); break;
    case 128: hipLaunchKernelGGL((pre_kernel<TO, T, 128>), dim3(nblk), dim3(256), 0, st, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_bwd_pre(const PreParams& p, hipStream_t st) {
  switch (p.s.dtype) {
    case 0: return launch_pre_t<float, float>(p, st);
    case 1: return p.o_f32 ? launch_pre_t<float, _Float16>(p, st) : launch_pre_t<_Float16, _Float16>(p, st);
    case 2: return p.o_f32 ? launch_pre_t<float, __bf16>(p, st) : launch_pre_t<__bf16, __bf16>(p, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_dq_convert(const DqParams& p, hipStream_t st) {
  const int64_t total = (int64_t)p.s.B * p.s.H * p.s.T * p.s.D;
  if (total == 0) return hipSuccess;
  int64_t nblk = (total + 255) / 256;
  if (nblk > 8192) nblk = 8192;
  switch (p.s.dtype) {
    case 0: hipLaunchKernelGGL(dq_convert_kernel<float>, dim3((unsigned)nblk), dim3(256), 0, st, p); break;
    case 1: hipLaunchKernelGGL(dq_convert_kernel<_Float16>, dim3((unsigned)nblk), dim3(256), 0, st, p); break;
    case 2: hipLaunchKernelGGL(dq_convert_kernel<__bf16>, dim3((unsigned)nblk), dim3(256), 0, st, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace theria
