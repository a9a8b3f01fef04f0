// Materialised score kernels behind the partial-fusion sdpa_custom backends on gfx950.
//
// qk_scores_kernel:  S = Q K^T (unscaled), written as a (B, H, T, M) tensor in float32 or in the input
//                    dtype. Replaces _qk_kernel / _qk_kernel_fast (reference theria/attention/
//                    triton_qk.py:24-64 and 402-453); the softmax and PV stay in PyTorch there too.
// qk_softmax_kernel: P = softmax_row(scale Q K^T), written as a float32 (B, H, T, M) tensor. Replaces
//                    _qk_softmax_kernel (triton_qk.py:128-194).
//
// Both compute the dot products with MFMA (32x32 output tiles per wave, fp32 accumulation: for float32
// inputs v_mfma_f32_32x32x2_f32 forms exact float32 products and sums, the reference's "ieee" dot).
// Operand fragments come straight from global memory (these backends exist for experiments; the fused
// operator is the fast path). qk_softmax makes two passes over the keys: pass 1 with this lane's query
// in the column (S^T = K Q^T) keeps an online row max and row sum per lane; pass 2 recomputes S with
// the query in the row, so that each store instruction writes 32 consecutive keys of a row.
#include "dispatch.hpp"
#include "sdpa_common.hpp"

namespace theria {

template <typename T, int DP, bool OUT_F32>
__global__ __launch_bounds__(256) void qk_scores_kernel(const ScoresParams p) {
  using MM = Mfma<T>;
  using F = typename MM::frag_t;
  constexpr int NKC = DP / MM::KC;
  const Shape& s = p.s;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, li = lane & 31, g = lane >> 5;
  const int nqb = (s.T + 63) / 64, nkb = (s.M + 63) / 64;
  const int bid = blockIdx.x;
  const int bh = bid / (nqb * nkb);
  const int rem = bid - bh * nqb * nkb;
  const int qb = rem / nkb, kb = rem - qb * nkb;
  const int b = bh / s.H, h = bh - b * s.H;
  const T* Q = (const T*)p.q.p + b * p.q.sb + h * p.q.sh;
  const T* K = (const T*)p.k.p + b * p.k.sb + h * p.k.sh;
  const int q0 = qb * 64 + (wave >> 1) * 32, k0 = kb * 64 + (wave & 1) * 32;

  f32x16_t acc = zero16();
#pragma unroll
  for (int c = 0; c < NKC; ++c) {
    const F a = gload_frag<T>(Q, p.q.sr, q0 + li, s.T, c, s.D, s.vec);
    const F bf = gload_frag<T>(K, p.k.sr, k0 + li, s.M, c, s.D, s.vec);
    acc = MM::mma(a, bf, acc);
  }
  const int key = k0 + li;
  if (key >= s.M) return;
  const int64_t base = (int64_t)bh * s.T * s.M;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int row = q0 + acc_row(r, g);
    if (row < s.T) {
      if (OUT_F32)
        ((float*)p.out)[base + (int64_t)row * s.M + key] = acc[r];
      else
        ((T*)p.out)[base + (int64_t)row * s.M + key] = (T)acc[r];
    }
  }
}

template <typename T, int DP>
__global__ __launch_bounds__(256) void qk_softmax_kernel(const ScoresParams p) {
  using MM = Mfma<T>;
  using F = typename MM::frag_t;
  constexpr int NKC = DP / MM::KC;
  __shared__ __attribute__((aligned(16))) float sM[4][32];
  __shared__ __attribute__((aligned(16))) float sL[4][32];
  const Shape& s = p.s;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, li = lane & 31, g = lane >> 5;
  const int nqb = (s.T + 127) / 128;
  const int bh = blockIdx.x / nqb;
  const int qb = blockIdx.x - bh * nqb;
  const int b = bh / s.H, h = bh - b * s.H;
  const T* Q = (const T*)p.q.p + b * p.q.sb + h * p.q.sh;
  const T* K = (const T*)p.k.p + b * p.k.sb + h * p.k.sh;
  const int q0 = qb * 128 + wave * 32;
  const float c2 = s.scale * kLog2e;

  F qf[NKC];
#pragma unroll
  for (int c = 0; c < NKC; ++c) qf[c] = gload_frag<T>(Q, p.q.sr, q0 + li, s.T, c, s.D, s.vec);

  // pass 1: per-query max and sum of exp (this lane's query li, keys acc_row(r, g) of each tile)
  float m = -THERIA_INF, l = 0.f;
  for (int k0 = 0; k0 < s.M; k0 += 32) {
    f32x16_t st = zero16();
#pragma unroll
    for (int c = 0; c < NKC; ++c) st = MM::mma(gload_frag<T>(K, p.k.sr, k0 + li, s.M, c, s.D, s.vec), qf[c], st);
    float mx = -THERIA_INF;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      if (k0 + acc_row(r, g) >= s.M) st[r] = -THERIA_INF;
      mx = fmaxf(mx, st[r]);
    }
    const float mnew = fmaxf(m, mx * c2);
    if (mnew != -THERIA_INF) {
      float part = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) part += fast_exp2(fmaf(st[r], c2, -mnew));
      l = l * fast_exp2(m - mnew) + part;
      m = mnew;
    }
  }
  // combine the two lane halves (each saw half of the keys of every tile)
  const float mt = pair_max(m);
  const float lt = pair_sum(m == -THERIA_INF ? 0.f : l * fast_exp2(m - mt));
  if (g == 0) {
    sM[wave][li] = mt;
    sL[wave][li] = lt > 0.f ? 1.f / lt : 0.f;
  }
  __syncthreads();

  // pass 2: P with the query in the row (register r <-> query acc_row(r, g)), 32 keys per store
  const int64_t base = (int64_t)bh * s.T * s.M;
  float mrow[16], irow[16];
#pragma unroll
  for (int qd = 0; qd < 4; ++qd) {
    const f32x4_t m4 = *reinterpret_cast<const f32x4_t*>(&sM[wave][8 * qd + 4 * g]);
    const f32x4_t i4 = *reinterpret_cast<const f32x4_t*>(&sL[wave][8 * qd + 4 * g]);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      mrow[4 * qd + e] = m4[e];
      irow[4 * qd + e] = i4[e];
    }
  }
  for (int k0 = 0; k0 < s.M; k0 += 32) {
    f32x16_t st = zero16();
#pragma unroll
    for (int c = 0; c < NKC; ++c) st = MM::mma(qf[c], gload_frag<T>(K, p.k.sr, k0 + li, s.M, c, s.D, s.vec), st);
    const int key = k0 + li;
    if (key < s.M) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = q0 + acc_row(r, g);
        if (row < s.T) {
          const float pv = mrow[r] == -THERIA_INF ? 0.f : fast_exp2(fmaf(st[r], c2, -mrow[r])) * irow[r];
          ((float*)p.out)[base + (int64_t)row * s.M + key] = pv;
        }
      }
    }
  }
}

struct ScoresLauncher {
  template <typename T, int DP, bool CAUSAL>
  static hipError_t run(const ScoresParams& p, hipStream_t st) {
    if constexpr (CAUSAL) {
      return hipErrorInvalidValue;  // the score backends have no mask
    } else {
      const int64_t bh = (int64_t)p.s.B * p.s.H;
      if (p.softmax) {
        const int64_t nblk = (int64_t)((p.s.T + 127) / 128) * bh;
        if (nblk == 0) return hipSuccess;
        hipLaunchKernelGGL((qk_softmax_kernel<T, DP>), dim3((unsigned)nblk), dim3(256), 0, st, p);
      } else {
        const int64_t nblk = (int64_t)((p.s.T + 63) / 64) * ((p.s.M + 63) / 64) * bh;
        if (nblk == 0) return hipSuccess;
        if (p.out_f32)
          hipLaunchKernelGGL((qk_scores_kernel<T, DP, true>), dim3((unsigned)nblk), dim3(256), 0, st, p);
        else
          hipLaunchKernelGGL((qk_scores_kernel<T, DP, false>), dim3((unsigned)nblk), dim3(256), 0, st, p);
      }
      return hipGetLastError();
    }
  }
};

hipError_t launch_scores(const ScoresParams& p, hipStream_t st) { return dispatch_all<ScoresLauncher>(p, st); }

}  // namespace theria
