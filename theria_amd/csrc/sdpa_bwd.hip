// Explicit SDPA backward (dQ, dK, dV) for gfx950.
//
// Replaces the reference's three kernels _sdpa_bwd_dv_kernel, _sdpa_bwd_dk_kernel and
// _sdpa_bwd_dq_kernel (theria/attention/triton_sdpa_backward.py:106-191, 269-398, 505-632) with one
// pass. Math (docs/phase9.md:19-26 of the reference): P from the saved lse, dV = P^T dO,
// dP = dO V^T, dS = P o (dP - delta), dQ = scale dS K, dK = scale dS^T Q, where delta_i = dO_i . O_i
// equals the reference's z_i = sum_j dP_ij P_ij and is computed once per row beforehand.
//
// Work decomposition: one workgroup = 4 waves owns 128 keys of one (batch, head) for the whole
// kernel (32 per wave) and walks over the query rows in tiles of 64 (32 for float32). Score tiles
// are computed as S = Q K^T so that, in the accumulator layout, each lane owns one key: the P and dS
// tiles are then directly the A operands of dV += P^T dO and dK += dS^T Q, whose B operands
// (dO^T, Q^T) come from the LDS transpose read, and dV/dK live in registers until the end. K and V
// fragments stay in registers as the B operands of S and dP. dP is seeded with -delta so the MFMA
// produces dP - delta directly. dQ needs the other orientation: each wave writes its scale*dS block
// to LDS, and after one barrier every wave computes one 32x32 dQ tile over all 128 keys of the
// workgroup (A = dS rows, B = K^T by transpose read of the LDS copy of K) and adds it into a float32
// accumulator with global float atomics; a final pass converts that accumulator to the input dtype.
// Causal: query tiles entirely above the block's first key are never visited, fully masked
// (wave, tile) pairs skip their MFMAs, and only diagonal tiles are masked element-wise.
#include "dispatch.hpp"
#include "sdpa_common.hpp"

namespace theria {

template <typename T, int DP, bool CAUSAL>
__global__ __launch_bounds__(256) void bwd_kernel(const BwdParams p) {
  using MM = Mfma<T>;
  using F = typename MM::frag_t;
  constexpr int KC = MM::KC;
  constexpr int NW = 4, BN = 32 * NW, NT = 64 * NW;
  constexpr int BM = sizeof(T) == 2 ? 64 : 32;
  constexpr int PITCH = DP + 16 / (int)sizeof(T);
  constexpr int SPITCH = BN + 16 / (int)sizeof(T);
  constexpr int NDT = DP / 32, NKC = DP / KC, NPC = 32 / KC, NQT = BM / 32;
  __shared__ __attribute__((aligned(16))) T sQ[BM * PITCH];
  __shared__ __attribute__((aligned(16))) T sdO[BM * PITCH];
  __shared__ __attribute__((aligned(16))) T sK[BN * PITCH];
  __shared__ __attribute__((aligned(16))) T sdS[BM * SPITCH];
  __shared__ __attribute__((aligned(16))) float sLse[BM];
  __shared__ __attribute__((aligned(16))) float sDel[BM];

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
  const bool dv_only = p.dv_only;
  const bool want_dq = p.want_dq && !dv_only;
  const bool want_dk = p.want_dk && !dv_only;

  const int key0 = kb * BN;
  const int kw0 = key0 + wave * 32;
  const int mykey = kw0 + li;
  const bool kvalid = mykey < s.M;

  F kf[NKC], vf[NKC];
#pragma unroll
  for (int c = 0; c < NKC; ++c) kf[c] = gload_frag<T>(K, p.k.sr, mykey, s.M, c, s.D, s.vec);
  if (!dv_only) {
    const T* V = (const T*)p.v.p + b * p.v.sb + h * p.v.sh;
#pragma unroll
    for (int c = 0; c < NKC; ++c) vf[c] = gload_frag<T>(V, p.v.sr, mykey, s.M, c, s.D, s.vec);
  } else {
#pragma unroll
    for (int c = 0; c < NKC; ++c) vf[c] = F{};
  }
  if (want_dq) {
    TileStage<T, BN, DP, NT> stK;
    stK.load(K, p.k.sr, key0, s.M, s.D, s.vec);
    stK.store(sK, PITCH);  // published by the first barrier of the query loop
  }

  f32x16_t dv[NDT], dk[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
    dv[dt] = zero16();
    dk[dt] = zero16();
  }
  const float c2 = s.scale * kLog2e;
  const int qbeg = CAUSAL ? (key0 / BM) * BM : 0;
  const int nqt = s.T > qbeg ? (s.T - qbeg + BM - 1) / BM : 0;
  const int64_t rowbase = (int64_t)bh * s.T;

  TileStage<T, BM, DP, NT> stQ, stO;
  float pre_lse = THERIA_INF, pre_del = 0.f;
  auto prefetch = [&](int q0) {
    stQ.load(Q, p.q.sr, q0, s.T, s.D, s.vec);
    stO.load(dO, p.dout.sr, q0, s.T, s.D, s.vec);
    if (tid < BM) {
      const int qq = q0 + tid;
      pre_lse = qq < s.T ? p.lse[rowbase + qq] * kLog2e : THERIA_INF;
      pre_del = (qq < s.T && !dv_only) ? p.delta[rowbase + qq] : 0.f;
    }
  };
  if (nqt > 0) prefetch(qbeg);

  for (int it = 0; it < nqt; ++it) {
    const int q0 = qbeg + it * BM;
    __syncthreads();
    stQ.store(sQ, PITCH);
    stO.store(sdO, PITCH);
    if (tid < BM) {
      sLse[tid] = pre_lse;
      sDel[tid] = pre_del;
    }
    __syncthreads();
    if (it + 1 < nqt) prefetch(q0 + BM);

#pragma unroll
    for (int qt = 0; qt < NQT; ++qt) {
      const int qr0 = qt * 32;
      const int q0t = q0 + qr0;
      const bool active = q0t < s.T && (!CAUSAL || kw0 <= q0t + 31);
      if (!active) {
        if (want_dq) {
#pragma unroll
          for (int r = 0; r < 16; ++r) sdS[(qr0 + acc_row(r, g)) * SPITCH + wave * 32 + li] = (T)0.f;
        }
        continue;
      }
      f32x16_t sc = zero16();
#pragma unroll
      for (int c = 0; c < NKC; ++c) sc = MM::mma(lds_cols<T, KLIN>(sQ, PITCH, qr0 + li, 0, c), kf[c], sc);
      f32x4_t lse4[4];
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) lse4[qd] = *reinterpret_cast<const f32x4_t*>(sLse + qr0 + 8 * qd + 4 * g);
      f32x16_t dp;
      if (!dv_only) {
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
          const f32x4_t d4 = *reinterpret_cast<const f32x4_t*>(sDel + qr0 + 8 * qd + 4 * g);
#pragma unroll
          for (int e = 0; e < 4; ++e) dp[4 * qd + e] = -d4[e];
        }
#pragma unroll
        for (int c = 0; c < NKC; ++c) dp = MM::mma(lds_cols<T, KLIN>(sdO, PITCH, qr0 + li, 0, c), vf[c], dp);
      }
      const bool diag = CAUSAL && (kw0 + 31 > q0t);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float pv = fast_exp2(fmaf(sc[r], c2, -lse4[r >> 2][r & 3]));
        if (!kvalid) pv = 0.f;
        if (diag && mykey > q0t + acc_row(r, g)) pv = 0.f;
        sc[r] = pv;
      }
#pragma unroll
      for (int cc = 0; cc < NPC; ++cc) {
        const F pa = acc_frag<T>(sc, cc);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) dv[dt] = MM::mma(pa, lds_rows<T, KACC>(sdO, PITCH, qr0, cc, dt * 32), dv[dt]);
      }
      if (!dv_only) {
#pragma unroll
        for (int r = 0; r < 16; ++r) dp[r] *= sc[r];  // dS
        if (want_dk) {
#pragma unroll
          for (int cc = 0; cc < NPC; ++cc) {
            const F da = acc_frag<T>(dp, cc);
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt)
              dk[dt] = MM::mma(da, lds_rows<T, KACC>(sQ, PITCH, qr0, cc, dt * 32), dk[dt]);
          }
        }
        if (want_dq) {
#pragma unroll
          for (int r = 0; r < 16; ++r) sdS[(qr0 + acc_row(r, g)) * SPITCH + wave * 32 + li] = (T)(dp[r] * s.scale);
        }
      }
    }

    if (want_dq) {
      __syncthreads();
#pragma unroll
      for (int tile = wave; tile < NQT * NDT; tile += NW) {
        const int qt = tile / NDT, dt = tile - (tile / NDT) * NDT;
        const int qr0 = qt * 32;
        if (q0 + qr0 >= s.T) continue;
        f32x16_t acc = zero16();
#pragma unroll
        for (int kc = 0; kc < BN / KC; ++kc)
          acc = MM::mma(lds_cols<T, KLIN>(sdS, SPITCH, qr0 + li, 0, kc), lds_rows<T, KLIN>(sK, PITCH, 0, kc, dt * 32), acc);
        const int d = dt * 32 + li;
        if (d < s.D) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int q = q0 + qr0 + acc_row(r, g);
            if (q < s.T) unsafeAtomicAdd(p.dq_accum + (rowbase + q) * s.D + d, acc[r]);
          }
        }
      }
    }
  }

  // Epilogue: lane holds column d = dt*32 + li of rows (keys) kw0 + acc_row(r, g).
  {
    T* DV = (T*)p.dv.p + b * p.dv.sb + h * p.dv.sh;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const int d = dt * 32 + li;
      if (d < s.D) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kw0 + acc_row(r, g);
          if (key < s.M) DV[(int64_t)key * p.dv.sr + d] = (T)dv[dt][r];
        }
      }
    }
  }
  if (want_dk) {
    T* DK = (T*)p.dk.p + b * p.dk.sb + h * p.dk.sh;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const int d = dt * 32 + li;
      if (d < s.D) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kw0 + acc_row(r, g);
          if (key < s.M) DK[(int64_t)key * p.dk.sr + d] = (T)(dk[dt][r] * s.scale);
        }
      }
    }
  }
}

struct BwdLauncher {
  template <typename T, int DP, bool CAUSAL>
  static hipError_t run(const BwdParams& p, hipStream_t st) {
    const int nkb = (p.s.M + 127) / 128;
    const int64_t nblk = (int64_t)nkb * p.s.B * p.s.H;
    if (nblk == 0) return hipSuccess;
    hipLaunchKernelGGL((bwd_kernel<T, DP, CAUSAL>), dim3((unsigned)nblk), dim3(256), 0, st, p);
    return hipGetLastError();
  }
};

hipError_t launch_bwd(const BwdParams& p, hipStream_t st) { return dispatch_all<BwdLauncher>(p, st); }

}  // namespace theria
