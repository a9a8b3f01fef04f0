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
//   keys as two 32-key subtiles for 16-bit inputs at head dim <= 64, else 32) accumulates the four D-wide products of the G_Q expression plus r and t, writes G_Q, r, t.
// cols kernel: lane per key (as in the backward). One pass over query tiles (64 queries as two 32-query
//   subtiles for 16-bit inputs at head dim <= 64, else 32) with r, t, z, lse per row staged in LDS
//   accumulates G_V and G_K in registers.
#include "dispatch.hpp"
#include "sdpa_common.hpp"

namespace theria {

template <typename T, int DP, bool CAUSAL>
__global__ __launch_bounds__(256) void bwdbwd_rows_kernel(const BwdBwdParams p) {
  using MM = Mfma<T>;
  using F = typename MM::frag_t;
  constexpr int KC = MM::KC;
  constexpr int NW = 4, BM = 32 * NW, NT = 64 * NW;
  // keys per tile: two 32-key subtiles per pair of barriers where the registers allow (one wave per SIMD)
  constexpr int BN = (DP == 128 || sizeof(T) == 4) ? 32 : 64;
  constexpr int PITCH = DP + 16 / (int)sizeof(T);
  constexpr int NDT = DP / 32, NKC = DP / KC, NPC = 32 / KC, NST = BN / 32;
  __shared__ __attribute__((aligned(16))) T sK[BN * PITCH];
  __shared__ __attribute__((aligned(16))) T sV[BN * PITCH];
  __shared__ __attribute__((aligned(16))) T sgK[BN * PITCH];
  __shared__ __attribute__((aligned(16))) T sgV[BN * PITCH];

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
  const bool has_gq = p.gq.p != nullptr, has_gk = p.gk.p != nullptr, has_gv = p.gv.p != nullptr;
  const T* GQ = has_gq ? (const T*)p.gq.p + b * p.gq.sb + h * p.gq.sh : nullptr;
  const T* GK = has_gk ? (const T*)p.gk.p + b * p.gk.sb + h * p.gk.sh : nullptr;
  const T* GV = has_gv ? (const T*)p.gv.p + b * p.gv.sb + h * p.gv.sh : nullptr;
  const int q0w = qb * BM + wave * 32;
  const int myq = q0w + li;
  const bool qvalid = myq < s.T;
  const int64_t row_id = (int64_t)bh * s.T + myq;

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
  const float z = qvalid ? p.delta[row_id] : 0.f;
  float r_part = 0.f, t_part = 0.f;

  int kend = s.M;
  if (CAUSAL) kend = min(s.M, qb * BM + BM);
  const int nkt = (kend + BN - 1) / BN;
  TileStage<T, BN, DP, NT> gsK, gsV, gsgK, gsgV;
  auto prefetch = [&](int k0) {
    gsK.load(K, p.k.sr, k0, s.M, s.D, s.vec);
    gsV.load(V, p.v.sr, k0, s.M, s.D, s.vec);
    if (has_gk) gsgK.load(GK, p.gk.sr, k0, s.M, s.D, s.vec);
    if (has_gv) gsgV.load(GV, p.gv.sr, k0, s.M, s.D, s.vec);
  };
  if (nkt > 0) prefetch(0);
  for (int kt = 0; kt < nkt; ++kt) {
    const int k0 = kt * BN;
    __syncthreads();
    gsK.store(sK, PITCH);
    gsV.store(sV, PITCH);
    if (has_gk) gsgK.store(sgK, PITCH);
    if (has_gv) gsgV.store(sgV, PITCH);
    __syncthreads();
    if (kt + 1 < nkt) prefetch(k0 + BN);
#pragma unroll
    for (int st = 0; st < NST; ++st) {
    const int k0s = k0 + 32 * st;  // this 32-key subtile
    if (CAUSAL && k0s > q0w + 31) continue;

    f32x16_t sc = zero16(), gm = zero16(), w = zero16(), dpz;
#pragma unroll
    for (int r = 0; r < 16; ++r) dpz[r] = -z;
#pragma unroll
    for (int c = 0; c < NKC; ++c) {
      const F kfr = lds_cols<T, KLIN>(sK, PITCH, 32 * st + li, 0, c);
      sc = MM::mma(kfr, qf[c], sc);
      dpz = MM::mma(lds_cols<T, KLIN>(sV, PITCH, 32 * st + li, 0, c), dof[c], dpz);
      if (has_gq) gm = MM::mma(kfr, gqf[c], gm);
      if (has_gk) gm = MM::mma(lds_cols<T, KLIN>(sgK, PITCH, 32 * st + li, 0, c), qf[c], gm);
      if (has_gv) w = MM::mma(lds_cols<T, KLIN>(sgV, PITCH, 32 * st + li, 0, c), dof[c], w);
    }
    const bool need_mask = (k0s + 32 > s.M) || (CAUSAL && k0s + 31 > q0w);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float pv = fast_exp2(fmaf(sc[r], c2, -moff));
      if (need_mask) {
        const int key = k0s + acc_row(r, g);
        if (key >= s.M || (CAUSAL && key > myq)) pv = 0.f;
      }
      const float gam = s.scale * gm[r];
      const float e1 = fmaf(gam, dpz[r], w[r]);
      const float pe1 = pv * e1;
      r_part = fmaf(pv, gam, r_part);
      t_part += pe1;
      sc[r] = pv;
      gm[r] = pe1;
      dpz[r] = pv * dpz[r];  // dS
    }
#pragma unroll
    for (int cc = 0; cc < NPC; ++cc) {
      const F pf = acc_frag<T>(sc, cc);
      const F pe1f = acc_frag<T>(gm, cc);
      const F dsf = acc_frag<T>(dpz, cc);
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const F kr = lds_rows<T, KACC>(sK, PITCH, 32 * st, cc, dt * 32);
        x13[dt] = MM::mma(kr, pe1f, x13[dt]);
        x2[dt] = MM::mma(kr, dsf, x2[dt]);
        x4[dt] = MM::mma(kr, pf, x4[dt]);
        if (has_gk) yk[dt] = MM::mma(lds_rows<T, KACC>(sgK, PITCH, 32 * st, cc, dt * 32), dsf, yk[dt]);
      }
    }
    }  // subtile
  }

  const float rr = pair_sum(r_part), tt = pair_sum(t_part);
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
            r4[e] = s.scale * (x13[dt][i] - rr * x2[dt][i] - tt * x4[dt][i] + yk[dt][i]);
          }
          store4<T>(OG, p.out_gq.sr, myq, d0, s.D, r4[0], r4[1], r4[2], r4[3], s.vec);
        }
      }
    if (g == 0) {
      p.r_row[row_id] = rr;
      p.t_row[row_id] = tt;
    }
  }
}

template <typename T, int DP, bool CAUSAL>
__global__ __launch_bounds__(256) void bwdbwd_cols_kernel(const BwdBwdParams p) {
  using MM = Mfma<T>;
  using F = typename MM::frag_t;
  constexpr int KC = MM::KC;
  constexpr int NW = 4, BN = 32 * NW, NT = 64 * NW;
  // queries per tile: two 32-query subtiles per pair of barriers where the registers allow
  constexpr int BM = (DP == 128 || sizeof(T) == 4) ? 32 : 64;
  constexpr int PITCH = DP + 16 / (int)sizeof(T);
  constexpr int NDT = DP / 32, NKC = DP / KC, NPC = 32 / KC, NSQ = BM / 32;
  __shared__ __attribute__((aligned(16))) T sQ[BM * PITCH];
  __shared__ __attribute__((aligned(16))) T sdO[BM * PITCH];
  __shared__ __attribute__((aligned(16))) T sgQ[BM * PITCH];
  __shared__ __attribute__((aligned(16))) float sLse[BM];
  __shared__ __attribute__((aligned(16))) float sZ[BM];
  __shared__ __attribute__((aligned(16))) float sR[BM];
  __shared__ __attribute__((aligned(16))) float sT[BM];

  const Shape& s = p.s;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6, li = lane & 31, g = lane >> 5;
  const int nkb = (s.M + BN - 1) / BN;
  const int bid = xcd_remap(blockIdx.x, gridDim.x);
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

  TileStage<T, BM, DP, NT> gsQ, gsO, gsgQ;
  float pre[4] = {THERIA_INF, 0.f, 0.f, 0.f};
  auto prefetch = [&](int q0) {
    gsQ.load(Q, p.q.sr, q0, s.T, s.D, s.vec);
    gsO.load(dO, p.dout.sr, q0, s.T, s.D, s.vec);
    if (has_gq) gsgQ.load(GQ, p.gq.sr, q0, s.T, s.D, s.vec);
    if (tid < BM) {
      const int qq = q0 + tid;
      const bool ok = qq < s.T;
      const float l2 = ok ? p.lse[rowbase + qq] * kLog2e : THERIA_INF;
      pre[0] = l2 == -THERIA_INF ? THERIA_INF : l2;
      pre[1] = ok ? p.delta[rowbase + qq] : 0.f;
      pre[2] = ok ? p.r_row[rowbase + qq] : 0.f;
      pre[3] = ok ? p.t_row[rowbase + qq] : 0.f;
    }
  };
  if (nqt > 0) prefetch(qbeg);
  for (int it = 0; it < nqt; ++it) {
    const int q0 = qbeg + it * BM;
    __syncthreads();
    gsQ.store(sQ, PITCH);
    gsO.store(sdO, PITCH);
    if (has_gq) gsgQ.store(sgQ, PITCH);
    if (tid < BM) {
      sLse[tid] = pre[0];
      sZ[tid] = pre[1];
      sR[tid] = pre[2];
      sT[tid] = pre[3];
    }
    __syncthreads();
    if (it + 1 < nqt) prefetch(q0 + BM);
    if (CAUSAL && kw0 > q0 + BM - 1) continue;
#pragma unroll
    for (int sq = 0; sq < NSQ; ++sq) {
    const int q0s = q0 + 32 * sq;  // this 32-query subtile
    if (CAUSAL && kw0 > q0s + 31) continue;

    f32x16_t sc = zero16(), gm = zero16(), w = zero16(), dpz;
    f32x4_t l4[4], z4[4], r4[4], t4[4];
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) {
      const int o = 32 * sq + 8 * qd + 4 * g;
      l4[qd] = *reinterpret_cast<const f32x4_t*>(sLse + o);
      z4[qd] = *reinterpret_cast<const f32x4_t*>(sZ + o);
      r4[qd] = *reinterpret_cast<const f32x4_t*>(sR + o);
      t4[qd] = *reinterpret_cast<const f32x4_t*>(sT + o);
#pragma unroll
      for (int e = 0; e < 4; ++e) dpz[4 * qd + e] = -z4[qd][e];
    }
#pragma unroll
    for (int c = 0; c < NKC; ++c) {
      const F qfr = lds_cols<T, KLIN>(sQ, PITCH, 32 * sq + li, 0, c);
      const F ofr = lds_cols<T, KLIN>(sdO, PITCH, 32 * sq + li, 0, c);
      sc = MM::mma(qfr, kf[c], sc);
      dpz = MM::mma(ofr, vf[c], dpz);
      if (has_gq) gm = MM::mma(lds_cols<T, KLIN>(sgQ, PITCH, 32 * sq + li, 0, c), kf[c], gm);
      if (has_gk) gm = MM::mma(qfr, gkf[c], gm);
      if (has_gv) w = MM::mma(ofr, gvf[c], w);
    }
    const bool diag = CAUSAL && (kw0 + 31 > q0s);
    f32x16_t gdp, gs;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int qd = r >> 2, e = r & 3;
      float pv = fast_exp2(fmaf(sc[r], c2, -l4[qd][e]));
      if (!kvalid) pv = 0.f;
      if (diag && mykey > q0s + acc_row(r, g)) pv = 0.f;
      const float gam = s.scale * gm[r];
      const float ds = pv * dpz[r];
      const float e1 = fmaf(gam, dpz[r], w[r]);
      gdp[r] = pv * (gam - r4[qd][e]);
      gs[r] = pv * e1 - r4[qd][e] * ds - t4[qd][e] * pv;
      dpz[r] = ds;
    }
#pragma unroll
    for (int cc = 0; cc < NPC; ++cc) {
      const F gdpf = acc_frag<T>(gdp, cc);
      const F gsf = acc_frag<T>(gs, cc);
      const F dsf = acc_frag<T>(dpz, cc);
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        accV[dt] = MM::mma(gdpf, lds_rows<T, KACC>(sdO, PITCH, 32 * sq, cc, dt * 32), accV[dt]);
        accK[dt] = MM::mma(gsf, lds_rows<T, KACC>(sQ, PITCH, 32 * sq, cc, dt * 32), accK[dt]);
        if (has_gq) accK[dt] = MM::mma(dsf, lds_rows<T, KACC>(sgQ, PITCH, 32 * sq, cc, dt * 32), accK[dt]);
      }
    }
    }  // subtile
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

struct RowsLauncher {
  template <typename T, int DP, bool CAUSAL>
  static hipError_t run(const BwdBwdParams& p, hipStream_t st) {
    const int nqb = (p.s.T + 127) / 128;
    const int64_t nblk = (int64_t)nqb * p.s.B * p.s.H;
    if (nblk == 0) return hipSuccess;
    hipLaunchKernelGGL((bwdbwd_rows_kernel<T, DP, CAUSAL>), dim3((unsigned)nblk), dim3(256), 0, st, p);
    return hipGetLastError();
  }
};

struct ColsLauncher {
  template <typename T, int DP, bool CAUSAL>
  static hipError_t run(const BwdBwdParams& p, hipStream_t st) {
    const int nkb = (p.s.M + 127) / 128;
    const int64_t nblk = (int64_t)nkb * p.s.B * p.s.H;
    if (nblk == 0) return hipSuccess;
    hipLaunchKernelGGL((bwdbwd_cols_kernel<T, DP, CAUSAL>), dim3((unsigned)nblk), dim3(256), 0, st, p);
    return hipGetLastError();
  }
};

hipError_t launch_bwdbwd_rows(const BwdBwdParams& p, hipStream_t st) { return dispatch_all<RowsLauncher>(p, st); }
hipError_t launch_bwdbwd_cols(const BwdBwdParams& p, hipStream_t st) { return dispatch_all<ColsLauncher>(p, st); }

}  // namespace theria
