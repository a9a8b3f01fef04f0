// Materialised score kernels behind the partial-fusion sdpa_custom backends on gfx950.
//
// S = Q K^T (unscaled) as a (B, H, T, M) tensor in float32 or in the input dtype: replaces _qk_kernel /
//   _qk_kernel_fast (reference theria/attention/triton_qk.py:24-64 and 402-453); the softmax and PV stay in
//   PyTorch there too.
// P = softmax_row(scale Q K^T) as a float32 (B, H, T, M) tensor: replaces _qk_softmax_kernel
//   (triton_qk.py:128-194).
//
// These kernels are bound by the write of the (B, H, T, M) output (1.07 GB in float32 at B4 H16 S2048), not by
// the dot products, so the layout serves the stores:
//  * one workgroup = 4 waves = 128 query rows of one (batch, head); each wave keeps its 32 queries' Q fragments
//    in registers and the workgroup streams K in 64-key tiles through LDS (one global read of K per workgroup,
//    register-prefetched one tile ahead);
//  * scores are formed lane-per-query (S^T = K Q^T with MFMA, float32 accumulation: for float32 inputs
//    v_mfma_f32_32x32x2_f32 forms exact float32 products and sums, the reference's "ieee" dot);
//  * each wave writes its 32 x 32 subtiles of results into its own padded LDS buffer and reads them back
//    row-major, 16 bytes per lane, with non-temporal stores (the output is not read again by this kernel; K stays
//    in L2). For 16-bit inputs up to head dim 64 the buffer holds four subtiles (16.5 KiB per wave), so that one
//    store instruction writes 2 rows x 128 consecutive keys (512 bytes each in float32): two workgroups fit a
//    CU's LDS, config 2's 4096 waves run in two rounds, and the stores reach 5.9 TB/s where 8 rows x 32 keys per
//    instruction from a one-subtile buffer (five workgroups per CU, every wave resident) reached 5.3 TB/s.
//    Otherwise the buffer holds one subtile (4.5 KiB per wave);
//  * P: a first pass over the key tiles keeps a running offset and row sum per lane (the offset only moves when
//    a subtile's partial sum leaves (0, 2^20], so the pass has no per-score max; the two lane halves of a query
//    are combined at the end), the second forms exp2(S scale log2 e - m) / l and stores it;
//  * the register budget matches the occupancy the LDS allows (two waves per SIMD with the four-subtile buffer,
//    four with the one-subtile buffer at head dim <= 64), so the MFMA accumulators stay in VGPRs instead of
//    AGPRs, which the statistics pass would read back one v_accvgpr_read per score.
#include <type_traits>

#include "dispatch.hpp"
#include "sdpa_common.hpp"

namespace theria {

enum ScoreMode { kScoresF32 = 0, kScoresT = 1, kProbs = 2 };

// Stores of 128 consecutive keys per row (four subtiles staged per wave, 16.5 KiB of LDS each, which leaves two
// workgroups per CU) for 16-bit inputs up to head dim 64; one subtile (4.5 KiB) otherwise.
template <typename T, int DP>
constexpr bool scores_wide() {
  return sizeof(T) == 2 && DP <= 64;
}

template <typename T, int DP, int MODE>
__global__ __launch_bounds__(256, (scores_wide<T, DP>() || DP > 64) ? 2 : 4) void scores_kernel(const ScoresParams p) {
  using MM = Mfma<T>;
  using F = typename MM::frag_t;
  constexpr int NKC = DP / MM::KC;
  constexpr int NW = 4, NT = 64 * NW, BN = 64, NU = BN / 32;
  constexpr int PITCH = DP + 16 / (int)sizeof(T);  // K tile rows (padded)
  constexpr int SW = scores_wide<T, DP>() ? 4 : 1;  // 32-key subtiles staged per store round
  constexpr int OP = 32 * SW + 4;                   // output staging rows, in floats (padded against bank conflicts)
  __shared__ __attribute__((aligned(16))) T sK[BN * PITCH];
  __shared__ __attribute__((aligned(16))) float sO[NW][32 * OP];

  const Shape& s = p.s;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, li = lane & 31, g = lane >> 5;
  const int nqb = (s.T + 127) / 128;
  const int bid = xcd_remap(blockIdx.x, gridDim.x);  // the query blocks of one head on one XCD (K shared in L2)
  const int bh = bid / nqb;
  const int qb = bid - bh * nqb;
  const int b = bh / s.H, h = bh - b * s.H;
  const T* Q = (const T*)p.q.p + b * p.q.sb + h * p.q.sh;
  const T* K = (const T*)p.k.p + b * p.k.sb + h * p.k.sh;
  const int q0w = qb * 128 + wave * 32;
  const float c2 = s.scale * kLog2e;

  F qf[NKC];
#pragma unroll
  for (int c = 0; c < NKC; ++c) qf[c] = gload_frag<T>(Q, p.q.sr, q0w + li, s.T, c, s.D, s.vec);

  const int nkt = (s.M + BN - 1) / BN;
  TileStage<T, BN, DP, NT> stK;
  // Stages key tile kt (two barriers) and prefetches the next one.
  auto stage = [&](int kt) {
    __syncthreads();  // every wave is done with the previous tile
    stK.store(sK, PITCH);
    __syncthreads();
    if (kt + 1 < nkt) stK.load_any(K, p.k.sr, (kt + 1) * BN, s.M, s.D, s.vec);
  };
  // S^T of subtile u of the staged tile kt for this wave's 32 queries: keys kt*BN + 32u + acc_row(r, g) of
  // query li; keys past the end are -inf.
  auto sub_scores = [&](int kt, int u) {
    f32x16_t st = zero16();
#pragma unroll
    for (int c = 0; c < NKC; ++c) st = MM::mma(lds_cols<T, KLIN>(sK, PITCH, 32 * u + li, 0, c), qf[c], st);
    if (kt * BN + 32 * u + 32 > s.M) {
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (kt * BN + 32 * u + acc_row(r, g) >= s.M) st[r] = -THERIA_INF;
    }
    return st;
  };
  // One sweep over the key tiles: body(kt, u) for each 32-key subtile.
  auto sweep = [&](auto&& body) {
    if (nkt > 0) stK.load_any(K, p.k.sr, 0, s.M, s.D, s.vec);
    for (int kt = 0; kt < nkt; ++kt) {
      stage(kt);
#pragma unroll
      for (int u = 0; u < NU; ++u) body(kt, u);
    }
  };

  // softmax statistics of query li (log2 domain): a running offset `off` and the sum l of exp2(S c2 - off) over
  // its keys. The offset only moves when a subtile's lane partial sum leaves (0, 2^20] (always on the lane's
  // first visible subtile): then it becomes the running max and l is rescaled. Below 2^20 every term is finite
  // and far from float32 overflow, and P = exp2(S c2 - off) / l does not depend on which offset was used.
  auto stats_add = [&](const f32x16_t& st, float& off, float& l) {
    float part = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) part += fast_exp2(fmaf(st[r], c2, -off));
    if (!(part <= 0x1p20f)) {  // first visible subtile of the lane, or scores far above the offset
      float mx = st[0];
#pragma unroll
      for (int r = 1; r < 16; ++r) mx = fmaxf(mx, st[r]);
      mx = fmaxf(off, mx * c2);
      if (mx == -THERIA_INF) return;  // no visible key yet
      part = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) part += fast_exp2(fmaf(st[r], c2, -mx));
      l = l * fast_exp2(off - mx);
      off = mx;
    }
    l += part;
  };
  // The lane halves of a query combined: P = exp2(S c2 - mrow) * inv_l.
  auto stats_end = [&](float off, float l, float& mrow, float& inv_l) {
    const float mt = pair_max(off);
    const float lt = pair_sum(off == -THERIA_INF ? 0.f : l * fast_exp2(off - mt));
    mrow = mt == -THERIA_INF ? 0.f : mt;  // finite, so exp2(-inf * c2 - mrow) = 0 for masked keys
    inv_l = lt > 0.f ? 1.f / lt : 0.f;
  };

  using OutT = typename std::conditional<MODE == kScoresT, T, float>::type;
  OutT* out = (OutT*)p.out + (int64_t)bh * s.T * s.M;
  float* so = sO[wave];
  const bool vrows = (s.M % 4) == 0;
  // Subtile (kt, u) of S (scores) or P into the wave's buffer, row li (query), keys 32 (sub % SW) + 8j + 4g ..+3;
  // once SW subtiles (or the last one) are staged, the 32 rows x 32 SW keys go out: each store instruction writes
  // 8 / SW rows x 32 SW consecutive keys (two rows x 512 bytes in float32 at SW = 4), 16 bytes per lane, vector
  // stores when the rows are aligned.
  auto emit = [&](int kt, int u, const f32x16_t& st, float mrow, float inv_l) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      f32x4_t v;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x = st[4 * j + e];
        v[e] = MODE == kProbs ? fast_exp2(fmaf(x, c2, -mrow)) * inv_l : x;
      }
      *reinterpret_cast<f32x4_t*>(so + li * OP + 32 * ((kt * NU + u) % SW) + 8 * j + 4 * g) = v;
    }
    const int sub = kt * NU + u;
    if (sub % SW != SW - 1 && sub != nkt * NU - 1) return;  // the round's subtiles are not all staged yet
    __builtin_amdgcn_wave_barrier();
    constexpr int LPR = 8 * SW, RPI = 64 / LPR;  // lanes per row, rows per store instruction
    const int col = 4 * (lane % LPR);
    const int key = (sub / SW) * SW * 32 + col;  // keys past the staged subtiles are past the end
#pragma unroll
    for (int it = 0; it < 32 / RPI; ++it) {
      const int row = RPI * it + lane / LPR;
      const int q = q0w + row;
      const f32x4_t v = *reinterpret_cast<const f32x4_t*>(so + row * OP + col);
      if (q >= s.T || key >= s.M) continue;
      OutT* dst = out + (int64_t)q * s.M + key;
      if (vrows && key + 4 <= s.M) {
        if constexpr (sizeof(OutT) == 4) {
          __builtin_nontemporal_store(v, reinterpret_cast<f32x4_t*>(dst));
        } else {
          OutT w[4] = {(OutT)v[0], (OutT)v[1], (OutT)v[2], (OutT)v[3]};
          __builtin_nontemporal_store(__builtin_bit_cast(i16x4_t, w), reinterpret_cast<i16x4_t*>(dst));
        }
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (key + e < s.M) dst[e] = (OutT)v[e];
      }
    }
    __builtin_amdgcn_wave_barrier();  // the buffer is rewritten by the next round
  };

  float mrow = 0.f, inv_l = 0.f;
  if constexpr (MODE == kProbs) {
    float off = -THERIA_INF, l = 0.f;
    sweep([&](int kt, int u) { stats_add(sub_scores(kt, u), off, l); });
    stats_end(off, l, mrow, inv_l);
  }
  sweep([&](int kt, int u) { emit(kt, u, sub_scores(kt, u), mrow, inv_l); });
}

struct ScoresLauncher {
  template <typename T, int DP, bool CAUSAL>
  static hipError_t run(const ScoresParams& p, hipStream_t st) {
    if constexpr (CAUSAL) {
      return hipErrorInvalidValue;  // the score backends have no mask
    } else {
      const int64_t nblk = (int64_t)((p.s.T + 127) / 128) * p.s.B * p.s.H;
      if (nblk == 0) return hipSuccess;
      const dim3 grid((unsigned)nblk), block(256);
      if (p.softmax)
        hipLaunchKernelGGL((scores_kernel<T, DP, kProbs>), grid, block, 0, st, p);
      else if (p.out_f32 || sizeof(T) == 4)
        hipLaunchKernelGGL((scores_kernel<T, DP, kScoresF32>), grid, block, 0, st, p);
      else
        hipLaunchKernelGGL((scores_kernel<T, DP, kScoresT>), grid, block, 0, st, p);
      return hipGetLastError();
    }
  }
};

hipError_t launch_scores(const ScoresParams& p, hipStream_t st) { return dispatch_all<ScoresLauncher>(p, st); }

}  // namespace theria
