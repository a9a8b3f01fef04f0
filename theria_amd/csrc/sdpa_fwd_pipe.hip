// Pipelined SDPA forward for 16-bit inputs on gfx950.
//
// Same contract as fwd_kernel (sdpa_fwd.hip): O = softmax(scale Q K^T) V with lse and the optional
// reference statistics (m, l) (reference theria/attention/triton_qk.py:242-304). It is used when
// the head dim is a multiple of 8 in 8..128 (computed at DP = 32, 64 or 128, the columns past D zero),
// every view allows 16-byte access and there are more than 128 queries.
//
// Work decomposition: one workgroup = NW waves x QT tiles of 32 queries (QT = 2 at DP = 32 and 64 without the
// causal mask, else 1); keys in tiles of 64. Scores are
// transposed (S^T = K Q^T), so each lane owns one query and the row sums are per-lane. Every SIMD runs two
// waves. With NW = 8 both are waves of one workgroup, kept in step by the per-tile barrier; two
// independent 4-wave workgroups on one CU do not share the SIMDs evenly (the older one is issued
// first and finishes well before the other), so NW = 8 is used whenever it still fills every CU.
//  * K and V tiles reach LDS by DMA (sdpa_lds.hpp) into double buffers, one barrier per key tile: the
//    loads for tile k+1 are in flight during the whole of iteration k.
//  * Software pipeline: iteration k issues the products O += V(k-1)^T P(k-1)^T next to S(k) = K(k) Q^T
//    and the exponentials of S(k), so MFMA and VALU work of adjacent tiles can overlap.
//  * No row max in the common path. P = exp2(S * scale * log2(e) - m_use) uses the current offset
//    m_use, and each lane's partial row sum of the tile is checked instead: while it is <= 2^20 every
//    P of the tile is finite and small enough for float32 accumulation. A tile that fails the check
//    (always the first tile, where m_use = -inf, and any tile whose scores exceed the offset by more
//    than ~14 in the log2 domain) takes a slow path that recomputes S, moves m_use to the exact running
//    max and rescales O and the row sum. lse = m_use + log2(l) does not depend on the offset.
//  * Row sums are accumulated from the rounded 16-bit P values that feed the PV product (v_dot2), so
//    numerator and denominator use the same probabilities.
#include <type_traits>

#include "sdpa_common.hpp"
#include "sdpa_lds.hpp"
#include "tile_count.hpp"
#include "sdpa_params.hpp"

namespace theria {

// QT query tiles of 32 per wave: two at DP = 32 and 64 without the causal mask, where each K / V^T fragment then
// feeds two MFMAs, unless the grid would then leave CUs without two waves per SIMD; one at DP = 128, where
// the registers would not allow two, and one with the causal mask, whose paired blocks need the smaller
// block to fill the GPU.
// FD: the head dim is DP itself (compile-time bounds); otherwise the runtime head dim s.D < DP bounds the
// loads, stores and DMA chunks.
#ifdef THERIA_TILE_COUNT
// 32 x 32 (query, key) units whose products the forward kernel ran (counter-enabled build only)
static __device__ unsigned long long g_tiles_fwd;
hipError_t tile_counts_fwd(unsigned long long* fwd, bool reset) {
  hipError_t e = hipMemcpyFromSymbol(fwd, HIP_SYMBOL(g_tiles_fwd), sizeof(*fwd));
  if (e == hipSuccess && reset) {
    const unsigned long long zero = 0;
    e = hipMemcpyToSymbol(HIP_SYMBOL(g_tiles_fwd), &zero, sizeof(zero));
  }
  return e;
}
#endif

template <typename T, bool CAUSAL, bool STATS, int NW, int DP, int QT, bool FD>
__global__ __launch_bounds__(64 * NW, 2) void fwd_pipe_kernel(const FwdParams p) {
  using MM = Mfma<T>;
  using F = typename MM::frag_t;
  // NKC k-chunks of 16 and NDT output tiles of 32 across the head dim.
  constexpr int NKC = DP / 16, NDT = DP / 32;
  constexpr int BM = 32 * NW * QT, BN = 64, TILE = BN * 2 * DP;
  // Separate arrays (not one [2][TILE] array) so that the compiler can tell the tile being read from the
  // tile being filled and does not wait for the DMA in flight before every LDS read.
  __shared__ __attribute__((aligned(1024))) char sK0[TILE];
  __shared__ __attribute__((aligned(1024))) char sK1[TILE];
  __shared__ __attribute__((aligned(1024))) char sV0[TILE];
  __shared__ __attribute__((aligned(1024))) char sV1[TILE];

  const Shape& s = p.s;
  const int Dh = FD ? DP : s.D;  // head dim
  const int lane = threadIdx.x & 63, li = lane & 31, g = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nqb = (s.T + BM - 1) / BM;
  // Causal: workgroup `unit` runs query block nqb - 1 - unit (the longest rows) and then its mirror
  // block `unit`, so every workgroup gets the same number of key tiles; an odd middle block runs once.
  // Unpaired (grids too small to fill the CUs in pairs): one block per workgroup, the longest first.
  const bool pair = CAUSAL && !s.unpaired;
  const int nunit = pair ? (nqb + 1) / 2 : nqb;
  const int bid = xcd_remap(blockIdx.x, gridDim.x);
  const int bh = bid / nunit;
  const int unit = bid - bh * nunit;
  const int b = bh / s.H, h = bh - b * s.H;
  const T* Q = (const T*)p.q.p + b * p.q.sb + h * p.q.sh;
  const T* K = (const T*)p.k.p + b * p.k.sb + h * p.k.sh;
  const T* V = (const T*)p.v.p + b * p.v.sb + h * p.v.sh;
  const int64_t rowbase = (int64_t)bh * s.T;
  const float c2 = s.scale * kLog2e;
  THERIA_TILES_DECL;

  for (int pass = 0; pass < (pair ? 2 : 1); ++pass) {
  const int qb = CAUSAL ? (pass == 0 ? nqb - 1 - unit : unit) : unit;
  if (pass == 1) {
    if (qb == nqb - 1 - unit) break;  // odd number of blocks: the middle one ran in pass 0
    __syncthreads();                  // every wave is done with the LDS tiles of the first block
  }
  const int q0w = qb * BM + wave * 32 * QT;  // query tile j of this wave starts at q0w + 32 j

    int kend = s.M;
    if (CAUSAL) kend = min(s.M, qb * BM + BM);
    const int nkt = (kend + BN - 1) / BN;
    // Tiles [0, nfull) have every key in range and visible to every query of the block.
    int nfull = s.M / BN;
    if (CAUSAL) nfull = min(nfull, qb * BM / BN);

    using Dma = SwzDma<NW, DP>;
    const Dma dma(wave, lane, Dh / 8);  // head dims below DP: zero-filled chunks past D
    constexpr int NSLAB = BN / Dma::SLAB_ROWS;
    static_assert(NSLAB * Dma::SLAB_ROWS == BN, "key tiles must be whole DMA slabs");
    // Byte offsets fit in 32 bits: the host only selects this kernel when every (batch, head) slab of K
    // and V spans less than 2^31 bytes.
    const uint32_t krs = (uint32_t)p.k.sr * 2, vrs = (uint32_t)p.v.sr * 2;
    const rsrc_t krsrc = make_rsrc(K, (uint32_t)slab_span(s.M, krs, 2 * Dh));
    const rsrc_t vrsrc = make_rsrc(V, (uint32_t)slab_span(s.M, vrs, 2 * Dh));
    uint32_t koff[NSLAB], voff[NSLAB];
#pragma unroll
    for (int i = 0; i < NSLAB; ++i) {
      koff[i] = dma.lane_offset(krs, i);
      voff[i] = dma.lane_offset(vrs, i);
    }
    if (nkt > 0) dma.template issue_clamped<NSLAB>(krsrc, krs, 0, s.M, sK0);

    F qf[QT][NKC];
#pragma unroll
    for (int j = 0; j < QT; ++j)
#pragma unroll
      for (int c = 0; c < NKC; ++c) qf[j][c] = gload_frag8<T>(Q, p.q.sr, q0w + 32 * j + li, s.T, c, Dh);

    f32x16_t o[QT][NDT];
    // pk_max: an upper bound of the row's largest P (relative to the current offset) that marks the peaked rows
    // in lse: the largest lane partial row sum of any tile (32 keys), one max per tile; causal (FINE), the largest
    // 8-key partial sum, one max per 8 keys: rows that see few keys would otherwise be flagged by the 32-key
    // sums of rows up to ~160 keys long, and every flagged row sends its block down the backward's exact path.
    constexpr bool FINE = CAUSAL;
    float m_use[QT], l_part[QT], m_max[QT], pk_max[QT];
#pragma unroll
    for (int j = 0; j < QT; ++j) {
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) o[j][dt] = zero16();
      m_use[j] = -THERIA_INF;
      l_part[j] = 0.f;
      m_max[j] = -THERIA_INF;
      pk_max[j] = 0.f;
    }
    F pf[QT][2][2];  // P of the previous tile as MFMA B fragments: [query tile][32-key subtile][16-key chunk]
    bool pf_skip = false;

    // S^T = K Q^T for both query tiles, key subtile t (32 keys) of the K tile in `kt`.
    auto scores_t = [&](const char* kt, int t, f32x16_t (&st)[QT]) {
#pragma unroll
      for (int j = 0; j < QT; ++j) st[j] = zero16();
#pragma unroll
      for (int c = 0; c < NKC; ++c) {
        const F kf = swz_cols<T, DP>(kt, 32 * t + li, c);
#pragma unroll
        for (int j = 0; j < QT; ++j) st[j] = MM::mma(kf, qf[j][c], st[j]);
      }
    };
    auto scores = [&](const char* kt, f32x16_t (&sc)[QT][2]) {
      f32x16_t s0[QT], s1[QT];
      scores_t(kt, 0, s0);
      scores_t(kt, 1, s1);
#pragma unroll
      for (int j = 0; j < QT; ++j) {
        sc[j][0] = s0[j];
        sc[j][1] = s1[j];
      }
    };
    // O^T += V^T P^T with the previous tile's P and the V tile in `vt`.
    auto pv_mma = [&](const char* vt) __attribute__((always_inline)) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int cc = 0; cc < 2; ++cc)
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) {
            const F vf = swz_rows<T, DP>(vt, 32 * t, cc, 32 * dt);
#pragma unroll
            for (int j = 0; j < QT; ++j) o[j][dt] = MM::mma(vf, pf[j][t][cc], o[j][dt]);
          }
    };
    // Keys out of range, or (causal) after the query, get -inf. Only boundary tiles pay for the test.
    auto mask = [&](f32x16_t (&sc)[QT][2], int k0) {
      if ((k0 + BN > s.M) || (CAUSAL && k0 + BN - 1 > q0w)) {
#pragma unroll
        for (int j = 0; j < QT; ++j) {
          const int lim = CAUSAL ? min(s.M, q0w + 32 * j + li + 1) : s.M;  // first key this query cannot see
#pragma unroll
          for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r)
              if (k0 + 32 * t + acc_row(r, g) >= lim) sc[j][t][r] = -THERIA_INF;
        }
      }
    };
    // P = exp2(S c2 - off) as 16-bit fragments into pn, this tile's lane partial row sums into ps and (FINE) the
    // largest 8-key partial sum into pk.
    auto exps = [&](const f32x16_t (&sc)[QT][2], const float (&off)[QT], F (&pn)[QT][2][2], float (&ps)[QT],
                    float (&pk)[QT]) {
#pragma unroll
      for (int j = 0; j < QT; ++j) {
        float acc = 0.f, mx = 0.f;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int cc = 0; cc < 2; ++cc) {
            F f;
#pragma unroll
            for (int e = 0; e < 8; ++e) f[e] = (T)fast_exp2(fmaf(sc[j][t][8 * cc + e], c2, -off[j]));
            pn[j][t][cc] = f;
            if constexpr (FINE) {
              const float fs = frag_sum<T>(f, 0.f);
              acc += fs;
              mx = fmaxf(mx, fs);
            } else {
              acc = frag_sum<T>(f, acc);
            }
          }
        ps[j] = acc;
        pk[j] = mx;
      }
    };
    // The same for key subtile t only, accumulating into ps and pk.
    auto exps_t = [&](const f32x16_t (&st)[QT], int t, F (&pn)[QT][2][2], float (&ps)[QT], float (&pk)[QT]) {
#pragma unroll
      for (int j = 0; j < QT; ++j)
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
          F f;
#pragma unroll
          for (int e = 0; e < 8; ++e) f[e] = (T)fast_exp2(fmaf(st[j][8 * cc + e], c2, -m_use[j]));
          pn[j][t][cc] = f;
          if constexpr (FINE) {
            const float fs = frag_sum<T>(f, 0.f);
            ps[j] += fs;
            pk[j] = fmaxf(pk[j], fs);
          } else {
            ps[j] = frag_sum<T>(f, ps[j]);
          }
        }
    };
    auto tile_max = [&](const f32x16_t (&sc)[QT][2], int j) {
      float mx = -THERIA_INF;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sc[j][t][r]);
      return pair_max(mx) * c2;
    };
    // Exact path: the running max becomes the offset; O and the row sums are rescaled to it.
    auto exact = [&](const f32x16_t (&sc)[QT][2], F (&pn)[QT][2][2], float (&ps)[QT], float (&pk)[QT]) {
      float off[QT];
#pragma unroll
      for (int j = 0; j < QT; ++j) {
        const float mx = tile_max(sc, j);
        m_max[j] = fmaxf(m_max[j], mx);
        const float mnew = fmaxf(m_use[j], mx);
        const float alpha = mnew == -THERIA_INF ? 1.f : fast_exp2(m_use[j] - mnew);
        m_use[j] = mnew;
        l_part[j] *= alpha;
        pk_max[j] *= alpha;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
          for (int r = 0; r < 16; ++r) o[j][dt][r] *= alpha;
        off[j] = mnew == -THERIA_INF ? 0.f : mnew;  // all keys so far masked: P = exp2(-inf) = 0
      }
      exps(sc, off, pn, ps, pk);
    };

    // One key tile. On entry K(k) and V(k-1) have been requested (one iteration earlier); this step
    // requests K(k+1) and V(k), issues O += V(k-1)^T P(k-1)^T, S(k) and P(k). kc/vp are the buffers holding
    // K(k)/V(k-1), kn/vn the buffers for K(k+1)/V(k). FAST: tile k is full (every key in range and visible
    // to every query of the block), tile k+1 is in range, and the buffers are compile-time distinct arrays.
    auto step = [&](auto fast_tag, int k, const char* kc, const char* vp, char* kn, char* vn) {
      constexpr bool FAST = decltype(fast_tag)::value;
      const int k0 = k * BN;
      wait_vm_all();
      __syncthreads();  // K(k), V(k-1) visible to all waves; the buffers of K(k-1), V(k-2) are free
      if (FAST) {
        dma.template issue<NSLAB>(krsrc, koff, (uint32_t)(k0 + BN) * krs, kn);
        dma.template issue<NSLAB>(vrsrc, voff, (uint32_t)k0 * vrs, vn);
      } else {
        if (k + 1 < nkt) dma.template issue_clamped<NSLAB>(krsrc, krs, k0 + BN, s.M, kn);
        dma.template issue_clamped<NSLAB>(vrsrc, vrs, k0, s.M, vn);
      }
      F pn[QT][2][2];
      // QT query tiles x two 32-key subtiles, unless every key of the tile follows every query of the wave
      if (FAST || !(CAUSAL && k0 > q0w + 32 * QT - 1)) THERIA_TILES_ADD(2 * QT);
      if constexpr (FAST) {
        // Phase order (kept by scheduling barriers, which also bound the live registers):
        //   S(k) subtile 0 | S(k) subtile 1 with exp of subtile 0 | O += V(k-1)^T P(k-1)^T with exp of subtile 1.
        f32x16_t s0[QT], s1[QT];
        float ps[QT], pk[QT];
#pragma unroll
        for (int j = 0; j < QT; ++j) ps[j] = pk[j] = 0.f;
        scores_t(kc, 0, s0);
        __builtin_amdgcn_sched_barrier(0);
        scores_t(kc, 1, s1);
        if (STATS) {
#pragma unroll
          for (int j = 0; j < QT; ++j) {
            float mx = -THERIA_INF;
#pragma unroll
            for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s0[j][r]);
            m_max[j] = fmaxf(m_max[j], pair_max(mx) * c2);
          }
        }
        exps_t(s0, 0, pn, ps, pk);
        if constexpr (DP == 64) {
          // Issue order inside the phase: the four K fragment reads first, then each of the 8 MFMAs
          // followed by 12 VALU instructions of the exponentials (measured ~5% faster than the
          // compiler's own order at head dim 64).
#pragma unroll
          for (int i = 0; i < 4; ++i) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 12, 0);  // VALU
          }
        }
        __builtin_amdgcn_sched_barrier(0);
        pv_mma(vp);
        if (STATS) {
#pragma unroll
          for (int j = 0; j < QT; ++j) {
            float mx = -THERIA_INF;
#pragma unroll
            for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s1[j][r]);
            m_max[j] = fmaxf(m_max[j], pair_max(mx) * c2);
          }
        }
        exps_t(s1, 1, pn, ps, pk);
        if constexpr (DP == 64) {
          // V fragment reads first, then each of the 16 PV MFMAs followed by 6 VALU instructions.
#pragma unroll
          for (int i = 0; i < 8; ++i) __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
            __builtin_amdgcn_sched_group_barrier(0x002, 6, 1);
          }
        }
        bool bad = false;
#pragma unroll
        for (int j = 0; j < QT; ++j) bad |= !(ps[j] <= 0x1p20f);
        if (__any(bad)) {
          f32x16_t sc2[QT][2];
          scores(kc, sc2);
          exact(sc2, pn, ps, pk);
        }
#pragma unroll
        for (int j = 0; j < QT; ++j) {
          l_part[j] += ps[j];
          pk_max[j] = fmaxf(pk_max[j], FINE ? pk[j] : ps[j]);
        }
#pragma unroll
        for (int j = 0; j < QT; ++j)
#pragma unroll
          for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int cc = 0; cc < 2; ++cc) pf[j][t][cc] = pn[j][t][cc];
        pf_skip = false;
      } else {
        const bool skip = CAUSAL && (k0 > q0w + 32 * QT - 1);  // every key after every query of the wave
        f32x16_t sc[QT][2];
        if (!skip) scores(kc, sc);
        if (k > 0 && !pf_skip) pv_mma(vp);
        if (!skip) {
          float ps[QT], pk[QT];
          mask(sc, k0);
          if (k == 0) {
            exact(sc, pn, ps, pk);
          } else {
            if (STATS) {
#pragma unroll
              for (int j = 0; j < QT; ++j) m_max[j] = fmaxf(m_max[j], tile_max(sc, j));
            }
            exps(sc, m_use, pn, ps, pk);
            bool bad = false;
#pragma unroll
            for (int j = 0; j < QT; ++j) bad |= !(ps[j] <= 0x1p20f);
            if (__any(bad)) {
              f32x16_t sc2[QT][2];
              scores(kc, sc2);
              mask(sc2, k0);
              exact(sc2, pn, ps, pk);
            }
          }
#pragma unroll
          for (int j = 0; j < QT; ++j) {
            l_part[j] += ps[j];
            pk_max[j] = fmaxf(pk_max[j], FINE ? pk[j] : ps[j]);
          }
#pragma unroll
          for (int j = 0; j < QT; ++j)
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
              for (int cc = 0; cc < 2; ++cc) pf[j][t][cc] = pn[j][t][cc];
        }
        pf_skip = skip;
      }
    };
    const std::integral_constant<bool, true> fast;
    const std::integral_constant<bool, false> general;
    if (nkt > 0) {
      // Tile 0 always takes the exact path (m_use = -inf); then the full tiles two at a time, so that
      // every buffer is a fixed array; then the boundary tiles.
      step(general, 0, sK0, sV1, sK1, sV0);
      // fast steps: k < nfull and K(k+1) in range
      const int nfast = min(nfull, s.M / BN - 1);
      int k = 1;
      for (; k + 1 < nfast; k += 2) {
        step(fast, k, sK1, sV0, sK0, sV1);      // k odd
        step(fast, k + 1, sK0, sV1, sK1, sV0);  // k + 1 even
      }
      if (k < nfast) {
        step(fast, k, sK1, sV0, sK0, sV1);
        ++k;
      }
      for (; k < nkt; ++k) {
        const bool odd = k & 1;
        step(general, k, odd ? sK1 : sK0, odd ? sV0 : sV1, odd ? sK0 : sK1, odd ? sV1 : sV0);
      }
      // drain: the last tile's PV
      wait_vm_all();
      __syncthreads();
      if (!pf_skip) pv_mma(((nkt - 1) & 1) ? sV1 : sV0);
    }

#pragma unroll
    for (int j = 0; j < QT; ++j) {
      const int myq = q0w + 32 * j + li;
      const float l = pair_sum(l_part[j]);
      const float inv = l > 0.f ? 1.f / l : 0.f;
      // cross-lane, so taken by every lane before the per-row branches
      const bool peaked = pair_max(pk_max[j]) > kPeakedFrac * l;
      if (myq < s.T) {
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
          for (int qd = 0; qd < 4; ++qd) {
            const int d0 = dt * 32 + 8 * qd + 4 * g;
            const float a0 = o[j][dt][4 * qd] * inv, a1 = o[j][dt][4 * qd + 1] * inv;
            const float a2 = o[j][dt][4 * qd + 2] * inv, a3 = o[j][dt][4 * qd + 3] * inv;
            if (p.o_f32) {
              float* O = (float*)p.o.p + b * p.o.sb + h * p.o.sh;
              store4_8<float>(O, p.o.sr, myq, d0, Dh, a0, a1, a2, a3);
            } else {
              T* O = (T*)p.o.p + b * p.o.sb + h * p.o.sh;
              store4_8<T>(O, p.o.sr, myq, d0, Dh, a0, a1, a2, a3);
            }
          }
        if (g == 0) {
          const int64_t row_id = rowbase + myq;
          p.lse[row_id] = l > 0.f ? lse_with_flag((m_use[j] + __builtin_log2f(l)) * kLn2, peaked) : -THERIA_INF;
          if (STATS) {
            if (p.row_max) p.row_max[row_id] = m_max[j] * kLn2;
            if (p.row_sum) p.row_sum[row_id] = l > 0.f ? l * fast_exp2(m_use[j] - m_max[j]) : 0.f;
          }
        }
      }
    }
  }  // pass
  THERIA_TILES_FLUSH(g_tiles_fwd);
}

template <typename T, bool CAUSAL, int NW, int DP, int QT>
static void fwd_pipe_go(const FwdParams& p, int64_t nblk, hipStream_t st) {
  const dim3 grid((unsigned)nblk), block(64 * NW);
  const bool stats = p.row_max || p.row_sum;
  if (p.s.D == DP) {
    if (stats)
      hipLaunchKernelGGL((fwd_pipe_kernel<T, CAUSAL, true, NW, DP, QT, true>), grid, block, 0, st, p);
    else
      hipLaunchKernelGGL((fwd_pipe_kernel<T, CAUSAL, false, NW, DP, QT, true>), grid, block, 0, st, p);
  } else {
    if (stats)
      hipLaunchKernelGGL((fwd_pipe_kernel<T, CAUSAL, true, NW, DP, QT, false>), grid, block, 0, st, p);
    else
      hipLaunchKernelGGL((fwd_pipe_kernel<T, CAUSAL, false, NW, DP, QT, false>), grid, block, 0, st, p);
  }
}

template <typename T, bool CAUSAL, int DP>
static void fwd_pipe_launch(const FwdParams& p0, hipStream_t st) {
  constexpr int QT = (DP <= 64 && !CAUSAL) ? 2 : 1;
  FwdParams p = p0;
  const int64_t bh = (int64_t)p.s.B * p.s.H;
  const int64_t cus = device_cu_count();
  // workgroups per (batch, head): query blocks, or (causal) pairs of mirrored query blocks
  auto units = [](int64_t nqb) { return CAUSAL ? (nqb + 1) / 2 : nqb; };
  const int64_t nblk8 = units((p.s.T + 256 * QT - 1) / (256 * QT)) * bh;
  const int64_t nblk4 = units((p.s.T + 128 * QT - 1) / (128 * QT)) * bh;
  // eight waves fill a 64-key DMA slab only at head dims 64 and 128 (at 32 one wave instruction copies 16 rows)
  if (DP >= 64 && nblk8 >= cus) {
    if constexpr (DP >= 64) fwd_pipe_go<T, CAUSAL, 8, DP, QT>(p, nblk8, st);
    return;
  }
  if constexpr (QT == 2) {
    // Too few query blocks to give every CU two four-wave workgroups: one query tile per wave doubles them.
    if (nblk4 < 2 * cus) {
      fwd_pipe_go<T, CAUSAL, 4, DP, 1>(p, units((p.s.T + 127) / 128) * bh, st);
      return;
    }
  }
  if (CAUSAL && nblk4 < cus) {
    // mirrored pairs would leave CUs without a workgroup: one block each, the longest first
    p.s.unpaired = true;
    fwd_pipe_go<T, CAUSAL, 4, DP, QT>(p, (p.s.T + 128 * QT - 1) / (128 * QT) * bh, st);
    return;
  }
  fwd_pipe_go<T, CAUSAL, 4, DP, QT>(p, nblk4, st);
}

// Launch if the pipelined kernel covers this problem (16-bit, head dim a multiple of 8 in 8..32 (run at
// DP = 32), 40..64 (DP = 64) or 72..128 (DP = 128), vector access, more than 128 queries); returns false
// otherwise.
template <typename T, bool CAUSAL>
bool launch_fwd_pipe(const FwdParams& p, hipStream_t st, hipError_t* err) {
  if (!(p.s.vec && p.s.D % 8 == 0 && p.s.D >= 8 && p.s.T > 128)) return false;
  // 32-bit byte offsets inside each (batch, head) slab of K and V
  if (!slab_fits_dma(p.s.M, p.k.sr, p.s.D) || !slab_fits_dma(p.s.M, p.v.sr, p.s.D)) return false;
  if ((int64_t)p.s.B * p.s.H == 0) {
    *err = hipSuccess;
    return true;
  }
  if (p.s.dp == 32)
    fwd_pipe_launch<T, CAUSAL, 32>(p, st);
  else if (p.s.dp == 64)
    fwd_pipe_launch<T, CAUSAL, 64>(p, st);
  else
    fwd_pipe_launch<T, CAUSAL, 128>(p, st);
  *err = hipGetLastError();
  return true;
}

template bool launch_fwd_pipe<__bf16, false>(const FwdParams&, hipStream_t, hipError_t*);
template bool launch_fwd_pipe<__bf16, true>(const FwdParams&, hipStream_t, hipError_t*);
template bool launch_fwd_pipe<_Float16, false>(const FwdParams&, hipStream_t, hipError_t*);
template bool launch_fwd_pipe<_Float16, true>(const FwdParams&, hipStream_t, hipError_t*);

}  // namespace theria
