// Pipelined dQ and dK/dV passes of the SDPA backward for 16-bit inputs on gfx950 (head dim a multiple of 8
// in 8..128, computed at DP = 32, 64 or 128 with the columns past D zero).
//
// dkdv_pipe_kernel has the contract of dkdv_kernel (sdpa_bwd.hip): dV = P^T dO and dK = scale dS^T Q with
// P = exp(scale Q K^T - lse) rebuilt from the saved row statistic and dS = P o (dO V^T - delta)
// (reference theria/attention/triton_sdpa_backward.py:106-266 and 269-462). It is used when the head
// dim qualifies and every view allows 16-byte access; the general kernel covers the rest.
//
// Work decomposition: one workgroup = NW waves, each owning 32 keys (K and V fragments in registers,
// dK and dV accumulated in registers); the workgroup streams the query tiles (64 or 128 rows) of its head.
//  * Q and dO tiles reach LDS by DMA (sdpa_lds.hpp) into double buffers with one barrier per tile;
//    the row terms -lse * log2(e) and -delta of the next tile are loaded by the first 64 threads during
//    the current tile and written beside them, with a flag for a tile holding a peaked row (largest
//    probability above 1/4, flagged in lse): the tile loop skips such tiles, and a workgroup that skipped
//    any runs them after the loop (found from the lse flags) from exact float32 scores, with P and dS as
//    two 16-bit terms (hi + lo), into the same dK / dV accumulators.
//  * Scores are S = Q K^T with this lane's key in the column, so dV += P^T dO and dK += dS^T Q take
//    P and dS straight from the accumulators (KACC order) and dO^T / Q^T from LDS transpose reads.
//  * Phase order per 64-row half of a tile, i.e. two 32-query subtiles (scheduling barriers keep it):
//      S, dP of subtile 0 | S, dP of subtile 1 with exp / dS of subtile 0
//      | dV, dK of subtile 0 with exp / dS of subtile 1 | dV, dK of subtile 1.
//  * dP starts from -delta as the MFMA accumulator input, so dS = P o dP is one multiply; K is held
//    pre-multiplied by scale * log2(e) (rounded once to 16 bits) and S starts from -lse * log2(e), so
//    P = exp2(S) takes no multiply per score. That rounding moves each score by ~2^-9 of its terms, below the
//    16-bit rounding of P on rows without a peaked flag; the peaked tiles (above) form exact scores from the
//    unscaled K instead.
#include <type_traits>

#include "sdpa_common.hpp"
#include "sdpa_lds.hpp"
#include "sdpa_params.hpp"
#include "tile_count.hpp"

// Waves per workgroup (compile-time knobs; the defaults are the measured best on MI355X).
#ifndef DQ_PIPE_NW
#define DQ_PIPE_NW 4
#endif
#ifndef DKDV_PIPE_NW
#define DKDV_PIPE_NW 4  // head dim 128 (head dim 64 picks 8 or 4 per problem size in the launcher)
#endif
// 64-row halves per tile (one barrier per tile): the query tile of dK/dV and the key tile of dQ. At head
// dim 128 (one wave per SIMD) 128-row tiles halve the barriers, which shortens dK/dV by a quarter; at 64
// (two waves per SIMD) they shorten dQ by ~1% and change nothing measurable for dK/dV.
#ifndef DQ64_HALVES
#define DQ64_HALVES 2
#endif
#ifndef DKDV64_HALVES
#define DKDV64_HALVES 1
#endif
#ifndef DQ128_HALVES
#define DQ128_HALVES 2
#endif
#ifndef DKDV128_HALVES
#define DKDV128_HALVES 2
#endif
// Head dim 128: subtile overlap and waves per SIMD
#ifndef DQ128_OVERLAP
#define DQ128_OVERLAP true
#endif
#ifndef DQ128_WPS
#define DQ128_WPS 1
#endif
#ifndef DKDV128_OVERLAP
#define DKDV128_OVERLAP true
#endif
#ifndef DKDV128_WPS
#define DKDV128_WPS 1
#endif

namespace theria {

#ifdef THERIA_TILE_COUNT
// 32 x 32 (query, key) units whose products the dQ and dK/dV kernels ran (counter-enabled build only)
static __device__ unsigned long long g_tiles_dq, g_tiles_dkdv;
hipError_t tile_counts_bwd(unsigned long long* dq, unsigned long long* dkdv, bool reset) {
  hipError_t e = hipMemcpyFromSymbol(dq, HIP_SYMBOL(g_tiles_dq), sizeof(*dq));
  if (e == hipSuccess) e = hipMemcpyFromSymbol(dkdv, HIP_SYMBOL(g_tiles_dkdv), sizeof(*dkdv));
  if (e == hipSuccess && reset) {
    const unsigned long long zero = 0;
    e = hipMemcpyToSymbol(HIP_SYMBOL(g_tiles_dq), &zero, sizeof(zero));
    if (e == hipSuccess) e = hipMemcpyToSymbol(HIP_SYMBOL(g_tiles_dkdv), &zero, sizeof(zero));
  }
  return e;
}
#endif

// FD: the head dim is DP itself (compile-time bounds); otherwise the runtime head dim s.D < DP bounds the
// loads, stores and DMA chunks (both kernels).
// dkdv_pipe_kernel runs the query tiles without a peaked row (flagged in lse: largest probability above 1/4)
// with K pre-multiplied by scale * log2(e) and S started from -lse2, so P = exp2(S), and skips the others;
// after the last tile, a workgroup that skipped any finds them again (a scan of the lse flags) and runs them
// from the exact float32 scores with P and dS as two 16-bit terms each, into the same dK, dV accumulators.
// Running them apart from the tile loop keeps the loop's registers and schedule.
template <typename T, bool CAUSAL, int NW, int DP, bool OVERLAP, int WPS, int HALVES, bool FD>
__global__ __launch_bounds__(64 * NW, WPS) void dkdv_pipe_kernel(const DkdvParams p) {
  using MM = Mfma<T>;
  using F = typename MM::frag_t;
  using Dma = SwzDma<NW, DP>;
  constexpr int NKC = DP / 16, NDT = DP / 32;
  constexpr int BN = 32 * NW, BM = 64 * HALVES, TILE = BM * 2 * DP, NSLAB = BM / Dma::SLAB_ROWS;
  static_assert(NSLAB * Dma::SLAB_ROWS == BM, "query tiles must be whole DMA slabs");
  static_assert(64 * NW >= BM, "the row terms of a tile are loaded one per thread");
  // OVERLAP: the exp / dS work of one subtile overlaps the products of the next (more live registers);
  // otherwise subtiles run one after the other. WPS: waves per SIMD the register budget is sized for.
  __shared__ __attribute__((aligned(1024))) char sQ0[TILE];
  __shared__ __attribute__((aligned(1024))) char sQ1[TILE];
  __shared__ __attribute__((aligned(1024))) char sO0[TILE];
  __shared__ __attribute__((aligned(1024))) char sO1[TILE];
  __shared__ __attribute__((aligned(16))) float sR0[2 * BM];  // [-lse * log2(e) | -delta] of a tile
  __shared__ __attribute__((aligned(16))) float sR1[2 * BM];
  __shared__ int sF0[2], sF1[2];  // per 64-row half: the tile holds a peaked row

  const Shape& s = p.s;
  const int tid = threadIdx.x;
  const int lane = tid & 63, li = lane & 31, g = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nkb = (s.M + BN - 1) / BN;
  // Causal at head dim <= 64: workgroup `unit` runs key block `unit` (the longest query range) and then its
  // mirror block nkb - 1 - unit, so every workgroup gets the same number of query tiles; an odd middle
  // block runs once. At head dim 128 (one workgroup per CU) the plain longest-first order measured faster.
  // Unpaired (grids too small to fill the CUs in pairs): one block per workgroup, the longest first.
  const bool pair = CAUSAL && DP <= 64 && !s.unpaired;
  const int nunit = pair ? (nkb + 1) / 2 : nkb;
  const int bid = xcd_remap(blockIdx.x, gridDim.x);
  const int bh = bid / nunit;
  const int unit = bid - bh * nunit;
  const int b = bh / s.H, h = bh - b * s.H;
  const T* Q = (const T*)p.q.p + b * p.q.sb + h * p.q.sh;
  const T* K = (const T*)p.k.p + b * p.k.sb + h * p.k.sh;
  const T* V = (const T*)p.v.p + b * p.v.sb + h * p.v.sh;
  const T* dO = (const T*)p.dout.p + b * p.dout.sb + h * p.dout.sh;
  const int64_t rowbase = (int64_t)bh * s.T;
  const float c2 = s.scale * kLog2e;
  THERIA_TILES_DECL;

  for (int pass = 0; pass < (pair ? 2 : 1); ++pass) {
  const int kb = pass == 0 ? unit : nkb - 1 - unit;
  if (pass == 1) {
    if (kb == unit) break;  // odd number of blocks: the middle one ran in pass 0
    __syncthreads();        // every wave is done with the LDS tiles of the first block
  }
  const int key0 = kb * BN;
  const int kw0 = key0 + wave * 32;  // this wave's keys: kw0 + li

    // K pre-multiplied by scale * log2(e) and S started from -lse * log2(e): P = exp2(S) with no per-score
    // scaling. The tiles holding a peaked row form the exact scores from K itself (kraw below).
    F kf[NKC], vf[NKC];
    auto load_v = [&]() {
#pragma unroll
      for (int c = 0; c < NKC; ++c) vf[c] = gload_frag8<T>(V, p.v.sr, kw0 + li, s.M, c, FD ? DP : s.D);
    };
#pragma unroll
    for (int c = 0; c < NKC; ++c) kf[c] = scaled_frag<T>(gload_frag8<T>(K, p.k.sr, kw0 + li, s.M, c, FD ? DP : s.D), c2);
    load_v();
    f32x16_t dv[NDT], dk[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      dv[dt] = zero16();
      dk[dt] = zero16();
    }

    const int qbeg = CAUSAL ? (key0 / BM) * BM : 0;
    const int nqt = s.T > qbeg ? (s.T - qbeg + BM - 1) / BM : 0;
    // Tiles with every query in range and (causal) every key of the block visible to every query,
    // in a key block whose keys are all in range, take the unmasked path.
    // Causal: tiles before ifull straddle the diagonal (q0 < last key of the block). Full tiles end at fend.
    const int ifull = CAUSAL ? min(nqt, (key0 + BN - 1 - qbeg + BM - 1) / BM) : 0;
    const int fend = (key0 + BN <= s.M) ? max(ifull, min(nqt, (s.T - qbeg) / BM)) : ifull;

    const Dma dma(wave, lane, FD ? DP / 8 : s.D / 8);  // head dims below DP: zero-filled chunks past D
    const uint32_t qrs = (uint32_t)p.q.sr * 2, ors = (uint32_t)p.dout.sr * 2;
    const rsrc_t qrsrc = make_rsrc(Q, (uint32_t)slab_span(s.T, qrs, 2 * (FD ? DP : s.D)));
    const rsrc_t orsrc = make_rsrc(dO, (uint32_t)slab_span(s.T, ors, 2 * (FD ? DP : s.D)));
    // K unscaled for the exact body: chunk c of key kw0 + li by a buffer load (zeros past the head dim and the
    // last key), so that no per-chunk address stays live across the tile loop.
    const uint32_t krs = (uint32_t)p.k.sr * 2;
    const rsrc_t krsrc = make_rsrc(K, (uint32_t)slab_span(s.M, krs, 2 * (FD ? DP : s.D)));
    auto kraw = [&](int c) {
      const int key = kw0 + li, col = c * 16 + 8 * g;
      const bool ok = key < s.M && (FD || col < s.D);
      return __builtin_bit_cast(F, buf_load16(krsrc, ok ? (uint32_t)key * krs + 2 * col : 0x80000000u, 0));
    };

    // Row terms of tile `it` for thread tid < BM, loaded two tiles ahead as raw lse and delta (rows past the
    // end: lse = +inf) and converted only when stored, so that no instruction waits for these loads (or for
    // the DMA issued just before them) until the next tile. Stored: -lse * log2(e) (-inf for rows past the
    // end or without visible keys, so P = 0), -delta, and per 64-row half whether it holds a row flagged
    // peaked in its lse.
    float r_lse = THERIA_INF, r_del = 0.f;
    auto load_rows = [&](int it) {
      if (tid < BM && it < nqt) {
        const int qq = qbeg + it * BM + tid;
        r_lse = qq < s.T ? p.lse[rowbase + qq] : THERIA_INF;
        r_del = qq < s.T ? p.delta[rowbase + qq] : 0.f;
      }
    };
    auto store_rows = [&](float* sr, int* sf) {
      if (tid < BM) {  // whole waves (BM is a multiple of 64)
        sr[tid] = __builtin_isinf(r_lse) ? -THERIA_INF : -r_lse * kLog2e;
        sr[BM + tid] = -r_del;
        const bool pk = __any(lse_peaked(r_lse));
        if (lane == 0) sf[tid >> 6] = pk;
      }
    };
    auto peaked_tile = [&](const int* sf) {
      return __builtin_amdgcn_readfirstlane(BM > 64 ? (sf[0] | sf[1]) : sf[0]) != 0;
    };

    // S = c2 Q K^T - lse2 and dP = dO V^T - delta for subtile qs (32 queries) of the tile in (tq, to, tr).
    auto sdp = [&](const char* tq, const char* to, const float* tr, int qs, f32x16_t& sc, f32x16_t& dp) {
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        const f32x4_t l4 = *reinterpret_cast<const f32x4_t*>(tr + 32 * qs + 8 * qd + 4 * g);
        const f32x4_t d4 = *reinterpret_cast<const f32x4_t*>(tr + BM + 32 * qs + 8 * qd + 4 * g);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          sc[4 * qd + e] = l4[e];
          dp[4 * qd + e] = d4[e];
        }
      }
#pragma unroll
      for (int c = 0; c < NKC; ++c) {
        sc = MM::mma(swz_cols<T, DP>(tq, 32 * qs + li, c), kf[c], sc);
        dp = MM::mma(swz_cols<T, DP>(to, 32 * qs + li, c), vf[c], dp);
      }
    };
    // Masks of a general tile: keys out of range and (causal) keys after the query get S = -inf.
    auto mask = [&](f32x16_t& sc, int q0s) {
      const int mykey = kw0 + li;
      if (kw0 + 31 >= s.M || (CAUSAL && kw0 + 31 > q0s)) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (mykey >= s.M || (CAUSAL && mykey > q0s + acc_row(r, g))) sc[r] = -THERIA_INF;
      }
    };
    // P = exp2(S) and dS = P o dP as 16-bit fragments (KACC chunks 0, 1).
    auto pds = [&](const f32x16_t& sc, const f32x16_t& dp, F (&pf)[2], F (&df)[2]) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float pv = fast_exp2(sc[r]);
        pf[r >> 3][r & 7] = (T)pv;
        df[r >> 3][r & 7] = (T)(pv * dp[r]);
      }
    };
    // dV += P^T dO and dK += dS^T Q for subtile qs.
    auto dvdk = [&](const char* tq, const char* to, int qs, const F (&pf)[2], const F (&df)[2]) {
#pragma unroll
      for (int cc = 0; cc < 2; ++cc)
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
          dv[dt] = MM::mma(pf[cc], swz_rows<T, DP>(to, 32 * qs, cc, 32 * dt), dv[dt]);
          dk[dt] = MM::mma(df[cc], swz_rows<T, DP>(tq, 32 * qs, cc, 32 * dt), dk[dt]);
        }
    };
    // Subtiles of query tile `it` in (tq, to, tr). FAST: every query in range and every key visible.
    auto body = [&](auto fast_tag, int it, const char* tq, const char* to, const float* tr) {
      constexpr bool FAST = decltype(fast_tag)::value;
      const int q0 = qbeg + it * BM;
      if constexpr (FAST && OVERLAP) {
        THERIA_TILES_ADD(2 * HALVES);
#pragma unroll
        for (int hf = 0; hf < HALVES; ++hf) {
          f32x16_t s0, p0, s1, p1;
          F pf0[2], df0[2], pf1[2], df1[2];
          sdp(tq, to, tr, 2 * hf, s0, p0);
          __builtin_amdgcn_sched_barrier(0);
          sdp(tq, to, tr, 2 * hf + 1, s1, p1);
          pds(s0, p0, pf0, df0);
          __builtin_amdgcn_sched_barrier(0);
          dvdk(tq, to, 2 * hf, pf0, df0);
          pds(s1, p1, pf1, df1);
          __builtin_amdgcn_sched_barrier(0);
          dvdk(tq, to, 2 * hf + 1, pf1, df1);
          __builtin_amdgcn_sched_barrier(0);
        }
      } else {
#pragma unroll
        for (int qs = 0; qs < 2 * HALVES; ++qs) {
          const int q0s = q0 + 32 * qs;
          if (!FAST && (q0s >= s.T || (CAUSAL && kw0 > q0s + 31))) continue;  // wave-uniform
          THERIA_TILES_ADD(1);
          f32x16_t sc, dp;
          F pf[2], df[2];
          sdp(tq, to, tr, qs, sc, dp);
          if (!FAST) mask(sc, q0s);
          pds(sc, dp, pf, df);
          dvdk(tq, to, qs, pf, df);
        }
      }
    };
    // A tile holding a peaked row instead: the exact float32 scores (from K reloaded unscaled, seeded with
    // -lse2 through the FMA) and P, dS as two 16-bit terms each (hi + lo, ~2^-16 relative), subtiles one after
    // the other.
    auto exact_body = [&](auto fast_tag, int it, const char* tq, const char* to, const float* tr) {
      constexpr bool FAST = decltype(fast_tag)::value;
      const int q0 = qbeg + it * BM;
#pragma unroll
      for (int qs = 0; qs < 2 * HALVES; ++qs) {
        const int q0s = q0 + 32 * qs;
        if (!FAST && (q0s >= s.T || (CAUSAL && kw0 > q0s + 31))) continue;  // wave-uniform
        THERIA_TILES_ADD(1);
        f32x16_t se = zero16(), dp;
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
          const f32x4_t d4 = *reinterpret_cast<const f32x4_t*>(tr + BM + 32 * qs + 8 * qd + 4 * g);
#pragma unroll
          for (int e = 0; e < 4; ++e) dp[4 * qd + e] = d4[e];
        }
#pragma unroll
        for (int c = 0; c < NKC; ++c) {
          se = MM::mma(swz_cols<T, DP>(tq, 32 * qs + li, c), kraw(c), se);
          dp = MM::mma(swz_cols<T, DP>(to, 32 * qs + li, c), vf[c], dp);
        }
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
          const f32x4_t l4 = *reinterpret_cast<const f32x4_t*>(tr + 32 * qs + 8 * qd + 4 * g);
#pragma unroll
          for (int e = 0; e < 4; ++e) se[4 * qd + e] = fmaf(se[4 * qd + e], c2, l4[e]);
        }
        if (!FAST) mask(se, q0s);
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
          F ph, pl, dh, dl;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float pv = fast_exp2(se[8 * cc + e]);
            const float ds = pv * dp[8 * cc + e];
            ph[e] = (T)pv;
            pl[e] = (T)(pv - (float)ph[e]);
            dh[e] = (T)ds;
            dl[e] = (T)(ds - (float)dh[e]);
          }
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) {
            const F ro = swz_rows<T, DP>(to, 32 * qs, cc, 32 * dt);
            dv[dt] = MM::mma(ph, ro, dv[dt]);
            dv[dt] = MM::mma(pl, ro, dv[dt]);
            const F rq = swz_rows<T, DP>(tq, 32 * qs, cc, 32 * dt);
            dk[dt] = MM::mma(dh, rq, dk[dt]);
            dk[dt] = MM::mma(dl, rq, dk[dt]);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    const std::integral_constant<bool, true> fast;
    const std::integral_constant<bool, false> general;

    bool pk_any = false;  // uniform: a tile holding a peaked row was skipped
    // One query tile `it` from buffers (tq, to, tr, tf); the next tile goes to (nq, no, nr, nf).
    auto step = [&](auto fast_tag, int it, const char* tq, const char* to, const float* tr, const int* tf, char* nq,
                    char* no, float* nr, int* nf) {
      const int q0 = qbeg + it * BM;
      wait_vm_all();
      __syncthreads();  // tile it visible to all waves; the other buffers (tile it-1) are free
      if (it + 1 < nqt) {
        dma.template issue_clamped<NSLAB>(qrsrc, qrs, q0 + BM, s.T, nq);
        dma.template issue_clamped<NSLAB>(orsrc, ors, q0 + BM, s.T, no);
        store_rows(nr, nf);
        load_rows(it + 2);
      }
      const bool pk = peaked_tile(tf);
      pk_any |= pk;  // run after the loop
      if (!pk) body(fast_tag, it, tq, to, tr);
    };

    // The tiles holding a peaked row, run from the exact scores into dK, dV; returns whether any ran (uniform).
    auto peaked_tiles = [&]() __attribute__((always_inline)) {
      // Tiles holding a peaked row, found 64 at a time from the lse flags, one after the other.
      __shared__ int sPk[64];
      bool touched = false;  // uniform
      for (int t0 = 0; t0 < nqt; t0 += 64) {
        const int nt = min(64, nqt - t0);
        __syncthreads();  // every thread is done with the previous flags
        if (tid < 64) sPk[tid] = 0;
        __syncthreads();
        // every row of the chunk (at most 64 tiles) in one batch of loads per thread
        constexpr int RPT = (64 * BM + 64 * NW - 1) / (64 * NW);
        const int r0 = qbeg + t0 * BM, r1 = min(s.T, qbeg + (t0 + nt) * BM);
        float lv[RPT];
#pragma unroll
        for (int j = 0; j < RPT; ++j) {
          const int r = r0 + tid + 64 * NW * j;
          lv[j] = r < r1 ? p.lse[rowbase + r] : THERIA_INF;  // rows past the end: no flag
        }
#pragma unroll
        for (int j = 0; j < RPT; ++j)
          if (lse_peaked(lv[j])) sPk[(tid + 64 * NW * j) / BM] = 1;
        __syncthreads();
        for (int i = 0; i < nt; ++i) {
          if (!sPk[i]) continue;  // uniform: every thread reads the same flag
          const int it = t0 + i;
          dma.template issue_clamped<NSLAB>(qrsrc, qrs, qbeg + it * BM, s.T, sQ0);
          dma.template issue_clamped<NSLAB>(orsrc, ors, qbeg + it * BM, s.T, sO0);
          load_rows(it);
          wait_vm_all();
          store_rows(sR0, sF0);
          __syncthreads();
          if (it >= ifull && it < fend)
            exact_body(fast, it, sQ0, sO0, sR0);
          else
            exact_body(general, it, sQ0, sO0, sR0);
          __syncthreads();  // the tile buffers are free again
          touched = true;
        }
      }
      return touched;
    };
    if (nqt > 0) {
      dma.template issue_clamped<NSLAB>(qrsrc, qrs, qbeg, s.T, sQ0);
      dma.template issue_clamped<NSLAB>(orsrc, ors, qbeg, s.T, sO0);
      load_rows(0);
      wait_vm_all();
      store_rows(sR0, sF0);
      load_rows(1);
      int it = 0;
      // causal diagonal tiles first (general), then the full tiles two at a time (fixed buffers), then the rest
      for (; it < ifull; ++it) {
        if (it & 1)
          step(general, it, sQ1, sO1, sR1, sF1, sQ0, sO0, sR0, sF0);
        else
          step(general, it, sQ0, sO0, sR0, sF0, sQ1, sO1, sR1, sF1);
      }
      if (it < fend && (it & 1)) {
        step(fast, it, sQ1, sO1, sR1, sF1, sQ0, sO0, sR0, sF0);
        ++it;
      }
      for (; it + 1 < fend; it += 2) {
        step(fast, it, sQ0, sO0, sR0, sF0, sQ1, sO1, sR1, sF1);
        step(fast, it + 1, sQ1, sO1, sR1, sF1, sQ0, sO0, sR0, sF0);
      }
      for (; it < nqt; ++it) {
        if (it & 1)
          step(general, it, sQ1, sO1, sR1, sF1, sQ0, sO0, sR0, sF0);
        else
          step(general, it, sQ0, sO0, sR0, sF0, sQ1, sO1, sR1, sF1);
      }
    }
    if (pk_any) peaked_tiles();  // into the same accumulators

    // Epilogue: lane holds column d = dt*32 + li of keys kw0 + acc_row(r, g).
    T* DV = (T*)p.dv.p + b * p.dv.sb + h * p.dv.sh;
    T* DK = p.dk.p ? (T*)p.dk.p + b * p.dk.sb + h * p.dk.sh : nullptr;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const int d = dt * 32 + li;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kw0 + acc_row(r, g);
        if (key < s.M && (FD || d < s.D)) {
          DV[(int64_t)key * p.dv.sr + d] = (T)dv[dt][r];
          if (DK) DK[(int64_t)key * p.dk.sr + d] = (T)(dk[dt][r] * s.scale);
        }
      }
    }
  }  // pass
  THERIA_TILES_FLUSH(g_tiles_dkdv);
}

// dQ pass with the contract of dq_kernel (sdpa_bwd.hip): dQ = scale dS K with dS = P o (dO V^T - delta)
// (reference triton_sdpa_backward.py:505-696), and delta = rowsum(dO o O) computed here when O is given.
// One workgroup = NW waves of 32 queries each (Q and dO fragments, dQ accumulated in registers); K and V
// tiles of 64 or 128 keys stream through DMA-filled swizzled double buffers, one barrier per tile. Scores
// are transposed (S^T = K Q^T, this lane's query in the column), so lse and delta are per-lane scalars and
// dQ^T += K^T dS^T takes dS^T from the accumulators. Phase order per 64-key half of a tile, i.e. two 32-key
// subtiles:
//   S, dP of subtile 0 | S, dP of subtile 1 with exp / dS of subtile 0
//   | dQ of subtile 0 with exp / dS of subtile 1 | dQ of subtile 1.
// Two paths per query block. The common one takes the blocks without a peaked row (flagged in lse: largest
// probability above 1/4): Q pre-multiplied by scale * log2(e), S^T started from -lse2, P = exp2(S^T), the row
// term dO . O. The peaked one takes the others (and every block for the frozen / normalised row terms): the
// row term from a pass over the keys, exact float32 scores and dS as two 16-bit terms in the waves holding a
// peaked row. PK = 2 compiles both and takes each block's own (one launch); PK = 0 / 1 compile one each, for
// two launches: at head dim 128 the second path's registers change the common path's schedule (~20% slower
// at config 3), at head dim 64 the common path's loop compiles to the same instructions either way.
template <typename T, bool CAUSAL, int NW, int DP, bool OVERLAP, int WPS, int HALVES, bool FD, int PK>
__global__ __launch_bounds__(64 * NW, WPS) void dq_pipe_kernel(const DqParams p) {
  using MM = Mfma<T>;
  using F = typename MM::frag_t;
  using Dma = SwzDma<NW, DP>;
  constexpr int NKC = DP / 16, NDT = DP / 32;
  constexpr int BM = 32 * NW, BN = 64 * HALVES, TILE = BN * 2 * DP, NSLAB = BN / Dma::SLAB_ROWS;
  static_assert(NSLAB * Dma::SLAB_ROWS == BN, "key tiles must be whole DMA slabs");
  __shared__ __attribute__((aligned(1024))) char sK0[TILE];
  __shared__ __attribute__((aligned(1024))) char sK1[TILE];
  __shared__ __attribute__((aligned(1024))) char sV0[TILE];
  __shared__ __attribute__((aligned(1024))) char sV1[TILE];

  const Shape& s = p.s;
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
  const T* dO = (const T*)p.dout.p + b * p.dout.sb + h * p.dout.sh;
  THERIA_TILES_DECL;

  for (int pass = 0; pass < (pair ? 2 : 1); ++pass) {
  const int qb = CAUSAL ? (pass == 0 ? nqb - 1 - unit : unit) : unit;
  if (pass == 1) {
    if (qb == nqb - 1 - unit) break;  // odd number of blocks: the middle one ran in pass 0
    __syncthreads();                  // every wave is done with the LDS tiles of the first block
  }
  const int q0w = qb * BM + wave * 32;
    const int myq = q0w + li;
    const bool qvalid = myq < s.T;
    const int64_t rowbase = (int64_t)bh * s.T;

    const float lse = qvalid ? p.lse[rowbase + myq] : THERIA_INF;
    const float lse2 = lse == -THERIA_INF ? THERIA_INF : lse * kLog2e;  // a row without visible keys has P = 0
    const int rt = p.row_term;
    // Rows flagged peaked in lse: the whole wave runs the split loop when any of its rows is, and the block
    // takes the peaked path.
    const bool peaked = qvalid && lse_peaked(lse);
    const bool split = __any(peaked);
    const bool block_peaked = rt >= kRowFrozen || __syncthreads_or(split);
    if (PK != 2 && block_peaked != (PK == 1)) continue;  // uniform over the workgroup

    // The block's work for one path (PEAKED: compile-time); the fused kernel (PK = 2) picks it per block.
    auto run = [&](auto peaked_tag) __attribute__((always_inline)) {
    constexpr bool PEAKED = decltype(peaked_tag)::value;

    F qf[NKC], of[NKC];
#pragma unroll
    for (int c = 0; c < NKC; ++c) {
      qf[c] = gload_frag8<T>(Q, p.q.sr, myq, s.T, c, FD ? DP : s.D);
      of[c] = gload_frag8<T>(dO, p.dout.sr, myq, s.T, c, FD ? DP : s.D);
    }
    float del = 0.f;
    if (!PEAKED && rt == kRowFromO) {
      // delta = dO . O over this lane's half of the head dim (the dO fragment's columns), then the pair
      float part = 0.f;
      if (qvalid) {
#pragma unroll
        for (int c = 0; c < NKC; ++c) {
          const int col = c * 16 + 8 * g;
          if (!FD && col >= s.D) continue;  // head dim below DP (a multiple of 8): whole 8-column groups only
          const int64_t off = (int64_t)myq * p.o.sr + col;
          if (p.o_f32) {
            const float* Op = (const float*)p.o.p + b * p.o.sb + h * p.o.sh + off;
            const f32x4_t a0 = *reinterpret_cast<const f32x4_t*>(Op);
            const f32x4_t a1 = *reinterpret_cast<const f32x4_t*>(Op + 4);
#pragma unroll
            for (int e = 0; e < 4; ++e) part += a0[e] * (float)of[c][e] + a1[e] * (float)of[c][4 + e];
          } else {
            const F ov = __builtin_bit_cast(F, *reinterpret_cast<const i16x8_t*>((const T*)p.o.p + b * p.o.sb +
                                                                               h * p.o.sh + off));
#pragma unroll
            for (int e = 0; e < 8; ++e) part += (float)ov[e] * (float)of[c][e];
          }
        }
      }
      del = pair_sum(part);
      if (qvalid && g == 0) p.delta[rowbase + myq] = del;
    } else if (rt == kRowGiven) {
      del = qvalid ? p.delta[rowbase + myq] : 0.f;
    }
    if (!PEAKED && !p.dq.p) return;  // only dO . O was requested (uniform over the grid)

    f32x16_t acc[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) acc[dt] = zero16();
    // c2 = scale * log2(e): split waves form P = exp2(S^T c2 - lse2) from the exact float32 scores; the others
    // hold Q pre-multiplied by c2 (one more 16-bit rounding of each score's factors, ~2^-9 of the score).
    const float c2 = s.scale * kLog2e;

    int kend = s.M;
    if (CAUSAL) kend = min(s.M, qb * BM + BM);
    const int nkt = (kend + BN - 1) / BN;
    // Tiles [0, nfull) have every key in range and visible to every query of the block.
    int nfull = s.M / BN;
    if (CAUSAL) nfull = min(nfull, qb * BM / BN);

    const Dma dma(wave, lane, FD ? DP / 8 : s.D / 8);  // head dims below DP: zero-filled chunks past D
    const uint32_t krs = (uint32_t)p.k.sr * 2, vrs = (uint32_t)p.v.sr * 2;
    const rsrc_t krsrc = make_rsrc(K, (uint32_t)slab_span(s.M, krs, 2 * (FD ? DP : s.D)));
    const rsrc_t vrsrc = make_rsrc(V, (uint32_t)slab_span(s.M, vrs, 2 * (FD ? DP : s.D)));

    // S^T = K Q^T and dP^T = V dO^T - delta for key subtile t of the tile in (tk, tv).
    // Split waves: S^T = K Q^T exactly; other waves: Q is pre-multiplied by scale * log2(e) (below) and S^T
    // starts from -lse2, so P = exp2(S^T) with no per-score scaling.
    auto sdp = [&](auto split_tag, const char* tk, const char* tv, int t, f32x16_t& sc, f32x16_t& dp) {
      constexpr bool SPLIT = decltype(split_tag)::value;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        sc[r] = SPLIT ? 0.f : -lse2;
        dp[r] = -del;
      }
#pragma unroll
      for (int c = 0; c < NKC; ++c) {
        sc = MM::mma(swz_cols<T, DP>(tk, 32 * t + li, c), qf[c], sc);
        dp = MM::mma(swz_cols<T, DP>(tv, 32 * t + li, c), of[c], dp);
      }
    };
    auto mask = [&](f32x16_t& sc, int k0t) {
      if ((k0t + 32 > s.M) || (CAUSAL && k0t + 31 > q0w)) {
        const int lim = CAUSAL ? min(s.M, myq + 1) : s.M;  // first key this query cannot see
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (k0t + acc_row(r, g) >= lim) sc[r] = -THERIA_INF;
      }
    };
    // dS^T = P^T o dP^T as 16-bit fragments (KACC chunks 0, 1)
    auto pds = [&](auto split_tag, const f32x16_t& sc, const f32x16_t& dp, F (&df)[2]) {
      constexpr bool SPLIT = decltype(split_tag)::value;
#pragma unroll
      for (int r = 0; r < 16; ++r)
        df[r >> 3][r & 7] = (T)(fast_exp2(SPLIT ? fmaf(sc[r], c2, -lse2) : sc[r]) * dp[r]);
    };
    auto dqm = [&](const char* tk, int t, const F (&df)[2]) {
#pragma unroll
      for (int cc = 0; cc < 2; ++cc)
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) acc[dt] = MM::mma(swz_rows<T, DP>(tk, 32 * t, cc, 32 * dt), df[cc], acc[dt]);
    };
    // The residual product of a split wave: dQ^T += K^T (dS - hi(dS))^T with the residual recomputed from the
    // float32 S and dP, so that dS enters as two 16-bit terms in total.
    auto dqm_lo = [&](const char* tk, int t, const f32x16_t& sc, const f32x16_t& dp) {
#pragma unroll
      for (int cc = 0; cc < 2; ++cc) {
        F dl;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float ds = fast_exp2(fmaf(sc[8 * cc + e], c2, -lse2)) * dp[8 * cc + e];
          dl[e] = (T)(ds - (float)(T)ds);
        }
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) acc[dt] = MM::mma(swz_rows<T, DP>(tk, 32 * t, cc, 32 * dt), dl, acc[dt]);
      }
    };

    auto step = [&](auto fast_tag, auto split_tag, int k, const char* tk, const char* tv, char* nk,
                    char* nv) __attribute__((always_inline)) {
      constexpr bool FAST = decltype(fast_tag)::value;
      constexpr bool SPLIT = decltype(split_tag)::value;
      const int k0 = k * BN;
      wait_vm_all();
      __syncthreads();  // tile k visible to all waves; the other buffers (tile k-1) are free
      if (k + 1 < nkt) {
        dma.template issue_clamped<NSLAB>(krsrc, krs, k0 + BN, s.M, nk);
        dma.template issue_clamped<NSLAB>(vrsrc, vrs, k0 + BN, s.M, nv);
      }
      if constexpr (FAST && OVERLAP && !SPLIT) {
        THERIA_TILES_ADD(2 * HALVES);
#pragma unroll
        for (int hf = 0; hf < HALVES; ++hf) {
          f32x16_t s0, p0, s1, p1;
          F d0[2], d1[2];
          sdp(split_tag, tk, tv, 2 * hf, s0, p0);
          __builtin_amdgcn_sched_barrier(0);
          sdp(split_tag, tk, tv, 2 * hf + 1, s1, p1);
          pds(split_tag, s0, p0, d0);
          __builtin_amdgcn_sched_barrier(0);
          dqm(tk, 2 * hf, d0);
          pds(split_tag, s1, p1, d1);
          __builtin_amdgcn_sched_barrier(0);
          dqm(tk, 2 * hf + 1, d1);
          __builtin_amdgcn_sched_barrier(0);
        }
      } else {
#pragma unroll
        for (int t = 0; t < 2 * HALVES; ++t) {
          const int k0t = k0 + 32 * t;
          if (!FAST && CAUSAL && k0t > q0w + 31) continue;  // every key after every query of the wave (uniform)
          THERIA_TILES_ADD(1);
          f32x16_t sc, dp;
          F df[2];
          sdp(split_tag, tk, tv, t, sc, dp);
          if (!FAST) mask(sc, k0t);
          pds(split_tag, sc, dp, df);
          dqm(tk, t, df);
          if constexpr (SPLIT) {
            dqm_lo(tk, t, sc, dp);
            __builtin_amdgcn_sched_barrier(0);  // one subtile at a time (registers)
          }
        }
      }
    };
    const std::integral_constant<bool, true> fast, with_split;
    const std::integral_constant<bool, false> general, no_split;

    // Both forms of the loop are inlined: a call that is not would take every register array it captures
    // (Q, dO fragments and the dQ accumulators) by address, i.e. into scratch memory.
    auto loop = [&](auto split_tag) __attribute__((always_inline)) {
      if (nkt <= 0) return;
      dma.template issue_clamped<NSLAB>(krsrc, krs, 0, s.M, sK0);
      dma.template issue_clamped<NSLAB>(vrsrc, vrs, 0, s.M, sV0);
      int k = 0;
      for (; k + 1 < nfull; k += 2) {
        step(fast, split_tag, k, sK0, sV0, sK1, sV1);
        step(fast, split_tag, k + 1, sK1, sV1, sK0, sV0);
      }
      for (; k < nkt; ++k) {
        if (k & 1)
          step(general, split_tag, k, sK1, sV1, sK0, sV0);
        else
          step(general, split_tag, k, sK0, sV0, sK1, sV1);
      }
    };
    // Peaked launch: the row term from a pass over the keys, for the frozen / normalised forms and in place of
    // dO . O, whose 16-bit P rounding in the forward's PV product (~2^-9 |dP|) a peaked row does not average
    // out while dS = P o (dP - delta) is a small difference there.
    if (PEAKED && rt != kRowGiven) {
      // a = sum_j P_ij dP_ij and l = sum_j P_ij over every key of the row (one more pass over the key tiles)
      float a_part = 0.f, l_part = 0.f, p_mx = 0.f;
      if (nkt > 0) {
        dma.template issue_clamped<NSLAB>(krsrc, krs, 0, s.M, sK0);
        dma.template issue_clamped<NSLAB>(vrsrc, vrs, 0, s.M, sV0);
      }
      for (int k = 0; k < nkt; ++k) {
        const int k0 = k * BN;
        const char* tk = (k & 1) ? sK1 : sK0;
        const char* tv = (k & 1) ? sV1 : sV0;
        wait_vm_all();
        __syncthreads();
        if (k + 1 < nkt) {
          dma.template issue_clamped<NSLAB>(krsrc, krs, k0 + BN, s.M, (k & 1) ? sK0 : sK1);
          dma.template issue_clamped<NSLAB>(vrsrc, vrs, k0 + BN, s.M, (k & 1) ? sV0 : sV1);
        }
#pragma unroll
        for (int t = 0; t < 2 * HALVES; ++t) {
          const int k0t = k0 + 32 * t;
          if (CAUSAL && k0t > q0w + 31) continue;  // wave-uniform
          f32x16_t sc = zero16(), dpp = zero16();
#pragma unroll
          for (int c = 0; c < NKC; ++c) {
            sc = MM::mma(swz_cols<T, DP>(tk, 32 * t + li, c), qf[c], sc);
            dpp = MM::mma(swz_cols<T, DP>(tv, 32 * t + li, c), of[c], dpp);
          }
          mask(sc, k0t);
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const float pv = fast_exp2(fmaf(sc[r], c2, -lse2));
            a_part = fmaf(pv, dpp[r], a_part);
            l_part += pv;
            p_mx = fmaxf(p_mx, pv);
          }
        }
      }
      __syncthreads();  // every wave is done with the tiles before the main loop refills the buffers
      const float a = pair_sum(a_part), l = pair_sum(l_part), pm = pair_max(p_mx);
      del = rt == kRowFrozen ? a : (l > 0.f ? a / l : 0.f);
      if (qvalid && g == 0) {
        p.delta[rowbase + myq] = del;
        if (p.lse_out)  // flagged from the exact largest probability
          p.lse_out[rowbase + myq] = l > 0.f ? lse_with_flag(lse + __builtin_log2f(l) * kLn2, pm > kPeakedFrac * l) : lse;
      }
    }
    if (!p.dq.p) return;  // only the row term was requested
    if (PEAKED && split) {
      loop(with_split);
    } else {
#pragma unroll
      for (int c = 0; c < NKC; ++c) qf[c] = scaled_frag<T>(qf[c], c2);
      loop(no_split);
    }

    if (qvalid) {
      T* DQ = (T*)p.dq.p + b * p.dq.sb + h * p.dq.sh;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
          const int d0 = dt * 32 + 8 * qd + 4 * g;
          const f32x16_t& a = acc[dt];
          store4_8<T>(DQ, p.dq.sr, myq, d0, FD ? DP : s.D, a[4 * qd] * s.scale, a[4 * qd + 1] * s.scale, a[4 * qd + 2] * s.scale,
                      a[4 * qd + 3] * s.scale);
        }
    }
    };  // run
    if constexpr (PK == 0) {
      run(std::false_type{});
    } else if constexpr (PK == 1) {
      run(std::true_type{});
    } else {
      if (block_peaked)
        run(std::true_type{});
      else
        run(std::false_type{});
    }
  }  // pass
  THERIA_TILES_FLUSH(g_tiles_dq);
}

// Launches with FD = (head dim == DP): one fused launch at head dim 64; at 128 the common launch (unless every
// block takes the row-term pass), then the peaked launch.
template <typename T, bool CAUSAL, int NW, int DP, bool OVERLAP, int WPS, int HALVES, bool FD>
static void dq_go_fd(const DqParams& p, int64_t nblk, hipStream_t st) {
  if constexpr (DP <= 64) {
    hipLaunchKernelGGL((dq_pipe_kernel<T, CAUSAL, NW, DP, OVERLAP, WPS, HALVES, FD, 2>), dim3((unsigned)nblk),
                       dim3(64 * NW), 0, st, p);
  } else {
    if (p.row_term < kRowFrozen)
      hipLaunchKernelGGL((dq_pipe_kernel<T, CAUSAL, NW, DP, OVERLAP, WPS, HALVES, FD, 0>), dim3((unsigned)nblk),
                         dim3(64 * NW), 0, st, p);
    hipLaunchKernelGGL((dq_pipe_kernel<T, CAUSAL, NW, DP, OVERLAP, WPS, HALVES, FD, 1>), dim3((unsigned)nblk),
                       dim3(64 * NW), 0, st, p);
  }
}
template <typename T, bool CAUSAL, int NW, int DP, bool OVERLAP, int WPS, int HALVES>
static void dq_go(const DqParams& p, int64_t nblk, hipStream_t st) {
  if (p.s.D == DP)
    dq_go_fd<T, CAUSAL, NW, DP, OVERLAP, WPS, HALVES, true>(p, nblk, st);
  else
    dq_go_fd<T, CAUSAL, NW, DP, OVERLAP, WPS, HALVES, false>(p, nblk, st);
}
template <typename T, bool CAUSAL, int NW, int DP, bool OVERLAP, int WPS, int HALVES, bool FD>
static void dkdv_go_fd(const DkdvParams& p, int64_t nblk, hipStream_t st) {
  hipLaunchKernelGGL((dkdv_pipe_kernel<T, CAUSAL, NW, DP, OVERLAP, WPS, HALVES, FD>), dim3((unsigned)nblk),
                     dim3(64 * NW), 0, st, p);
}
template <typename T, bool CAUSAL, int NW, int DP, bool OVERLAP, int WPS, int HALVES>
static void dkdv_go(const DkdvParams& p, int64_t nblk, hipStream_t st) {
  if (p.s.D == DP)
    dkdv_go_fd<T, CAUSAL, NW, DP, OVERLAP, WPS, HALVES, true>(p, nblk, st);
  else
    dkdv_go_fd<T, CAUSAL, NW, DP, OVERLAP, WPS, HALVES, false>(p, nblk, st);
}

// Head dims the pipelined kernels take: a multiple of 8 in 8..32 (run at DP = 32), 40..64 (DP = 64) or 72..128
// (DP = 128); columns past D are zero in every tile and are never stored.
static bool pipe_head_dim(const Shape& s) { return s.vec && s.D % 8 == 0 && s.D >= 8; }

template <typename T, bool CAUSAL>
bool launch_dq_pipe(const DqParams& p0, hipStream_t st, hipError_t* err) {
  if (!pipe_head_dim(p0.s)) return false;
  // 32-bit byte offsets inside each (batch, head) slab of K and V
  if (!slab_fits_dma(p0.s.M, p0.k.sr, p0.s.D) || !slab_fits_dma(p0.s.M, p0.v.sr, p0.s.D)) return false;
  constexpr int NW = DQ_PIPE_NW;
  DqParams p = p0;
  const int64_t nqb = (p.s.T + 32 * NW - 1) / (32 * NW);
  int64_t nblk = (CAUSAL ? (nqb + 1) / 2 : nqb) * p.s.B * p.s.H;  // causal: mirrored pairs
  if (CAUSAL && nblk > 0 && nblk < device_cu_count()) {
    // the pairs would leave CUs without a workgroup: one block each, the longest first
    p.s.unpaired = true;
    nblk = nqb * p.s.B * p.s.H;
  }
  if (nblk == 0) {
    *err = hipSuccess;
    return true;
  }
  if (p.s.dp == 32)
    dq_go<T, CAUSAL, NW, 32, true, 2, DQ64_HALVES>(p, nblk, st);
  else if (p.s.dp == 64)
    dq_go<T, CAUSAL, NW, 64, true, 2, DQ64_HALVES>(p, nblk, st);
  else
    dq_go<T, CAUSAL, NW, 128, DQ128_OVERLAP, DQ128_WPS, DQ128_HALVES>(p, nblk, st);
  *err = hipGetLastError();
  return true;
}

template bool launch_dq_pipe<__bf16, false>(const DqParams&, hipStream_t, hipError_t*);
template bool launch_dq_pipe<__bf16, true>(const DqParams&, hipStream_t, hipError_t*);
template bool launch_dq_pipe<_Float16, false>(const DqParams&, hipStream_t, hipError_t*);
template bool launch_dq_pipe<_Float16, true>(const DqParams&, hipStream_t, hipError_t*);

// Launch if the pipelined kernel covers this problem (16-bit, a head dim pipe_head_dim takes, vector
// access, dK and dV both wanted); returns false otherwise.
template <typename T, bool CAUSAL>
bool launch_dkdv_pipe(const DkdvParams& p0, hipStream_t st, hipError_t* err) {
  if (!(pipe_head_dim(p0.s) && !p0.dv_only)) return false;
  // 32-bit byte offsets inside each (batch, head) slab of Q, dO and K
  if (!slab_fits_dma(p0.s.T, p0.q.sr, p0.s.D) || !slab_fits_dma(p0.s.T, p0.dout.sr, p0.s.D) ||
      !slab_fits_dma(p0.s.M, p0.k.sr, p0.s.D))
    return false;
  DkdvParams p = p0;
  const int64_t cus = device_cu_count();
  // workgroups of nw waves (32 keys each): key blocks, or (causal head dim <= 64) pairs of mirrored blocks
  auto blocks = [&](int nw) {
    const int64_t nkb = (p.s.M + 32 * nw - 1) / (32 * nw);
    return ((CAUSAL && p.s.dp <= 64 && !p.s.unpaired) ? (nkb + 1) / 2 : nkb) * p.s.B * p.s.H;
  };
  // Causal grids whose pairs of four-wave workgroups would leave CUs without one (two-wave workgroups, half the
  // waves per SIMD): one block per workgroup, the longest first.
  if (CAUSAL && p.s.dp <= 64 && blocks(4) < cus) p.s.unpaired = true;
  if (blocks(4) == 0) {
    *err = hipSuccess;
    return true;
  }
  if (p.s.dp == 32) {
    // Four-wave workgroups (eight waves would copy 128-row DMA slabs into 64-row query tiles), two-wave ones
    // where four-wave ones would leave CUs idle.
    if (blocks(4) >= cus)
      dkdv_go<T, CAUSAL, 4, 32, true, 2, DKDV64_HALVES>(p, blocks(4), st);
    else
      dkdv_go<T, CAUSAL, 2, 32, true, 2, DKDV64_HALVES>(p, blocks(2), st);
  } else if (p.s.dp == 64) {
    // Eight-wave workgroups (both waves of a SIMD in one workgroup) whenever they still fill every CU:
    // two independent four-wave workgroups on a CU progress unevenly (the older one is issued first), and
    // with two rounds of them the CUs that finish early idle through a ~10% tail at config 2.
    // Grids that would leave CUs without a four-wave workgroup use two-wave ones (twice as many; per
    // workgroup they are slower, so only then).
    const int64_t nblk8 = blocks(8);
    if (nblk8 >= cus)
      dkdv_go<T, CAUSAL, 8, 64, true, 2, DKDV64_HALVES>(p, nblk8, st);
    else if (blocks(4) >= cus)
      dkdv_go<T, CAUSAL, 4, 64, true, 2, DKDV64_HALVES>(p, blocks(4), st);
    else
      dkdv_go<T, CAUSAL, 2, 64, true, 2, DKDV64_HALVES>(p, blocks(2), st);
  } else {
    constexpr int NW = DKDV_PIPE_NW;
    dkdv_go<T, CAUSAL, NW, 128, DKDV128_OVERLAP, DKDV128_WPS, DKDV128_HALVES>(p, blocks(NW), st);
  }
  *err = hipGetLastError();
  return true;
}

template bool launch_dkdv_pipe<__bf16, false>(const DkdvParams&, hipStream_t, hipError_t*);
template bool launch_dkdv_pipe<__bf16, true>(const DkdvParams&, hipStream_t, hipError_t*);
template bool launch_dkdv_pipe<_Float16, false>(const DkdvParams&, hipStream_t, hipError_t*);
template bool launch_dkdv_pipe<_Float16, true>(const DkdvParams&, hipStream_t, hipError_t*);

}  // namespace theria
