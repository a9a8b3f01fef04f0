// Shared device building blocks for the gfx950 SDPA kernels.
//
// Tiling vocabulary used by every kernel:
//  * All matrix products use 32x32 MFMA output tiles. For 16-bit inputs the instruction is
//    v_mfma_f32_32x32x16_{bf16,f16} (k extent 16, 8 elements per lane); for float32 inputs it is
//    v_mfma_f32_32x32x2_f32 (k extent 2, 1 element per lane). Accumulation is float32 in both.
//  * Operand fragment of lane l (li = l % 32, g = l / 32): the row (A) or column (B) index is li, and
//    the k elements depend on g. Output ("accumulator") layout: register r of lane l holds the element
//    at row acc_row(r, g) = 8*(r/4) + 4*g + r%4 and column li. These layouts were checked bit-exactly
//    on the MI355X against a host matrix product.
//  * Because the k reduction is order-free, the k elements of a fragment may follow any mapping as long
//    as both operands use the same one. Two mappings are used:
//      KLIN: element e of chunk c sits at k = c*KC + g*EPL + e (contiguous per lane);
//      KACC: element e of chunk c sits at k = acc_row(c*EPL + e, g) (k inside a 32-row block), which is
//            exactly how an accumulator tile's registers are laid out. An accumulator tile can then be
//            fed straight back as an operand (P, dS, ...) whose k index is the tile's row index.
//  * Row-major LDS tiles are read two ways: "cols" fragments (k runs along a row, lane-fixed row) with
//    ds_read_b128 / ds_read_b64, and "rows" fragments (k runs down a column, lane-fixed column) with the
//    gfx950 transpose read ds_read_b64_tr_b16. Its semantics, measured on the device: within each group
//    of 16 lanes, result lane j element e = 16-bit element (j % 4) of the 8 bytes addressed by source
//    lane 4*e + j/4. Giving source lane s the address of row (k0 + s/4), column (c0 + 4*(s%4)) therefore
//    hands lane j the column c0 + j for rows k0..k0+3. No transposed copies are kept in LDS.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace theria {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef short i16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
#define THERIA_INF (__builtin_inff())

enum KOrder { KLIN = 0, KACC = 1 };

__device__ __forceinline__ int acc_row(int r, int g) { return 8 * (r >> 2) + 4 * g + (r & 3); }

// ----------------------------------------------------------------------------------------------
// MFMA traits
// ----------------------------------------------------------------------------------------------
template <typename T> struct Mfma;

template <> struct Mfma<__bf16> {
  using frag_t = bf16x8_t;
  static constexpr int KC = 16;
  static constexpr int EPL = 8;
  __device__ __forceinline__ static f32x16_t mma(frag_t a, frag_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};

template <> struct Mfma<_Float16> {
  using frag_t = f16x8_t;
  static constexpr int KC = 16;
  static constexpr int EPL = 8;
  __device__ __forceinline__ static f32x16_t mma(frag_t a, frag_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

template <> struct Mfma<float> {
  using frag_t = float;
  static constexpr int KC = 2;
  static constexpr int EPL = 1;
  __device__ __forceinline__ static f32x16_t mma(frag_t a, frag_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
};

template <typename T> __device__ __forceinline__ T to_t(float x) { return (T)x; }

__device__ __forceinline__ f32x16_t zero16() {
  f32x16_t z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// Lane l and lane l^32 combined (both halves receive the result).
__device__ __forceinline__ float pair_max(float x) {
  auto w = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(w[0]), __uint_as_float(w[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
  auto w = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(w[0]) + __uint_as_float(w[1]);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// a * b rounded once and never fused into a following add: the float32 kernels form x = fl(S c) - m2 from
// the same fl(S c) that the row max m2 was taken over, so the row's largest score gives x = 0 exactly.
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}

// float32 probability from the row's own statistics (kRowOwnStats): exp2((fl(S c) - m2) - L2). m2 = +inf
// (a row without visible keys, or past the end) gives 0.
__device__ __forceinline__ float own_prob(float s_raw, float c2, float m2, float l2) {
  return fast_exp2((mul_rn(s_raw, c2) - m2) - l2);
}

// Peaked rows. With 16-bit inputs the lowest mantissa bit of each lse the forward writes marks a row whose
// largest probability may exceed 1/4 (kPeakedFrac); the backward kernels read it to take their exact path
// there (two-term 16-bit operands, the row term from a pass over the keys). Setting the bit moves lse by at
// most one unit in the last place. Infinite lse (rows without visible keys) carries no flag.
constexpr float kPeakedFrac = 0.25f;
__device__ __forceinline__ float lse_with_flag(float lse, bool peaked) {
  if (!__builtin_isfinite(lse)) return lse;
  return __uint_as_float((__float_as_uint(lse) & ~1u) | (peaked ? 1u : 0u));
}
__device__ __forceinline__ bool lse_peaked(float lse) {
  return __builtin_isfinite(lse) && (__float_as_uint(lse) & 1u);
}

// ----------------------------------------------------------------------------------------------
// k-index mapping of fragment element 0 / element EPL/2 for 16-bit types, and the single element of
// float32 fragments. c is the chunk index (KC wide), g the lane half.
// ----------------------------------------------------------------------------------------------
template <int ORDER> __device__ __forceinline__ int k16_first(int c, int g) {
  return ORDER == KLIN ? c * 16 + 8 * g : c * 16 + 4 * g;
}
template <int ORDER> __device__ __forceinline__ int k16_second(int c, int g) {
  return ORDER == KLIN ? c * 16 + 8 * g + 4 : c * 16 + 4 * g + 8;
}
template <int ORDER> __device__ __forceinline__ int k32(int c, int g) {
  return ORDER == KLIN ? 2 * c + g : acc_row(c, g);
}

// ----------------------------------------------------------------------------------------------
// LDS fragment reads
// ----------------------------------------------------------------------------------------------
// "cols" fragment: lane-fixed row `row`, k along the row starting at column kbase.
template <typename T, int ORDER>
__device__ __forceinline__ typename Mfma<T>::frag_t lds_cols(const T* base, int pitch, int row, int kbase, int c) {
  const int g = (threadIdx.x >> 5) & 1;
  if constexpr (sizeof(T) == 2) {
    using F = typename Mfma<T>::frag_t;
    const T* p0 = base + row * pitch + kbase + k16_first<ORDER>(c, g);
    if constexpr (ORDER == KLIN) {
      return __builtin_bit_cast(F, *reinterpret_cast<const i16x8_t*>(p0));
    } else {
      const T* p1 = base + row * pitch + kbase + k16_second<ORDER>(c, g);
      i16x4_t a = *reinterpret_cast<const i16x4_t*>(p0);
      i16x4_t b = *reinterpret_cast<const i16x4_t*>(p1);
      i16x8_t v = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
      return __builtin_bit_cast(F, v);
    }
  } else {
    return base[row * pitch + kbase + k32<ORDER>(c, g)];
  }
}

typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;

__device__ __forceinline__ i16x4_t ds_read_tr16(const void* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(p));
}

// "rows" fragment: lane-fixed column col0 + li, k down the column starting at row kbase.
template <typename T, int ORDER>
__device__ __forceinline__ typename Mfma<T>::frag_t lds_rows(const T* base, int pitch, int kbase, int c, int col0) {
  const int lane = threadIdx.x & 63;
  const int g = lane >> 5;
  if constexpr (sizeof(T) == 2) {
    using F = typename Mfma<T>::frag_t;
    const int s = lane & 15, hh = (lane >> 4) & 1;
    const int col = col0 + 16 * hh + 4 * (s & 3);
    const T* p0 = base + (kbase + k16_first<ORDER>(c, g) + (s >> 2)) * pitch + col;
    const T* p1 = base + (kbase + k16_second<ORDER>(c, g) + (s >> 2)) * pitch + col;
    i16x4_t a = ds_read_tr16(p0);
    i16x4_t b = ds_read_tr16(p1);
    i16x8_t v = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
    return __builtin_bit_cast(F, v);
  } else {
    return base[(kbase + k32<ORDER>(c, g)) * pitch + col0 + (lane & 31)];
  }
}

// Accumulator tile -> operand fragment whose k index is the tile row (KACC order), chunk c.
// c must be a compile-time constant after unrolling so the register indices stay static.
template <typename T>
__device__ __forceinline__ typename Mfma<T>::frag_t acc_frag(const f32x16_t& a, int c) {
  if constexpr (sizeof(T) == 2) {
    typename Mfma<T>::frag_t f;
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = (T)a[c * 8 + e];
    return f;
  } else {
    return a[c];
  }
}

// Fragment with every element multiplied by x (in float32, rounded once to T).
template <typename T>
__device__ __forceinline__ typename Mfma<T>::frag_t scaled_frag(const typename Mfma<T>::frag_t& f, float x) {
  if constexpr (sizeof(T) == 2) {
    typename Mfma<T>::frag_t r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = (T)((float)f[e] * x);
    return r;
  } else {
    return f * x;
  }
}

// Two-term 16-bit split of accumulator chunk c (16-bit T only): hi = round(x), lo = round(x - hi), so
// hi + lo carries x to ~2^-16 relative and an MFMA pair over (hi, lo) sums x-weighted products with no
// operand rounding of consequence.
template <typename T>
__device__ __forceinline__ void split_frag(const f32x16_t& a, int c, typename Mfma<T>::frag_t& hi,
                                           typename Mfma<T>::frag_t& lo) {
  static_assert(sizeof(T) == 2, "split_frag is for 16-bit operands");
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const T h = (T)a[c * 8 + e];
    hi[e] = h;
    lo[e] = (T)(a[c * 8 + e] - (float)h);
  }
}

// ----------------------------------------------------------------------------------------------
// Global memory access
// ----------------------------------------------------------------------------------------------
// Fragment of row `row` straight from global memory (k along the row, KLIN order). Rows >= nrows
// and columns >= D read as zero. vec: 16-byte loads are legal (alignment checked by the host).
template <typename T>
__device__ __forceinline__ typename Mfma<T>::frag_t gload_frag(const T* base, int64_t rs, int row, int nrows, int c,
                                                              int D, bool vec) {
  using F = typename Mfma<T>::frag_t;
  const int g = (threadIdx.x >> 5) & 1;
  if constexpr (sizeof(T) == 2) {
    const int col = c * 16 + 8 * g;
    i16x8_t v = {0, 0, 0, 0, 0, 0, 0, 0};
    if (row < nrows) {
      const T* p = base + (int64_t)row * rs + col;
      if (vec && col + 8 <= D) {
        v = *reinterpret_cast<const i16x8_t*>(p);
      } else {
        const short* ps = reinterpret_cast<const short*>(p);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (col + e < D) ? ps[e] : (short)0;
      }
    }
    return __builtin_bit_cast(F, v);
  } else {
    const int col = 2 * c + g;
    return (row < nrows && col < D) ? base[(int64_t)row * rs + col] : 0.f;
  }
}

// Cooperative tile staging: a [ROWS][DP] tile of rows row0.. of a (rows, D) matrix, loaded into
// registers (16 bytes per chunk) and later stored to a row-major LDS tile of pitch `pitch`.
// Out-of-range rows and columns are zero, so every LDS column < DP is defined.
template <typename T, int ROWS, int DP, int NT>
struct TileStage {
  static constexpr int VEC = 16 / (int)sizeof(T);
  static constexpr int CPR = DP / VEC;
  static constexpr int NCH = ROWS * CPR;
  static constexpr int PER = (NCH + NT - 1) / NT;
  i16x8_t r[PER];

  // Straight-line 16-byte loads; only for tiles whose rows and columns are all in range with
  // vector-legal alignment (callers check `row0 + ROWS <= nrows && D == DP && vec` first).
  __device__ __forceinline__ void load_fast(const T* base, int64_t rs, int row0) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int ch = (int)threadIdx.x + i * NT;
      if (NCH % NT == 0 || ch < NCH) {
        const int row = ch / CPR, col = (ch % CPR) * VEC;
        r[i] = *reinterpret_cast<const i16x8_t*>(base + (int64_t)(row0 + row) * rs + col);
      }
    }
  }

  // Picks the fast path when the whole tile is in range (a uniform branch).
  __device__ __forceinline__ void load_any(const T* base, int64_t rs, int row0, int nrows, int D, bool vec) {
    if (vec && D == DP && row0 + ROWS <= nrows)
      load_fast(base, rs, row0);
    else
      load(base, rs, row0, nrows, D, vec);
  }

  __device__ __forceinline__ void load(const T* base, int64_t rs, int row0, int nrows, int D, bool vec) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int ch = (int)threadIdx.x + i * NT;
      i16x8_t v = {0, 0, 0, 0, 0, 0, 0, 0};
      if (NCH % NT == 0 || ch < NCH) {
        const int row = ch / CPR, col = (ch % CPR) * VEC;
        const int grow = row0 + row;
        if (grow < nrows && col < D) {
          const T* p = base + (int64_t)grow * rs + col;
          if (vec && col + VEC <= D) {
            v = *reinterpret_cast<const i16x8_t*>(p);
          } else {
            T tmp[VEC];
#pragma unroll
            for (int e = 0; e < VEC; ++e) tmp[e] = (col + e < D) ? p[e] : (T)0.f;
            v = __builtin_bit_cast(i16x8_t, tmp);
          }
        }
      }
      r[i] = v;
    }
  }

  __device__ __forceinline__ void store(T* lds, int pitch) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int ch = (int)threadIdx.x + i * NT;
      if (NCH % NT == 0 || ch < NCH) {
        const int row = ch / CPR, col = (ch % CPR) * VEC;
        *reinterpret_cast<i16x8_t*>(lds + row * pitch + col) = r[i];
      }
    }
  }
};

// ----------------------------------------------------------------------------------------------
// Block scheduling
// ----------------------------------------------------------------------------------------------
// The dispatcher hands workgroup ids to the 8 XCDs round-robin, and each XCD has its own L2. This
// renumbering gives consecutive logical ids (the tiles of one (batch, head), which share K and V) to
// the same XCD, so each head's K/V is fetched from HBM into one L2 instead of eight.
__device__ __forceinline__ int xcd_remap(int bid, int nblocks) {
  constexpr int NX = 8;
  const int q = nblocks / NX, rem = nblocks % NX;
  const int xcd = bid % NX, local = bid / NX;
  return xcd < rem ? xcd * (q + 1) + local : rem * (q + 1) + (xcd - rem) * q + local;
}

// Store 4 consecutive elements (columns col..col+3 of row `row`) from float values, bounds-checked.
template <typename T>
__device__ __forceinline__ void store4(T* base, int64_t rs, int row, int col, int D, float a, float b, float c,
                                       float d, bool vec) {
  T* p = base + (int64_t)row * rs + col;
  if (vec && col + 4 <= D) {
    if constexpr (sizeof(T) == 2) {
      T v[4] = {(T)a, (T)b, (T)c, (T)d};
      *reinterpret_cast<i16x4_t*>(p) = __builtin_bit_cast(i16x4_t, v);
    } else {
      *reinterpret_cast<f32x4_t*>(p) = f32x4_t{a, b, c, d};
    }
  } else {
    if (col + 0 < D) p[0] = (T)a;
    if (col + 1 < D) p[1] = (T)b;
    if (col + 2 < D) p[2] = (T)c;
    if (col + 3 < D) p[3] = (T)d;
  }
}

// gload_frag for 16-bit T and a head dim D that is a multiple of 8, with 16-byte aligned rows: a lane's 8
// columns are all in range or all out of range, so one vector load (or zero) covers them.
template <typename T>
__device__ __forceinline__ typename Mfma<T>::frag_t gload_frag8(const T* base, int64_t rs, int row, int nrows, int c,
                                                               int D) {
  static_assert(sizeof(T) == 2, "16-bit operands only");
  const int col = c * 16 + 8 * ((threadIdx.x >> 5) & 1);
  i16x8_t v = {0, 0, 0, 0, 0, 0, 0, 0};
  if (row < nrows && col < D) v = *reinterpret_cast<const i16x8_t*>(base + (int64_t)row * rs + col);
  return __builtin_bit_cast(typename Mfma<T>::frag_t, v);
}

// store4 for a head dim D that is a multiple of 8 and a column that is a multiple of 4 (vector access).
template <typename T>
__device__ __forceinline__ void store4_8(T* base, int64_t rs, int row, int col, int D, float a, float b, float c,
                                         float d) {
  if (col >= D) return;
  T* p = base + (int64_t)row * rs + col;
  if constexpr (sizeof(T) == 2) {
    T v[4] = {(T)a, (T)b, (T)c, (T)d};
    *reinterpret_cast<i16x4_t*>(p) = __builtin_bit_cast(i16x4_t, v);
  } else {
    *reinterpret_cast<f32x4_t*>(p) = f32x4_t{a, b, c, d};
  }
}

// Load 4 consecutive elements (columns col..col+3 of row `row`) as float, zero beyond D.
template <typename T>
__device__ __forceinline__ f32x4_t load4(const T* base, int64_t rs, int row, int col, int D, bool vec) {
  const T* p = base + (int64_t)row * rs + col;
  f32x4_t out;
  if (vec && col + 4 <= D) {
    if constexpr (sizeof(T) == 2) {
      i16x4_t v = *reinterpret_cast<const i16x4_t*>(p);
      T t[4];
      __builtin_memcpy(t, &v, 8);
      out = f32x4_t{(float)t[0], (float)t[1], (float)t[2], (float)t[3]};
    } else {
      out = *reinterpret_cast<const f32x4_t*>(p);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) out[e] = (col + e < D) ? (float)p[e] : 0.f;
  }
  return out;
}

}  // namespace theria
