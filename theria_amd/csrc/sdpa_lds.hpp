// LDS tiles filled by DMA for 16-bit inputs with a head dimension DP of 32, 64 or 128 (gfx950).
//
// A tile holds R rows x DP columns of a 16-bit type, RB = 2 DP bytes per row (64, 128 or 256), with no
// padding. Its global rows are copied by LDS DMA (buffer_load_dwordx4 ... lds), which writes the 16
// bytes of lane l of a wave to LDS address M0 + 16 * l (checked on the device), so one wave instruction
// fills 1024 / RB consecutive rows and the data never passes through VGPRs.
//
// The RB/16 chunks (16 bytes) of row r are stored XOR-swizzled: logical chunk c sits at slot
// c ^ swz<DP>(r), and the DMA lane that fills slot s of row r fetches logical chunk s ^ swz<DP>(r). The
// swizzle makes both read patterns bank-conflict free:
//  * "cols" fragments (ds_read_b128, one lane-fixed row, k along the row): 16 lanes read the same logical
//    chunk of 16 consecutive rows (16-aligned). DP = 32: four rows span the 64 banks, so rows r and r + 4
//    share banks and swz = (r >> 2) & 3 sends the four rows of each residue r & 3 to distinct slots. DP = 64:
//    rows of one parity share a 32-bank half and
//    swz = bits 1..3 of r (bit-reversed) gives them distinct slots. DP = 128: every row spans all 64
//    banks and swz = ((r & 3) << 2) | ((r >> 2) & 3) is a bijection of r & 15.
//  * "rows" (transpose) fragments (ds_read_b64_tr_b16, k down a column): 32 lanes read 4 consecutive rows
//    (4-aligned) x 4 consecutive chunks (4-aligned). DP = 32: the 4 rows are the 64 banks, whatever the slots.
//    DP = 64: the two rows of one parity differ in bit 1,
//    which flips slot bit 2. DP = 128: the 4 rows XOR by 0, 4, 8, 12, i.e. land in 4 different chunk quads.
#pragma once

#include "sdpa_common.hpp"

namespace theria {

template <int DP>
__device__ __forceinline__ int swz(int r) {
  static_assert(DP == 32 || DP == 64 || DP == 128, "tile rows of 64, 128 or 256 bytes");
  if constexpr (DP == 32)
    return (r >> 2) & 3;
  else if constexpr (DP == 64)
    return (((r >> 1) & 1) << 2) | (((r >> 2) & 1) << 1) | ((r >> 3) & 1);
  else
    return ((r & 3) << 2) | ((r >> 2) & 3);
}

// Wait until every global load (and LDS DMA) this wave issued has completed (s_waitcnt vmcnt(0)).
__device__ __forceinline__ void wait_vm_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }

typedef __attribute__((address_space(3))) void lds_void_t;

// Buffer resource (V#). The type only exists in the device pass; the host pass parses the kernels but
// never runs them, so it gets a placeholder of the same size.
#if defined(__HIP_DEVICE_COMPILE__)
typedef __amdgpu_buffer_rsrc_t rsrc_t;
#else
typedef struct {
  unsigned w[4];
} rsrc_t;
#endif

// Bytes spanned by `rows` rows of `row_bytes` bytes at a row stride of `rs_bytes`. The stride may be smaller
// than a row (overlapping rows) or zero (one row broadcast over all of them), so the span is that of the last
// row's end, not rows * stride. A buffer resource over fewer bytes would read the missing rows as zeros.
__host__ __device__ __forceinline__ int64_t slab_span(int64_t rows, int64_t rs_bytes, int64_t row_bytes) {
  return rows > 0 ? (rows - 1) * rs_bytes + row_bytes : 0;
}

// The DMA kernels address each (batch, head) slab with 32-bit byte offsets (and an out-of-range offset of
// 2^31 for the chunks past the head dim), so the slab must span less than 2^31 bytes.
__host__ __device__ __forceinline__ bool slab_fits_dma(int64_t rows, int64_t rs_elems, int64_t head_dim) {
  return slab_span(rows, 2 * rs_elems, 2 * head_dim) < (int64_t(1) << 31);
}

// Buffer resource over `bytes` bytes from `base` (raw buffer, stride 0; gfx9 data-format word). Loads
// beyond `bytes` return zero instead of faulting.
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
#else
  return rsrc_t{};
#endif
}

// 16 bytes per lane from the buffer at voffset + soffset into registers (zeros beyond the resource's range).
__device__ __forceinline__ i16x8_t buf_load16(rsrc_t rsrc, uint32_t voffset, uint32_t soffset) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_bit_cast(i16x8_t, __builtin_amdgcn_raw_buffer_load_b128(rsrc, voffset, soffset, 0));
#else
  return i16x8_t{};
#endif
}

// One 16-byte-per-lane LDS DMA: lane l's 16 bytes at voffset + soffset in the buffer go to lds + 16 l.
__device__ __forceinline__ void dma16(rsrc_t rsrc, char* lds, uint32_t voffset, uint32_t soffset) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void_t*)lds, 16, voffset, soffset, 0, 0);
#endif
}

// Per-lane constants of the cooperative DMA of slabs by a workgroup of NW waves. One wave instruction
// fills RPW = 1024 / RB rows; wave w fills rows RPW w .. RPW w + RPW - 1 of every slab of RPW * NW rows
// (bytes [1024 w, 1024 w + 1024) of it). `wave` must be wave-uniform (an SGPR value), since it selects
// the LDS destination. The copies are buffer_load_dwordx4 ... lds with a per-lane 32-bit offset and a
// wave-uniform offset for the tile, so no 64-bit address math is needed. Rows shorter than DP (a head dim
// D < DP, a multiple of 8) fill only their nck = D / 8 leading chunks from memory: the lanes of the other
// chunks use an offset past the end of the buffer (kOutOfRange, >= 2^31 > any buffer the host admits),
// for which the buffer load returns zero, so the tile's columns D .. DP - 1 read as zero.
template <int NW, int DP>
struct SwzDma {
  static constexpr int RB = 2 * DP;            // bytes per row
  static constexpr int CPR = RB / 16;          // chunks per row
  static constexpr int RPW = 1024 / RB;        // rows per wave instruction
  static constexpr int SLAB_ROWS = RPW * NW;
  static constexpr int SLAB_BYTES = SLAB_ROWS * RB;
  // A lane derives its swizzle from its row inside the slab; that equals the swizzle of the tile row
  // only if slabs start on multiples of the swizzle's period (16 rows).
  static_assert(SLAB_ROWS % 16 == 0, "LDS DMA slabs must span a multiple of 16 rows (more waves per workgroup)");
  static constexpr uint32_t kOutOfRange = 0x80000000u;
  int row;     // row of the slab filled by this lane
  int chunk;   // logical 16-byte chunk this lane fetches
  int dst;     // byte offset of this wave's piece in a slab
  bool valid;  // the chunk lies inside the row (chunk < nck)

  __device__ __forceinline__ SwzDma(int wave, int lane, int nck = CPR)
      : row(RPW * wave + lane / CPR),
        chunk((lane % CPR) ^ swz<DP>(RPW * wave + lane / CPR)),
        dst(1024 * wave),
        valid(chunk < nck) {}

  // Byte offset, from the tile's first row, of what this lane fetches for slab i (out of range for a chunk
  // past the row; the tile offset added to it stays below 2^32).
  __device__ __forceinline__ uint32_t lane_offset(uint32_t rs_bytes, int i) const {
    return valid ? (uint32_t)(SLAB_ROWS * i + row) * rs_bytes + chunk * 16 : kOutOfRange;
  }

  // Rows [r0, r0 + SLAB_ROWS * NSLAB) all in range: tile_off = r0 * rs_bytes (wave-uniform), off[i] =
  // lane_offset(rs_bytes, i). r0 must be a multiple of 16 (the swizzle of a slab row then only depends on
  // its position in the slab).
  template <int NSLAB>
  __device__ __forceinline__ void issue(rsrc_t rsrc, const uint32_t (&off)[NSLAB], uint32_t tile_off, char* tile) const {
#pragma unroll
    for (int i = 0; i < NSLAB; ++i) dma16(rsrc, tile + SLAB_BYTES * i + dst, off[i], tile_off);
  }

  // Rows [r0, r0 + SLAB_ROWS * NSLAB) of a matrix with nrows rows (r0 a multiple of 16). Rows >= nrows
  // copy row nrows - 1, a valid row whose scores the caller masks; nrows must be positive.
  template <int NSLAB>
  __device__ __forceinline__ void issue_clamped(rsrc_t rsrc, uint32_t rs_bytes, int r0, int nrows, char* tile) const {
#pragma unroll
    for (int i = 0; i < NSLAB; ++i) {
      const uint32_t r = (uint32_t)min(r0 + SLAB_ROWS * i + row, nrows - 1);
      dma16(rsrc, tile + SLAB_BYTES * i + dst, valid ? r * rs_bytes + chunk * 16 : kOutOfRange, 0);
    }
  }
};

// "cols" fragment (KLIN order): lane row `row` of the tile, k = columns 16c + 8g .. 16c + 8g + 7.
template <typename T, int DP>
__device__ __forceinline__ typename Mfma<T>::frag_t swz_cols(const char* tile, int row, int c) {
  const int g = (threadIdx.x >> 5) & 1;
  const int slot = (2 * c + g) ^ swz<DP>(row);
  return __builtin_bit_cast(typename Mfma<T>::frag_t, *reinterpret_cast<const i16x8_t*>(tile + row * (2 * DP) + slot * 16));
}

// "rows" fragment (KACC order): lane-fixed column col0 + li, k = tile rows kbase + acc_row(8c + e, g)
// (the same rows as lds_rows<T, KACC> in sdpa_common.hpp, on the swizzled layout). kbase is a multiple of 16.
template <typename T, int DP>
__device__ __forceinline__ typename Mfma<T>::frag_t swz_rows(const char* tile, int kbase, int c, int col0) {
  const int lane = threadIdx.x & 63;
  const int s = lane & 15, hh = (lane >> 4) & 1, g = lane >> 5;
  const int col = col0 + 16 * hh + 4 * (s & 3);
  const int r0 = kbase + 16 * c + 4 * g + (s >> 2);
  const int r1 = r0 + 8;
  const i16x4_t a = ds_read_tr16(tile + r0 * (2 * DP) + (((col >> 3) ^ swz<DP>(r0)) << 4) + (col & 7) * 2);
  const i16x4_t b = ds_read_tr16(tile + r1 * (2 * DP) + (((col >> 3) ^ swz<DP>(r1)) << 4) + (col & 7) * 2);
  const i16x8_t v = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  return __builtin_bit_cast(typename Mfma<T>::frag_t, v);
}

// Sum of the 8 16-bit values of a fragment added to acc (v_dot2 with ones), in float32.
template <typename T>
__device__ __forceinline__ float frag_sum(const typename Mfma<T>::frag_t& f, float acc) {
  if constexpr (__is_same(T, __bf16)) {
    typedef __bf16 v2_t __attribute__((ext_vector_type(2)));
    const v2_t one = {(__bf16)1.0f, (__bf16)1.0f};
#pragma unroll
    for (int i = 0; i < 4; ++i) acc = __builtin_amdgcn_fdot2_f32_bf16(v2_t{f[2 * i], f[2 * i + 1]}, one, acc, false);
  } else {
    typedef _Float16 v2_t __attribute__((ext_vector_type(2)));
    const v2_t one = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
    for (int i = 0; i < 4; ++i) acc = __builtin_amdgcn_fdot2(v2_t{f[2 * i], f[2 * i + 1]}, one, acc, false);
  }
  return acc;
}

}  // namespace theria
