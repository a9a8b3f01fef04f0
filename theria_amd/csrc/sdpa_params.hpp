// Kernel parameter blocks and launcher declarations shared by the kernel files and the C ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace theria {

// A (B, H, rows, D) view: base pointer plus element strides (batch, head, row); last dim contiguous.
struct View {
  const void* p;
  int64_t sb, sh, sr;
};
struct MutView {
  void* p;
  int64_t sb, sh, sr;
};

struct Shape {
  int B, H, T, M, D;
  float scale;
  bool causal;
  int dtype;  // theria_dtype
  int dp;     // padded head dim: 32, 64 or 128
  bool vec;   // every view allows 16-byte vector access
};

// Forward (mode 0) or row term from saved stats (mode 1: delta_i = dO_i . sum_j P_ij V_j).
struct FwdParams {
  Shape s;
  View q, k, v, dout;
  MutView o;
  MutView o_lo;     // optional (mode 0, 16-bit O): rounding residual O - (float)o in the input dtype
  bool o_f32;
  float* lse;       // mode 0: out; mode 1: in
  float* row_max;   // optional (mode 0)
  float* row_sum;   // optional (mode 0)
  float* delta;     // mode 1: out
  // mode 1: delta from the normalised O = sum_j P_ij V_j / sum_j P_ij (the exact softmax's row term for the
  // operator's own lse) instead of sum_j P_ij dP_ij with P as given (the reference's frozen-stats term)
  bool row_normalize;
};

// Largest probability of a row above which the 16-bit backward forms P and dS as two 16-bit terms
// (hi + lo): exp(m - lse) > 1/16, i.e. m - lse > -ln 16.
constexpr float kPeakedLog = -2.7725887222397811f;

// dQ pass of the backward. When o.p is set, delta = rowsum(dO * (O + O_lo)) is computed and written to
// delta; otherwise delta is read. row_max (optional): the row maxima m that mark peaked rows (16-bit
// inputs); absent, every row is treated as peaked.
struct DqParams {
  Shape s;
  View q, k, v, dout, o, o_lo;
  bool o_f32;
  const float* lse;
  const float* row_max;
  float* delta;
  MutView dq;
};

// dK / dV pass of the backward (dv_only: no V, dK not computed).
struct DkdvParams {
  Shape s;
  View q, k, v, dout;
  const float* lse;
  const float* row_max;  // as in DqParams
  const float* delta;
  MutView dk, dv;
  bool dv_only;
};

// normalize: P divided by its own row sum (the exact-softmax JVP, for an lse of this library's forward);
// otherwise P = exp(S - lse) exactly as given (the reference's frozen-stats JVP).
struct JvpParams {
  Shape s;
  View q, k, v, o, tq, tk, tv;
  const float* lse;
  MutView tout;
  bool normalize;
};

struct BwdBwdParams {
  Shape s;
  View q, k, v, dout, gq, gk, gv;
  const float* lse;
  const float* delta;
  float* r_row;
  float* t_row;
  MutView out_gq, out_gk, out_gv;
};

// Materialised scores (partial-fusion backends): S = Q K^T or P = softmax(scale Q K^T), contiguous
// (B, H, T, M) output.
struct ScoresParams {
  Shape s;
  View q, k;
  void* out;
  bool out_f32;  // scores in float32 (else the input dtype); P is always float32
  bool softmax;
};

// Compute units of the current device (cached per device).
int device_cu_count();

hipError_t launch_fwd(const FwdParams& p, int mode, hipStream_t st);
hipError_t launch_bwd_dq(const DqParams& p, hipStream_t st);
hipError_t launch_bwd_dkdv(const DkdvParams& p, hipStream_t st);
hipError_t launch_jvp(const JvpParams& p, hipStream_t st);
hipError_t launch_bwdbwd_rows(const BwdBwdParams& p, hipStream_t st);
hipError_t launch_bwdbwd_cols(const BwdBwdParams& p, hipStream_t st);
hipError_t launch_scores(const ScoresParams& p, hipStream_t st);

}  // namespace theria
