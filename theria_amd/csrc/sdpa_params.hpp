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
  bool o_f32;
  float* lse;       // mode 0: out; mode 1: in
  float* row_max;   // optional (mode 0)
  float* row_sum;   // optional (mode 0)
  float* delta;     // mode 1: out
};

// dQ pass of the backward. When o.p is set, delta = rowsum(dO * O) is computed and written to
// delta; otherwise delta is read.
struct DqParams {
  Shape s;
  View q, k, v, dout, o;
  bool o_f32;
  const float* lse;
  float* delta;
  MutView dq;
};

// dK / dV pass of the backward (dv_only: no V, dK not computed).
struct DkdvParams {
  Shape s;
  View q, k, v, dout;
  const float* lse;
  const float* delta;
  MutView dk, dv;
  bool dv_only;
};

struct JvpParams {
  Shape s;
  View q, k, v, o, tq, tk, tv;
  const float* lse;
  MutView tout;
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
