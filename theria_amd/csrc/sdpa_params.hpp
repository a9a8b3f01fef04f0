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
  // causal pipelined kernels: one block per workgroup, longest first, instead of a block and its mirror (set by
  // the launchers when the mirrored pairs would leave CUs without a workgroup)
  bool unpaired;
};

// Forward: O, lse and the optional reference statistics m (row_max) and l (row_sum).
struct FwdParams {
  Shape s;
  View q, k, v;
  MutView o;
  bool o_f32;
  float* lse;
  float* row_max;  // optional
  float* row_sum;  // optional
};

// How the dQ kernel obtains the row term delta_i of dS = P o (dP - delta), which it writes to delta (the
// dK / dV kernel reads it there):
enum RowTerm : int {
  kRowFromO = 0,    // dO_i . O_i from the given O; with 16-bit inputs a workgroup holding a peaked row (flagged
                    // in its lse) forms it exactly instead (as kRowNormalized): the 16-bit P of the forward's
                    // PV product leave ~2^-9 |dP| in dO . O, which a peaked row does not average out
  kRowGiven = 1,    // read from delta
  kRowFrozen = 2,   // sum_j P_ij dP_ij with P = exp(S - lse) exactly as given (frozen statistics)
  kRowNormalized = 3,  // sum_j P_ij dP_ij / sum_j P_ij: the exact softmax's row term for this lse
  kRowOwnStats = 4,    // float32: the row's own statistics from this kernel's scores, ignoring lse: m2 = max_j
                       // fl(S_ij scale log2 e) (to lse_out), L2 = log2 sum_j exp2(fl(S_ij scale log2 e) - m2) (to
                       // l2_out) and sum_j P_ij dP_ij / sum_j P_ij (to delta), with dP formed from zero
};

// dQ pass of the backward (dq.p may be null: the row term only). 16-bit inputs: peaked rows are flagged in lse.
struct DqParams {
  Shape s;
  View q, k, v, dout, o;
  bool o_f32;
  int row_term;  // RowTerm
  const float* lse;
  float* delta;
  MutView dq;
  // optional, with a row-term pass (blocks taking it): lse + ln(sum_j P_ij), the row's exact normaliser for P
  // rebuilt from lse, flagged peaked from the row's exact largest probability (above 1/4); with kRowOwnStats
  // the row max m2 (+inf for a row without visible keys)
  float* lse_out;
  float* l2_out;  // kRowOwnStats: L2 (0 for a row without visible keys)
};

// dK / dV pass of the backward (dv_only: no V, dK not computed).
struct DkdvParams {
  Shape s;
  View q, k, v, dout;
  const float* lse;  // 16-bit inputs: peaked rows flagged
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

// lse: 16-bit inputs, the row normaliser (natural log, peaked rows flagged); float32 inputs, the row max m2 of
// fl(S scale log2 e) with row_l2 = L2, so that P = exp2((fl(S scale log2 e) - m2) - L2) (kRowOwnStats).
struct BwdBwdParams {
  Shape s;
  View q, k, v, dout, gq, gk, gv;
  const float* lse;
  const float* row_l2;  // float32 inputs only
  const float* delta;
  float* r_row;
  float* t_row;
  MutView out_gq, out_gk, out_gv;
  // The key-split row kernel (16-bit, head dim 64) forms the row statistics itself from the forward's lse
  // (lse_fwd) and writes the row term and the exact normaliser to z_out and lse_out, which the column kernel
  // then reads as delta and lse.
  const float* lse_fwd;
  float* z_out;
  float* lse_out;
  MutView out_gdo;  // the key-split row kernel also writes G_dO (no separate JVP launch)
};

// The row kernel of this problem forms the row term and the exact normaliser itself (no row-term pass needed).
bool bwdbwd_rows_make_row_terms(const BwdBwdParams& p);

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

hipError_t launch_fwd(const FwdParams& p, hipStream_t st);
hipError_t launch_bwd_dq(const DqParams& p, hipStream_t st);
hipError_t launch_bwd_dkdv(const DkdvParams& p, hipStream_t st);
hipError_t launch_jvp(const JvpParams& p, hipStream_t st);
hipError_t launch_bwdbwd_rows(const BwdBwdParams& p, hipStream_t st);
hipError_t launch_bwdbwd_cols(const BwdBwdParams& p, hipStream_t st);
hipError_t launch_scores(const ScoresParams& p, hipStream_t st);

#ifdef THERIA_TILE_COUNT
// Executed 32 x 32 tile units of the pipelined kernels (counter-enabled build only; reset: zero them after reading).
hipError_t tile_counts_fwd(unsigned long long* fwd, bool reset);
hipError_t tile_counts_bwd(unsigned long long* dq, unsigned long long* dkdv, bool reset);
// Float32 atomic adds (or, atomic = false, plain stores) over n floats, reps times, in dQ-tile-shaped workgroups.
hipError_t launch_atomic_probe(float* buf, int64_t n, int reps, bool atomic, hipStream_t st);
#endif

}  // namespace theria
