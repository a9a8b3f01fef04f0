/*
 * theria_sdpa.h - C ABI of the MI355X (gfx950) scaled-dot-product-attention operator family.
 *
 * One shared library, libtheria_sdpa.so, exports these entry points. They take caller-owned device
 * pointers, plain integer shapes and strides, and a hipStream_t passed as void*. The library never
 * allocates or frees device memory: every output and every workspace is caller-owned. Every entry
 * point is reentrant; the only mutable state is the thread-local message behind theria_last_error()
 * and a per-device cache of the compute-unit count (used to pick launch shapes).
 *
 * Semantics follow theria's operator contract (docs/phase9.md:12-39 in the reference):
 *   S = scale * Q K^T (+ causal mask), P = softmax_row(S), O = P V,
 *   m_i = max_j S_ij, l_i = sum_j exp(S_ij - m_i), lse_i = m_i + log(l_i).
 *
 * Tensors are (B, H, rows, D) views with element strides for batch, head and row; the last
 * dimension must be contiguous (stride 1). Row statistics (lse, m, l, delta, r, t) are contiguous
 * float32 arrays shaped (B, H, rows). Supported dtypes are float32, float16 and bfloat16 (the
 * reference's _ALLOWED_DTYPES, theria/attention/triton_sdpa_backward.py:20); head_dim <= 128.
 *
 * Return value: THERIA_OK, THERIA_ERR_CONTRACT (a shape, dtype, stride or pointer the contract
 * rejects: the reference raises AssertionError for these) or THERIA_ERR_HIP (a launch failure).
 * theria_last_error() returns the message of the last failing call on the calling thread.
 */
#ifndef THERIA_SDPA_H
#define THERIA_SDPA_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define THERIA_SDPA_ABI_VERSION 9

enum theria_dtype { THERIA_DTYPE_F32 = 0, THERIA_DTYPE_F16 = 1, THERIA_DTYPE_BF16 = 2 };
enum theria_status { THERIA_OK = 0, THERIA_ERR_CONTRACT = 1, THERIA_ERR_HIP = 2 };

/* A (B, H, rows, D) tensor view. data == NULL means "absent" where an entry point allows it. */
typedef struct {
  void* data;
  int64_t stride_b, stride_h, stride_row; /* element strides; the last dimension has stride 1 */
} theria_tensor_t;

/* Problem description shared by every entry point. tq = query rows (T), tk = key rows (M). */
typedef struct {
  int32_t dtype; /* enum theria_dtype of q, k, v and the other (B,H,rows,D) tensors */
  int32_t batch, heads, tq, tk, head_dim;
  float scale;    /* softmax scale; theria uses 1/sqrt(head_dim) */
  int32_t causal; /* 1: key j is visible to query i only when j <= i (top-left aligned) */
} theria_sdpa_problem_t;

/* ABI version (THERIA_SDPA_ABI_VERSION of the built library). */
int theria_abi_version(void);

/* Message of the last failing call on this thread ("" if none). */
const char* theria_last_error(void);

/*
 * Fused forward: O = softmax(scale Q K^T) V, saving lse (natural log) per query row.
 * Replaces triton_sdpa_fused + _fused_sdpa_kernel (theria/attention/triton_qk.py:242-369).
 * o_is_f32 selects float32 O (the reference kernel's output dtype, triton_qk.py:321) instead of
 * the input dtype. row_max / row_sum may be NULL; when given they receive the reference's saved
 * statistics m (row max of scaled scores) and l (sum of exp(S - m)) (triton_qk.py:299-304).
 * A query row with no visible key gets O = 0, lse = -inf, m = -inf, l = 0.
 * 16-bit inputs: the lowest mantissa bit of each finite lse marks a peaked row, one whose largest
 * probability may exceed 1/4 (set from an upper bound formed from 32-key partial row sums, so it may also
 * mark a row just below); it moves lse by at most one unit in the last place. The backward entry points
 * read it (see theria_sdpa_bwd).
 */
int theria_sdpa_fwd(const theria_sdpa_problem_t* p, const theria_tensor_t* q, const theria_tensor_t* k,
                    const theria_tensor_t* v, const theria_tensor_t* o, int32_t o_is_f32, float* lse,
                    float* row_max, float* row_sum, void* stream);

/*
 * Explicit backward given the forward output O: dQ, dK, dV.
 * Replaces sdpa_bwd_dq / sdpa_bwd_dk / sdpa_bwd_dv and their kernels
 * (theria/attention/triton_sdpa_backward.py:106-266, 269-462, 505-696) and the backward of
 * TritonFusedSDPAFunction (triton_qk.py:379-387). The row term z_i = sum_j dP_ij P_ij of the
 * reference (triton_sdpa_backward.py:312-353, 543-585) is computed once per row and written to delta_out
 * (B,H,tq) float32: as delta_i = dO_i . O_i for 16-bit inputs (see below for peaked rows), and for float32
 * inputs as sum_j P_ij dP_ij / sum_j P_ij in a pass over the keys with the same P and dP the gradient uses
 * (on a row whose probability sits on one key, dP - z is then a difference of consistently rounded values;
 * dO . O with the forward's O leaves ~2e-5 in dQ there). dout has the input dtype; o may be float32 (o_is_f32).
 * dq / dk may have data == NULL to skip that output. Deterministic (no atomics, no workspace).
 * theria_sdpa_bwd = theria_sdpa_bwd_dq followed by theria_sdpa_bwd_dkdv on the same stream.
 *
 * 16-bit inputs: the probabilities P and the score gradients dS enter the MFMA products as 16-bit
 * operands. On the rows lse flags as peaked (theria_sdpa_fwd), each is taken as two 16-bit terms (hi + lo,
 * ~2^-16 relative) from the exact float32 scores, so that sums over many such rows stay within the 16-bit
 * bars, and the row term of every row of a query block (128 or 256 rows) holding a peaked row is formed
 * exactly, sum_j P_ij dP_ij / sum_j P_ij, in one more pass over the keys (dO . O carries the 16-bit
 * rounding of the P in the forward's PV product, which a peaked row does not average out). Other rows take
 * Q or K pre-multiplied by scale * log2(e) in 16 bits. An lse from elsewhere is read the same way: its flag
 * bits choose the path (every row flagged: always the exact path). Float32 inputs ignore the flags.
 */
int theria_sdpa_bwd(const theria_sdpa_problem_t* p, const theria_tensor_t* q, const theria_tensor_t* k,
                    const theria_tensor_t* v, const theria_tensor_t* o, int32_t o_is_f32,
                    const theria_tensor_t* dout, const float* lse, float* delta_out,
                    const theria_tensor_t* dq, const theria_tensor_t* dk, const theria_tensor_t* dv, void* stream);

/*
 * The two kernels of theria_sdpa_bwd, for callers that schedule or time them separately.
 *  bwd_dq:   dQ. When o has data, delta = rowsum(dO * O) (or its exact form, as in theria_sdpa_bwd)
 *            is computed and written to delta; when o is absent, delta is read (the row term computed
 *            by an earlier call). dq may be absent: then only delta is produced.
 *  bwd_dkdv: dK and dV from delta (dk may be absent).
 */
int theria_sdpa_bwd_dq(const theria_sdpa_problem_t* p, const theria_tensor_t* q, const theria_tensor_t* k,
                       const theria_tensor_t* v, const theria_tensor_t* o, int32_t o_is_f32,
                       const theria_tensor_t* dout, const float* lse, float* delta,
                       const theria_tensor_t* dq, void* stream);
int theria_sdpa_bwd_dkdv(const theria_sdpa_problem_t* p, const theria_tensor_t* q, const theria_tensor_t* k,
                         const theria_tensor_t* v, const theria_tensor_t* dout, const float* lse,
                         const float* delta, const theria_tensor_t* dk,
                         const theria_tensor_t* dv, void* stream);

/*
 * Explicit backward from saved statistics only (no O), the reference's sdpa_bwd_* signature
 * (q, k, v, dout, m, l, scale) with lse = m + log(l). The row term is recomputed from P(lse) and
 * dP = dO V^T in a first pass over the keys (of the dQ kernel, which runs for it even without dq).
 * v may have data == NULL: then only dV is computed (sdpa_bwd_dv takes no v,
 * triton_sdpa_backward.py:194), and dq / dk must be absent. delta_out receives the row term.
 * 16-bit inputs: the flag bits of lse choose the exact path as in theria_sdpa_bwd; with the reference's
 * statistics a row is peaked when l_i < 4 (its largest probability 1 / l_i exceeds 1/4).
 * normalize = 0: the reference's frozen-stats backward, P = exp(S - lse) held as given and the row term
 *   z_i = sum_j P_ij dP_ij (triton_sdpa_backward.py:312-353, 543-585).
 * normalize = 1: the row term sum_j P_ij dP_ij / sum_j P_ij, i.e. the exact softmax gradient's, for an
 *   lse this library's forward wrote (a 16-bit forward's lse comes from rounded
 *   probabilities, so P(lse) sums to 1 only within ~2^-9, which the frozen row term passes on to dS).
 */
int theria_sdpa_bwd_from_stats(const theria_sdpa_problem_t* p, const theria_tensor_t* q, const theria_tensor_t* k,
                               const theria_tensor_t* v, const theria_tensor_t* dout, const float* lse,
                               float* delta_out, const theria_tensor_t* dq,
                               const theria_tensor_t* dk, const theria_tensor_t* dv, int32_t normalize,
                               void* stream);

/*
 * Frozen-stats JVP: tangent of O along (tq, tk, tv) with P rebuilt from lse.
 * Replaces sdpa_jvp (theria/attention/triton_sdpa_backward.py:465-503), which runs eager PyTorch:
 *   G = scale (tq K^T + Q tk^T), c_i = sum_j P_ij G_ij, tO = (P o G) V - c o O + P tv.
 * o may have data == NULL: O is then rebuilt from P(lse) and V inside the kernel. Any tangent may
 * have data == NULL (a zero tangent). tout has the input dtype.
 * normalize = 0: the frozen-stats JVP exactly as the reference defines it, P = exp(S - lse) held as given
 *   (the caller's stats need not be the exact ones; O is then rebuilt from that P, o is not read).
 * normalize = 1: the JVP of the exact softmax, for an lse this library's forward wrote: P is divided by
 *   its own row sum (a 16-bit forward's lse comes from rounded probabilities, so P(lse) sums to 1 only
 *   within ~2^-9).
 */
int theria_sdpa_jvp(const theria_sdpa_problem_t* p, const theria_tensor_t* q, const theria_tensor_t* k,
                    const theria_tensor_t* v, const theria_tensor_t* o, const float* lse, const theria_tensor_t* tq,
                    const theria_tensor_t* tk, const theria_tensor_t* tv, const theria_tensor_t* tout,
                    int32_t normalize, void* stream);

/*
 * Double backward: the vector-Jacobian product of the backward map (Q, K, V, dO) -> (dQ, dK, dV)
 * with cotangents (gq, gk, gv) of (dQ, dK, dV). Outputs out_gq, out_gk, out_gv, out_gdout.
 * The reference has no kernel for this: its HVP is a finite difference of the VJP
 * (theria/attention/hvp_utils.py:30-49) or autograd-in-backward (theria/autograd/sdpa_custom_function.py:32-53).
 * delta (the row term written by theria_sdpa_bwd) is not read and may be NULL: a pass over the keys recomputes
 * the row term into the workspace. Any cotangent may have data == NULL (zero).
 * For float32 inputs that pass also forms each row's own statistics from its float32 scores, m2 = max_j fl(S c)
 * and L2 = log2 sum_j exp2(fl(S c) - m2) with c = scale log2(e), and the row and column kernels rebuild
 * P = exp2((fl(S c) - m2) - L2) with dP formed as in that pass (lse is read only by the G_dO pass): on rows
 * whose probability sits on one key the second-order terms are differences (dP - z, Gam - r, E1 - t) that
 * P from a rounded lse would leave at ~1e-5.
 * For 16-bit inputs a pass over the keys recomputes, into the workspace, the row normaliser
 * lse + ln(sum_j P_ij) (a 16-bit forward's lse comes from rounded probabilities, so P rebuilt from it sums to
 * one only within ~2^-9) and the row term sum_j P_ij dP_ij / sum_j P_ij in float32 (delta from the 16-bit O
 * differs from it by the rounding of O); the second-order terms amplify both where they cancel. delta is
 * then not read. Query blocks holding a row flagged peaked in lse are redone by a second row pass (run as
 * part of the column kernel's grid) that forms G_Q's score-gradient in float32 from the first pass's row
 * terms; those blocks and tiles enter the G_Q, G_K, G_V products as two 16-bit terms.
 * row_ws is a caller-owned float32 workspace of 5*batch*heads*tq elements.
 */
int theria_sdpa_bwd_bwd(const theria_sdpa_problem_t* p, const theria_tensor_t* q, const theria_tensor_t* k,
                        const theria_tensor_t* v, const theria_tensor_t* o, const theria_tensor_t* dout,
                        const float* lse, const float* delta, const theria_tensor_t* gq, const theria_tensor_t* gk,
                        const theria_tensor_t* gv, const theria_tensor_t* out_gq, const theria_tensor_t* out_gk,
                        const theria_tensor_t* out_gv, const theria_tensor_t* out_gdout, float* row_ws, void* stream);

/*
 * theria_sdpa_bwd_bwd without a workspace argument and without any allocation. It has no counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). The row workspace is a static device array of 5 * 2^20 floats (20 MiB)
 * that each GPU the library runs on holds until the process ends, so 5 * batch * heads * tq must not exceed
 * 5 * 2^20 (a larger problem is rejected with THERIA_ERR_CONTRACT). Every call on one GPU shares that GPU's
 * array: calls that overlap on one GPU (other streams, other threads) race and must be serialised by the
 * caller. Results equal theria_sdpa_bwd_bwd's bit for bit. The first call on a device looks up that device's
 * scratch address (hipGetSymbolAddress, which may load the library's code object): make one call outside any
 * stream capture before capturing it in a HIP graph; captured calls then only launch kernels.
 */
int theria_sdpa_bwd_bwd_noalloc(const theria_sdpa_problem_t* p, const theria_tensor_t* q, const theria_tensor_t* k,
                                const theria_tensor_t* v, const theria_tensor_t* o, const theria_tensor_t* dout,
                                const float* lse, const float* delta, const theria_tensor_t* gq,
                                const theria_tensor_t* gk, const theria_tensor_t* gv, const theria_tensor_t* out_gq,
                                const theria_tensor_t* out_gk, const theria_tensor_t* out_gv,
                                const theria_tensor_t* out_gdout, void* stream);

/*
 * Materialised scores for the partial-fusion sdpa_custom backends (theria/attention/custom.py:30-49).
 * theria_qk_scores: unscaled S = Q K^T as a contiguous (B, H, tq, tk) tensor at `out`, float32 when
 *   out_f32 (or when the inputs are float32), else the input dtype. Replaces _qk_kernel and
 *   _qk_kernel_fast behind triton_qk / triton_qk_fast (theria/attention/triton_qk.py:24-125, 402-522).
 * theria_qk_softmax: P = softmax(scale Q K^T) over the keys as a contiguous float32 (B, H, tq, tk)
 *   tensor. Replaces _qk_softmax_kernel / triton_qk_softmax (triton_qk.py:128-240).
 * p->causal must be 0 (the reference's score backends have no mask); v-related fields are unused.
 */
int theria_qk_scores(const theria_sdpa_problem_t* p, const theria_tensor_t* q, const theria_tensor_t* k, void* out,
                     int32_t out_f32, void* stream);
int theria_qk_softmax(const theria_sdpa_problem_t* p, const theria_tensor_t* q, const theria_tensor_t* k, float* probs,
                      void* stream);

/*
 * Measurement hook with no counterpart in the reference: the executed tile units of the pipelined 16-bit
 * kernels, counted by the kernels themselves, for measuring causal tile skipping. counts[0..2] receive the
 * 32 x 32 (query, key) units whose products the forward, dQ and dK/dV kernels ran since the last reset (on the
 * current device, after the work is complete: the call synchronises with a device copy); reset = 1 zeroes
 * them afterwards. Only the counter-enabled build (libtheria_sdpa_tiles.so, the same sources compiled with
 * THERIA_TILE_COUNT) counts; libtheria_sdpa.so returns THERIA_ERR_CONTRACT and zeros.
 */
int theria_debug_tile_counts(uint64_t* counts, int32_t reset);

/*
 * Measurement only (no counterpart in the reference): float32 atomic-add throughput in the pattern a backward that
 * formed dQ inside the dK/dV kernel would need. Each 256-thread workgroup adds a constant to 128 x 64 consecutive
 * floats of buf (relaxed, device scope; atomic = 0: plain stores of the same shape), reps workgroups per
 * 8192-float block, consecutive workgroups on different blocks; n rounded down to whole blocks. Only the
 * counter-enabled build (libtheria_sdpa_tiles.so) runs it; libtheria_sdpa.so returns THERIA_ERR_CONTRACT.
 */
int theria_debug_atomic_probe(float* buf, int64_t n, int32_t reps, int32_t atomic, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* THERIA_SDPA_H */
