/*
 * msda_hip.h - C ABI of the MI355X (gfx950) multi-scale deformable attention
 * operator.
 *
 * The library (libmsda_hip.so) is the drop-in replacement for the two device
 * launches of the reference operator roulbac/msda-triton:
 *
 *   msda_forward   replaces the launch of `_msda_forward_kernel`
 *                  (src/msda_triton/ops.py:46-52, kernel at
 *                  src/msda_triton/kernels.py:58-163)
 *   msda_backward  replaces the zero-fill, the launch of
 *                  `_msda_backward_kernel` and the accumulator cast
 *                  (src/msda_triton/ops.py:76-92, kernel at
 *                  src/msda_triton/kernels.py:166-291)
 *
 * and, one step further out, msda_fused_forward / msda_fused_backward fold
 * the attention layer's front-end (softmax of the logits, reference point +
 * offset / (W, H); labs/solutions/lab00.py:194-208) into the same kernels.
 *
 * Conventions shared by every entry point
 *   - All pointers are device pointers to C-contiguous arrays.
 *   - value                (B, S, M, D)        dtype
 *     spatial_shapes       (L, 2) int64        (H_l, W_l), on the device
 *     level_start_index    (L,)   int64        offset of level l along S, on the device
 *     sampling_locations   (B, Q, M, L, K, 2)  dtype, normalised (x, y)
 *     attention_weights    (B, Q, M, L, K)     dtype
 *     output / grad_output (B, Q, M, D)        dtype
 *   - Bilinear sampling follows grid_sample(align_corners=False,
 *     padding_mode="zeros"): x = loc_x * W_l - 0.5, y = loc_y * H_l - 0.5,
 *     corners outside [0, W_l) x [0, H_l) contribute zero.
 *   - Arithmetic is fp32 for every storage dtype; results are rounded once to
 *     the storage dtype.
 *   - Work is enqueued on `stream` (a hipStream_t; NULL = the null stream).
 *     No entry point synchronises or allocates device memory, and none
 *     keeps state between calls apart from the launch overrides set by
 *     msda_set_launch_override (unset by default); all of them may be
 *     captured into a hipGraph.
 *   - The return value is MSDA_OK or one of the MSDA_ERR_* codes below; the
 *     device buffers are untouched when an argument error is returned.
 */
#ifndef MSDA_HIP_H_
#define MSDA_HIP_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Storage dtype codes. */
#define MSDA_DTYPE_F32 0
#define MSDA_DTYPE_F16 1
#define MSDA_DTYPE_BF16 2

/* Return codes. */
#define MSDA_OK 0
#define MSDA_ERR_INVALID_ARGUMENT 1 /* negative size, NULL pointer for a non-empty array */
#define MSDA_ERR_UNSUPPORTED_DTYPE 2
#define MSDA_ERR_UNSUPPORTED_SHAPE 3 /* L > MSDA_MAX_LEVELS, D*elem > 1024 bytes, S >= 2^31 */
#define MSDA_ERR_LAUNCH 4            /* hipGetLastError() after a launch */

#define MSDA_MAX_LEVELS 64

/*
 * Forward: output[b,q,m,:] = sum_{l,k} A[b,q,m,l,k] *
 *          bilinear(value[b, level l, m, :], sampling_locations[b,q,m,l,k]).
 *
 * Replaces src/msda_triton/ops.py:46-52 (allocation of `out` stays with the
 * caller, as there) and the kernel src/msda_triton/kernels.py:58-163.
 * batch..num_points are B, S, M, D, Q, L, K.  B*Q == 0 launches nothing.
 */
int msda_forward(const void* value, const int64_t* spatial_shapes,
                 const int64_t* level_start_index, const void* sampling_locations,
                 const void* attention_weights, void* output, int64_t batch,
                 int64_t num_keys, int64_t num_heads, int64_t head_dim,
                 int64_t num_queries, int64_t num_levels, int64_t num_points,
                 int dtype, void* stream);

/*
 * Backward: the three analytic gradients of msda_forward.
 *
 * Replaces src/msda_triton/ops.py:76-92 and the kernel
 * src/msda_triton/kernels.py:166-291.
 *   grad_value              (B, S, M, D) dtype, written in full; its contents
 *                           on entry do not matter.
 *   grad_value_accum        NULL: on the atomic paths grad_value is
 *                           accumulated in place with the dtype's own atomics
 *                           (fp32 add, packed fp16/bf16 add).  Non-NULL: an
 *                           fp32 scratch array of B*S*M*D floats; the atomic
 *                           and binned paths accumulate there in fp32 and
 *                           round once into grad_value.  This is the
 *                           reference's `fp32_grad_accum=True`
 *                           (src/msda_triton/ops.py:76-77,91-92).  For
 *                           dtype == MSDA_DTYPE_F32 it may alias grad_value.
 *   grad_sampling_locations (B, Q, M, L, K, 2) dtype, written in full.
 *   grad_attention_weights  (B, Q, M, L, K)    dtype, written in full.
 * The library picks one of four ways to form grad_value
 * (msda_backward_plan reports which): for few samples per (batch, head,
 * level) -- Q*K <= 2048, a head row of a multiple of 16 bytes up to 256,
 * Q*D*elem <= 40960, 16-byte aligned grad_output and grad_value -- workgroups
 * that own bands of value rows sum each element's contributions in fp32 and
 * store it once (no atomics, no zero-fill, grad_value_accum unused);
 * otherwise, for head rows of 32, 64 or 128 bytes with D a power of two,
 * the samples are binned by band of value rows (the bins kept in
 * grad_sampling_locations and grad_attention_weights before those are
 * written, a count matrix in the accumulator -- grad_value or
 * grad_value_accum -- before it is zero-filled on `stream`) and each band's
 * rows are summed in fp32 by one workgroup, which stores them, or by
 * several, which add them with atomics; for other shapes grad_value is
 * zero-filled and the atomics are issued by a kernel that merges samples
 * sharing a row within a workgroup or by the direct scatter.  On the owner
 * path grad_value is bitwise reproducible (each element one fp32 sum in an
 * order fixed by the inputs); on the binned path wherever no band is split
 * over workgroups; on the atomic paths it is not (the order of the atomics
 * varies).  The other two gradients are reproducible on every path.
 */
int msda_backward(const void* value, const int64_t* spatial_shapes,
                  const int64_t* level_start_index, const void* sampling_locations,
                  const void* attention_weights, const void* grad_output,
                  void* grad_value, float* grad_value_accum,
                  void* grad_sampling_locations, void* grad_attention_weights,
                  int64_t batch, int64_t num_keys, int64_t num_heads,
                  int64_t head_dim, int64_t num_queries, int64_t num_levels,
                  int64_t num_points, int dtype, void* stream);

/*
 * Fused MSDeformAttn front-end, forward.  Computes what the reference's
 * attention layer composes in PyTorch around the operator
 * (labs/solutions/lab00.py:194-208, MSDACrossAttention.forward):
 *
 *   weights   = softmax over the L*K points of attention_logits[b,q,m,:]
 *   locations = reference_points[b,q,(l),:] + sampling_offsets / (W_l, H_l)
 *   output    = msda_forward(value, ..., locations, weights)
 *
 * with the locations and weights formed in the kernel's staging step (fp32),
 * never stored.  No single reference function corresponds to it: it
 * replaces the three PyTorch ops of lab00.py:202-207 plus the operator
 * launch of src/msda_triton/ops.py:46-52.
 *   reference_points   (B, Q, 2) if reference_levels == 0, or
 *                      (B, Q, L, 2) if reference_levels == 1; dtype, normalised.
 *   sampling_offsets   (B, Q, M, L, K, 2) dtype, in level-l pixel units.
 *   attention_logits   (B, Q, M, L, K)    dtype (softmax over the last two).
 *   softmax_lse        (B, Q, M) fp32: receives log(sum_{l,k} exp(logit)) of
 *                      each (b, q, m) for the backward; may be NULL
 *                      (inference).  Not written when B*Q*M*D == 0.
 */
int msda_fused_forward(const void* value, const int64_t* spatial_shapes,
                       const int64_t* level_start_index, const void* reference_points,
                       const void* sampling_offsets, const void* attention_logits,
                       void* output, float* softmax_lse, int64_t batch,
                       int64_t num_keys, int64_t num_heads, int64_t head_dim,
                       int64_t num_queries, int64_t num_levels, int64_t num_points,
                       int reference_levels, int dtype, void* stream);

/*
 * Fused front-end, backward: gradients of msda_fused_forward.  Replaces the
 * operator's backward (src/msda_triton/ops.py:76-92) plus the autograd of
 * lab00.py:202-207 (softmax backward, the division by (W_l, H_l) and the
 * broadcast sum onto the reference points).
 *   softmax_lse, output     what msda_fused_forward returned for these inputs.
 *   grad_value, grad_value_accum  as in msda_backward.
 *   grad_reference_points   shape of reference_points, written in full; NULL
 *                           skips it.
 *   grad_sampling_offsets   (B, Q, M, L, K, 2) dtype, written in full.
 *   grad_attention_logits   (B, Q, M, L, K)    dtype, written in full.
 * The softmax backward uses delta = <grad_output, output> per (b, q, m).
 * All gradients but grad_value are bitwise deterministic.
 */
int msda_fused_backward(const void* value, const int64_t* spatial_shapes,
                        const int64_t* level_start_index, const void* reference_points,
                        const void* sampling_offsets, const void* attention_logits,
                        const float* softmax_lse, const void* output,
                        const void* grad_output, void* grad_value,
                        float* grad_value_accum, void* grad_reference_points,
                        void* grad_sampling_offsets, void* grad_attention_logits,
                        int64_t batch, int64_t num_keys, int64_t num_heads,
                        int64_t head_dim, int64_t num_queries, int64_t num_levels,
                        int64_t num_points, int reference_levels, int dtype,
                        void* stream);

/*
 * Deterministic backward.  The reference accumulates grad_value with
 * floating-point atomics, so its sums depend on their arrival order and are
 * not reproducible bit for bit (documented at src/msda_triton/ops.py:135-138).
 * These variants make it identical on every run.  Calls that take the owner
 * path (msda_backward_plan(..., 1) == MSDA_BACKWARD_OWNER; see msda_backward)
 * get it from there: every element is one fp32 sum over its contributions
 * in an order fixed by the inputs, no workspace needed.  Other calls
 * accumulate in int64 fixed point: on the binned path
 * (MSDA_BACKWARD_BINNED) each band's fp32 sums, formed in an order fixed by
 * the inputs, enter as round(sum * 2^e); on the atomic paths each
 * contribution c does, as round(c * 2^e); integer addition is exact, and
 * the result does not depend on the order.  e is chosen per call from Q*L*K * max|A| *
 * max|grad_output| (a bound on every element) so that no sum can overflow;
 * the resolution, that bound times 2^-60, is far below fp32 rounding.
 * grad_sampling_locations / grad_attention_weights (and the fused
 * gradients) are deterministic in every variant.
 *
 *   workspace   device scratch of msda_deterministic_workspace_bytes(B, S, M,
 *               D, Q, L, K, dtype) bytes (the int64 accumulator plus the scale
 *               words; 0 when the call takes the owner path, given 16-byte
 *               aligned grad_output and grad_value -- workspace may then be
 *               NULL; -1 for invalid sizes or dtype); its contents on entry
 *               do not matter.  With a misaligned grad_output the owner path
 *               is ruled out: pass the full B*S*M*D*8 + 64 bytes, or the
 *               call returns MSDA_ERR_INVALID_ARGUMENT before any launch.
 * Other arguments as in msda_backward / msda_fused_backward (no fp32
 * accumulator: the integer accumulator replaces it).
 */
int64_t msda_deterministic_workspace_bytes(int64_t batch, int64_t num_keys, int64_t num_heads,
                                           int64_t head_dim, int64_t num_queries,
                                           int64_t num_levels, int64_t num_points, int dtype);

int msda_backward_deterministic(const void* value, const int64_t* spatial_shapes,
                                const int64_t* level_start_index,
                                const void* sampling_locations, const void* attention_weights,
                                const void* grad_output, void* grad_value, void* workspace,
                                void* grad_sampling_locations, void* grad_attention_weights,
                                int64_t batch, int64_t num_keys, int64_t num_heads,
                                int64_t head_dim, int64_t num_queries, int64_t num_levels,
                                int64_t num_points, int dtype, void* stream);

int msda_fused_backward_deterministic(const void* value, const int64_t* spatial_shapes,
                                      const int64_t* level_start_index,
                                      const void* reference_points, const void* sampling_offsets,
                                      const void* attention_logits, const float* softmax_lse,
                                      const void* output, const void* grad_output,
                                      void* grad_value, void* workspace,
                                      void* grad_reference_points, void* grad_sampling_offsets,
                                      void* grad_attention_logits, int64_t batch,
                                      int64_t num_keys, int64_t num_heads, int64_t head_dim,
                                      int64_t num_queries, int64_t num_levels,
                                      int64_t num_points, int reference_levels, int dtype,
                                      void* stream);

/*
 * Projections either side of the operator.  They replace the four
 * nn.Linear calls of the reference's attention layer
 * (labs/solutions/lab00.py:199-201 value_proj / offset_proj / weight_proj,
 * :208 out_proj) and Deformable-DETR's masked_fill of padded value rows.
 *
 *   input   (rows, in_features)            dtype
 *   weight  (split, in_features)           dtype   output columns [0, split)
 *   weight2 (out - split, in_features)     dtype   columns [split, out); NULL if split == out
 *   bias / bias2 (split,) / (out - split,) dtype   nullable
 *   row_mask (rows,) uint8                 nullable; nonzero row -> output row 0
 *   output  (rows, split), output2 (rows, out - split)
 *
 * output = input weight^T + bias (row_mask rows zero), fp32 accumulation, one
 * rounding.  in_features (and, for the backward, split and out_features) must
 * be multiples of 16 bytes of the dtype; half precision takes reductions of
 * at most 512 (in_features forward, out_features for grad_input); the input,
 * weight and grad_output pointers must be 16-byte aligned.  Violations return
 * MSDA_ERR_UNSUPPORTED_SHAPE.  rows == 0 launches nothing.
 */
int msda_projection_forward(const void* input, const void* weight, const void* bias,
                            const void* weight2, const void* bias2, const uint8_t* row_mask,
                            void* output, void* output2, int64_t rows, int64_t in_features,
                            int64_t out_features, int64_t split, int dtype, void* stream);

/* Bytes of the workspace msda_projection_backward needs (the transposed
 * weights and the weight / bias gradients' fp32 partial sums; -1 for invalid
 * arguments). */
int64_t msda_projection_workspace_bytes(int64_t rows, int64_t in_features, int64_t out_features,
                                        int dtype);

/*
 * Backward of msda_projection_forward.  grad_output (rows, split) and
 * grad_output2 (rows, out - split) are the output gradients.  Every output is
 * nullable (skipped when NULL):
 *   grad_input   = [grad_output | grad_output2] [weight ; weight2], masked rows 0
 *   grad_weight  = grad_output^T input over unmasked rows, grad_weight2 likewise
 *   grad_bias    = column sums of grad_output over unmasked rows, grad_bias2 likewise
 * Every gradient, grad_input included, needs `workspace`
 * (msda_projection_workspace_bytes, 16-byte aligned, contents ignored; NULL
 * only when no gradient is asked for or rows == 0).  Weight / bias gradients
 * are fixed-order sums (no atomics), so every output is bitwise reproducible.  When grad_input and a weight or
 * bias gradient are both asked for, the weight/bias half runs on a second
 * stream of the library's (one per device, default priority, created on the
 * first such call), forked from and joined back into `stream` with events:
 * the call stays ordered on `stream` as a whole (and captures into a HIP
 * graph as two parallel branches).
 */
int msda_projection_backward(const void* input, const void* weight, const void* weight2,
                             const uint8_t* row_mask, const void* grad_output,
                             const void* grad_output2, void* grad_input, void* grad_weight,
                             void* grad_bias, void* grad_weight2, void* grad_bias2,
                             void* workspace, int64_t rows, int64_t in_features,
                             int64_t out_features, int64_t split, int dtype, void* stream);

/*
 * msda_projection_backward without the workspace argument: it allocates
 * nothing.  No counterpart in the reference; it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving or
 * training loops, harnesses that forbid hipMalloc).  The workspace is a
 * device array inside the library, 64 MiB per GPU, held by every GPU the
 * library runs on until the process ends; shapes whose workspace
 * (msda_projection_workspace_bytes) exceeds it return
 * MSDA_ERR_UNSUPPORTED_SHAPE.  Every call on one GPU uses that GPU's one
 * array: calls that overlap on one GPU (other streams, other threads) race
 * and give wrong results -- serialise them.  Arguments and results as in
 * msda_projection_backward (bitwise the same outputs); everything runs on
 * `stream` (no second stream).
 */
int msda_projection_backward_noalloc(const void* input, const void* weight, const void* weight2,
                                     const uint8_t* row_mask, const void* grad_output,
                                     const void* grad_output2, void* grad_input,
                                     void* grad_weight, void* grad_bias, void* grad_weight2,
                                     void* grad_bias2, int64_t rows, int64_t in_features,
                                     int64_t out_features, int64_t split, int dtype,
                                     void* stream);

/*
 * Human-readable text for a return code (static storage).  The reference has
 * no error channel below Python; this backs the RuntimeError that the host
 * raises for a non-zero code (src/msda_triton/ops.py:165-171 raise the
 * equivalent errors for a missing backend).
 */
const char* msda_error_string(int code);

/* Library ABI version, (major << 16) | minor. */
int msda_abi_version(void);

/*
 * Which way msda_backward / msda_fused_backward (deterministic == 0) or their
 * deterministic variants (deterministic != 0) form grad_value for these
 * sizes, assuming 16-byte aligned grad_output and grad_value (and, for the
 * binned path's bookkeeping, 256-byte aligned buffers, as torch allocates):
 * one of the MSDA_BACKWARD_* codes below, or minus an MSDA_ERR_* code for
 * sizes or a dtype the backward rejects.  Host-only (no device work); it
 * follows the same launch overrides (msda_set_launch_override) as the
 * backward.  No
 * counterpart in the reference, whose backward has a single kernel
 * (src/msda_triton/ops.py:76-92): it serves callers and benchmarks that
 * report which kernels ran.
 */
#define MSDA_BACKWARD_ATOMIC_DIRECT 0 /* zero-fill + direct atomic scatter */
#define MSDA_BACKWARD_ATOMIC_DEDUP 1  /* zero-fill + row-merging atomic kernel */
#define MSDA_BACKWARD_OWNER 2         /* row-owner kernel + scatter-free gradient kernel */
#define MSDA_BACKWARD_BINNED 3        /* samples binned by band of value rows, zero-fill,
                                         band sums + scatter-free gradient kernel */
int msda_backward_plan(int64_t batch, int64_t num_keys, int64_t num_heads, int64_t head_dim,
                       int64_t num_queries, int64_t num_levels, int64_t num_points, int dtype,
                       int deterministic);

/*
 * Launch-shape and path overrides, for sweeps and for tests that run every
 * kernel variant.  No counterpart in the reference, which picks its launch
 * configuration by Triton autotuning (src/msda_triton/kernels.py:54-65).
 * By default no knob is set and every call makes the automatic choice; the
 * library reads no environment variable.  The table is process-wide (every
 * device, every thread): set it before the calls it should affect.
 *   knob    one of the MSDA_KNOB_* codes below
 *   value   the knob's value, or MSDA_OVERRIDE_AUTO to restore the
 *           automatic choice
 * Returns MSDA_OK, or MSDA_ERR_INVALID_ARGUMENT for an unknown knob.
 */
#define MSDA_KNOB_FWD_TS 0      /* forward / scatter-free gradient: sample slots per pair */
#define MSDA_KNOB_FWD_CB 1      /* ... bytes per lane load, at most (16, 8, 4, 2) */
#define MSDA_KNOB_BWD_TS 2      /* atomic backward: sample slots per pair */
#define MSDA_KNOB_BWD_CB 3      /* atomic backward: bytes per lane load, at most */
#define MSDA_KNOB_BWD_PRIV 4    /* 0: direct atomic kernel instead of the row-dedup one */
#define MSDA_KNOB_BWD_OWNER 5   /* 0: no owner-computes backward */
#define MSDA_KNOB_BWD_BIN 6     /* 0: no binned backward */
#define MSDA_KNOB_OWN_MIX 7     /* owner launch order: 2 auto, 0 gradient workgroups last,
                                   1 first, -1 a launch of their own */
#define MSDA_KNOB_OWN_ROWS 8    /* owner path: rows per band, at most (64..2048) */
#define MSDA_KNOB_OWN_ENTRIES 9 /* owner path: corner entries per band the level split aims at */
#define MSDA_NUM_KNOBS 10
#define MSDA_OVERRIDE_AUTO (-2147483647 - 1)
int msda_set_launch_override(int knob, int value);

#ifdef __cplusplus
}
#endif

#endif /* MSDA_HIP_H_ */
