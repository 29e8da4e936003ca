// Host-side launch plumbing shared by the forward/backward translation units
// and the C ABI (msda_capi.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "msda_device.h"

namespace msda {

// Launch shape of one kernel call: CB bytes per lane load, G lanes per value
// row (power of two, g_real of them live), TS sample slots per (b, q, m) pair.
struct Shape {
  int cb;
  int g;
  int g_real;
  int ts;
};

FastDiv make_fastdiv(uint32_t d);

// Launch-shape and path overrides (msda_set_launch_override; sweeps and the
// tests that run every kernel variant).  Knob ids are the MSDA_KNOB_* codes
// of the header.  A call that nobody has overridden reads one relaxed atomic
// per knob it consults and gets `dflt`.
constexpr int kNumKnobs = 10;
int launch_override(int knob, int dflt);
bool launch_override_set(int knob);

// Picks CB/G for a row of `row_bytes` and the slot count TS for LK samples
// over `npairs` (b, q, m) pairs; *_pref > 0 override the choice (sweeps).
// Returns false if the row is too wide for one wave.
bool choose_shape(int row_bytes, int lk, int64_t npairs, bool backward, int ts_pref,
                  int cb_pref, Shape* out);

// Fills the pass/record fields of `p` for shape `s` (sch, npass, nblocks)
// for a kernel that stages at most `max_records` samples per pass.
void finish_params(const Shape& s, int max_records, Params* p);

// grad_value accumulator of the backward: the storage dtype's own atomics,
// an fp32 scratch, int64 fixed point (deterministic; see det_scale), or none
// (grad_loc / grad_attn only, grad_value written by the owner kernel).
enum AccMode : int { kAccNative = 0, kAccF32 = 1, kAccI64 = 2, kAccNone = 3 };

// `fused`: the fused front-end variants (offsets + logits instead of
// locations + weights; see Params).
hipError_t launch_forward(int dtype, bool fused, const Shape& s, const Params& p,
                          hipStream_t st);
hipError_t launch_backward(int dtype, AccMode acc, bool fused, const Shape& s,
                           const Params& p, hipStream_t st);
// Row-dedup backward (msda_backward_priv.hip).
bool priv_supported(const Shape& s, int D, int K, int elem_bytes);
void priv_params(const Shape& s, int elem_bytes, Params* p);
hipError_t launch_backward_priv(int dtype, AccMode acc, bool fused, const Shape& s,
                                const Params& p, hipStream_t st);
// Owner-computes grad_value (msda_backward_owner.hip): every element written
// once with plain stores, no atomics and no zero-fill; for calls with few
// samples per (b, m, level).  owner_plan fills the owner fields of `p` and
// returns false when the call does not qualify.
bool owner_plan(int64_t B, int64_t Q, int64_t K, int64_t D, int64_t S, int64_t L,
                int elem_bytes, Params* p);
// One launch: the owner workgroups (params p) followed by pd.nblocks
// workgroups computing grad_loc / grad_attn (params pd, runtime shape).
hipError_t launch_owner(int dtype, bool fused, const Params& p, const Params& pd,
                        hipStream_t st);
// Binned owner backward (msda_backward_binned.hip): grad_value for calls
// with many samples per (b, m, level), summed per band of value rows in LDS.
// Its bookkeeping lives in the call's grad_loc / grad_attn buffers, which
// the gradient kernel overwrites afterwards.
constexpr int kBinAccFloats = 8192;  // fp32 band accumulator: P * D floats (32 KB)
constexpr int kBinMaxBands = 4096;   // bands per level
constexpr int kBinMaxGroups = 1024;  // (b, m, level) groups per launch
constexpr int kBinChunk = 4096;      // entries per work item (at most, unless items run short)
struct BinArgs {
  uint32_t* entries;  // [group][Q*K] sample ids q*K + k, by key (in grad_loc)
  uint32_t* mat;      // [group][nqb][nbmax] per sample block: its samples per key,
                      // then their first slot within the key (in the accumulator)
  uint32_t* cursors;  // [group][nbmax] first entry of each key
  uint32_t* nitems;   // [group] work items
  uint32_t* next;     // [8] work-item counters of bin_acc_kernel, one per XCD (zeroed by
                      // bin_scan_kernel)
  uint4* items;       // [group][cap] (band | split << 31, first entry, end entry, 0)
  uint32_t loc_bytes, attn_bytes;
  int32_t ngroups, nbmax, cap, nqb, log2p, log2k, chunk;  // bands of 2^log2p pixels
};
// Fills `a` for a slice of B batches; false when the shapes or the buffers
// (size, alignment) do not suit the path.  `acc` (B*S*M*D elements of
// acc_elem_bytes: grad_value or the fp32 scratch) holds the count matrix
// during the binning.
bool bin_plan(int64_t B, int64_t Q, int64_t M, int64_t K, int64_t D, int64_t S, int64_t L,
              int elem_bytes, void* grad_loc, void* grad_attn, void* acc, int acc_elem_bytes,
              BinArgs* a);
// Bins the samples, zeroes p.grad_acc (the accumulator: grad_value, or the
// fp32 scratch when f32acc, fp32 for fp32 dtype; det: the int64 fixed-point
// accumulator of the deterministic backward, scale from p.det_max) and sums
// the bands into it.
hipError_t launch_binned(int dtype, bool fused, bool f32acc, bool det, const Params& p,
                         const BinArgs& a, hipStream_t st);
// Fused front-end: reference-point gradient from the offset gradients, one
// wave per (b, q) of the nbq in the call.
hipError_t launch_ref_grad(int dtype, const Params& p, uint64_t nbq, hipStream_t st);
hipError_t launch_zero(void* ptr, uint64_t bytes, hipStream_t st);
hipError_t launch_cast(int dtype, const float* src, void* dst, uint64_t n, hipStream_t st);
// Deterministic backward: max|A| (or 1 for softmax weights, `attn` NULL) and
// max|grad_out| into det_max[0..1] (zeroed beforehand), then, after the
// backward kernel, the int64 accumulator rounded into grad_value.
hipError_t launch_det_max(int dtype, const void* attn, uint64_t n_attn, const void* grad_out,
                          uint64_t n_gout, uint32_t* det_max, hipStream_t st);
hipError_t launch_det_cast(int dtype, const Params& p, const long long* acc, void* dst,
                           uint64_t n, hipStream_t st);

// ---------------------------------------------------------------------------
// Projections either side of the operator (msda_proj.hip).
// y(r, c) = sum_k A(r, k) W(c, k) (+ bias, masked rows zero); see proj_kernel.
struct ProjArgs {
  const void* a0;
  const void* a1;
  int64_t lda0, lda1;
  int ksplit;  // reduction index k >= ksplit reads a1
  const void* w0;
  const void* w1;
  int64_t ldw;
  const void* b0;  // nullable
  const void* b1;  // nullable
  const uint8_t* mask;  // nullable, one byte per row
  void* y0;
  void* y1;
  int64_t ldy0, ldy1;
  int nsplit;  // output column c >= nsplit reads w1 / b1 and goes to y1
  int64_t rows;
  int K, N;
  // Set per row slice by launch_projection (buffer ranges, 32-bit).
  int nblocks;
  uint32_t abytes0, abytes1, ybytes0, ybytes1;
};
// Largest reduction length one launch takes (fp32 callers split larger ones
// into launches that accumulate).
int proj_max_reduction(int dtype);
hipError_t launch_projection(int dtype, bool accumulate, const ProjArgs& a, hipStream_t st);
// wt (N x K) = [w0; w1]^T, w0 rows [0, ksplit), w1 rows [ksplit, K), both N wide.
hipError_t launch_transpose(int dtype, const void* w0, const void* w1, int ksplit, int K, int N,
                            void* wt, hipStream_t st);

struct WgradArgs {
  const void* g0;
  const void* g1;
  int64_t ldg0, ldg1;
  int nsplit;
  const void* x;
  int64_t ldx;
  const uint8_t* mask;
  float* ws;   // [nchunks][N][K]
  float* wsb;  // [nchunks][N], NULL: no bias gradient
  int64_t rows;
  int K, N;
  int nchunks;
  int64_t rows_per_chunk;
  int ntile_n, ntile_k;
  int nset;  // steps in flight per workgroup: 4 (one workgroup per CU) or 2 (two)
};
void wgrad_plan(int64_t rows, int n, int k, int dtype, WgradArgs* a);
int64_t wgrad_workspace_bytes(int64_t rows, int n, int k, int dtype);
hipError_t launch_wgrad(int dtype, const WgradArgs& a, void* dw0, void* dw1, void* db0, void* db1,
                        hipStream_t st);

}  // namespace msda
