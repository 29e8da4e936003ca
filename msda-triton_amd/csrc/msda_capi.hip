// C ABI of the MSDA operator: argument checks, batch slicing and launch-shape
// selection around the kernels in msda_forward.hip / msda_backward.hip.
// Declarations and the contract live in include/msda_hip.h.
#include <atomic>
#include <mutex>

#include "../../include/msda_hip.h"
#include "msda_launch.h"

namespace msda {

FastDiv make_fastdiv(uint32_t d) {
  FastDiv f;
  uint32_t l = 0;
  while ((1ull << l) < d) ++l;
  f.mul = (uint32_t)((((1ull << l) - d) << 32) / d + 1);
  f.shift = l;
  f.d = d;
  return f;
}

static int next_pow2(int x) {
  int p = 1;
  while (p < x) p <<= 1;
  return p;
}

static int log2i(int x) {
  int l = 0;
  while ((1 << l) < x) ++l;
  return l;
}

bool choose_shape(int row_bytes, int lk, int64_t npairs, bool backward, int ts_pref,
                  int cb_pref, Shape* out) {
  Shape s;
  // Widest lane chunk (<= 16 bytes) that divides the row.
  s.cb = row_bytes % 16 == 0 ? 16 : row_bytes % 8 == 0 ? 8 : row_bytes % 4 == 0 ? 4 : 2;
  // The backward wants >= 16 lanes per row (4-byte chunks at least) so that
  // its atomics cover whole 64-byte segments per instruction.
  if (backward)
    while (s.cb > 4 && row_bytes / s.cb < 16) s.cb >>= 1;
  while (cb_pref > 0 && s.cb > cb_pref && s.cb > 2) s.cb >>= 1;
  s.g_real = row_bytes / s.cb;
  s.g = next_pow2(s.g_real);
  if (s.g > kWave) return false;
  int ts_max = kWave / s.g;
  const int lk2 = next_pow2(lk);
  if (ts_max > lk2) ts_max = lk2;
  int ts;
  if (ts_pref > 0) {
    ts = next_pow2(ts_pref);
  } else if (backward) {
    // One slot: an atomic instruction then spans different (b, q, m) pairs,
    // whose rows differ, instead of neighbouring points of one query.
    ts = 1;
  } else {
    // Split a pair's samples over 4 slots unless one slot per pair already
    // yields >= 8192 waves (32 per CU).
    ts = npairs * s.g / kWave >= 8192 ? 1 : 4;
  }
  if (ts > ts_max) ts = ts_max;
  s.ts = ts;
  *out = s;
  return true;
}

void finish_params(const Shape& s, int max_records, Params* p) {
  const int team = s.g * s.ts;
  const int ppb = (kWave / team) * (kBlock / kWave);
  int sch = next_pow2(p->LK);
  if (sch > max_records / ppb) sch = max_records / ppb;
  p->sch = sch;
  p->log2_sch = log2i(sch);
  p->npass = (p->LK + sch - 1) / sch;
  p->nblocks = (p->npairs + ppb - 1) / ppb;
  p->g_real = s.g_real;
  p->g_rt = s.g;
  p->ts_rt = s.ts;
}

// Override table: 0 = automatic, else (value << 1) | 1.  Process-wide, set
// only through msda_set_launch_override; relaxed atomics, so a call racing
// a change sees either value of each knob.
static std::atomic<int64_t> g_override[kNumKnobs];

int launch_override(int knob, int dflt) {
  const int64_t v = g_override[knob].load(std::memory_order_relaxed);
  return (v & 1) ? (int)(v >> 1) : dflt;
}

bool launch_override_set(int knob) {
  return (g_override[knob].load(std::memory_order_relaxed) & 1) != 0;
}

// Slots per pair (power of two), upper bound on the bytes per lane load (16,
// 8, 4, 2; 0 = automatic), and the backward path switches (0 = off).
static int fwd_ts_pref() { return launch_override(MSDA_KNOB_FWD_TS, 0); }
static int bwd_ts_pref() { return launch_override(MSDA_KNOB_BWD_TS, 0); }
static int fwd_cb_pref() { return launch_override(MSDA_KNOB_FWD_CB, 0); }
static int bwd_cb_pref() { return launch_override(MSDA_KNOB_BWD_CB, 0); }
// Off: the direct backward instead of the row-dedup one.
static bool bwd_priv_enabled() { return launch_override(MSDA_KNOB_BWD_PRIV, 1) != 0; }
// Off: atomic (or binned) backward even where the owner-computes one applies.
static bool bwd_owner_enabled() { return launch_override(MSDA_KNOB_BWD_OWNER, 1) != 0; }
// Off: no binned owner path (the atomic kernels instead).
static bool bwd_bin_enabled() { return launch_override(MSDA_KNOB_BWD_BIN, 1) != 0; }
static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

static int elem_bytes(int dtype) { return dtype == kF32 ? 4 : 2; }

struct Dims {
  int64_t B, S, M, D, Q, L, K;
};

static int check_dims(const Dims& d, int dtype) {
  if (dtype != kF32 && dtype != kF16 && dtype != kBF16) return MSDA_ERR_UNSUPPORTED_DTYPE;
  if (d.B < 0 || d.S < 0 || d.M < 0 || d.D < 0 || d.Q < 0 || d.L < 0 || d.K < 0)
    return MSDA_ERR_INVALID_ARGUMENT;
  if (d.L > kMaxLevels) return MSDA_ERR_UNSUPPORTED_SHAPE;
  if (d.S >= (1ll << 31) || d.Q >= (1ll << 31) || d.M >= (1 << 16) || d.D >= (1 << 16) ||
      d.K >= (1 << 16))
    return MSDA_ERR_UNSUPPORTED_SHAPE;
  return MSDA_OK;
}

// Largest batch slice whose value / output / sample counts fit the 32-bit
// addressing of the kernels (0 if one batch element alone does not fit).
static int64_t slice_batch(const Dims& d) {
  const int64_t lim = (int64_t)kMaxSliceElems;
  int64_t bs = d.B;
  const int64_t per_val = d.S * d.M * d.D;
  const int64_t per_out = d.Q * d.M * d.D;
  const int64_t per_smp = d.Q * d.M * d.L * d.K;
  if (per_val > 0 && lim / per_val < bs) bs = lim / per_val;
  if (per_out > 0 && lim / per_out < bs) bs = lim / per_out;
  if (per_smp > 0 && lim / per_smp < bs) bs = lim / per_smp;
  return bs;
}

static int status(hipError_t e) { return e == hipSuccess ? MSDA_OK : MSDA_ERR_LAUNCH; }

static const char* at(const void* base, int64_t elems, int e) {
  return static_cast<const char*>(base) + elems * e;
}
static char* at(void* base, int64_t elems, int e) { return static_cast<char*>(base) + elems * e; }

// Binned owner path: batch slices of at most kBinMaxGroups (b, m, level)
// groups, each within the 32-bit slice limits, whose grad_loc / grad_attn
// and accumulator (acc, acc_e bytes per element) hold the slice's
// bookkeeping (bin_plan).  On success *bs_out is the slice size.  NULL
// buffers (msda_backward_plan): buffers at 256-byte aligned addresses are
// assumed, so the alignment padding is the one a torch allocation would see.
static bool binned_slices(const Dims& d, int e, void* grad_loc, void* grad_attn, void* acc,
                          int acc_e, int64_t* bs_out) {
  const int64_t per_b = d.M * d.L;
  int64_t bs = slice_batch(d);
  if (per_b <= 0 || per_b > kBinMaxGroups || bs <= 0) return false;
  if (bs > kBinMaxGroups / per_b) bs = kBinMaxGroups / per_b;
  for (int64_t b0 = 0; b0 < d.B; b0 += bs) {
    const int64_t nb = d.B - b0 < bs ? d.B - b0 : bs;
    const int64_t so = b0 * d.Q * d.M * d.L * d.K;
    void* gl = grad_loc ? at(grad_loc, so * 2, e)
                        : reinterpret_cast<void*>((uintptr_t)(so * 2 * e));
    void* ga = grad_attn ? at(grad_attn, so, e) : reinterpret_cast<void*>((uintptr_t)(so * e));
    const int64_t vo = b0 * d.S * d.M * d.D;
    void* ac = acc ? at(acc, vo, acc_e) : reinterpret_cast<void*>((uintptr_t)(vo * acc_e));
    BinArgs ba;
    if (!bin_plan(nb, d.Q, d.M, d.K, d.D, d.S, d.L, e, gl, ga, ac, acc_e, &ba)) return false;
  }
  *bs_out = bs;
  return true;
}

static void base_params(const Dims& d, int64_t b0, int64_t bs, int dtype, Params* p) {
  const int e = elem_bytes(dtype);
  p->S = (int32_t)d.S;
  p->M = (int32_t)d.M;
  p->D = (int32_t)d.D;
  p->Q = (int32_t)d.Q;
  p->L = (int32_t)d.L;
  p->K = (int32_t)d.K;
  p->LK = (int32_t)(d.L * d.K);
  p->MD = (int32_t)(d.M * d.D);
  p->npairs = (int32_t)(bs * d.Q * d.M);
  p->value_bytes = (uint32_t)(bs * d.S * d.M * d.D * e);
  p->gout_bytes = (uint32_t)(bs * d.Q * d.M * d.D * e);
  p->div_qm = make_fastdiv((uint32_t)(d.Q * d.M > 0 ? d.Q * d.M : 1));
  p->div_m = make_fastdiv((uint32_t)(d.M > 0 ? d.M : 1));
  p->div_k = make_fastdiv((uint32_t)(d.K > 0 ? d.K : 1));
  (void)b0;
}

// Fused front-end arguments (NULL when the call takes locations + weights).
struct FusedArgs {
  const void* ref;     // reference points
  float* lse;          // forward: output (may be NULL); backward: input
  const void* output;  // backward: the forward output
  void* grad_ref;      // backward: may be NULL
  int ref_levels;      // 0: (B, Q, 2); 1: (B, Q, L, 2)
};

static int forward_impl(const void* value, const int64_t* spatial_shapes,
                        const int64_t* level_start_index, const void* loc, const void* attn,
                        void* output, const Dims& d, int dtype, void* stream,
                        const FusedArgs* f) {
  int rc = check_dims(d, dtype);
  if (rc != MSDA_OK) return rc;
  const int64_t n_out = d.B * d.Q * d.M * d.D;
  if (n_out == 0) return MSDA_OK;
  const int64_t n_smp = d.B * d.Q * d.M * d.L * d.K;
  if (!output || (d.L > 0 && (!spatial_shapes || !level_start_index)) ||
      (n_smp > 0 && (!loc || !attn || (f && !f->ref))) || (d.B * d.S * d.M * d.D > 0 && !value))
    return MSDA_ERR_INVALID_ARGUMENT;
  const int e = elem_bytes(dtype);
  Shape sh;
  if (!choose_shape((int)(d.D * e), (int)(d.L * d.K), d.B * d.Q * d.M, false, fwd_ts_pref(),
                    fwd_cb_pref(), &sh))
    return MSDA_ERR_UNSUPPORTED_SHAPE;
  const int64_t bs = slice_batch(d);
  if (bs <= 0) return MSDA_ERR_UNSUPPORTED_SHAPE;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t ref_per_b = d.Q * (f && f->ref_levels ? d.L : 1) * 2;
  for (int64_t b0 = 0; b0 < d.B; b0 += bs) {
    const int64_t nb = d.B - b0 < bs ? d.B - b0 : bs;
    Params p = {};
    base_params(d, b0, nb, dtype, &p);
    const int64_t so = b0 * d.Q * d.M * d.L * d.K;
    p.value = value ? at(value, b0 * d.S * d.M * d.D, e) : nullptr;
    p.shapes = spatial_shapes;
    p.starts = level_start_index;
    p.loc = loc ? at(loc, so * 2, e) : nullptr;
    p.attn = attn ? at(attn, so, e) : nullptr;
    p.out = at(output, b0 * d.Q * d.M * d.D, e);
    if (f) {
      p.ref = f->ref ? at(f->ref, b0 * ref_per_b, e) : nullptr;
      p.lse = f->lse ? f->lse + b0 * d.Q * d.M : nullptr;
      p.ref_levels = f->ref_levels;
    }
    finish_params(sh, kMaxRecords, &p);
    rc = status(launch_forward(dtype, f != nullptr, sh, p, st));
    if (rc != MSDA_OK) return rc;
  }
  return MSDA_OK;
}

// deterministic: bitwise-reproducible grad_value -- the owner path where it
// applies, else int64 fixed-point accumulation in det_workspace (n_val * 8
// bytes followed by the two max words of the scale, det_scale).
static int backward_impl(const void* value, const int64_t* spatial_shapes,
                         const int64_t* level_start_index, const void* loc, const void* attn,
                         const void* grad_output, void* grad_value, float* grad_value_accum,
                         void* grad_loc, void* grad_attn, const Dims& d, int dtype, void* stream,
                         const FusedArgs* f, bool deterministic = false,
                         void* det_workspace = nullptr) {
  int rc = check_dims(d, dtype);
  if (rc != MSDA_OK) return rc;
  const int e = elem_bytes(dtype);
  const int64_t n_val = d.B * d.S * d.M * d.D;
  const int64_t n_smp = d.B * d.Q * d.M * d.L * d.K;
  const int64_t n_out = d.B * d.Q * d.M * d.D;
  if ((n_val > 0 && (!value || !grad_value)) ||
      (n_smp > 0 && (!loc || !attn || !grad_loc || !grad_attn)) ||
      (n_out > 0 && !grad_output) || (d.L > 0 && (!spatial_shapes || !level_start_index)))
    return MSDA_ERR_INVALID_ARGUMENT;
  if (f && n_smp > 0 && n_out > 0 && d.S > 0 && (!f->ref || !f->lse || !f->output))
    return MSDA_ERR_INVALID_ARGUMENT;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool compute = n_smp > 0 && n_out > 0 && d.S > 0;
  // Owner-computes grad_value (few samples per (b, m, level)): every element
  // stored once from an fp32 sum in a fixed order -- bitwise reproducible,
  // so it also serves the deterministic entry points -- and neither the
  // zero-fill, the fp32 scratch nor the deterministic workspace is used.
  Params own = {};
  base_params(d, 0, d.B, dtype, &own);
  const bool owner = compute && bwd_owner_enabled() && aligned16(grad_output) &&
                     aligned16(grad_value) && owner_plan(d.B, d.Q, d.K, d.D, d.S, d.L, e, &own);
  if (deterministic && !owner && !det_workspace && n_val > 0) return MSDA_ERR_INVALID_ARGUMENT;
  const bool det = deterministic && !owner && n_val > 0;
  bool ref_inline = false;  // fused: grad_ref formed by the backward workgroups
  // fp32 accumulation is only a separate path for half storage.
  const bool fp32_acc =
      !owner && !det && grad_value_accum != nullptr && dtype != kF32 && n_val > 0;
  // Binned owner path (many samples per (b, m, level)): every slice's
  // grad_loc / grad_attn must hold its bookkeeping (bin_plan).
  int64_t bs_bin = 0;
  const bool binned =
      compute && !owner && bwd_bin_enabled() &&
      binned_slices(d, e, grad_loc, grad_attn,
                    det ? det_workspace
                        : fp32_acc ? static_cast<void*>(grad_value_accum) : grad_value,
                    det ? 8 : fp32_acc ? 4 : e, &bs_bin);
  const AccMode mode = det ? kAccI64 : fp32_acc ? kAccF32 : kAccNative;
  void* acc = det ? det_workspace : fp32_acc ? static_cast<void*>(grad_value_accum) : grad_value;
  const int acc_e = det ? 8 : fp32_acc ? 4 : e;
  uint32_t* det_max =
      det ? reinterpret_cast<uint32_t*>(static_cast<char*>(det_workspace) + n_val * 8) : nullptr;

  if (!owner && !binned) {  // the binned path zeroes its accumulator after binning
    rc = status(launch_zero(acc, (uint64_t)(n_val * acc_e) + (det ? 8u : 0u), st));
    if (rc != MSDA_OK) return rc;
  } else if (det) {  // binned: only the two max words start at zero here
    rc = status(launch_zero(det_max, 8u, st));
    if (rc != MSDA_OK) return rc;
  }
  if (det && compute) {
    rc = status(launch_det_max(dtype, f ? nullptr : attn, f ? 0 : (uint64_t)n_smp, grad_output,
                               (uint64_t)n_out, det_max, st));
    if (rc != MSDA_OK) return rc;
  }
  const float det_samples = (float)(d.Q * d.L * d.K);
  if (n_smp > 0 && !compute) {
    // No channels or no keys: every sampled value is zero, so are the
    // location and weight gradients (and, fused, the offset, logit and
    // reference-point gradients: delta = <grad_out, 0> = 0).
    rc = status(launch_zero(grad_loc, (uint64_t)(n_smp * 2 * e), st));
    if (rc == MSDA_OK) rc = status(launch_zero(grad_attn, (uint64_t)(n_smp * e), st));
    if (rc != MSDA_OK) return rc;
  } else if (compute) {
    // The owner paths run the direct kernel without its scatter: no atomics
    // to spread over pairs, so it takes the forward's launch shape.
    // Binned path: 4 sample slots per pair by default (measured faster than
    // the forward's 1 for the encoder / pixel-decoder grids it serves).
    const bool no_scatter = owner || binned;
    const int ts_pref = !no_scatter ? bwd_ts_pref()
                        : binned && fwd_ts_pref() <= 0 ? 4 : fwd_ts_pref();
    Shape sh;
    if (!choose_shape((int)(d.D * e), (int)(d.L * d.K), d.B * d.Q * d.M, !no_scatter, ts_pref,
                      no_scatter ? fwd_cb_pref() : bwd_cb_pref(), &sh))
      return MSDA_ERR_UNSUPPORTED_SHAPE;
    const int64_t bs = binned ? bs_bin : slice_batch(d);
    if (bs <= 0) return MSDA_ERR_UNSUPPORTED_SHAPE;
    const int64_t ref_per_b = d.Q * (f && f->ref_levels ? d.L : 1) * 2;
    // Fused, owner path: the gradient workgroups also form grad_ref when
    // each holds whole queries and all their samples in one pass (then no
    // ref_grad_kernel launch).
    if (owner && f && f->grad_ref) {
      Params t = {};
      base_params(d, 0, bs, dtype, &t);
      finish_params(sh, kBwdRecords, &t);
      const int ppb = (kWave / (sh.g * sh.ts)) * (kBlock / kWave);
      ref_inline = t.npass == 1 && ppb % d.M == 0;
    }
    for (int64_t b0 = 0; b0 < d.B; b0 += bs) {
      const int64_t nb = d.B - b0 < bs ? d.B - b0 : bs;
      Params p = {};
      base_params(d, b0, nb, dtype, &p);
      const int64_t vo = b0 * d.S * d.M * d.D, so = b0 * d.Q * d.M * d.L * d.K;
      const int64_t oo = b0 * d.Q * d.M * d.D;
      p.value = at(value, vo, e);
      p.shapes = spatial_shapes;
      p.starts = level_start_index;
      p.loc = at(loc, so * 2, e);
      p.attn = at(attn, so, e);
      p.grad_out = at(grad_output, oo, e);
      p.grad_acc = at(acc, vo, acc_e);
      p.acc_bytes = (uint32_t)(nb * d.S * d.M * d.D * acc_e);
      p.grad_loc = at(grad_loc, so * 2, e);
      p.grad_attn = at(grad_attn, so, e);
      p.det_max = det_max;
      p.det_samples = det_samples;
      if (f) {
        if (ref_inline) {
          p.ref_inline = 1;
          p.grad_ref = at(f->grad_ref, b0 * ref_per_b, e);
        }
        p.ref = at(f->ref, b0 * ref_per_b, e);
        p.lse = f->lse + b0 * d.Q * d.M;
        p.out_fwd = at(f->output, oo, e);
        p.ref_levels = f->ref_levels;
      }
      if (binned) {
        BinArgs ba;
        if (!bin_plan(nb, d.Q, d.M, d.K, d.D, d.S, d.L, e, p.grad_loc, p.grad_attn, p.grad_acc,
                      acc_e, &ba))
          return MSDA_ERR_LAUNCH;  // checked for every slice above
        if (f) p.ref_bytes = (uint32_t)(nb * ref_per_b * e);
        finish_params(sh, kBwdRecords, &p);
        rc = status(launch_binned(dtype, f != nullptr, fp32_acc, det, p, ba, st));
        // grad_loc / grad_attn (their bookkeeping contents overwritten).
        if (rc == MSDA_OK) rc = status(launch_backward(dtype, kAccNone, f != nullptr, sh, p, st));
        if (rc != MSDA_OK) return rc;
        continue;
      }
      if (owner) {
        Params po = p;
        po.grad_acc = at(grad_value, vo, e);
        po.own_rows = own.own_rows;
        po.own_split = own.own_split;
        po.own_groups = own.own_groups;
        po.g_real = own.g_real;
        po.g_rt = own.g_rt;
        po.own_lg = own.own_lg;
        po.own_est = own.own_est;
        po.own_big = own.own_big;
        po.div_g = make_fastdiv((uint32_t)own.g_real);
        // Sweeps: 0 gradient workgroups last, 1 first, -1 a launch of their own.
        po.own_mix = launch_override(MSDA_KNOB_OWN_MIX, 2);
        if (f) po.ref_bytes = (uint32_t)(nb * ref_per_b * e);
        finish_params(sh, kBwdRecords, &p);
        // The owner launch carries the grad_loc / grad_attn workgroups when
        // they gather 16-byte chunks (the chunk size it is compiled for);
        // other shapes (sweep overrides) run them as a launch of their own.
        const bool merged = sh.cb == 16 && po.own_mix >= 0;
        Params pd = p;
        if (!merged) pd.nblocks = 0;
        rc = status(launch_owner(dtype, f != nullptr, po, pd, st));
        if (rc == MSDA_OK && !merged)
          rc = status(launch_backward(dtype, kAccNone, f != nullptr, sh, p, st));
        if (rc != MSDA_OK) return rc;
        continue;
      }
      finish_params(sh, kBwdRecords, &p);
      if (bwd_priv_enabled() && priv_supported(sh, (int)d.D, (int)d.K, e)) {
        priv_params(sh, e, &p);
        rc = status(launch_backward_priv(dtype, mode, f != nullptr, sh, p, st));
      } else {
        rc = status(launch_backward(dtype, mode, f != nullptr, sh, p, st));
      }
      if (rc != MSDA_OK) return rc;
    }
  }
  if (fp32_acc) {
    rc = status(launch_cast(dtype, grad_value_accum, grad_value, (uint64_t)n_val, st));
    if (rc != MSDA_OK) return rc;
  }
  if (det) {
    Params p = {};
    p.det_max = det_max;
    p.det_samples = det_samples;
    rc = status(launch_det_cast(dtype, p, static_cast<const long long*>(det_workspace),
                                grad_value, (uint64_t)n_val, st));
    if (rc != MSDA_OK) return rc;
  }
  if (f && f->grad_ref && !ref_inline) {
    const int64_t nbq = d.B * d.Q;
    if (compute) {
      Params p = {};
      base_params(d, 0, d.B, dtype, &p);
      p.shapes = spatial_shapes;
      p.starts = level_start_index;
      p.grad_loc = grad_loc;
      p.grad_ref = f->grad_ref;
      p.ref_levels = f->ref_levels;
      rc = status(launch_ref_grad(dtype, p, (uint64_t)nbq, st));
    } else {
      rc = status(launch_zero(f->grad_ref,
                              (uint64_t)(nbq * (f->ref_levels ? d.L : 1) * 2 * e), st));
    }
    if (rc != MSDA_OK) return rc;
  }
  return MSDA_OK;
}

}  // namespace msda

using namespace msda;

extern "C" int msda_forward(const void* value, const int64_t* spatial_shapes,
                            const int64_t* level_start_index, const void* sampling_locations,
                            const void* attention_weights, void* output, int64_t batch,
                            int64_t num_keys, int64_t num_heads, int64_t head_dim,
                            int64_t num_queries, int64_t num_levels, int64_t num_points,
                            int dtype, void* stream) {
  const Dims d{batch, num_keys, num_heads, head_dim, num_queries, num_levels, num_points};
  return forward_impl(value, spatial_shapes, level_start_index, sampling_locations,
                      attention_weights, output, d, dtype, stream, nullptr);
}

extern "C" int msda_backward(const void* value, const int64_t* spatial_shapes,
                             const int64_t* level_start_index, const void* sampling_locations,
                             const void* attention_weights, const void* grad_output,
                             void* grad_value, float* grad_value_accum,
                             void* grad_sampling_locations, void* grad_attention_weights,
                             int64_t batch, int64_t num_keys, int64_t num_heads,
                             int64_t head_dim, int64_t num_queries, int64_t num_levels,
                             int64_t num_points, int dtype, void* stream) {
  const Dims d{batch, num_keys, num_heads, head_dim, num_queries, num_levels, num_points};
  return backward_impl(value, spatial_shapes, level_start_index, sampling_locations,
                       attention_weights, grad_output, grad_value, grad_value_accum,
                       grad_sampling_locations, grad_attention_weights, d, dtype, stream,
                       nullptr);
}

extern "C" int msda_fused_forward(const void* value, const int64_t* spatial_shapes,
                                  const int64_t* level_start_index, const void* reference_points,
                                  const void* sampling_offsets, const void* attention_logits,
                                  void* output, float* softmax_lse, int64_t batch,
                                  int64_t num_keys, int64_t num_heads, int64_t head_dim,
                                  int64_t num_queries, int64_t num_levels, int64_t num_points,
                                  int reference_levels, int dtype, void* stream) {
  if (reference_levels != 0 && reference_levels != 1) return MSDA_ERR_INVALID_ARGUMENT;
  const Dims d{batch, num_keys, num_heads, head_dim, num_queries, num_levels, num_points};
  const FusedArgs f{reference_points, softmax_lse, nullptr, nullptr, reference_levels};
  return forward_impl(value, spatial_shapes, level_start_index, sampling_offsets,
                      attention_logits, output, d, dtype, stream, &f);
}

extern "C" int msda_fused_backward(const void* value, const int64_t* spatial_shapes,
                                   const int64_t* level_start_index, const void* reference_points,
                                   const void* sampling_offsets, const void* attention_logits,
                                   const float* softmax_lse, const void* output,
                                   const void* grad_output, void* grad_value,
                                   float* grad_value_accum, void* grad_reference_points,
                                   void* grad_sampling_offsets, void* grad_attention_logits,
                                   int64_t batch, int64_t num_keys, int64_t num_heads,
                                   int64_t head_dim, int64_t num_queries, int64_t num_levels,
                                   int64_t num_points, int reference_levels, int dtype,
                                   void* stream) {
  if (reference_levels != 0 && reference_levels != 1) return MSDA_ERR_INVALID_ARGUMENT;
  const Dims d{batch, num_keys, num_heads, head_dim, num_queries, num_levels, num_points};
  const FusedArgs f{reference_points, const_cast<float*>(softmax_lse), output,
                    grad_reference_points, reference_levels};
  return backward_impl(value, spatial_shapes, level_start_index, sampling_offsets,
                       attention_logits, grad_output, grad_value, grad_value_accum,
                       grad_sampling_offsets, grad_attention_logits, d, dtype, stream, &f);
}

extern "C" int64_t msda_deterministic_workspace_bytes(int64_t batch, int64_t num_keys,
                                                      int64_t num_heads, int64_t head_dim,
                                                      int64_t num_queries, int64_t num_levels,
                                                      int64_t num_points, int dtype) {
  const Dims d{batch, num_keys, num_heads, head_dim, num_queries, num_levels, num_points};
  if (check_dims(d, dtype) != MSDA_OK) return -1;
  // None on the owner path (16-byte aligned grad_output / grad_value assumed).
  if (msda_backward_plan(batch, num_keys, num_heads, head_dim, num_queries, num_levels,
                         num_points, dtype, 1) == MSDA_BACKWARD_OWNER)
    return 0;
  return batch * num_keys * num_heads * head_dim * 8 + 64;
}

extern "C" int msda_backward_deterministic(
    const void* value, const int64_t* spatial_shapes, const int64_t* level_start_index,
    const void* sampling_locations, const void* attention_weights, const void* grad_output,
    void* grad_value, void* workspace, void* grad_sampling_locations,
    void* grad_attention_weights, int64_t batch, int64_t num_keys, int64_t num_heads,
    int64_t head_dim, int64_t num_queries, int64_t num_levels, int64_t num_points, int dtype,
    void* stream) {
  const Dims d{batch, num_keys, num_heads, head_dim, num_queries, num_levels, num_points};
  return backward_impl(value, spatial_shapes, level_start_index, sampling_locations,
                       attention_weights, grad_output, grad_value, nullptr,
                       grad_sampling_locations, grad_attention_weights, d, dtype, stream, nullptr,
                       true, workspace);
}

extern "C" int msda_fused_backward_deterministic(
    const void* value, const int64_t* spatial_shapes, const int64_t* level_start_index,
    const void* reference_points, const void* sampling_offsets, const void* attention_logits,
    const float* softmax_lse, const void* output, const void* grad_output, void* grad_value,
    void* workspace, void* grad_reference_points, void* grad_sampling_offsets,
    void* grad_attention_logits, int64_t batch, int64_t num_keys, int64_t num_heads,
    int64_t head_dim, int64_t num_queries, int64_t num_levels, int64_t num_points,
    int reference_levels, int dtype, void* stream) {
  if (reference_levels != 0 && reference_levels != 1) return MSDA_ERR_INVALID_ARGUMENT;
  const Dims d{batch, num_keys, num_heads, head_dim, num_queries, num_levels, num_points};
  const FusedArgs f{reference_points, const_cast<float*>(softmax_lse), output,
                    grad_reference_points, reference_levels};
  return backward_impl(value, spatial_shapes, level_start_index, sampling_offsets,
                       attention_logits, grad_output, grad_value, nullptr, grad_sampling_offsets,
                       grad_attention_logits, d, dtype, stream, &f, true, workspace);
}

// ---------------------------------------------------------------------------
// Projections either side of the operator.
// ---------------------------------------------------------------------------

struct ProjDims {
  int64_t rows, in, out, split;
};

// Shared argument checks.  `epu`: elements per 16 bytes; row lengths and the
// output split must be multiples of it so every 16-byte load stays inside one
// row of one tensor.
static int check_proj(const ProjDims& d, int dtype) {
  if (dtype != kF32 && dtype != kF16 && dtype != kBF16) return MSDA_ERR_UNSUPPORTED_DTYPE;
  if (d.rows < 0 || d.in < 1 || d.out < 1 || d.split < 1 || d.split > d.out)
    return MSDA_ERR_INVALID_ARGUMENT;
  const int64_t epu = 16 / elem_bytes(dtype);
  if (d.in % epu != 0 || d.in >= (1 << 20) || d.out >= (1 << 20) || d.rows >= (1ll << 36))
    return MSDA_ERR_UNSUPPORTED_SHAPE;
  if (dtype != kF32 && d.in > proj_max_reduction(dtype)) return MSDA_ERR_UNSUPPORTED_SHAPE;
  return MSDA_OK;
}

extern "C" int msda_projection_forward(const void* input, const void* weight, const void* bias,
                                       const void* weight2, const void* bias2,
                                       const uint8_t* row_mask, void* output, void* output2,
                                       int64_t rows, int64_t in_features, int64_t out_features,
                                       int64_t split, int dtype, void* stream) {
  const ProjDims d{rows, in_features, out_features, split};
  int rc = check_proj(d, dtype);
  if (rc != MSDA_OK) return rc;
  const bool two = split < out_features;
  if (rows == 0) return MSDA_OK;
  if (!input || !weight || !output || (two && (!weight2 || !output2)))
    return MSDA_ERR_INVALID_ARGUMENT;
  if (!aligned16(input) || !aligned16(weight) || (two && !aligned16(weight2)))
    return MSDA_ERR_UNSUPPORTED_SHAPE;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int e = elem_bytes(dtype);
  const int64_t step = dtype == kF32 ? proj_max_reduction(dtype) : in_features;
  for (int64_t k0 = 0; k0 < in_features && rc == MSDA_OK; k0 += step) {
    const int64_t kc = in_features - k0 < step ? in_features - k0 : step;
    ProjArgs a{};
    a.a0 = at(input, k0, e);
    a.lda0 = in_features;
    a.ksplit = (int)kc;
    a.w0 = at(weight, k0, e);
    a.w1 = two ? at(weight2, k0, e) : nullptr;
    a.ldw = in_features;
    a.b0 = k0 == 0 ? bias : nullptr;
    a.b1 = k0 == 0 && two ? bias2 : nullptr;
    a.mask = row_mask;
    a.y0 = output;
    a.y1 = two ? output2 : nullptr;
    a.ldy0 = split;
    a.ldy1 = out_features - split;
    a.nsplit = (int)split;
    a.rows = rows;
    a.K = (int)kc;
    a.N = (int)out_features;
    rc = status(launch_projection(dtype, k0 > 0, a, st));
  }
  return rc;
}

// Workspace of the backward: the transposed weight [W; W2]^T (in x out, for
// grad_input), then the fp32 partials of the weight / bias gradients.
static int64_t wt_bytes(const ProjDims& d, int dtype) {
  return (d.in * d.out * elem_bytes(dtype) + 255) / 256 * 256;
}

extern "C" int64_t msda_projection_workspace_bytes(int64_t rows, int64_t in_features,
                                                   int64_t out_features, int dtype) {
  const ProjDims d{rows, in_features, out_features, out_features};
  if (check_proj(d, dtype) != MSDA_OK) return -1;
  return wt_bytes(d, dtype) +
         wgrad_workspace_bytes(rows, (int)out_features, (int)in_features, dtype);
}

// A second stream per device for the projection backward: the weight
// gradient (partials + fixed-order reduction) does not depend on grad_input,
// so it runs beside the transpose and the grad_input launch, forked from and
// joined back into the caller's stream with events (also under graph
// capture, where the two become parallel branches).  Default priority,
// non-blocking; created on a device's first such call made outside graph
// capture, and kept until the process ends.  The mutex covers the fork/join enqueue, so concurrent
// callers on one device share the stream without mixing their events.
constexpr int kSideMaxDevices = 64;
struct SideStream {
  hipStream_t s = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
};
static SideStream g_side[kSideMaxDevices];
static std::mutex g_side_mu;

static SideStream* side_stream_locked(hipStream_t caller) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kSideMaxDevices) return nullptr;
  // The caller's stream must belong to the current device (the side stream
  // is that device's); otherwise the call runs on the caller's stream alone.
  hipDevice_t sdev = -1;
  if (hipStreamGetDevice(caller, &sdev) != hipSuccess || sdev != dev) return nullptr;
  SideStream& ss = g_side[dev];
  if (!ss.s) {
    // Not created under graph capture (creation may be illegal there): a
    // first call made while capturing runs on the caller's stream alone.
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(caller, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone)
      return nullptr;
    hipStream_t s = nullptr;
    hipEvent_t f = nullptr, j = nullptr;
    if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) return nullptr;
    if (hipEventCreateWithFlags(&f, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&j, hipEventDisableTiming) != hipSuccess) {
      if (f) (void)hipEventDestroy(f);
      (void)hipStreamDestroy(s);
      return nullptr;
    }
    ss.fork = f;
    ss.join = j;
    ss.s = s;
  }
  return &ss;
}

// overlap: run the weight gradient on the side stream (msda_projection_backward);
// the allocation-free entry point runs everything on the caller's stream.
static int projection_backward_impl(const void* input, const void* weight, const void* weight2,
                                    const uint8_t* row_mask, const void* grad_output,
                                    const void* grad_output2, void* grad_input, void* grad_weight,
                                    void* grad_bias, void* grad_weight2, void* grad_bias2,
                                    void* workspace, int64_t rows, int64_t in_features,
                                    int64_t out_features, int64_t split, int dtype, void* stream,
                                    bool overlap) {
  const ProjDims d{rows, in_features, out_features, split};
  int rc = check_proj(d, dtype);
  if (rc != MSDA_OK) return rc;
  const bool two = split < out_features;
  const int64_t epu = 16 / elem_bytes(dtype);
  if (split % epu != 0 || out_features % epu != 0) return MSDA_ERR_UNSUPPORTED_SHAPE;
  if (dtype != kF32 && out_features > proj_max_reduction(dtype) && grad_input)
    return MSDA_ERR_UNSUPPORTED_SHAPE;
  const bool wgrad = grad_weight || grad_bias || (two && (grad_weight2 || grad_bias2));
  const bool dx = grad_input != nullptr && rows > 0;
  if ((rows > 0 && (!grad_output || (two && !grad_output2))) ||
      (dx && (!weight || (two && !weight2))) || ((dx || wgrad) && !workspace) ||
      (wgrad && rows > 0 && !input))
    return MSDA_ERR_INVALID_ARGUMENT;
  if ((rows > 0 && (!aligned16(grad_output) || (two && !aligned16(grad_output2)))) ||
      (wgrad && rows > 0 && !aligned16(input)) || ((dx || wgrad) && !aligned16(workspace)))
    return MSDA_ERR_UNSUPPORTED_SHAPE;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int e = elem_bytes(dtype);
  char* wt = static_cast<char*>(workspace);
  float* partials = reinterpret_cast<float*>(wt + wt_bytes(d, dtype));

  // Weight and bias gradients: on the side stream when both halves run.
  std::unique_lock<std::mutex> lock(g_side_mu, std::defer_lock);
  SideStream* side = nullptr;
  if (overlap && dx && wgrad) {
    lock.lock();
    side = side_stream_locked(st);
    if (side && (hipEventRecord(side->fork, st) != hipSuccess ||
                 hipStreamWaitEvent(side->s, side->fork, 0) != hipSuccess))
      return MSDA_ERR_LAUNCH;
  }
  if (wgrad) {
    WgradArgs w{};
    wgrad_plan(rows, (int)out_features, (int)in_features, dtype, &w);
    w.g0 = grad_output;
    w.g1 = two ? grad_output2 : nullptr;
    w.ldg0 = split;
    w.ldg1 = out_features - split;
    w.nsplit = (int)split;
    w.x = input;
    w.ldx = in_features;
    w.mask = row_mask;
    w.ws = partials;
    w.wsb = (grad_bias || (two && grad_bias2))
                ? w.ws + (int64_t)w.nchunks * out_features * in_features
                : nullptr;
    rc = status(launch_wgrad(dtype, w, grad_weight, two ? grad_weight2 : nullptr, grad_bias,
                             two ? grad_bias2 : nullptr, side ? side->s : st));
  }

  // grad_input = [g | g2] [W ; W2] = [g | g2] wt^T with wt = [W ; W2]^T
  // (in x out): proj_kernel over the output features as its reduction,
  // segment 0 from grad_output, segment 1 from grad_output2; fp32 splits it
  // into launches of <= 256 that accumulate.
  if (dx && rc == MSDA_OK) {
    rc = status(launch_transpose(dtype, weight, two ? weight2 : nullptr, (int)split,
                                 (int)out_features, (int)in_features, wt, st));
    const int64_t step = dtype == kF32 ? proj_max_reduction(dtype) : out_features;
    for (int64_t k0 = 0; k0 < out_features && rc == MSDA_OK; k0 += step) {
      const int64_t k1 = k0 + step < out_features ? k0 + step : out_features;
      ProjArgs a{};
      if (k1 <= split) {
        a.a0 = at(grad_output, k0, e);
        a.lda0 = split;
        a.ksplit = (int)(k1 - k0);
      } else if (k0 >= split) {
        a.a0 = at(grad_output2, k0 - split, e);
        a.lda0 = out_features - split;
        a.ksplit = (int)(k1 - k0);
      } else {
        a.a0 = at(grad_output, k0, e);
        a.lda0 = split;
        a.a1 = grad_output2;
        a.lda1 = out_features - split;
        a.ksplit = (int)(split - k0);
      }
      a.w0 = wt + k0 * e;
      a.ldw = out_features;
      a.mask = row_mask;
      a.y0 = grad_input;
      a.ldy0 = in_features;
      a.nsplit = (int)in_features;
      a.rows = rows;
      a.K = (int)(k1 - k0);
      a.N = (int)in_features;
      rc = status(launch_projection(dtype, k0 > 0, a, st));
    }
  }
  if (side) {  // join: the caller's stream waits for the weight gradient
    if (hipEventRecord(side->join, side->s) != hipSuccess ||
        hipStreamWaitEvent(st, side->join, 0) != hipSuccess)
      rc = MSDA_ERR_LAUNCH;
  }
  return rc;
}

extern "C" int msda_projection_backward(const void* input, const void* weight,
                                        const void* weight2, const uint8_t* row_mask,
                                        const void* grad_output, const void* grad_output2,
                                        void* grad_input, void* grad_weight, void* grad_bias,
                                        void* grad_weight2, void* grad_bias2, void* workspace,
                                        int64_t rows, int64_t in_features, int64_t out_features,
                                        int64_t split, int dtype, void* stream) {
  return projection_backward_impl(input, weight, weight2, row_mask, grad_output, grad_output2,
                                  grad_input, grad_weight, grad_bias, grad_weight2, grad_bias2,
                                  workspace, rows, in_features, out_features, split, dtype, stream,
                                  true);
}

// ---------------------------------------------------------------------------
// Projection backward without allocation: the workspace lives in the
// library's own device memory.
// ---------------------------------------------------------------------------

// The workspace of msda_projection_backward_noalloc: a file-scope device
// array, so every GPU the library runs on holds one copy of it from module
// load until the process ends.  64 MiB covers every half-precision
// projection the library takes (reductions of at most 512: ~35 MB at 512 x
// 512 on 256 CUs) and fp32 ones up to 512 x 512.
constexpr int64_t kNoAllocScratchBytes = (int64_t)64 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

// Device address of `scratch` on each device.  In host code the array's
// name is a host-side stand-in, not a device address: kernels and copies
// get these addresses, looked up once per device with that device current.
constexpr int kNoAllocMaxDevices = 64;
static std::atomic<void*> g_scratch_addr[kNoAllocMaxDevices];
static std::mutex g_scratch_mu;

static void* scratch_address() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kNoAllocMaxDevices) return nullptr;
  void* ptr = g_scratch_addr[dev].load(std::memory_order_acquire);
  if (ptr) return ptr;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  ptr = g_scratch_addr[dev].load(std::memory_order_relaxed);
  if (!ptr) {
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return nullptr;
    g_scratch_addr[dev].store(ptr, std::memory_order_release);
  }
  return ptr;
}

extern "C" int msda_projection_backward_noalloc(
    const void* input, const void* weight, const void* weight2, const uint8_t* row_mask,
    const void* grad_output, const void* grad_output2, void* grad_input, void* grad_weight,
    void* grad_bias, void* grad_weight2, void* grad_bias2, int64_t rows, int64_t in_features,
    int64_t out_features, int64_t split, int dtype, void* stream) {
  const ProjDims d{rows, in_features, out_features, split};
  const int rc = check_proj(d, dtype);
  if (rc != MSDA_OK) return rc;
  const bool two = split < out_features;
  const bool wgrad = grad_weight || grad_bias || (two && (grad_weight2 || grad_bias2));
  const bool dx = grad_input != nullptr && rows > 0;
  void* ws = nullptr;
  if (dx || wgrad) {
    if (msda_projection_workspace_bytes(rows, in_features, out_features, dtype) >
        kNoAllocScratchBytes)
      return MSDA_ERR_UNSUPPORTED_SHAPE;
    ws = scratch_address();
    if (!ws) return MSDA_ERR_LAUNCH;
  }
  return projection_backward_impl(input, weight, weight2, row_mask, grad_output, grad_output2,
                                  grad_input, grad_weight, grad_bias, grad_weight2, grad_bias2, ws,
                                  rows, in_features, out_features, split, dtype, stream, false);
}

extern "C" const char* msda_error_string(int code) {
  switch (code) {
    case MSDA_OK: return "success";
    case MSDA_ERR_INVALID_ARGUMENT: return "invalid argument (negative size or NULL pointer)";
    case MSDA_ERR_UNSUPPORTED_DTYPE: return "unsupported dtype (expected fp32, fp16 or bf16)";
    case MSDA_ERR_UNSUPPORTED_SHAPE:
      return "unsupported shape (more than 64 levels, head_dim row wider than one wave, one "
             "batch element beyond 2^28 elements; projections: feature counts not a multiple of "
             "16 bytes, a half-precision reduction longer than 512, or a pointer not 16-byte "
             "aligned)";
    case MSDA_ERR_LAUNCH: return "HIP kernel launch failed";
    default: return "unknown msda error code";
  }
}

extern "C" int msda_abi_version(void) { return (1 << 16) | 5; }

static_assert(MSDA_NUM_KNOBS == kNumKnobs, "knob table");

extern "C" int msda_set_launch_override(int knob, int value) {
  if (knob < 0 || knob >= kNumKnobs) return MSDA_ERR_INVALID_ARGUMENT;
  const int64_t v = value == MSDA_OVERRIDE_AUTO ? 0 : ((int64_t)value * 2) | 1;
  g_override[knob].store(v, std::memory_order_relaxed);
  return MSDA_OK;
}

extern "C" int msda_backward_plan(int64_t batch, int64_t num_keys, int64_t num_heads,
                                  int64_t head_dim, int64_t num_queries, int64_t num_levels,
                                  int64_t num_points, int dtype, int deterministic) {
  const Dims d{batch, num_keys, num_heads, head_dim, num_queries, num_levels, num_points};
  const int rc = check_dims(d, dtype);
  if (rc != MSDA_OK) return -rc;
  const int e = elem_bytes(dtype);
  const bool compute = d.B * d.Q * d.M * d.L * d.K > 0 && d.B * d.Q * d.M * d.D > 0 && d.S > 0;
  Params own = {};
  base_params(d, 0, d.B, dtype, &own);
  if (compute && bwd_owner_enabled() && owner_plan(d.B, d.Q, d.K, d.D, d.S, d.L, e, &own))
    return MSDA_BACKWARD_OWNER;
  int64_t bs_bin = 0;
  if (compute && bwd_bin_enabled() &&
      binned_slices(d, e, nullptr, nullptr, nullptr, deterministic ? 8 : e, &bs_bin))
    return MSDA_BACKWARD_BINNED;
  Shape sh;
  if (compute && !choose_shape((int)(d.D * e), (int)(d.L * d.K), d.B * d.Q * d.M, true,
                               bwd_ts_pref(), bwd_cb_pref(), &sh))
    return -MSDA_ERR_UNSUPPORTED_SHAPE;
  if (compute && bwd_priv_enabled() && priv_supported(sh, (int)d.D, (int)d.K, e))
    return MSDA_BACKWARD_ATOMIC_DEDUP;
  return MSDA_BACKWARD_ATOMIC_DIRECT;
}
