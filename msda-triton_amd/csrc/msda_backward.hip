// MSDA backward kernel for gfx950, plus the fill and cast kernels around it.
//
// Computes the reference's `_msda_backward_kernel`
// (src/msda_triton/kernels.py:166-291).  With g = grad_out[b,q,m,:] and the
// corner dot products G_c = <g, value[corner c]> (c = 00, 01, 10, 11):
//   grad_attn[p]    = sum_c w_c G_c                                (254-260)
//   grad_loc[p, x]  = A W ((1-ly)(G01 - G00) + ly (G11 - G10))     (264, 266)
//   grad_loc[p, y]  = A H ((1-lx)(G10 - G00) + lx (G11 - G01))     (265, 267)
//   grad_value[c]  += A w_c g            (atomic scatter, 278-291)
// The reference forms dx/dy per channel and then reduces; because every term
// is linear in the corner values, reducing the four corner dots first gives
// the same sums with 4 instead of ~15 operations per channel.
//
// Work decomposition mirrors the forward (see msda_forward.hip): sample
// records are staged in LDS by the whole workgroup, a pair is served by G*TS
// lanes, G lanes span one value row.  The four G_c are folded across the G
// chunk lanes with DPP, the per-sample results go back through LDS and leave
// as one coalesced store per pass.  The scatter (see Scatter below) issues
// buffer atomics whose lanes cover consecutive words of each corner row: fp32
// adds into an fp32 accumulator, or packed fp16 / bf16 adds straight into
// grad_value.  Out-of-map corners carry an out-of-range offset, so their
// atomics are dropped by the hardware.  The backward prefers 16 lanes per
// value row (4-byte gathers for a 64-byte bf16 row) and one sample slot per
// pair, so that one atomic instruction covers four full rows of four
// different (b, q, m) pairs.
//
// FUSED = true is the backward of the fused front-end (see msda_forward.hip).
// A sample's weight is A = softmax(logits)[s] = exp(logit - lse), its location
// ref + offset / (W, H), so
//   d/d(logit_s)  = A_s (grad_attn_s - delta),  delta = sum_s' A_s' grad_attn_s'
//   d/d(offset_s) = grad_loc_s / (W, H)         (the A*W, A*H factors cancel)
// and delta equals <grad_out[pair], out[pair]> (out = sum_s A_s sampled_s), a
// per-pair dot that each team computes from the saved forward output -- no
// reduction over the pair's levels is needed.  Reference points receive the
// sum of their samples' grad_loc in ref_grad_kernel below.
#include "msda_bwd_body.h"
#include "msda_launch.h"

namespace msda {

namespace {

// T: storage dtype.  A: accumulator dtype (F32, or T for in-place atomics).
template <class T, class A, int CB, int G, int TS, bool FUSED>
__global__ __launch_bounds__(kBlock) void bwd_kernel(Params p) {
  __shared__ BwdLds sm;
  bwd_body<T, A, CB, G, TS, FUSED>(p, xcd_remap(blockIdx.x, p.nblocks), sm);
}

template <class T, class A, int CB, int G, int TS, bool FUSED>
hipError_t launch_one(const Params& p, hipStream_t st) {
  hipLaunchKernelGGL((bwd_kernel<T, A, CB, G, TS, FUSED>), dim3(p.nblocks), dim3(kBlock), 0, st,
                     p);
  return hipGetLastError();
}

template <class T, class A, bool FUSED>
hipError_t dispatch(const Shape& s, const Params& p, hipStream_t st) {
  switch (s.cb * 10000 + s.g * 100 + s.ts) {
    case 40801: return launch_one<T, A, 4, 8, 1, FUSED>(p, st);
    case 41601: return launch_one<T, A, 4, 16, 1, FUSED>(p, st);
    case 41604: return launch_one<T, A, 4, 16, 4, FUSED>(p, st);
    case 81601: return launch_one<T, A, 8, 16, 1, FUSED>(p, st);
    case 161601: return launch_one<T, A, 16, 16, 1, FUSED>(p, st);
    case 160404: return launch_one<T, A, 16, 4, 4, FUSED>(p, st);
    case 160804: return launch_one<T, A, 16, 8, 4, FUSED>(p, st);
    default: break;
  }
  if (s.cb == 16) return launch_one<T, A, 16, 0, 0, FUSED>(p, st);
  if (s.cb == 8) return launch_one<T, A, 8, 0, 0, FUSED>(p, st);
  if (s.cb == 4) return launch_one<T, A, 4, 0, 0, FUSED>(p, st);
  if constexpr (T::kBytes == 2) {
    if (s.cb == 2) return launch_one<T, A, 2, 0, 0, FUSED>(p, st);
  }
  return hipErrorInvalidValue;
}

template <bool FUSED>
hipError_t dispatch_dtype(int dtype, AccMode acc, const Shape& s, const Params& p,
                          hipStream_t st) {
  if (acc == kAccNone) {
    switch (dtype) {
      case kF32: return dispatch<F32, NoAcc, FUSED>(s, p, st);
      case kF16: return dispatch<F16, NoAcc, FUSED>(s, p, st);
      case kBF16: return dispatch<BF16, NoAcc, FUSED>(s, p, st);
      default: return hipErrorInvalidValue;
    }
  }
  switch (dtype) {
    case kF32:
      return acc == kAccI64 ? dispatch<F32, I64, FUSED>(s, p, st)
                            : dispatch<F32, F32, FUSED>(s, p, st);
    case kF16:
      return acc == kAccI64   ? dispatch<F16, I64, FUSED>(s, p, st)
             : acc == kAccF32 ? dispatch<F16, F32, FUSED>(s, p, st)
                              : dispatch<F16, F16, FUSED>(s, p, st);
    case kBF16:
      return acc == kAccI64   ? dispatch<BF16, I64, FUSED>(s, p, st)
             : acc == kAccF32 ? dispatch<BF16, F32, FUSED>(s, p, st)
                              : dispatch<BF16, BF16, FUSED>(s, p, st);
    default: return hipErrorInvalidValue;
  }
}

// ---------------------------------------------------------------------------
// Fused front-end: gradient of the reference points.  A reference point
// moves every location built from it, so its gradient is the sum of those
// samples' d/d(loc) = (W_l, H_l) * d/d(offset), read back from the offset
// gradients the backward kernel stored.  One wave per (b, q): lane j covers
// the (m, k, coordinate) items j, j + 64, ... of one level at a time; since
// 64 is even a lane always holds the same coordinate (j & 1), and an xor
// butterfly over lane distances 2..32 (fixed order: deterministic) leaves the
// x sum in lane 0 and the y sum in lane 1.  Per-level reference points
// (B,Q,L,2) get one sum per level, shared ones (B,Q,2) one over all levels.
// ---------------------------------------------------------------------------
template <class T>
__global__ __launch_bounds__(kBlock) void ref_grad_kernel(Params p, uint64_t nbq) {
  __shared__ LevelTable lt;
  load_levels(p, lt);
  __syncthreads();
  const int lane = threadIdx.x % kWave;
  const uint64_t bq = (uint64_t)blockIdx.x * (kBlock / kWave) + threadIdx.x / kWave;
  if (bq >= nbq) return;  // whole waves
  const int n = p.M * p.K * 2;
  float acc = 0.f;
  for (int l = 0; l < p.L; ++l) {
    const float sc = (lane & 1) ? (float)lt.h[l] : (float)lt.w[l];
    for (int j = lane; j < n; j += kWave) {
      const uint32_t mk = (uint32_t)j >> 1;
      const uint32_t m = fdiv(mk, p.div_k);
      const uint32_t k = mk - m * (uint32_t)p.K;
      const uint64_t e =
          ((bq * (uint32_t)p.M + m) * (uint32_t)p.LK + (uint32_t)(l * p.K) + k) * 2 + (j & 1);
      acc += load1<T>(p.grad_loc, e) * sc;
    }
    if (p.ref_levels) {
      float v = acc;
#pragma unroll
      for (int d = 2; d < kWave; d <<= 1) v += __shfl_xor(v, d);
      if (lane < 2) store1<T>(p.grad_ref, (bq * (uint32_t)p.L + l) * 2 + lane, v);
      acc = 0.f;
    }
  }
  if (!p.ref_levels) {
#pragma unroll
    for (int d = 2; d < kWave; d <<= 1) acc += __shfl_xor(acc, d);
    if (lane < 2) store1<T>(p.grad_ref, bq * 2 + lane, acc);
  }
}

// ---------------------------------------------------------------------------
// Zero fill (a kernel rather than hipMemsetAsync so that captured graphs hold
// only kernel nodes) and the fp32 -> dtype cast of the fp32 accumulator.
// ---------------------------------------------------------------------------
// Bytes [0, nhead) and [tail, tail + ntail) are cleared one by one (an
// unaligned start or end), the 16-byte-aligned middle with two 16-byte stores
// per lane and iteration (measured fastest: 7.45 us for the decoder's 45.5 MB
// on 1024 workgroups, vs 7.9 us with one store on 8192).
__global__ __launch_bounds__(kBlock) void zero_kernel(uint8_t* head, int nhead, uint4* p,
                                                      uint64_t n16, uint8_t* tail, int ntail) {
  const uint64_t stride = (uint64_t)gridDim.x * kBlock * 2;
  for (uint64_t i = (uint64_t)blockIdx.x * kBlock * 2 + threadIdx.x; i < n16; i += stride) {
    p[i] = make_uint4(0u, 0u, 0u, 0u);
    if (i + kBlock < n16) p[i + kBlock] = make_uint4(0u, 0u, 0u, 0u);
  }
  if (blockIdx.x == 0 && (int)threadIdx.x < nhead) head[threadIdx.x] = 0;
  if (blockIdx.x == 0 && (int)threadIdx.x < ntail) tail[threadIdx.x] = 0;
}

template <class T>
__global__ __launch_bounds__(kBlock) void cast_kernel(const float* src, void* dst, uint64_t n) {
  const uint64_t stride = (uint64_t)gridDim.x * kBlock;
  const uint64_t n4 = n / 4;
  for (uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x; i < n4; i += stride) {
    const float4 v = reinterpret_cast<const float4*>(src)[i];
    reinterpret_cast<uint2*>(dst)[i] = make_uint2(pack2<T>(v.x, v.y), pack2<T>(v.z, v.w));
  }
  if (blockIdx.x == 0 && threadIdx.x < (n & 3)) {
    const uint64_t i = n4 * 4 + threadIdx.x;
    store1<T>(dst, i, src[i]);
  }
}

// Deterministic backward, before the scatter: max|A| (1 for softmax
// weights, attn == NULL) and max|grad_out| into det_max[0..1].  For
// non-negative floats the bit patterns order like the values, so an unsigned
// integer atomicMax gives the exact maximum whatever the order.  Atomics on
// one address serialise at the memory side, so each workgroup reduces first
// (wave xor butterfly, then LDS) and issues one atomic per word.
// max |x| over n elements of T at base, this thread's share (thread t of
// nt): element-wise up to the first 16-byte boundary, then 16-byte loads,
// four in flight per thread, then the tail.
template <class T>
__device__ __forceinline__ float absmax_range(const void* base, uint64_t n, uint64_t t,
                                              uint64_t nt) {
  float m = 0.f;
  if (base == nullptr || n == 0) return m;
  constexpr int kE = 16 / T::kBytes;  // elements per 16 bytes
  uint64_t head = ((16u - (reinterpret_cast<uintptr_t>(base) & 15u)) & 15u) / T::kBytes;
  if (head > n) head = n;
  for (uint64_t i = t; i < head; i += nt) m = fmaxf(m, fabsf(load1<T>(base, i)));
  const uint64_t nv = (n - head) / kE;
  const uint4* v = reinterpret_cast<const uint4*>(static_cast<const char*>(base) + head * T::kBytes);
  for (uint64_t i = t; i < nv; i += 4 * nt) {
    uint4 x[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) x[u] = i + u * nt < nv ? v[i + u * nt] : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const uint32_t w[4] = {x[u].x, x[u].y, x[u].z, x[u].w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        if constexpr (T::kBytes == 4) {
          m = fmaxf(m, fabsf(__uint_as_float(w[k])));
        } else {
          float lo, hi;
          unpack2<T>(w[k], lo, hi);
          m = fmaxf(m, fmaxf(fabsf(lo), fabsf(hi)));
        }
      }
    }
  }
  for (uint64_t i = head + nv * kE + t; i < n; i += nt) m = fmaxf(m, fabsf(load1<T>(base, i)));
  return m;
}

template <class T>
__global__ __launch_bounds__(kBlock) void det_max_kernel(const void* attn, uint64_t n_attn,
                                                         const void* gout, uint64_t n_gout,
                                                         uint32_t* det_max) {
  __shared__ float s_m[2][kBlock / kWave];
  const uint64_t nt = (uint64_t)gridDim.x * kBlock;
  const uint64_t t0 = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
  float ma = absmax_range<T>(attn, n_attn, t0, nt);
  const float mg = absmax_range<T>(gout, n_gout, t0, nt);
  if (attn == nullptr) ma = 1.f;
  float mgr = mg;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    ma = fmaxf(ma, __shfl_xor(ma, d));
    mgr = fmaxf(mgr, __shfl_xor(mgr, d));
  }
  const int wave = threadIdx.x / kWave;
  if (threadIdx.x % kWave == 0) {
    s_m[0][wave] = ma;
    s_m[1][wave] = mgr;
  }
  __syncthreads();
  if (threadIdx.x < 2) {
    float m = 0.f;
    for (int w = 0; w < kBlock / kWave; ++w) m = fmaxf(m, s_m[threadIdx.x][w]);
    atomicMax(&det_max[threadIdx.x], __float_as_uint(m));
  }
}

// Deterministic backward, after the scatter: grad_value = acc / scale,
// rounded once to the storage dtype.
template <class T>
__global__ __launch_bounds__(kBlock) void det_cast_kernel(Params p, const long long* acc,
                                                          void* dst, uint64_t n) {
  const double inv = 1.0 / (double)det_scale(p);
  const uint64_t stride = (uint64_t)gridDim.x * kBlock;
  for (uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
    store1<T>(dst, i, (float)((double)acc[i] * inv));
  }
}

int grid_for(uint64_t items) {
  // Enough workgroups to cover 256 CUs several times; grid-stride beyond.
  const uint64_t want = (items + kBlock - 1) / kBlock;
  return (int)(want < 8192 ? (want ? want : 1) : 8192);
}

}  // namespace

hipError_t launch_backward(int dtype, AccMode acc, bool fused, const Shape& s,
                           const Params& p, hipStream_t st) {
  return fused ? dispatch_dtype<true>(dtype, acc, s, p, st)
               : dispatch_dtype<false>(dtype, acc, s, p, st);
}

hipError_t launch_det_max(int dtype, const void* attn, uint64_t n_attn, const void* grad_out,
                          uint64_t n_gout, uint32_t* det_max, hipStream_t st) {
  const uint64_t n = n_attn > n_gout ? n_attn : n_gout;
  int grid = grid_for(n);
  if (grid > 256) grid = 256;
  switch (dtype) {
    case kF32:
      hipLaunchKernelGGL(det_max_kernel<F32>, dim3(grid), dim3(kBlock), 0, st, attn, n_attn,
                         grad_out, n_gout, det_max);
      break;
    case kF16:
      hipLaunchKernelGGL(det_max_kernel<F16>, dim3(grid), dim3(kBlock), 0, st, attn, n_attn,
                         grad_out, n_gout, det_max);
      break;
    case kBF16:
      hipLaunchKernelGGL(det_max_kernel<BF16>, dim3(grid), dim3(kBlock), 0, st, attn, n_attn,
                         grad_out, n_gout, det_max);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_det_cast(int dtype, const Params& p, const long long* acc, void* dst,
                           uint64_t n, hipStream_t st) {
  if (n == 0) return hipSuccess;
  const int grid = grid_for(n);
  switch (dtype) {
    case kF32:
      hipLaunchKernelGGL(det_cast_kernel<F32>, dim3(grid), dim3(kBlock), 0, st, p, acc, dst, n);
      break;
    case kF16:
      hipLaunchKernelGGL(det_cast_kernel<F16>, dim3(grid), dim3(kBlock), 0, st, p, acc, dst, n);
      break;
    case kBF16:
      hipLaunchKernelGGL(det_cast_kernel<BF16>, dim3(grid), dim3(kBlock), 0, st, p, acc, dst, n);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_ref_grad(int dtype, const Params& p, uint64_t nbq, hipStream_t st) {
  if (nbq == 0) return hipSuccess;
  const dim3 grid((unsigned)((nbq + kBlock / kWave - 1) / (kBlock / kWave)));
  switch (dtype) {
    case kF32: hipLaunchKernelGGL(ref_grad_kernel<F32>, grid, dim3(kBlock), 0, st, p, nbq); break;
    case kF16: hipLaunchKernelGGL(ref_grad_kernel<F16>, grid, dim3(kBlock), 0, st, p, nbq); break;
    case kBF16: hipLaunchKernelGGL(ref_grad_kernel<BF16>, grid, dim3(kBlock), 0, st, p, nbq); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_zero(void* ptr, uint64_t bytes, hipStream_t st) {
  if (bytes == 0) return hipSuccess;
  uint8_t* b = static_cast<uint8_t*>(ptr);
  // Unaligned head (pointers into the middle of a buffer), aligned middle, tail.
  uint64_t head = (16 - (reinterpret_cast<uintptr_t>(b) & 15)) & 15;
  if (head > bytes) head = bytes;
  const uint64_t n16 = (bytes - head) / 16;
  const uint64_t ntail = bytes - head - n16 * 16;
  uint64_t want = (n16 + 2 * kBlock - 1) / (2 * kBlock);
  const int grid = (int)(want < 1 ? 1 : want > 1024 ? 1024 : want);
  hipLaunchKernelGGL(zero_kernel, dim3(grid), dim3(kBlock), 0, st, b, (int)head,
                     reinterpret_cast<uint4*>(b + head), n16, b + head + n16 * 16, (int)ntail);
  return hipGetLastError();
}

hipError_t launch_cast(int dtype, const float* src, void* dst, uint64_t n, hipStream_t st) {
  if (n == 0) return hipSuccess;
  const int grid = grid_for(n / 4 ? n / 4 : 1);
  switch (dtype) {
    case kF16: hipLaunchKernelGGL(cast_kernel<F16>, dim3(grid), dim3(kBlock), 0, st, src, dst, n); break;
    case kBF16: hipLaunchKernelGGL(cast_kernel<BF16>, dim3(grid), dim3(kBlock), 0, st, src, dst, n); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace msda
