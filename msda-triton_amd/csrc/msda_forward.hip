// MSDA forward kernel for gfx950.
//
// Computes the reference's `_msda_forward_kernel`
// (src/msda_triton/kernels.py:58-163):
//   out[b,q,m,:] = sum_{l,k} A * sum_corners w_corner * value[b, row, m, :]
// with fp32 accumulation and one rounding to the storage dtype.
//
// Work decomposition (one workgroup = 256 lanes = 4 wave64):
//   * a workgroup owns `ppb` consecutive (b, q, m) pairs; their sampling
//     parameters are one contiguous run of memory;
//   * stage: each lane turns one sample into a record in LDS (4 corner byte
//     offsets + 4 fp32 weights A*w_corner), so the bilinear set-up is done once
//     per sample rather than once per channel chunk;
//   * gather: a pair is served by a team of G*TS lanes.  G lanes cover the D
//     channels of a value row with CB-byte buffer loads (16 B = 8 bf16 or 4
//     fp32), TS slots split the L*K samples, U samples per slot are kept in
//     flight (4 corner loads each);
//   * the TS partial sums are folded with DPP / permlane exchanges and slot 0
//     stores its CB bytes of the output row.
//
// FUSED = true is the fused MSDeformAttn front-end (labs/solutions/lab00.py:
// 194-208): the staging turns reference points, per-level pixel offsets and
// attention logits into locations and softmax weights, after a prologue that
// computes each pair's log-sum-exp (kept in LDS and, for the backward, in
// p.lse).  The (B,Q,M,L,K) locations and weights never exist in memory.
#include "msda_launch.h"

namespace msda {

namespace {

constexpr int kUnroll = 4;

template <class T, int CB, int G, int TS, bool FUSED>
__global__ __launch_bounds__(kBlock) void fwd_kernel(Params p) {
  using C = Chunk<T, CB>;
  constexpr int kVec = C::kVec;
  constexpr int kWords = C::kWords;
  constexpr bool kStatic = G > 0;

  __shared__ LevelTable lt;
  __shared__ uint4 s_off[kMaxRecords];
  __shared__ float4 s_w[kMaxRecords];
  __shared__ float s_lse[FUSED ? kBlock : 1];

  const int g = kStatic ? G : p.g_rt;
  const int ts = kStatic ? TS : p.ts_rt;
  const int team = g * ts;
  const int ppw = kWave / team;
  const int ppb = ppw * (kBlock / kWave);
  const int blk = xcd_remap(blockIdx.x, p.nblocks);
  const int pair0 = blk * ppb;

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int ch = lane & (g - 1);
  const int sl = (lane / g) & (ts - 1);
  const int pl = wave * ppw + lane / team;
  const int pair = pair0 + pl;
  const bool live = ch < p.g_real;
  const uint32_t chb = live ? (uint32_t)(ch * CB) : kDeadLaneBytes;

  // Fused: when a pair's L*K logits are staged in one pass by lanes of one
  // wave, its log-sum-exp is formed in the staging step itself (no separate
  // prologue round trip); otherwise by pair_lse first.
  const bool lse_inline = FUSED && p.npass == 1 && p.sch <= kWave;
  load_levels(p, lt);
  if constexpr (FUSED) {
    if (!lse_inline) pair_lse<T>(p, pair0, ppb, team, s_lse);
  }
  __syncthreads();

  const __amdgpu_buffer_rsrc_t rv = make_rsrc(p.value, p.value_bytes);
  float acc[kVec];
#pragma unroll
  for (int k = 0; k < kVec; ++k) acc[k] = 0.f;

  const int nrec = ppb * p.sch;
  const int nps = p.sch / ts;  // samples per slot per pass (uniform)
  const int rbase = pl * p.sch + sl;

  for (int pass = 0; pass < p.npass; ++pass) {
    for (int j = threadIdx.x; j < nrec; j += kBlock) {
      const int jp = j >> p.log2_sch;
      const int s = pass * p.sch + (j & (p.sch - 1));
      const int pr = pair0 + jp;
      const bool valid = pr < p.npairs && s < p.LK;
      float lse = 0.f;
      if constexpr (FUSED) {
        if (lse_inline) {
          // The pair's sch records sit on sch consecutive lanes of one wave.
          const float x = valid ? load1<T>(p.attn, (uint64_t)pr * (uint32_t)p.LK + s) : -INFINITY;
          float mx = x;
          for (int d = 1; d < p.sch; d <<= 1) mx = fmaxf(mx, __shfl_xor(mx, d));
          float z = valid ? expf(x - mx) : 0.f;
          for (int d = 1; d < p.sch; d <<= 1) z += __shfl_xor(z, d);
          lse = mx + logf(z);
          if (s == 0 && pr < p.npairs && p.lse != nullptr) p.lse[pr] = lse;
        } else {
          lse = s_lse[jp];
        }
      }
      const Sample q = make_sample<T, FUSED>(p, lt, (uint32_t)pr, (uint32_t)s, valid, lse);
      const float w1x = 1.f - q.lx, w1y = 1.f - q.ly;
      s_off[j] = make_uint4(q.off[0] * T::kBytes, q.off[1] * T::kBytes, q.off[2] * T::kBytes,
                            q.off[3] * T::kBytes);
      s_w[j] = make_float4(q.a * (w1x * w1y), q.a * (q.lx * w1y), q.a * (w1x * q.ly),
                           q.a * (q.lx * q.ly));
    }
    __syncthreads();

    for (int i = 0; i < nps; i += kUnroll) {
      uint32_t raw[kUnroll][4][kWords];
      float4 w[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        if (i + u < nps) {  // wave-uniform
          const int j = rbase + (i + u) * ts;
          const uint4 o = s_off[j];
          w[u] = s_w[j];
          C::load_raw(rv, o.x + chb, raw[u][0]);
          C::load_raw(rv, o.y + chb, raw[u][1]);
          C::load_raw(rv, o.z + chb, raw[u][2]);
          C::load_raw(rv, o.w + chb, raw[u][3]);
        }
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        if (i + u < nps) {
          float v0[kVec], v1[kVec], v2[kVec], v3[kVec];
          C::unpack(raw[u][0], v0);
          C::unpack(raw[u][1], v1);
          C::unpack(raw[u][2], v2);
          C::unpack(raw[u][3], v3);
#pragma unroll
          for (int k = 0; k < kVec; ++k) {
            acc[k] += w[u].x * v0[k] + w[u].y * v1[k] + w[u].z * v2[k] + w[u].w * v3[k];
          }
        }
      }
    }
    if (pass + 1 < p.npass) __syncthreads();
  }

#pragma unroll
  for (int k = 0; k < kVec; ++k) {
    if constexpr (kStatic) {
      acc[k] = xsum_range<G, G * TS / 2, G * TS>(acc[k]);
    } else {
      acc[k] = xsum_runtime(acc[k], g, team);
    }
  }
  if (sl == 0 && live && pair < p.npairs) {
    char* dst = static_cast<char*>(p.out) +
                ((uint64_t)pair * (uint32_t)p.D) * T::kBytes + (uint32_t)(ch * CB);
    C::store(dst, acc);
  }
}

template <class T, int CB, int G, int TS, bool FUSED>
hipError_t launch_one(const Params& p, hipStream_t st) {
  hipLaunchKernelGGL((fwd_kernel<T, CB, G, TS, FUSED>), dim3(p.nblocks), dim3(kBlock), 0, st, p);
  return hipGetLastError();
}

template <class T, bool FUSED>
hipError_t dispatch(const Shape& s, const Params& p, hipStream_t st) {
  switch (s.cb * 10000 + s.g * 100 + s.ts) {
    case 160201: return launch_one<T, 16, 2, 1, FUSED>(p, st);
    case 160204: return launch_one<T, 16, 2, 4, FUSED>(p, st);
    case 160216: return launch_one<T, 16, 2, 16, FUSED>(p, st);
    case 160401: return launch_one<T, 16, 4, 1, FUSED>(p, st);
    case 160404: return launch_one<T, 16, 4, 4, FUSED>(p, st);
    case 160416: return launch_one<T, 16, 4, 16, FUSED>(p, st);
    case 160801: return launch_one<T, 16, 8, 1, FUSED>(p, st);
    case 160804: return launch_one<T, 16, 8, 4, FUSED>(p, st);
    case 161601: return launch_one<T, 16, 16, 1, FUSED>(p, st);
    case 161604: return launch_one<T, 16, 16, 4, FUSED>(p, st);
    default: break;
  }
  if (s.cb == 16) return launch_one<T, 16, 0, 0, FUSED>(p, st);
  if (s.cb == 8) return launch_one<T, 8, 0, 0, FUSED>(p, st);
  if (s.cb == 4) return launch_one<T, 4, 0, 0, FUSED>(p, st);
  if constexpr (T::kBytes == 2) {
    if (s.cb == 2) return launch_one<T, 2, 0, 0, FUSED>(p, st);
  }
  return hipErrorInvalidValue;
}

template <bool FUSED>
hipError_t dispatch_dtype(int dtype, const Shape& s, const Params& p, hipStream_t st) {
  switch (dtype) {
    case kF32: return dispatch<F32, FUSED>(s, p, st);
    case kF16: return dispatch<F16, FUSED>(s, p, st);
    case kBF16: return dispatch<BF16, FUSED>(s, p, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_forward(int dtype, bool fused, const Shape& s, const Params& p,
                          hipStream_t st) {
  return fused ? dispatch_dtype<true>(dtype, s, p, st) : dispatch_dtype<false>(dtype, s, p, st);
}

}  // namespace msda
