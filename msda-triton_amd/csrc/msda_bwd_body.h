// Body of the direct MSDA backward (bwd_kernel in msda_backward.hip), as a
// device function over an LDS struct so that another kernel can run it for
// some of its workgroups (the owner backward computes grad_loc / grad_attn
// this way, NoAcc, in the same launch as grad_value).
//
// Computes the reference's `_msda_backward_kernel`
// (src/msda_triton/kernels.py:166-291); the formulas and the work
// decomposition are described in msda_backward.hip.
#pragma once

#include "msda_scatter.h"

namespace msda {

constexpr int kBwdUnroll = 4;

struct BwdLds {
  LevelTable lt;
  uint4 s_off[kBwdRecords];
  float4 s_geo[kBwdRecords];  // lx, ly, A, -
  float2 s_scl[kBwdRecords];  // A*W, A*H
  float4 s_res[kBwdRecords];  // grad_attn, grad_x, grad_y, -
};

// T: storage dtype.  A: accumulator dtype (F32, or T for in-place atomics;
// NoAcc: no scatter).  `blk` is the workgroup's logical block.
template <class T, class A, int CB, int G, int TS, bool FUSED>
__device__ __forceinline__ void bwd_body(const Params& p, int blk, BwdLds& sm) {
  using C = Chunk<T, CB>;
  constexpr int kVec = C::kVec;
  constexpr int kWords = C::kWords;
  constexpr bool kStatic = G > 0;
  // NoAcc: grad_loc / grad_attn only (grad_value comes from the owner kernel).
  constexpr bool kScatter = A::kBytes > 0;
  // Accumulator byte offset = value byte offset * kAccScale.
  constexpr uint32_t kAccScale = A::kBytes / T::kBytes;

  LevelTable& lt = sm.lt;
  uint4* const s_off = sm.s_off;
  float4* const s_geo = sm.s_geo;
  float2* const s_scl = sm.s_scl;
  float4* const s_res = sm.s_res;

  const int g = kStatic ? G : p.g_rt;
  const int ts = kStatic ? TS : p.ts_rt;
  const int team = g * ts;
  const int ppw = kWave / team;
  const int ppb = ppw * (kBlock / kWave);
  const int pair0 = blk * ppb;

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int ch = lane & (g - 1);
  const int sl = (lane / g) & (ts - 1);
  const int pl = wave * ppw + lane / team;
  const int pair = pair0 + pl;
  const bool live = ch < p.g_real;
  const uint32_t chb = live ? (uint32_t)(ch * CB) : kDeadLaneBytes;

  load_levels(p, lt);

  const __amdgpu_buffer_rsrc_t rv = make_rsrc(p.value, p.value_bytes);
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.grad_acc, p.acc_bytes);
  const __amdgpu_buffer_rsrc_t rg = make_rsrc(p.grad_out, p.gout_bytes);
  const float det_s = A::kBytes == 8 ? det_scale(p) : 0.f;  // int64 fixed-point scale

  // grad_out of this lane's pair: its gather chunk (for the dot products)
  // and the words it scatters (zeros for tail pairs and padding lanes).
  float gv[kVec];
  C::load(rg, (uint32_t)pair * (uint32_t)(p.D * T::kBytes) + chb, gv);
  using Sc = Scatter<T, A, CB>;
  float sg[Sc::kSlots];
  if constexpr (kScatter) Sc::load_g(p, pair, ch, live, sg);
  float delta = 0.f;  // fused: <grad_out, out> of this lane's pair
  if constexpr (FUSED) {
    float ov[kVec];
    C::load(make_rsrc(p.out_fwd, p.gout_bytes),
            (uint32_t)pair * (uint32_t)(p.D * T::kBytes) + chb, ov);
#pragma unroll
    for (int k = 0; k < kVec; ++k) delta += gv[k] * ov[k];
    if constexpr (kStatic) {
      delta = xsum_range<1, G / 2, G>(delta);
    } else {
      delta = xsum_runtime(delta, 1, g);
    }
  }

  __syncthreads();

  const int nrec = ppb * p.sch;
  const int nps = p.sch / ts;
  const int rbase = pl * p.sch + sl;

  for (int pass = 0; pass < p.npass; ++pass) {
    for (int j = threadIdx.x; j < nrec; j += kBlock) {
      const int jp = j >> p.log2_sch;
      const int s = pass * p.sch + (j & (p.sch - 1));
      const int pr = pair0 + jp;
      const bool valid = pr < p.npairs && s < p.LK;
      const Sample q = make_sample<T, FUSED>(p, lt, (uint32_t)pr, (uint32_t)s, valid,
                                             FUSED && valid ? p.lse[pr] : 0.f);
      s_off[j] = make_uint4(q.off[0] * T::kBytes, q.off[1] * T::kBytes, q.off[2] * T::kBytes,
                            q.off[3] * T::kBytes);
      s_geo[j] = make_float4(q.lx, q.ly, q.a, 0.f);
      s_scl[j] = make_float2(q.a * q.fw, q.a * q.fh);
    }
    __syncthreads();

    for (int i = 0; i < nps; i += kBwdUnroll) {
      uint32_t raw[kBwdUnroll][4][kWords];
      uint4 o[kBwdUnroll];
#pragma unroll
      for (int u = 0; u < kBwdUnroll; ++u) {
        if (i + u < nps) {  // wave-uniform
          const int j = rbase + (i + u) * ts;
          o[u] = s_off[j];
          C::load_raw(rv, o[u].x + chb, raw[u][0]);
          C::load_raw(rv, o[u].y + chb, raw[u][1]);
          C::load_raw(rv, o[u].z + chb, raw[u][2]);
          C::load_raw(rv, o[u].w + chb, raw[u][3]);
        }
      }
#pragma unroll
      for (int u = 0; u < kBwdUnroll; ++u) {
        if (i + u < nps) {
          const int j = rbase + (i + u) * ts;
          float d[4];
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            float v[kVec];
            C::unpack(raw[u][c], v);
            float acc = 0.f;
#pragma unroll
            for (int k = 0; k < kVec; ++k) acc += gv[k] * v[k];
            if constexpr (kStatic) {
              d[c] = xsum_range<1, G / 2, G>(acc);
            } else {
              d[c] = xsum_runtime(acc, 1, g);
            }
          }
          const float4 geo = s_geo[j];
          const float lx = geo.x, ly = geo.y, a = geo.z;
          const float mx = 1.f - lx, my = 1.f - ly;
          const float w00 = mx * my, w01 = lx * my, w10 = mx * ly, w11 = lx * ly;
          if (ch == 0) {
            const float2 sc = s_scl[j];
            const float ga = w00 * d[0] + w01 * d[1] + w10 * d[2] + w11 * d[3];
            const float tx = my * (d[1] - d[0]) + ly * (d[3] - d[2]);
            const float ty = mx * (d[2] - d[0]) + lx * (d[3] - d[1]);
            if constexpr (FUSED) {
              s_res[j] = make_float4(a * (ga - delta), a * tx, a * ty, 0.f);
            } else {
              s_res[j] = make_float4(ga, sc.x * tx, sc.y * ty, 0.f);
            }
          }
          // Atomics interleaved with the next samples' gathers measured
          // faster than issuing them all after the gathers (decoder preset).
          if constexpr (kScatter) {
            if (live) {
              Sc::add(ra, o[u].x * kAccScale, ch, p.g_real, a * w00, sg, det_s);
              Sc::add(ra, o[u].y * kAccScale, ch, p.g_real, a * w01, sg, det_s);
              Sc::add(ra, o[u].z * kAccScale, ch, p.g_real, a * w10, sg, det_s);
              Sc::add(ra, o[u].w * kAccScale, ch, p.g_real, a * w11, sg, det_s);
            }
          }
        }
      }
    }
    __syncthreads();

    for (int j = threadIdx.x; j < nrec; j += kBlock) {
      const int jp = j >> p.log2_sch;
      const int s = pass * p.sch + (j & (p.sch - 1));
      const int pr = pair0 + jp;
      if (pr < p.npairs && s < p.LK) {
        const uint64_t pi = (uint64_t)pr * (uint32_t)p.LK + (uint32_t)s;
        const float4 r = s_res[j];
        store1<T>(p.grad_attn, pi, r.x);
        store_xy<T>(p.grad_loc, pi, r.y, r.z);
      }
    }
    if constexpr (FUSED) {
      // Reference-point gradient of the workgroup's queries, when it holds
      // whole queries (ppb a multiple of M) and one pass holds all their
      // samples (host-checked): grad_ref = sum over heads and points (and
      // levels, for one point per query) of grad_offset * (W, H), summed in
      // a fixed order -- what the separate ref_grad_kernel does from memory.
      if (p.ref_inline) {
        const int nl = p.ref_levels ? p.L : 1;
        const int nqw = ppb / p.M;
        for (int t = threadIdx.x; t < nqw * nl * 2; t += kBlock) {
          const int c = t & 1, gi = t >> 1;
          const int qi = gi / nl, lr = gi - qi * nl;
          const int pr0 = pair0 + qi * p.M;
          if (pr0 >= p.npairs) continue;
          float acc = 0.f;
          const int l_lo = p.ref_levels ? lr : 0, l_hi = p.ref_levels ? lr + 1 : p.L;
          for (int l = l_lo; l < l_hi; ++l) {
            float al = 0.f;
            for (int m = 0; m < p.M; ++m) {
              const float4* rr = s_res + (qi * p.M + m) * p.sch + l * p.K;
              for (int k = 0; k < p.K; ++k) al += c ? rr[k].z : rr[k].y;
            }
            acc += al * (c ? (float)lt.h[l] : (float)lt.w[l]);
          }
          store1<T>(p.grad_ref, ((uint64_t)(pr0 / p.M) * (uint32_t)nl + (uint32_t)lr) * 2u + c, acc);
        }
      }
    }
    if (pass + 1 < p.npass) __syncthreads();
  }
}

}  // namespace msda
