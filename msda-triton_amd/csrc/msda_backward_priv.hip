// LDS-deduplicated MSDA backward for gfx950.
//
// Same gradients as bwd_kernel (msda_backward.hip, reference
// src/msda_triton/kernels.py:166-291), organised to issue fewer atomics.
// Measured on MI355X: grad_value's buffer atomics are forwarded by L2 to the
// memory side (TCC_EA0_ATOMIC == TCC_ATOMIC), one request per 64-byte row
// segment, at a fixed chip-wide rate -- so the scatter costs one request per
// (corner row, sample), and samples that share a corner row waste requests.
// Here one workgroup owns (batch b, head m, level l, nq consecutive queries):
// up to 128 samples, 512 corner entries.  It
//
//   1. stages the block's samples (corner offsets, lx, ly, A) and grad_out
//      rows (fp32) in LDS and inserts every in-map corner row into an LDS hash
//      table (open addressing, ds_cmpst);
//   2. groups the entries of rows hit more than once (CSR over hash
//      positions: integer LDS counts taken at insertion, a block prefix sum,
//      a fill pass);
//   3. gathers the corners, reduces the four corner dot products across the
//      row's lanes (DPP) into grad_attn / grad_loc;
//   4. gives each row hit by >= 2 entries to one team of lanes, which sums
//      the row's contributions A*w_c*g in registers and issues ONE coalesced
//      atomic row update; a row hit once is scattered directly in step 3, as
//      in the direct kernel, so random sampling pays little for the dedup.
//
// No floating-point LDS atomics: a first version accumulated with ds_add_f32
// and spent ~93% of its wait cycles on LDS (address conflicts serialise).
// Query blocks of one head sample nearby pixels in encoder-style
// self-attention (Q = S, reference points on the pixel grid) and when
// sampling is concentrated, so those cases see the largest reduction.
//
// FUSED = true: backward of the fused front-end (formulas in
// msda_backward.hip).  The block holds one level of each pair, but the
// softmax couples all L*K samples; the coupling enters only through
// delta = <grad_out, out>, which each block computes for its queries from the
// staged grad_out rows and the saved forward output.
#include <type_traits>

#include "msda_launch.h"
#include "msda_scatter.h"

namespace msda {

namespace {

// ~29 KB of LDS per workgroup.
constexpr int kPrivSamples = 128;  // samples per workgroup
constexpr int kEntries = 4 * kPrivSamples;
constexpr int kHashBits = 10;
constexpr int kHashCap = 1 << kHashBits;  // >= 2x the corner entries: probing always ends
constexpr uint32_t kEmpty = 0xFFFFFFFFu;
// Staged grad_out floats (nq * D): 1024 for rows of <= 32 elements, else
// 2048.  Sized per launch shape so that the common D <= 32 case fits six
// workgroups per CU (LDS) instead of five.
__host__ __device__ constexpr int g_floats(int row_elems) { return row_elems <= 32 ? 1024 : 2048; }
constexpr int kGFloatsMax = 2048;
constexpr uint16_t kNoPos = 0xFFFF;
constexpr int kUnroll = 4;

__device__ __forceinline__ uint32_t hash_row(uint32_t key) {
  return (key * 2654435761u) >> (32 - kHashBits);  // Fibonacci hashing
}

// grad_out rows staged in LDS in their storage dtype (half types as raw
// 16-bit values: no precision is lost, and the half LDS footprint lets eight
// workgroups share a CU).
template <class T>
using GElem = std::conditional_t<T::kBytes == 4, float, uint16_t>;

template <class T>
__device__ __forceinline__ float g_at(const GElem<T>* g, int i) {
  if constexpr (T::kBytes == 4) {
    return g[i];
  } else {
    return unpack1<T>(g[i]);
  }
}

// Elements i and i + 1 (i even for half storage: one 32-bit LDS read).
template <class T>
__device__ __forceinline__ void g_at2(const GElem<T>* g, int i, float& lo, float& hi) {
  if constexpr (T::kBytes == 4) {
    lo = g[i];
    hi = g[i + 1];
  } else {
    unpack2<T>(*reinterpret_cast<const uint32_t*>(g + i), lo, hi);
  }
}

// Exclusive prefix sum of v over the 256 lanes of the workgroup; `tot`
// receives the total.  `warp_sums` holds 4 ints of LDS.
__device__ __forceinline__ int block_exclusive_scan(int v, int* warp_sums, int* tot) {
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  int x = v;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int y = __shfl_up(x, d);
    if (lane >= d) x += y;
  }
  if (lane == kWave - 1) warp_sums[wave] = x;
  __syncthreads();
  int base = 0;
  for (int w = 0; w < wave; ++w) base += warp_sums[w];
  *tot = warp_sums[0] + warp_sums[1] + warp_sums[2] + warp_sums[3];
  return base + x - v;
}

template <class T, class A, int CB, int G, bool FUSED>
__global__ __launch_bounds__(kBlock) void bwd_priv_kernel(Params p) {
  using C = Chunk<T, CB>;
  using Sc = Scatter<T, A, CB>;
  constexpr int kVec = C::kVec;
  constexpr int kWords = C::kWords;
  constexpr int kTeams = kBlock / G;
  constexpr int kWpl = Sc::kWordsPerLane;  // accumulator words per lane
  constexpr int kEpw = Sc::kElemsPerWord;
  static_assert(kWpl > 0, "row dedup needs word-aligned rows");
  constexpr uint32_t kAccScale = A::kBytes / T::kBytes;
  static_assert(kHashCap == 4 * kBlock, "four hash positions per lane in the scan");
  static_assert(kEntries == 2 * kBlock, "two corner entries per lane");

  // A row is identified by its hash-table position h (0..kHashCap-1).
  __shared__ uint32_t h_key[kHashCap];
  // Entries per row, then the CSR fill cursor; dead after the fill, when the
  // same LDS holds the per-sample results (grad_attn, grad_x, grad_y, -).
  __shared__ union {
    int cnt[kHashCap];
    float4 res[kPrivSamples];
  } u_cnt_res;
  int* const h_cnt = u_cnt_res.cnt;
  float4* const s_res = u_cnt_res.res;
  // CSR segment per row (offsets <= kEntries fit 16 bits); empty for rows
  // hit once, which are scattered directly.
  __shared__ uint16_t h_start[kHashCap + 1];
  __shared__ uint4 s_off[kPrivSamples];
  __shared__ float4 s_geo[kPrivSamples];  // lx, ly, A, -
  __shared__ uint16_t s_pos[kEntries];    // row of entry 4*sample+corner; kNoPos if outside
  __shared__ uint16_t s_csr[kEntries];
  __shared__ uint16_t s_multi[kEntries];  // rows with >= 2 entries
  constexpr int kGFloats = g_floats(G * CB / T::kBytes);
  __shared__ __align__(16) GElem<T> s_g[kGFloats];
  __shared__ float s_delta[FUSED ? kPrivSamples : 1];  // fused: <grad_out, out> per query
  __shared__ int s_wsum[4];
  __shared__ int n_multi;

  const int tid = threadIdx.x;
  const int D = p.D;
  const int K = p.K;
  const int nq = p.nq;
  const int ns = nq * K;

  // Block -> (b, m, l, query block), query block fastest.
  int blk = xcd_remap(blockIdx.x, p.nblocks);
  const int qb = blk % p.nqblk;
  blk /= p.nqblk;
  const int l = blk % p.L;
  blk /= p.L;
  const int m = blk % p.M;
  const int b = blk / p.M;
  const int q0 = qb * nq;
  // The block's level: read once (no LDS level table, no extra round trip).
  const int32_t lh = (int32_t)p.shapes[2 * l], lw = (int32_t)p.shapes[2 * l + 1];
  const int32_t lst = (int32_t)p.starts[l];
  const float fw = (float)lw, fh = (float)lh;

  for (int h = tid; h < kHashCap; h += kBlock) {
    h_key[h] = kEmpty;
    h_cnt[h] = 0;
  }
  if (tid == 0) n_multi = 0;
  // grad_out rows of the block's pairs (loads batched for latency).
  {
    constexpr int kIt = kGFloats / kBlock;
    GElem<T> gtmp[kIt];
    const int n = nq * D;
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
      const int idx = tid + it * kBlock;
      gtmp[it] = 0;
      if (idx < n) {
        const int qi = (int)fdiv((uint32_t)idx, p.div_d);
        const int d = idx - qi * D;
        const int q = q0 + qi;
        if (q < p.Q) {
          const uint64_t pair = ((uint64_t)b * (uint32_t)p.Q + (uint32_t)q) * (uint32_t)p.M + m;
          gtmp[it] = static_cast<const GElem<T>*>(p.grad_out)[pair * (uint32_t)D + d];
        }
      }
    }
    // 1. Stage samples (their parameter loads issued together with the
    //    grad_out loads above, one round trip), then insert and count corner
    //    rows.  Lanes t and t + 128 both build sample t's geometry and
    //    insert two of its four corners each.
    const int si = tid % kPrivSamples;
    const int half = tid / kPrivSamples;
    const int qi = (int)fdiv((uint32_t)si, p.div_k);
    const int k = si - qi * K;
    const int q = q0 + qi;
    const bool valid = si < ns && q < p.Q;
    const uint32_t pair = (uint32_t)(((int64_t)b * p.Q + q) * p.M + m);
    const Sample smp = make_sample_at<T, FUSED>(p, valid ? pair : 0u, (uint32_t)(l * K + k),
                                                valid, FUSED && valid ? p.lse[pair] : 0.f,
                                                lh, lw, lst);
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
      const int idx = tid + it * kBlock;
      if (idx < n) s_g[idx] = gtmp[it];
    }
    if (half == 0) {
      s_off[si] = make_uint4(smp.off[0] * T::kBytes, smp.off[1] * T::kBytes,
                             smp.off[2] * T::kBytes, smp.off[3] * T::kBytes);
      s_geo[si] = make_float4(smp.lx, smp.ly, smp.a, 0.f);
    }
    __syncthreads();
#pragma unroll
    for (int cc = 0; cc < 2; ++cc) {
      const int c = 2 * half + cc;
      // (select, not smp.off[c]: a runtime index would put the array in scratch)
      const uint32_t key = half ? (cc ? smp.off[3] : smp.off[2]) : (cc ? smp.off[1] : smp.off[0]);
      uint16_t pos = kNoPos;
      if (key != kOobElem) {
        uint32_t h = hash_row(key);
        for (int it = 0; it < kHashCap; ++it) {
          const uint32_t prev = atomicCAS(&h_key[h], kEmpty, key);
          if (prev == kEmpty || prev == key) break;
          h = (h + 1) & (kHashCap - 1);
        }
        atomicAdd(&h_cnt[h], 1);
        pos = (uint16_t)h;
      }
      s_pos[4 * si + c] = pos;
    }
  }
  if constexpr (FUSED) {
    // delta per query: tq lanes (a power of two <= 64) per query, strided
    // over the D channels, merged by an xor butterfly (deterministic order).
    int nqp = 1;
    while (nqp < nq) nqp <<= 1;
    const int tq = kBlock / nqp < kWave ? kBlock / nqp : kWave;
    const int sub = tid % tq;
    for (int qb = 0; qb < nq; qb += kBlock / tq) {
      const int qi = qb + tid / tq;
      const int q = q0 + qi;
      float acc = 0.f;
      if (qi < nq && q < p.Q) {
        const uint64_t pair = ((uint64_t)b * (uint32_t)p.Q + (uint32_t)q) * (uint32_t)p.M + m;
        for (int d = sub; d < D; d += tq) {
          acc += g_at<T>(s_g, qi * D + d) * load1<T>(p.out_fwd, pair * (uint32_t)D + d);
        }
      }
      for (int x = 1; x < tq; x <<= 1) acc += __shfl_xor(acc, x);
      if (sub == 0 && qi < nq) s_delta[qi] = acc;
    }
  }
  __syncthreads();

  // 2. Rows hit by >= 2 entries get a CSR segment and an owner team; an entry
  //    alone on its row is scattered directly during the gathers.
  {
    int cnt[4], mc[4], msum = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      cnt[i] = h_cnt[4 * tid + i];
      mc[i] = cnt[i] >= 2 ? cnt[i] : 0;
      msum += mc[i];
    }
    int total;
    int base = block_exclusive_scan(msum, s_wsum, &total);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = 4 * tid + i;
      h_start[h] = (uint16_t)base;
      h_cnt[h] = mc[i] ? base : -1;  // fill cursor, or -1: single-entry row
      if (mc[i]) s_multi[atomicAdd(&n_multi, 1)] = (uint16_t)h;
      base += mc[i];
    }
    if (tid == kBlock - 1) h_start[kHashCap] = (uint16_t)base;
  }
  __syncthreads();
  for (int e = tid; e < kEntries; e += kBlock) {
    const uint16_t pos = s_pos[e];
    if (pos != kNoPos && h_cnt[pos] >= 0) s_csr[atomicAdd(&h_cnt[pos], 1)] = (uint16_t)e;
  }
  __syncthreads();

  // 3. Gathers, corner dots, and the direct atomics of single-entry rows
  //    (interleaved with the gathers, as in the direct kernel).  A
  //    single-entry row has an empty CSR segment; h_cnt's LDS now holds
  //    s_res.
  const int team = tid / G;
  const int ch = tid % G;
  const bool live = ch < p.g_real;
  const uint32_t chb = live ? (uint32_t)(ch * CB) : kDeadLaneBytes;
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(p.value, p.value_bytes);
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.grad_acc, p.acc_bytes);
  constexpr bool kDet = A::kBytes == 8;  // int64 fixed point (deterministic)
  const float det_s = kDet ? det_scale(p) : 0.f;

  for (int s0 = team; s0 < ns; s0 += kTeams * kUnroll) {
    uint32_t raw[kUnroll][4][kWords];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int s = s0 + u * kTeams;
      if (s < ns) {  // uniform per team
        const uint4 o = s_off[s];
        C::load_raw(rv, o.x + chb, raw[u][0]);
        C::load_raw(rv, o.y + chb, raw[u][1]);
        C::load_raw(rv, o.z + chb, raw[u][2]);
        C::load_raw(rv, o.w + chb, raw[u][3]);
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int s = s0 + u * kTeams;
      if (s < ns) {
        const int qi = (int)fdiv((uint32_t)s, p.div_k);
        const GElem<T>* gq = s_g + qi * D;
        float gv[kVec];
        if constexpr (T::kBytes == 2) {
#pragma unroll
          for (int k = 0; k < kVec; k += 2) g_at2<T>(gq, live ? ch * kVec + k : 0, gv[k], gv[k + 1]);
        } else {
#pragma unroll
          for (int k = 0; k < kVec; ++k) gv[k] = g_at<T>(gq, live ? ch * kVec + k : 0);
        }
        if (!live) {
#pragma unroll
          for (int k = 0; k < kVec; ++k) gv[k] = 0.f;
        }
        float d[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          float v[kVec];
          C::unpack(raw[u][c], v);
          float acc = 0.f;
#pragma unroll
          for (int k = 0; k < kVec; ++k) acc += gv[k] * v[k];
          d[c] = xsum_range<1, G / 2, G>(acc);
        }
        const float4 geo = s_geo[s];
        const float lx = geo.x, ly = geo.y, a = geo.z;
        const float mx = 1.f - lx, my = 1.f - ly;
        if (ch == 0) {
          const float ga = mx * my * d[0] + lx * my * d[1] + mx * ly * d[2] + lx * ly * d[3];
          const float tx = my * (d[1] - d[0]) + ly * (d[3] - d[2]);
          const float ty = mx * (d[2] - d[0]) + lx * (d[3] - d[1]);
          if constexpr (FUSED) {
            s_res[s] = make_float4(a * (ga - s_delta[qi]), a * tx, a * ty, 0.f);
          } else {
            s_res[s] = make_float4(ga, a * fw * tx, a * fh * ty, 0.f);
          }
        }
        if (live) {
          float sg[Sc::kSlots];
#pragma unroll
          for (int i = 0; i < kWpl; ++i) {
            if constexpr (kEpw == 2) {
              g_at2<T>(gq, (ch + p.g_real * i) * 2, sg[2 * i], sg[2 * i + 1]);
            } else {
              sg[i] = g_at<T>(gq, ch + p.g_real * i);
            }
          }
          const uint4 o = s_off[s];
          const uint32_t offs[4] = {o.x, o.y, o.z, o.w};
          const float w[4] = {mx * my, lx * my, mx * ly, lx * ly};
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const uint16_t pos = s_pos[4 * s + c];
            if (pos != kNoPos && h_start[pos] == h_start[pos + 1]) {  // single-entry row
              Sc::add(ra, offs[c] * kAccScale, ch, p.g_real, a * w[c], sg, det_s);
            }
          }
        }
      }
    }
  }

  // 4. One team per shared row: sum its entries in registers, one atomic row
  //    update.  Two rows per team per step keep two LDS chains in flight.
  //    (s_csr, h_start and s_multi were complete before step 3.)  The CSR
  //    order of a row's entries depends on scheduling; the deterministic
  //    variant therefore sums their int64 fixed-point values, which is exact.
  using Acc = std::conditional_t<kDet, long long, float>;
  const int nm = n_multi;
  if (live) {
    for (int r0 = team; r0 < nm; r0 += 2 * kTeams) {
      Acc acc[2][kWpl * kEpw];
      int rows[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int ri = r0 + u * kTeams;
        rows[u] = ri < nm ? (int)s_multi[ri] : -1;
#pragma unroll
        for (int i = 0; i < kWpl * kEpw; ++i) acc[u][i] = 0;
        if (rows[u] < 0) continue;
        const int e1 = h_start[rows[u] + 1];
        for (int idx = h_start[rows[u]]; idx < e1; ++idx) {
          const int e = s_csr[idx];
          const int sa = e >> 2, c = e & 3;
          const float4 geo = s_geo[sa];
          const float wx = (c & 1) ? geo.x : 1.f - geo.x;
          const float wy = (c & 2) ? geo.y : 1.f - geo.y;
          const float coef = geo.z * wx * wy;
          const GElem<T>* gq = s_g + (int)fdiv((uint32_t)sa, p.div_k) * D;
#pragma unroll
          for (int i = 0; i < kWpl; ++i) {
            float gw[kEpw];
            if constexpr (kEpw == 2) {
              g_at2<T>(gq, (ch + p.g_real * i) * 2, gw[0], gw[1]);
            } else {
              gw[0] = g_at<T>(gq, ch + p.g_real * i);
            }
#pragma unroll
            for (int j = 0; j < kEpw; ++j) {
              const float v = coef * gw[j];
              if constexpr (kDet) {
                acc[u][i * kEpw + j] += to_fixed(v, det_s);
              } else {
                acc[u][i * kEpw + j] += v;
              }
            }
          }
        }
      }
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        if (rows[u] < 0) continue;
        const uint32_t row = h_key[rows[u]] * (uint32_t)A::kBytes;
#pragma unroll
        for (int i = 0; i < kWpl; ++i) {
          const uint32_t off = row + (uint32_t)Sc::kWordBytes * (uint32_t)(ch + p.g_real * i);
          if constexpr (kDet) {
            raw_buffer_atomic_add_i64(acc[u][i], ra, (int)off, 0, 0);
          } else if constexpr (kEpw == 1) {
            atomic_add_word<A>(ra, off, acc[u][i], 0.f);
          } else {
            atomic_add_word<A>(ra, off, acc[u][2 * i], acc[u][2 * i + 1]);
          }
        }
      }
    }
  }
  __syncthreads();

  // grad_attn / grad_loc of the block's samples.
  if (tid < ns) {
    const int qi = (int)fdiv((uint32_t)tid, p.div_k);
    const int k = tid - qi * K;
    const int q = q0 + qi;
    if (q < p.Q) {
      const uint64_t pair = ((uint64_t)b * (uint32_t)p.Q + (uint32_t)q) * (uint32_t)p.M + m;
      const uint64_t pi = pair * (uint32_t)p.LK + (uint32_t)(l * K + k);
      const float4 r = s_res[tid];
      store1<T>(p.grad_attn, pi, r.x);
      store_xy<T>(p.grad_loc, pi, r.y, r.z);
    }
  }
}

template <class T, class A, int CB, int G, bool FUSED>
hipError_t launch_one(const Params& p, hipStream_t st) {
  hipLaunchKernelGGL((bwd_priv_kernel<T, A, CB, G, FUSED>), dim3(p.nblocks), dim3(kBlock), 0, st,
                     p);
  return hipGetLastError();
}

template <class T, class A, bool FUSED>
hipError_t dispatch(const Shape& s, const Params& p, hipStream_t st) {
  switch (s.cb * 100 + s.g) {
    case 408: return launch_one<T, A, 4, 8, FUSED>(p, st);
    case 416: return launch_one<T, A, 4, 16, FUSED>(p, st);
    case 816: return launch_one<T, A, 8, 16, FUSED>(p, st);
    case 1616: return launch_one<T, A, 16, 16, FUSED>(p, st);
    default: return hipErrorInvalidValue;
  }
}

template <bool FUSED>
hipError_t dispatch_dtype(int dtype, AccMode acc, const Shape& s, const Params& p,
                          hipStream_t st) {
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

}  // namespace

bool priv_supported(const Shape& s, int D, int K, int elem_bytes) {
  const int key = s.cb * 100 + s.g;
  const bool shape_ok = key == 408 || key == 416 || key == 816 || key == 1616;
  // Half storage needs word-aligned rows for the packed atomics.
  return shape_ok && D >= 1 && D <= g_floats(s.g * s.cb / elem_bytes) && K >= 1 &&
         K <= kPrivSamples &&
         (D * elem_bytes) % 4 == 0;
}

void priv_params(const Shape& s, int elem_bytes, Params* p) {
  int nq = kPrivSamples / p->K;
  const int gf = g_floats(s.g * s.cb / elem_bytes);
  if (nq * p->D > gf) nq = gf / p->D;
  p->nq = nq;
  p->nqblk = (p->Q + nq - 1) / nq;
  p->div_d = make_fastdiv((uint32_t)p->D);
  p->nblocks = (p->npairs / (p->Q > 0 ? p->Q : 1)) * p->L * p->nqblk;
}

hipError_t launch_backward_priv(int dtype, AccMode acc, bool fused, const Shape& s,
                                const Params& p, hipStream_t st) {
  return fused ? dispatch_dtype<true>(dtype, acc, s, p, st)
               : dispatch_dtype<false>(dtype, acc, s, p, st);
}

}  // namespace msda
