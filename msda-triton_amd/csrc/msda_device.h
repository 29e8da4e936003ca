// Device-side building blocks shared by the MSDA forward and backward kernels
// (gfx950 / CDNA4, wave64).
//
// Memory layouts follow the reference operator (src/msda_triton/kernels.py:
// 67-82, 167-185): value (B,S,M,D), sampling_locations (B,Q,M,L,K,2),
// attention_weights (B,Q,M,L,K), all C-contiguous.
//
// Addressing: every kernel works on a batch slice whose value tensor holds
// fewer than 2^28 elements, so element offsets are 32-bit and value rows are
// read with buffer loads (SGPR base + 32-bit VGPR byte offset).  A corner that
// falls outside the feature map is given the element offset kOobElem; its byte
// offset lies beyond the buffer's num_records, so the hardware range check
// returns zero for the load and drops the atomic.  That is exactly
// grid_sample's zeros padding and costs no per-element select.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace msda {

constexpr int kBlock = 256;  // threads per workgroup: 4 wave64
constexpr int kWave = 64;
constexpr int kMaxLevels = 64;
constexpr int kMaxRecords = 512;             // staged samples per workgroup pass (forward)
constexpr int kBwdRecords = 256;             // same, backward (keeps LDS for occupancy)
constexpr uint32_t kOobElem = 1u << 28;      // element-offset sentinel
constexpr uint32_t kDeadLaneBytes = 1u << 30;  // pushes padding lanes out of range
constexpr uint32_t kMaxSliceElems = (1u << 28) - 1;
// gfx9 buffer descriptor word 3: raw (untyped) 32-bit data format.
constexpr int kRsrcWord3 = 0x00020000;

enum DType : int { kF32 = 0, kF16 = 1, kBF16 = 2 };

typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Packed-bf16 buffer atomic; clang has no builtin for it, so bind the LLVM
// intrinsic by name (lowers to buffer_atomic_pk_add_bf16 on gfx950).
__device__ bf16x2 raw_buffer_atomic_fadd_v2bf16(bf16x2 v, __amdgpu_buffer_rsrc_t rsrc,
                                                int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.raw.ptr.buffer.atomic.fadd.v2bf16");
// 64-bit integer buffer atomic add (buffer_atomic_add_x2), bound the same way.
__device__ long long raw_buffer_atomic_add_i64(long long v, __amdgpu_buffer_rsrc_t rsrc,
                                               int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.raw.ptr.buffer.atomic.add.i64");

// --------------------------------------------------------------------------
// Division by a runtime constant: n / d == (umulhi(n, mul) + n) >> shift for
// 0 <= n < 2^31 (Granlund & Montgomery 1994, round-up multiplier).
// --------------------------------------------------------------------------
struct FastDiv {
  uint32_t mul;
  uint32_t shift;
  uint32_t d;
};

__device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv& f) {
  return (__umulhi(n, f.mul) + n) >> f.shift;
}

// --------------------------------------------------------------------------
// Storage dtypes.
// --------------------------------------------------------------------------
struct F32 {
  static constexpr int kBytes = 4;
  static constexpr int kCode = kF32;
};
struct F16 {
  static constexpr int kBytes = 2;
  static constexpr int kCode = kF16;
};
struct BF16 {
  static constexpr int kBytes = 2;
  static constexpr int kCode = kBF16;
};
// Accumulator of the deterministic backward (int64 fixed point, see
// det_scale); never a storage dtype.
struct I64 {
  static constexpr int kBytes = 8;
  static constexpr int kCode = -1;
};
// "Accumulator" of a backward launch that scatters nothing (grad_loc and
// grad_attn only; grad_value is written by the owner kernel).
struct NoAcc {
  static constexpr int kBytes = 0;
  static constexpr int kCode = -2;
};

// Two storage elements packed in one 32-bit word -> two floats.
template <class T>
__device__ __forceinline__ void unpack2(uint32_t w, float& lo, float& hi);
template <>
__device__ __forceinline__ void unpack2<BF16>(uint32_t w, float& lo, float& hi) {
  lo = __uint_as_float(w << 16);
  hi = __uint_as_float(w & 0xffff0000u);
}
template <>
__device__ __forceinline__ void unpack2<F16>(uint32_t w, float& lo, float& hi) {
  f16x2 h = __builtin_bit_cast(f16x2, w);
  lo = (float)h[0];
  hi = (float)h[1];
}

// One storage element held in the low 16 bits.
template <class T>
__device__ __forceinline__ float unpack1(uint32_t w);
template <>
__device__ __forceinline__ float unpack1<BF16>(uint32_t w) {
  return __uint_as_float(w << 16);
}
template <>
__device__ __forceinline__ float unpack1<F16>(uint32_t w) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)w);
}
template <>
__device__ __forceinline__ float unpack1<F32>(uint32_t w) {
  return __uint_as_float(w);
}

// Two floats -> two storage elements in one word (round to nearest even).
template <class T>
__device__ __forceinline__ uint32_t pack2(float lo, float hi);
template <>
__device__ __forceinline__ uint32_t pack2<BF16>(float lo, float hi) {
  bf16x2 v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}
template <>
__device__ __forceinline__ uint32_t pack2<F16>(float lo, float hi) {
  f16x2 v = {(_Float16)lo, (_Float16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

template <class T>
__device__ __forceinline__ void store1(void* base, uint64_t i, float v);
template <>
__device__ __forceinline__ void store1<F32>(void* base, uint64_t i, float v) {
  static_cast<float*>(base)[i] = v;
}
template <>
__device__ __forceinline__ void store1<F16>(void* base, uint64_t i, float v) {
  static_cast<_Float16*>(base)[i] = (_Float16)v;
}
template <>
__device__ __forceinline__ void store1<BF16>(void* base, uint64_t i, float v) {
  static_cast<__bf16*>(base)[i] = (__bf16)v;
}

// Elements 2i and 2i + 1 (an (x, y) pair): one store when the base allows
// it (16-bit types: 4-byte aligned; fp32: 8-byte aligned), else two.
template <class T>
__device__ __forceinline__ void store_xy(void* base, uint64_t i, float x, float y) {
  if constexpr (T::kBytes == 4) {
    if ((reinterpret_cast<uintptr_t>(base) & 7) == 0) {
      static_cast<float2*>(base)[i] = make_float2(x, y);
      return;
    }
  } else {
    if ((reinterpret_cast<uintptr_t>(base) & 3) == 0) {
      static_cast<uint32_t*>(base)[i] = pack2<T>(x, y);
      return;
    }
  }
  store1<T>(base, 2 * i, x);
  store1<T>(base, 2 * i + 1, y);
}

template <class T>
__device__ __forceinline__ float load1(const void* base, uint64_t i) {
  if constexpr (T::kBytes == 4) {
    return static_cast<const float*>(base)[i];
  } else {
    return unpack1<T>(static_cast<const uint16_t*>(base)[i]);
  }
}

// (x, y) pair at element index 2*i.
template <class T>
__device__ __forceinline__ void load_xy(const void* base, uint64_t i, float& x, float& y) {
  if constexpr (T::kBytes == 4) {
    float2 v = static_cast<const float2*>(base)[i];
    x = v.x;
    y = v.y;
  } else {
    unpack2<T>(static_cast<const uint32_t*>(base)[i], x, y);
  }
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes,
                                           kRsrcWord3);
}

// 16 bytes of T from 16 / elem floats (round to nearest even), as the four
// dwords of a 128-bit store.
template <class T>
__device__ __forceinline__ i32x4 pack16(const float (&v)[16 / T::kBytes]) {
  i32x4 w;
  if constexpr (T::kBytes == 4) {
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = __float_as_int(v[i]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = (int)pack2<T>(v[2 * i], v[2 * i + 1]);
  }
  return w;
}

// --------------------------------------------------------------------------
// Chunk = CB contiguous bytes of one value row, VEC = CB / elem floats.
// --------------------------------------------------------------------------
template <class T, int CB>
struct Chunk {
  static constexpr int kVec = CB / T::kBytes;
  static constexpr int kWords = CB >= 4 ? CB / 4 : 1;

  // Load CB bytes at byte offset `off` (out of range -> zeros), raw words.
  __device__ __forceinline__ static void load_raw(__amdgpu_buffer_rsrc_t r, uint32_t off,
                                                  uint32_t (&w)[kWords]) {
    if constexpr (CB == 16) {
      i32x4 x = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
      w[0] = x[0]; w[1] = x[1]; w[2] = x[2]; w[3] = x[3];
    } else if constexpr (CB == 8) {
      i32x2 x = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
      w[0] = x[0]; w[1] = x[1];
    } else if constexpr (CB == 4) {
      w[0] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
    } else {
      static_assert(CB == 2, "chunk bytes");
      w[0] = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
    }
  }

  // Raw words -> kVec floats.
  __device__ __forceinline__ static void unpack(const uint32_t (&w)[kWords], float (&v)[kVec]) {
    if constexpr (T::kBytes == 4) {
#pragma unroll
      for (int i = 0; i < kVec; ++i) v[i] = __uint_as_float(w[i]);
    } else if constexpr (CB == 2) {
      v[0] = unpack1<T>(w[0]);
    } else {
#pragma unroll
      for (int i = 0; i < kWords; ++i) unpack2<T>(w[i], v[2 * i], v[2 * i + 1]);
    }
  }

  __device__ __forceinline__ static void load(__amdgpu_buffer_rsrc_t r, uint32_t off,
                                              float (&v)[kVec]) {
    uint32_t w[kWords];
    load_raw(r, off, w);
    unpack(w, v);
  }

  // Store kVec floats as CB bytes of T at a 64-bit address.
  __device__ __forceinline__ static void store(void* p, const float (&v)[kVec]) {
    if constexpr (T::kBytes == 4) {
      if constexpr (CB == 16) {
        *static_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
      } else if constexpr (CB == 8) {
        *static_cast<float2*>(p) = make_float2(v[0], v[1]);
      } else {
        *static_cast<float*>(p) = v[0];
      }
    } else if constexpr (CB == 2) {
      store1<T>(p, 0, v[0]);
    } else {
      uint32_t w[kWords];
#pragma unroll
      for (int i = 0; i < kWords; ++i) w[i] = pack2<T>(v[2 * i], v[2 * i + 1]);
      if constexpr (CB == 16) {
        *static_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
      } else if constexpr (CB == 8) {
        *static_cast<uint2*>(p) = make_uint2(w[0], w[1]);
      } else {
        *static_cast<uint32_t*>(p) = w[0];
      }
    }
  }
};

// --------------------------------------------------------------------------
// Cross-lane sums.  `xsum<DIST, TEAM>` adds the value held DIST lanes away
// inside aligned teams of TEAM lanes, so that after the steps DIST = s,
// 2s, ..., TEAM/2 every lane of a team holds the sum over the lanes that
// differ from it in those index bits.  DPP forms are used where the pattern
// allows: quad_perm for 1 and 2, row_ror for 4 and 8 when a team covers whole
// 16-lane rows (rotation then stays inside the lane group), and the gfx950
// v_permlane16/32_swap pair exchanges for 16 and 32.  ds_swizzle (xor mode)
// covers 4 and 8 inside smaller teams.
// --------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}

template <int DIST, int TEAM>
__device__ __forceinline__ float xsum(float v) {
  static_assert(DIST >= 1 && DIST < TEAM && TEAM <= kWave, "xsum shape");
  if constexpr (DIST == 1) {
    return v + dpp<0xB1>(v);  // quad_perm [1,0,3,2]
  } else if constexpr (DIST == 2) {
    return v + dpp<0x4E>(v);  // quad_perm [2,3,0,1]
  } else if constexpr (DIST == 4 || DIST == 8) {
    if constexpr (TEAM >= 16) {
      return v + dpp<0x120 + DIST>(v);  // row_ror:DIST
    } else {
      return v + __builtin_bit_cast(
                     float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v),
                                                        (DIST << 10) | 0x1F));
    }
  } else if constexpr (DIST == 16) {
    auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, v),
                                              __builtin_bit_cast(uint32_t, v), false, false);
    return __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, (uint32_t)r[1]);
  } else {
    static_assert(DIST == 32, "xsum distance");
    auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, v),
                                              __builtin_bit_cast(uint32_t, v), false, false);
    return __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, (uint32_t)r[1]);
  }
}

// Sum over the lanes FIRST, 2*FIRST, ..., LAST (all powers of two) apart,
// inside teams of TEAM lanes.
template <int FIRST, int LAST, int TEAM>
__device__ __forceinline__ float xsum_range(float v) {
  if constexpr (FIRST > LAST) {
    return v;
  } else {
    return xsum_range<FIRST * 2, LAST, TEAM>(xsum<FIRST, TEAM>(v));
  }
}

// Runtime-distance variant (ds_bpermute) for launch shapes without a
// specialised kernel: sums over distances first, 2*first, ... < end.
__device__ __forceinline__ float xsum_runtime(float v, int first, int end) {
  for (int d = first; d < end; d <<= 1) v += __shfl_xor(v, d);
  return v;
}

// --------------------------------------------------------------------------
// Kernel parameters (by value).  One launch covers a batch slice.
// --------------------------------------------------------------------------
//
// Fused front-end (kernels instantiated with FUSED = true): `loc` holds the
// sampling offsets in each level's pixel units and `attn` the attention
// logits; a sample's location is ref + offset / (W_l, H_l) and its weight
// softmax over the pair's L*K logits, exp(logit - lse[pair]).  The backward
// then writes d/d(offset) into grad_loc and d/d(logit) into grad_attn.
struct Params {
  const void* value;
  const int64_t* shapes;
  const int64_t* starts;
  const void* loc;       // sampling locations (fused: sampling offsets)
  const void* attn;      // attention weights (fused: attention logits)
  void* out;             // forward output
  const void* grad_out;  // backward
  void* grad_acc;        // backward atomic target (grad_value or fp32 scratch)
  void* grad_loc;        // fused: grad of the offsets
  void* grad_attn;       // fused: grad of the logits
  const void* ref;       // fused: reference points (B,Q,2) or (B,Q,L,2)
  float* lse;            // fused: per-pair log-sum-exp of the logits (B,Q,M)
  const void* out_fwd;   // fused backward: the forward output (for <g, out>)
  void* grad_ref;        // fused backward: grad of the reference points
  int32_t ref_levels;    // fused: 1 if reference points are per level
  int32_t ref_inline;    // fused: the backward workgroups also write grad_ref
  const uint32_t* det_max;  // deterministic: bits of max|A| and max|grad_out| (>= 0)
  float det_samples;        // deterministic: samples per (b, m) = Q * L * K
  uint32_t value_bytes;  // num_records of the value buffer
  uint32_t acc_bytes;    // num_records of the accumulator buffer
  uint32_t gout_bytes;   // num_records of grad_out
  int32_t S, M, D, Q, L, K, LK;
  int32_t MD;
  int32_t npairs;   // pairs (b, q, m) in the slice
  int32_t nblocks;  // workgroups in the grid
  int32_t sch;      // staged samples per pair per pass (power of two)
  int32_t log2_sch;
  int32_t npass;    // ceil(LK / sch)
  int32_t g_real;   // live chunk lanes per value row
  int32_t g_rt;     // runtime G (generic kernels)
  int32_t ts_rt;    // runtime TS (generic kernels)
  int32_t nq;       // deduplicating backward: queries per workgroup
  int32_t nqblk;    //   query blocks per (b, m, l)
  int32_t own_rows;    // owner backward: most rows per band (<= kOwnRows)
  int32_t own_split;   //   least bands per level (entry balance)
  int32_t own_groups;  //   bands (workgroups) per (b, m) in the grid
  int32_t own_lg;      //   log2 of the lanes per row (g_rt)
  FastDiv div_g;       //   division by g_real (live lanes per row)
  uint32_t ref_bytes;  //   fused: num_records of the reference points
  int32_t own_mix;     //   order of band and gradient workgroups (0 last, 1 first, 2 after own_est)
  int32_t own_est;     //   bands per (b, m), estimated (host)
  int32_t own_cut;     //   band chunks (of 8 workgroups) dispatched before the gradient chunks
  int32_t own_big;     //   1: the 40 KB grad_out staging build of the kernel
  FastDiv div_qm, div_m, div_k, div_d;
};

// Deterministic backward: grad_value is accumulated in int64 fixed point,
// each contribution c entering as round(c * scale) with scale = 2^e, so the
// sum is exact and independent of the order in which atomics land.  A value
// row takes at most one corner of each sample of its (b, m), with corner
// weights <= 1, so |grad_value[row, ch]| <= Q*L*K * max|A| * max|grad_out|;
// e puts that bound below 2^60 (no int64 overflow, resolution bound * 2^-60).
__device__ __forceinline__ float det_scale(const Params& p) {
  const float bound = p.det_samples * __uint_as_float(p.det_max[0]) *
                      __uint_as_float(p.det_max[1]);
  int e = 100;  // bound == 0: every contribution is 0
  if (bound > 0.f) {
    int k = 0;
    frexpf(bound, &k);  // bound < 2^k
    e = 60 - k;
  }
  if (!(bound <= 3.0e38f)) e = -100;  // inf / NaN inputs: no overflow, result undefined
  e = e < -100 ? -100 : (e > 100 ? 100 : e);
  return ldexpf(1.f, e);
}

__device__ __forceinline__ long long to_fixed(float c, float scale) {
  return (long long)rintf(c * scale);
}

// Workgroups are dispatched to the 8 XCDs round-robin (id i -> XCD i % 8).
// Map them so that each XCD walks one contiguous range of logical blocks:
// neighbouring query blocks then share that XCD's L2.  Bijective for any n.
__device__ __forceinline__ int xcd_remap(int bid, int n) {
  constexpr int kXcd = 8;
  const int q = n / kXcd, r = n % kXcd;
  const int x = bid % kXcd, k = bid / kXcd;
  return (x < r) ? x * (q + 1) + k : r * (q + 1) + (x - r) * q + k;
}

// Level table (H, W, start) in LDS, loaded once per workgroup.
struct LevelTable {
  int32_t h[kMaxLevels];
  int32_t w[kMaxLevels];
  int32_t start[kMaxLevels];
};

__device__ __forceinline__ void load_levels(const Params& p, LevelTable& t) {
  for (int l = threadIdx.x; l < p.L; l += kBlock) {
    t.h[l] = (int32_t)p.shapes[2 * l];
    t.w[l] = (int32_t)p.shapes[2 * l + 1];
    t.start[l] = (int32_t)p.starts[l];
  }
}

// Fused front-end: log-sum-exp of the L*K logits of each of the workgroup's
// `ppb` pairs (pair0, pair0 + 1, ...) into s_lse[0..ppb) and, when p.lse is
// set, into p.lse.  `tpp` lanes (a power of two <= 64) share a pair: each
// keeps a running (max, sum of exp(x - max)) over a strided subset of the
// logits, then the lanes are merged by an xor butterfly in a fixed order, so
// the result does not depend on scheduling.  Every thread of the workgroup
// must call it (cross-lane exchanges).
template <class T>
__device__ __forceinline__ void pair_lse(const Params& p, int pair0, int ppb, int tpp,
                                         float* s_lse) {
  const int per_iter = kBlock / tpp;
  const int sub = threadIdx.x % tpp;
  for (int base = 0; base < ppb; base += per_iter) {
    const int jp = base + (int)threadIdx.x / tpp;
    const int pr = pair0 + jp;
    float mx = -INFINITY, z = 0.f;
    if (jp < ppb && pr < p.npairs) {
      const uint64_t i0 = (uint64_t)pr * (uint32_t)p.LK;
      for (int s = sub; s < p.LK; s += tpp) {
        const float x = load1<T>(p.attn, i0 + s);
        if (x > mx) {
          z = z * expf(mx - x) + 1.f;
          mx = x;
        } else {
          z += expf(x - mx);
        }
      }
    }
    for (int d = 1; d < tpp; d <<= 1) {
      const float mo = __shfl_xor(mx, d), zo = __shfl_xor(z, d);
      const float mn = fmaxf(mx, mo);
      z = mn == -INFINITY ? 0.f : z * expf(mx - mn) + zo * expf(mo - mn);
      mx = mn;
    }
    if (sub == 0 && jp < ppb) {
      const float lse = mx + logf(z);
      s_lse[jp] = lse;
      if (p.lse != nullptr && pr < p.npairs) p.lse[pr] = lse;
    }
  }
}

// Bilinear geometry of one sample (pair, s), shared by both directions.
// Coordinates follow x = loc_x * W - 0.5 (src/msda_triton/kernels.py:112-128),
// evaluated without contraction so that it rounds like grid_sample's
// unnormalisation.  Floors are clamped before the float->int conversion.
struct Sample {
  uint32_t off[4];  // element offsets of corners 00, 01, 10, 11 (kOobElem if outside)
  float lx, ly, a, fw, fh;
  int32_t pix;      // pixel index (start + y0 * W + x0) of corner 00; meaningful for in-map corners
  uint32_t vmask;   // bit c set when corner c lies in the map
};

// Image coordinate x = a * b + c - 0.5 as a cell (x0f = floor(x)) and a
// fraction.  The fp32 product and sum round by up to ulp(x) / 2 (W * 2^-25 px
// for a location times a width W), which the fraction alone cannot absorb:
// the exact rounding errors (two-product through an fma, two-sum) are added
// to the fraction, so it is good to ~1 ulp of itself.  A half-precision
// location times W is exact in fp32, so those inputs see no change; fp32
// decoders (W, H not powers of two) gain ~1e-3 in grad_loc against exact
// arithmetic.  kAdd (a sum c) is there for the fused form, which keeps its
// single fma for now.
template <bool kAdd>
__device__ __forceinline__ void split_coord(float a, float b, float c, float& x0f, float& fr) {
  const float p = __fmul_rn(a, b);
  float err = __fmaf_rn(a, b, -p);  // a * b - p, exact
  float s = p;
  if constexpr (kAdd) {
    s = __fadd_rn(p, c);
    const float bp = __fsub_rn(s, p);
    err = __fadd_rn(err, __fadd_rn(__fsub_rn(p, __fsub_rn(s, bp)), __fsub_rn(c, bp)));
  }
  const float t = __fsub_rn(s, 0.5f);
  x0f = floorf(t);
  float f = __fadd_rn(__fsub_rn(t, x0f), err);
  if (f < 0.f) {
    x0f -= 1.f;
    f = __fadd_rn(f, 1.f);
  } else if (f >= 1.f) {
    x0f += 1.f;
    f = __fsub_rn(f, 1.f);
  }
  fr = f;
}

// Cell and fraction of x = loc * size - 0.5 for a location in storage type
// T: a half-precision location times an integer size is exact in fp32, so
// one product, floor and subtraction give what split_coord gives at less
// cost; fp32 locations take split_coord.
template <class T>
__device__ __forceinline__ void coord_cell(float loc, float size, float& x0f, float& fr) {
  if constexpr (T::kBytes == 4) {
    split_coord<false>(loc, size, 0.f, x0f, fr);
  } else {
    const float x = __fsub_rn(__fmul_rn(loc, size), 0.5f);
    x0f = floorf(x);
    fr = x - x0f;
  }
}

//
// make_sample_at takes the sample's level (H, W, start) explicitly (kernels
// whose workgroup covers one level read them once instead of staging a
// table); make_sample looks them up in the workgroup's LDS level table.
//
// FUSED: the location is ref + offset / (W, H) (labs/solutions/lab00.py:
// 201-207), i.e. the image coordinate x = ref_x * W + offset_x - 0.5, which
// is evaluated in that form: one fma, exact for half-precision inputs of the
// usual magnitudes (so bilinear cells match exact arithmetic even at
// knots), and no division.  The weight is exp(logit - lse), `lse` being the
// pair's log-sum-exp.
template <class T, bool FUSED = false>
__device__ __forceinline__ Sample make_sample_at(const Params& p, uint32_t pair, uint32_t s,
                                                 bool valid, float lse, int32_t H, int32_t W,
                                                 int32_t st) {
  Sample r;
  if (!valid) {
    r.off[0] = r.off[1] = r.off[2] = r.off[3] = kOobElem;
    r.lx = r.ly = r.a = r.fw = r.fh = 0.f;
    r.pix = 0;
    r.vmask = 0;
    return r;
  }
  const uint32_t bq = fdiv(pair, p.div_m);
  const uint32_t b = fdiv(pair, p.div_qm);
  const uint32_t m = pair - bq * (uint32_t)p.M;
  const uint64_t pi = (uint64_t)pair * (uint32_t)p.LK + s;
  const float fw = (float)W, fh = (float)H;
  float a, x0f, y0f;
  if constexpr (FUSED) {
    const uint32_t l = fdiv(s, p.div_k);
    float rx, ry, ox, oy;
    load_xy<T>(p.ref, p.ref_levels ? (uint64_t)bq * (uint32_t)p.L + l : (uint64_t)bq, rx, ry);
    load_xy<T>(p.loc, pi, ox, oy);
    // One fma, rounded once (the owner backward forms the same value).
    const float x = __fsub_rn(__fmaf_rn(rx, fw, ox), 0.5f);
    const float y = __fsub_rn(__fmaf_rn(ry, fh, oy), 0.5f);
    x0f = floorf(x);
    y0f = floorf(y);
    r.lx = x - x0f;
    r.ly = y - y0f;
    a = expf(load1<T>(p.attn, pi) - lse);
  } else {
    float locx, locy;
    load_xy<T>(p.loc, pi, locx, locy);
    a = load1<T>(p.attn, pi);
    coord_cell<T>(locx, fw, x0f, r.lx);
    coord_cell<T>(locy, fh, y0f, r.ly);
  }
  x0f = fminf(fmaxf(x0f, -2.f), fw + 1.f);
  y0f = fminf(fmaxf(y0f, -2.f), fh + 1.f);
  const int32_t x0 = (int32_t)x0f, y0 = (int32_t)y0f;
  const bool vx0 = (x0 >= 0) & (x0 < W), vx1 = (x0 >= -1) & (x0 < W - 1);
  const bool vy0 = (y0 >= 0) & (y0 < H), vy1 = (y0 >= -1) & (y0 < H - 1);
  const uint32_t base = (b * (uint32_t)p.S * (uint32_t)p.M + m) * (uint32_t)p.D;
  const uint32_t o00 = base + (uint32_t)(st + y0 * W + x0) * (uint32_t)p.MD;
  const uint32_t o10 = o00 + (uint32_t)W * (uint32_t)p.MD;
  r.off[0] = (vy0 & vx0) ? o00 : kOobElem;
  r.off[1] = (vy0 & vx1) ? o00 + (uint32_t)p.MD : kOobElem;
  r.off[2] = (vy1 & vx0) ? o10 : kOobElem;
  r.off[3] = (vy1 & vx1) ? o10 + (uint32_t)p.MD : kOobElem;
  r.a = a;
  r.fw = fw;
  r.fh = fh;
  r.pix = st + y0 * W + x0;
  r.vmask = (uint32_t)(vy0 & vx0) | (uint32_t)(vy0 & vx1) << 1 | (uint32_t)(vy1 & vx0) << 2 |
            (uint32_t)(vy1 & vx1) << 3;
  return r;
}

template <class T, bool FUSED = false>
__device__ __forceinline__ Sample make_sample(const Params& p, const LevelTable& lt,
                                              uint32_t pair, uint32_t s, bool valid,
                                              float lse = 0.f) {
  const uint32_t l = valid ? fdiv(s, p.div_k) : 0u;
  return make_sample_at<T, FUSED>(p, pair, s, valid, lse, lt.h[l], lt.w[l], lt.start[l]);
}

}  // namespace msda
