// Projections either side of the operator (the attention layer's value,
// offset/logit and output projections, labs/solutions/lab00.py:187-208):
//
//   forward   y = x W^T + b, rows flagged in `mask` set to zero (Deformable-DETR's
//             value.masked_fill(padding_mask, 0)), output columns optionally split
//             over two weights / two output tensors (offset and logit projections
//             of the same query rows in one pass);
//   grad_x    dx = dy W  (same kernel on the transposed weight, masked rows zero);
//   grad_w/b  dW = sum_r keep_r dy_r^T x_r, db = sum_r keep_r dy_r (per-chunk
//             partials + a fixed-order reduction, no atomics: bitwise reproducible).
//
// gfx950 MFMA: v_mfma_f32_32x32x16_{bf16,f16} for half storage,
// v_mfma_f32_32x32x2_f32 for fp32; fp32 accumulation throughout, one rounding
// to the storage dtype at the end.
//
// Operand "units": every lane feeds 16 contiguous bytes of its row (A) or
// column (B) per unit.  Half: one 32x32x16 MFMA per unit, lanes 0-31 supply
// k = 16u + 0..7 and lanes 32-63 k = 16u + 8..15 (the instruction's layout).
// fp32: four 32x32x2 MFMAs per unit; lanes 0-31 hold k = 8u + 0..3, lanes
// 32-63 k = 8u + 4..7, and MFMA i pairs element i of both halves — any
// one-to-one assignment of k to (step, slot) gives the same sum as long as A
// and B agree, and this one keeps every lane's 16 bytes contiguous.
#include <type_traits>

#include "msda_device.h"
#include "msda_launch.h"

namespace msda {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

template <class T>
struct Mfma;
template <>
struct Mfma<BF16> {
  __device__ __forceinline__ static void unit(const i32x4& a, const i32x4& b, f32x16& c) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};
template <>
struct Mfma<F16> {
  __device__ __forceinline__ static void unit(const i32x4& a, const i32x4& b, f32x16& c) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                               __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};
template <>
struct Mfma<F32> {
  __device__ __forceinline__ static void unit(const i32x4& a, const i32x4& b, f32x16& c) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      c = __builtin_amdgcn_mfma_f32_32x32x2f32(__int_as_float(a[i]), __int_as_float(b[i]), c, 0,
                                               0, 0);
    }
  }
};

__device__ __forceinline__ i32x4 ld16(const void* p) { return *static_cast<const i32x4*>(p); }

// Element e (0..3) of a 32x32 MFMA accumulator quad i/4 lives at row
// 8*(i/4) + 4*(lane/32) + i%4, column lane%32.
__device__ __forceinline__ int acc_row(int i, int slot) { return (i >> 2) * 8 + slot * 4 + (i & 3); }

// ---------------------------------------------------------------------------
// y[r, c] = sum_k A(r, k) W(c, k)  (+ bias[c]; zero where mask[r]; += y if ACC)
//
// A(r, k): k <  ksplit -> a0[r*lda0 + k], else a1[r*lda1 + k - ksplit]  (SPLITA)
// W(c, k): c <  nsplit -> w0[c*ldw + k], else w1[(c-nsplit)*ldw + k]
// y(r, c): c <  nsplit -> y0[r*ldy0 + c], else y1[r*ldy1 + c - nsplit]  (SPLITN)
//
// Persistent workgroups of 4 waves; a workgroup owns 128 output columns
// (grid.y) and walks row blocks of 32 (grid.x stride); the column groups of
// one row block run on the same XCD (linear ids differ by a multiple of 8),
// so the second read of the block hits L2.  Each wave keeps its 32 weight
// columns x KP in registers for the whole kernel (KP = NU*UK, zero past K, so
// the MFMA loop has a fixed trip count): 64 registers for K <= 256 in half
// precision, and three workgroups share a CU.
//
// LDS rows are KP*E bytes, unpadded; 16-byte chunk c of row r sits at chunk
// position c ^ (r & 15), so the 16 rows a quarter-wave reads for one MFMA
// fragment fall on 16 distinct 4-bank groups.  The weights enter through the
// same buffers once (coalesced row loads).  Activation blocks are copied from
// memory straight into LDS (buffer_load_dwordx4 ... lds, one block ahead, two
// buffers, one barrier per block) -- no staging registers; with SPLITA the
// two source tensors need per-lane descriptors, so that variant stages through
// registers instead.  Buffer range checks turn rows past the end into zero
// reads and dropped stores, so every block issues the same instructions.
// The row mask of a block travels as one 32-bit word (wave 0's ballot).
// Output: lanes 2m, 2m+1 hold columns c, c+1; one DPP swap per row pair lets
// each lane store two adjacent columns of one row.
// ---------------------------------------------------------------------------
constexpr uint32_t kOob = 0x80000000u;  // beyond any num_records used here

template <class T>
using PairT = typename std::conditional<T::kBytes == 4, uint2, uint32_t>::type;

template <class T>
__device__ __forceinline__ PairT<T> make_pair(float lo, float hi) {
  if constexpr (T::kBytes == 4) {
    return uint2{__float_as_uint(lo), __float_as_uint(hi)};
  } else {
    return pack2<T>(lo, hi);
  }
}

template <class T>
__device__ __forceinline__ void store_pair(__amdgpu_buffer_rsrc_t r, uint32_t off, PairT<T> v) {
  if constexpr (T::kBytes == 4) {
    __builtin_amdgcn_raw_buffer_store_b64(i32x2{(int)v.x, (int)v.y}, r, off, 0, 0);
  } else {
    __builtin_amdgcn_raw_buffer_store_b32(v, r, off, 0, 0);
  }
}

__device__ __forceinline__ float swap_pair_lane(float v) {
  // quad_perm [1, 0, 3, 2]: exchange with lane ^ 1.
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false));
}

__device__ __forceinline__ int swz(int r, int c) { return c ^ (r & 15); }

template <int NU, bool SPLITA>
constexpr int proj_waves_per_eu() {
  return NU == 16 ? 3 : 2;
}

// WDIRECT: weights loaded straight into registers (launches with at most two
// row blocks per workgroup) instead of through LDS.
template <class T, int NU, bool ACC, bool SPLITA, bool SPLITN, bool WDIRECT>
__global__ __launch_bounds__(kBlock)
__attribute__((amdgpu_waves_per_eu(proj_waves_per_eu<NU, SPLITA>())))
void proj_kernel(ProjArgs p) {
  constexpr int E = T::kBytes;
  constexpr int EPU = 16 / E;          // elements per lane per unit
  constexpr int UK = 2 * EPU;          // k covered by one unit
  constexpr int KP = NU * UK;
  constexpr int ROWB = KP * E;         // LDS bytes per row
  constexpr int CPR = ROWB / 16;       // 16-byte chunks per row
  constexpr int BUFB = 32 * ROWB;      // one 32-row block
  constexpr int IPW = BUFB / 1024 / 4; // 1 KB direct-to-LDS loads per wave per block
  constexpr int ROUNDS = 32 * CPR / kBlock;
  // Half-precision outputs (K <= 256) leave through an LDS tile: each wave
  // parks its 32 x 32 results, then every lane stores 16-byte row chunks of
  // the workgroup's 32 x 128 block (full 256-byte row segments).
  constexpr bool WIDE = E == 2 && NU == 16;
  constexpr int OPITCH = 128 * E + 16;
  __shared__ __align__(16) unsigned char smem[2 * BUFB];
  __shared__ __align__(16) unsigned char sout[WIDE ? 2 : 1][WIDE ? 32 * OPITCH : 16];
  __shared__ uint32_t smask[2];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int rl = lane & 31, slot = lane >> 5;
  const int nrows = (int)p.rows;  // one row slice: < 2^31 bytes per operand
  const uint32_t lda0 = (uint32_t)p.lda0, lda1 = (uint32_t)p.lda1;
  const __amdgpu_buffer_rsrc_t ra0 = make_rsrc(p.a0, p.abytes0);
  const __amdgpu_buffer_rsrc_t ra1 = make_rsrc(SPLITA ? p.a1 : p.a0, SPLITA ? p.abytes1 : 0u);
  const __amdgpu_buffer_rsrc_t ry0 = make_rsrc(p.y0, p.ybytes0);
  const __amdgpu_buffer_rsrc_t ry1 = make_rsrc(SPLITN ? p.y1 : p.y0, SPLITN ? p.ybytes1 : 0u);
  const __amdgpu_buffer_rsrc_t rmask = make_rsrc(p.mask, p.mask != nullptr ? (uint32_t)p.rows : 0u);

  // ---- weights -> registers ----
  const int colw = blockIdx.y * 128;  // first output column of this workgroup
  const int col0 = colw + wave * 32;  // ... of this wave
  i32x4 w[NU];
  if constexpr (WDIRECT) {
    // Lane (rl, slot) of a wave holds, for its output column c = col0 + rl,
    // the 16-byte pieces 2u + slot (u < NU) of weight row c: loaded straight
    // into the MFMA operand layout, all NU loads in flight (one memory latency,
    // no LDS passes or barriers; the weights are L2-resident after the first
    // workgroups).  Buffer range checks give zeros past N and past K.
    {
      const int c = col0 + rl;
      const bool hi = c >= p.nsplit;
      const int cr = hi ? c - p.nsplit : c;  // row within its weight
      const int nw = hi ? p.N - p.nsplit : p.nsplit;
      const __amdgpu_buffer_rsrc_t rw =
          make_rsrc(hi ? p.w1 : p.w0, (uint32_t)((int64_t)nw * p.ldw * E));
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        const int k = (2 * u + slot) * EPU;
        const uint32_t off = (c < p.N && k < p.K) ? (uint32_t)(((int64_t)cr * p.ldw + k) * E) : kOob;
        w[u] = __builtin_amdgcn_raw_buffer_load_b128(rw, off, 0, 0);
      }
    }
  } else {
    // Two passes of 64 weight rows through LDS, loaded as coalesced row
    // chunks (for NU == 16 both passes' loads are issued before the first
    // LDS pass: one memory latency for the whole prologue).  Used by the
    // launches with several row blocks per workgroup: there hundreds of
    // workgroups start at once, and the direct path's scattered 32-byte
    // weight reads slowed the value projection's forward (24.8 -> 27.3 us).
    constexpr int WQ = 2 * ROUNDS;      // loads per thread per pass
    auto wload = [&](int pass, int q) {
      const int idx = tid + kBlock * q;
      const int r = idx / CPR;  // 0..63
      const int ch = idx - r * CPR;
      const int c = colw + pass * 64 + r;
      const int k = ch * EPU;
      i32x4 v = i32x4{0, 0, 0, 0};
      if (c < p.N && k < p.K) {
        const bool hi = c >= p.nsplit;
        const char* base = static_cast<const char*>(hi ? p.w1 : p.w0);
        v = ld16(base + ((int64_t)(hi ? c - p.nsplit : c) * p.ldw + k) * E);
      }
      return v;
    };
    auto wpark = [&](int q, const i32x4& v) {
      const int idx = tid + kBlock * q;
      const int r = idx / CPR;
      const int ch = idx - r * CPR;
      *reinterpret_cast<i32x4*>(smem + r * ROWB + swz(r, ch) * 16) = v;
    };
    auto wpick = [&](int pass) {
      __syncthreads();
      if ((wave >> 1) == pass) {
        const int r = (wave & 1) * 32 + rl;
#pragma unroll
        for (int u = 0; u < NU; ++u) {
          w[u] = *reinterpret_cast<const i32x4*>(smem + r * ROWB + swz(r, 2 * u + slot) * 16);
        }
      }
      __syncthreads();
    };
    if constexpr (NU == 16) {
      i32x4 st0[WQ], st1[WQ];
#pragma unroll
      for (int q = 0; q < WQ; ++q) st0[q] = wload(0, q);
#pragma unroll
      for (int q = 0; q < WQ; ++q) st1[q] = wload(1, q);
#pragma unroll
      for (int q = 0; q < WQ; ++q) wpark(q, st0[q]);
      wpick(0);
#pragma unroll
      for (int q = 0; q < WQ; ++q) wpark(q, st1[q]);
      wpick(1);
    } else {
      // NU == 32: a weight row is 1 KB, one wave instruction's worth of
      // 16-byte pieces, so each pass goes HBM -> LDS directly (lane `lane`
      // of the instruction for LDS row r fills position `lane`, i.e. chunk
      // swz(r, lane)); staging the pass in registers held 64 VGPRs beside
      // the 128 weight registers and spilled.
      static_assert(ROWB == kWave * 16, "one weight row per wave instruction");
      const __amdgpu_buffer_rsrc_t rw0 =
          make_rsrc(p.w0, (uint32_t)((int64_t)p.nsplit * p.ldw * E));
      const __amdgpu_buffer_rsrc_t rw1 =
          make_rsrc(p.w1 != nullptr ? p.w1 : p.w0,
                    p.w1 != nullptr ? (uint32_t)((int64_t)(p.N - p.nsplit) * p.ldw * E) : 0u);
#pragma unroll
      for (int pass = 0; pass < 2; ++pass) {
#pragma unroll
        for (int j = 0; j < 64 / (kBlock / kWave); ++j) {
          const int r = wave * (64 / (kBlock / kWave)) + j;  // LDS row
          const int c = colw + pass * 64 + r;                // weight row
          const int kk = swz(r, lane) * EPU;
          const bool hi = c >= p.nsplit;
          const int cr = hi ? c - p.nsplit : c;
          const uint32_t off =
              (c < p.N && kk < p.K) ? (uint32_t)(((int64_t)cr * p.ldw + kk) * E) : kOob;
          unsigned char* dst = smem + r * ROWB;
          if (hi) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rw1, dst, 16, off, 0, 0, 0);
          } else {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rw0, dst, 16, off, 0, 0, 0);
          }
        }
        __builtin_amdgcn_s_waitcnt(0);  // this pass's rows have landed in LDS
        wpick(pass);
      }
    }
  }
  const int c_lane = col0 + rl;
  float bias = 0.f;
  {
    const bool hi = c_lane >= p.nsplit;
    const void* bp = hi ? p.b1 : p.b0;
    if (c_lane < p.N && bp != nullptr) bias = load1<T>(bp, (uint64_t)(hi ? c_lane - p.nsplit : c_lane));
  }

  // ---- activation blocks ----
  // Rows are clamped to nrows, whose offsets lie at or past num_records.
  // Each lane's 16-byte piece goes HBM -> LDS directly (its LDS slot is fixed
  // by the lane id).  With a split input the lanes pick their source by a
  // branch: the two loads run under complementary EXEC masks, and a masked
  // lane neither fetches nor writes LDS (no staging registers: loading both
  // sources into registers and merging them held two 16-byte results per
  // piece in flight and spilled the weight registers).
  uint32_t pre_mask = 0u;
  auto issue_block = [&](int pb, int blk) {
    const int r0 = blk * 32;
    unsigned char* b = smem + pb * BUFB;
#pragma unroll
    for (int j = 0; j < IPW; ++j) {
      const int byte = (wave * IPW + j) * 1024 + lane * 16;
      const int r = byte / ROWB;
      const int c = swz(r, (byte - r * ROWB) / 16);
      const int k = c * EPU;
      const uint32_t row = (uint32_t)min(r0 + r, nrows);
      unsigned char* dst = b + (wave * IPW + j) * 1024;
      if constexpr (!SPLITA) {
        const uint32_t off = k < p.K ? (row * lda0 + k) * E : kOob;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(ra0, dst, 16, off, 0, 0, 0);
      } else {
        if (k < p.ksplit) {
          __builtin_amdgcn_raw_ptr_buffer_load_lds(ra0, dst, 16, (row * lda0 + k) * E, 0, 0, 0);
        } else {
          const uint32_t off = k < p.K ? (row * lda1 + k - p.ksplit) * E : kOob;
          __builtin_amdgcn_raw_ptr_buffer_load_lds(ra1, dst, 16, off, 0, 0, 0);
        }
      }
    }
    pre_mask = (wave == 0 && lane < 32)
                   ? (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(
                         rmask, (uint32_t)min(r0 + lane, nrows), 0, 0)
                   : 0u;
  };
  const int blk0 = blockIdx.x;
  issue_block(0, blk0);
  int pb = 0;
  // Blocks blk0 + j*G alternate between LDS buffers 0 and 1.  Buffer pb^1 is
  // refilled (issue_block) right after the barrier of block j, which every
  // wave passes only after finishing block j-1, the buffer's previous reader.
  for (int blk = blk0; blk < p.nblocks; blk += gridDim.x) {
    if (wave == 0) {
      const uint64_t bits = __ballot(pre_mask != 0u);
      if (lane == 0) smask[pb] = (uint32_t)bits;
    }
    __builtin_amdgcn_s_waitcnt(0);  // this block's copies into LDS have landed
    __syncthreads();
    issue_block(pb ^ 1, blk + gridDim.x);
    const unsigned char* b = smem + pb * BUFB;
    // The accumulator starts at the bias (every element of a lane's tile is
    // in its column), so the epilogue adds nothing.
    f32x16 acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = bias;
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const i32x4 a = *reinterpret_cast<const i32x4*>(b + rl * ROWB + swz(rl, 2 * u + slot) * 16);
      Mfma<T>::unit(a, w[u], acc);
    }
    const uint32_t mword = smask[pb];
    const int r0 = blk * 32;
    const bool odd = rl & 1;
    const int cp = c_lane - (odd ? 1 : 0);  // first column of this lane's pair
    const bool hi = SPLITN && cp >= p.nsplit;
    const int cc = hi ? cp - p.nsplit : cp;
    const uint32_t ldy = (uint32_t)(hi ? p.ldy1 : p.ldy0);
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      const int i0 = 2 * jj, i1 = 2 * jj + 1;
      const int ra = acc_row(i0, slot), rb = acc_row(i1, slot);
      float v0 = acc[i0], v1 = acc[i1];
      if (mword != 0u) {  // wave-uniform: blocks without padded rows skip the selects
        v0 = ((mword >> ra) & 1u) ? 0.f : v0;
        v1 = ((mword >> rb) & 1u) ? 0.f : v1;
      }
      // even lane keeps row ra and takes the partner's (row ra, c+1);
      // odd lane keeps row rb and takes the partner's (row rb, c-1).
      const float x = swap_pair_lane(odd ? v0 : v1);
      const int rr = odd ? rb : ra;
      PairT<T> pv = odd ? make_pair<T>(x, v1) : make_pair<T>(v0, x);
      if constexpr (WIDE) {
        *reinterpret_cast<PairT<T>*>(&sout[pb][rr * OPITCH + (cp - colw) * E]) = pv;
      } else {
        const int row = r0 + rr;
        const uint32_t off =
            (row < nrows && cp < p.N) ? ((uint32_t)row * ldy + (uint32_t)cc) * E : kOob;
        if constexpr (ACC) {
          const i32x2 old = __builtin_amdgcn_raw_buffer_load_b64(ry0, off, 0, 0);
          pv.x = __float_as_uint(__uint_as_float(pv.x) + __int_as_float(old[0]));
          pv.y = __float_as_uint(__uint_as_float(pv.y) + __int_as_float(old[1]));
        }
        if constexpr (SPLITN) {
          store_pair<T>(ry0, hi ? kOob : off, pv);
          store_pair<T>(ry1, hi ? off : kOob, pv);
        } else {
          store_pair<T>(ry0, off, pv);
        }
      }
    }
    if constexpr (WIDE) {
      // sout[pb] is rewritten two blocks later, behind the barrier of the
      // block in between (see above), so one barrier here suffices.
      __syncthreads();
#pragma unroll
      for (int i = 0; i < 32 * 16 / kBlock; ++i) {
        const int id = tid + kBlock * i;
        const int rr = id >> 4, ch = id & 15;
        const int col = colw + ch * 8;
        const int row = r0 + rr;
        const bool h2 = SPLITN && col >= p.nsplit;
        const uint32_t ld2 = (uint32_t)(h2 ? p.ldy1 : p.ldy0);
        const int c2 = h2 ? col - p.nsplit : col;
        const uint32_t off =
            (row < nrows && col < p.N) ? ((uint32_t)row * ld2 + (uint32_t)c2) * E : kOob;
        const i32x4 v = *reinterpret_cast<const i32x4*>(&sout[pb][rr * OPITCH + ch * 16]);
        if constexpr (SPLITN) {
          __builtin_amdgcn_raw_buffer_store_b128(v, ry0, h2 ? kOob : off, 0, 0);
          __builtin_amdgcn_raw_buffer_store_b128(v, ry1, h2 ? off : kOob, 0, 0);
        } else {
          __builtin_amdgcn_raw_buffer_store_b128(v, ry0, off, 0, 0);
        }
      }
    }
    pb ^= 1;
  }
}

// wt[c*K + k] = k < ksplit ? w0[k*N + c] : w1[(k - ksplit)*N + c]: the weights
// [w0; w1] (K x N) transposed, so that grad_input = grad_output [w0; w1] runs
// on proj_kernel with wt as its (N x K) weight.  32 x 32 tiles through LDS,
// four elements per thread.
template <class T>
__global__ __launch_bounds__(kBlock) void transpose_kernel(const void* w0, const void* w1,
                                                           int ksplit, int K, int N, void* wt) {
  __shared__ float tile[32][33];
  const int k0 = blockIdx.x * 32, c0 = blockIdx.y * 32;
  const int cr = threadIdx.x & 31, kq = threadIdx.x >> 5;  // 8 row groups of 4
  float v[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int k = min(k0 + kq * 4 + j, K - 1), c = min(c0 + cr, N - 1);
    v[j] = k < ksplit ? load1<T>(w0, (uint64_t)k * N + c)
                      : load1<T>(w1, (uint64_t)(k - ksplit) * N + c);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) tile[kq * 4 + j][cr] = v[j];
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = c0 + kq * 4 + j, k = k0 + cr;
    if (k < K && c < N) store1<T>(wt, (uint64_t)c * K + k, tile[cr][kq * 4 + j]);
  }
}

// ---------------------------------------------------------------------------
// Partial weight / bias gradients over one chunk of rows:
//   ws[chunk][n][k] = sum_{r in chunk} keep_r G(r, n) X(r, k)
//   wsb[chunk][n]   = sum_{r in chunk} keep_r G(r, n)
// G(r, n): n < nsplit -> g0[r*ldg0 + n], else g1[r*ldg1 + n - nsplit].
// A workgroup owns a 128 (n) x 128 (k) tile, each wave a 64 x 64 quarter
// (2 x 2 MFMA tiles).  The MFMA reduction runs over rows r, so every fragment
// is 8 (half) or 4 (fp32) consecutive rows of ONE column: the tiles are kept
// in LDS transposed (LDS row = one n or one k, RS consecutive r, pitch 136
// bytes, which spreads 32 consecutive columns over all 64 banks).  Staging
// per step (RS = 128/E rows): lane l loads columns 2l, 2l+1 of one row per
// load (a wave covers one 256/512-byte row segment, fully coalesced), one
// step ahead in registers; groups of 4 (half) / 2 (fp32) rows are repacked
// with v_perm into per-column 8-byte pieces and written with ds_write_b64.
// Workgroups are numbered so that the tiles of a chunk share an XCD
// (dispatch is round-robin over the 8 XCDs): the re-reads of each G and X
// row segment by the chunk's other tiles then hit the same L2.
// ---------------------------------------------------------------------------
template <class T, bool MASKED, bool SPLITG, int NSET>
__global__ __launch_bounds__(kBlock, NSET == 2 ? 2 : 1) void wgrad_kernel(WgradArgs p) {
  constexpr int E = T::kBytes;
  constexpr int EPU = 16 / E;
  constexpr int UK = 2 * EPU;
  constexpr int TW = 128;              // tile width in n and in k
  constexpr int RS = 128 / E;          // rows per step
  constexpr int RW = RS / 4;           // rows per wave per step
  constexpr int PITCH = RS * E + 8;    // LDS bytes per transposed column
  constexpr int TILE_BYTES = TW * PITCH;
  __shared__ __align__(16) unsigned char lds[2][2 * TILE_BYTES];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int rl = lane & 31, slot = lane >> 5;
  const int wn = wave >> 1, wk = wave & 1;

  const int ntiles = p.ntile_n * p.ntile_k;
  const int xcd = blockIdx.x & 7;
  const int j = blockIdx.x >> 3;
  const int tile = j % ntiles;
  const int chunk = (j / ntiles) * 8 + xcd;
  const int tn = tile / p.ntile_k, tk = tile - tn * p.ntile_k;
  const int n0 = tn * TW, k0 = tk * TW;
  const int64_t rbeg = (int64_t)chunk * p.rows_per_chunk;
  const int64_t rend = rbeg + p.rows_per_chunk < p.rows ? rbeg + p.rows_per_chunk : p.rows;

  // Staging: lane l covers CPL = 16/E consecutive columns (one 16-byte load)
  // of RG row groups; each group is NI = 4 consecutive rows, so one wave
  // instruction reads RG rows x 256 bytes (coalesced) and a lane ends up with a
  // 4-row x CPL-column block that it writes to LDS column by column.  G and X
  // are read through buffer descriptors based at the chunk's first row: the
  // row offset is a wave-uniform scalar (soffset), the lane's row group and
  // columns a per-lane constant (voffset), and rows past the chunk's end fall
  // outside num_records and read as zero.
  constexpr int CPL = 16 / E;      // columns per lane
  constexpr int LPR = TW / CPL;    // lanes per tile row
  constexpr int NI = 4;            // rows per group (loads per tensor per step)
  const int lc = lane % LPR, rg = lane / LPR;
  const int gc = n0 + lc * CPL, xc = k0 + lc * CPL;
  const bool g_hi = gc >= p.nsplit;
  const uint32_t ldg0 = (uint32_t)p.ldg0 * E, ldg1 = (uint32_t)p.ldg1 * E;
  const uint32_t ldx = (uint32_t)p.ldx * E;
  const int64_t nr = rend > rbeg ? rend - rbeg : 0;
  const __amdgpu_buffer_rsrc_t rg0 =
      make_rsrc(static_cast<const char*>(p.g0) + rbeg * p.ldg0 * E, (uint32_t)(nr * ldg0));
  const __amdgpu_buffer_rsrc_t rg1 =
      make_rsrc(SPLITG ? static_cast<const char*>(p.g1) + rbeg * p.ldg1 * E : p.g0,
                SPLITG ? (uint32_t)(nr * ldg1) : 0u);
  const __amdgpu_buffer_rsrc_t rx =
      make_rsrc(static_cast<const char*>(p.x) + rbeg * p.ldx * E, (uint32_t)(nr * ldx));
  const __amdgpu_buffer_rsrc_t rm = make_rsrc(MASKED ? p.mask + rbeg : p.x, MASKED ? (uint32_t)nr : 0u);
  const uint32_t rgo = (uint32_t)(rg * NI);
  const uint32_t vg0 = (gc < p.N && !g_hi) ? rgo * ldg0 + (uint32_t)gc * E : kOob;
  const uint32_t vg1 = (gc < p.N && g_hi) ? rgo * ldg1 + (uint32_t)(gc - p.nsplit) * E : kOob;
  const uint32_t vx = xc < p.K ? rgo * ldx + (uint32_t)xc * E : kOob;
  const int wv = __builtin_amdgcn_readfirstlane(wave);

  // NSET steps in flight per workgroup, register sets 0 .. NSET-1 rotating:
  // four (~128 KB) when the launch has one workgroup per CU; two when it
  // has more, which then fit two workgroups per CU (the registers of two
  // waves per SIMD).  Masked rows are zeroed when parked: lane i < RW of a
  // wave loads the mask byte of its share's row i, and a ballot turns them
  // into bits.
  i32x4 gp[NSET][NI], xp[NSET][NI];
  uint32_t mk[NSET];
  auto load_step = [&](int sset, int64_t r0) {
    const uint32_t row0 = (uint32_t)(r0 - rbeg) + (uint32_t)(wv * RW);
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      i32x4 g = __builtin_amdgcn_raw_buffer_load_b128(rg0, vg0, (row0 + i) * ldg0, 0);
      if constexpr (SPLITG) g |= __builtin_amdgcn_raw_buffer_load_b128(rg1, vg1, (row0 + i) * ldg1, 0);
      gp[sset][i] = g;
      xp[sset][i] = __builtin_amdgcn_raw_buffer_load_b128(rx, vx, (row0 + i) * ldx, 0);
    }
    if constexpr (MASKED) {
      mk[sset] = __builtin_amdgcn_raw_buffer_load_b8(rm, lane < RW ? (uint32_t)lane : kOob, row0, 0);
    }
  };
  auto park_step = [&](int sset, unsigned char* b) {
    uint32_t masked = 0;
    if constexpr (MASKED) masked = (uint32_t)__ballot(lane < RW && mk[sset] != 0u) >> rgo;
    i32x4 gq[NI], xq[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const bool off = (masked >> i) & 1u;
      gq[i] = off ? i32x4{0, 0, 0, 0} : gp[sset][i];
      xq[i] = off ? i32x4{0, 0, 0, 0} : xp[sset][i];
    }
    // Tile column c lives in LDS row c ^ ((c >> 5) & 3) (see cslot): the
    // writers of one instruction (columns 8*lc + j, or 4*lc + j for fp32)
    // then hit distinct bank groups, and the 32 consecutive columns a
    // fragment read covers stay a permutation of 32 rows.  Row span of this
    // lane: wave*RW + rgo + 0..3.
    unsigned char* rowoff = b + (wave * RW + (int)rgo) * E;
    const int a = (lc * CPL >> 5) & 3;
    auto col = [&](int j) { return rowoff + (lc * CPL + (j ^ a)) * PITCH; };
    if constexpr (E == 4) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        unsigned char* tg = col(j);
        unsigned char* tx = tg + TILE_BYTES;
        *reinterpret_cast<uint2*>(tg) = uint2{(uint32_t)gq[0][j], (uint32_t)gq[1][j]};
        *reinterpret_cast<uint2*>(tg + 8) = uint2{(uint32_t)gq[2][j], (uint32_t)gq[3][j]};
        *reinterpret_cast<uint2*>(tx) = uint2{(uint32_t)xq[0][j], (uint32_t)xq[1][j]};
        *reinterpret_cast<uint2*>(tx + 8) = uint2{(uint32_t)xq[2][j], (uint32_t)xq[3][j]};
      }
    } else {
      // dword m of a row = columns 2m (low half) and 2m+1 (high half);
      // [r0.lo16 | r1.lo16] = perm(r1, r0, 0x05040100), high halves 0x07060302.
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const uint32_t g0 = gq[0][m], g1 = gq[1][m], g2 = gq[2][m], g3 = gq[3][m];
        const uint32_t x0 = xq[0][m], x1 = xq[1][m], x2 = xq[2][m], x3 = xq[3][m];
        unsigned char* te = col(2 * m);
        unsigned char* to = col(2 * m + 1);
        *reinterpret_cast<uint2*>(te) =
            uint2{__builtin_amdgcn_perm(g1, g0, 0x05040100u), __builtin_amdgcn_perm(g3, g2, 0x05040100u)};
        *reinterpret_cast<uint2*>(to) =
            uint2{__builtin_amdgcn_perm(g1, g0, 0x07060302u), __builtin_amdgcn_perm(g3, g2, 0x07060302u)};
        *reinterpret_cast<uint2*>(te + TILE_BYTES) =
            uint2{__builtin_amdgcn_perm(x1, x0, 0x05040100u), __builtin_amdgcn_perm(x3, x2, 0x05040100u)};
        *reinterpret_cast<uint2*>(to + TILE_BYTES) =
            uint2{__builtin_amdgcn_perm(x1, x0, 0x07060302u), __builtin_amdgcn_perm(x3, x2, 0x07060302u)};
      }
    }
  };
  auto frag = [](const unsigned char* q) {
    const uint2 lo = *reinterpret_cast<const uint2*>(q);
    const uint2 hi = *reinterpret_cast<const uint2*>(q + 8);
    return i32x4{(int)lo.x, (int)lo.y, (int)hi.x, (int)hi.y};
  };

  const bool want_bias = p.wsb != nullptr && tk == 0 && wk == 0;
  f32x16 acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a) {
#pragma unroll
    for (int c = 0; c < 2; ++c) acc[a][c] = f32x16{};
  }
  float bsum[2] = {0.f, 0.f};
  // One step: park register set `sset` in LDS buffer sset & 1, refill the set
  // with the rows NSET steps ahead, MFMA.  An LDS buffer is rewritten two
  // steps after it was read, behind the barrier of the step in between, which
  // every wave passes only after finishing its reads.
  auto step = [&](int sset, int64_t r0) {
    unsigned char* b = lds[sset & 1];
    park_step(sset, b);
    __syncthreads();
    load_step(sset, r0 + NSET * RS);
    // Fragment rows: column c = base + rl with base = 64*w + 32*h, stored in
    // LDS row c ^ ((c >> 5) & 3) = base + (rl ^ ((2*w + h) & 3)).
    const unsigned char* ta[2];
    const unsigned char* tb[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      ta[h] = b + (wn * 64 + h * 32 + (rl ^ ((2 * wn + h) & 3))) * PITCH + slot * 16;
      tb[h] = b + TILE_BYTES + (wk * 64 + h * 32 + (rl ^ ((2 * wk + h) & 3))) * PITCH + slot * 16;
    }
#pragma unroll
    for (int u = 0; u < RS / UK; ++u) {
      i32x4 fa[2], fb[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        fa[h] = frag(ta[h] + u * 32);
        fb[h] = frag(tb[h] + u * 32);
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int g = 0; g < 2; ++g) Mfma<T>::unit(fa[h], fb[g], acc[h][g]);
      }
      if (want_bias) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
          for (int w2 = 0; w2 < 4; ++w2) {
            if constexpr (E == 4) {
              bsum[h] += __int_as_float(fa[h][w2]);
            } else {
              float lo, hi;
              unpack2<T>((uint32_t)fa[h][w2], lo, hi);
              bsum[h] += lo + hi;
            }
          }
        }
      }
    }
  };
  if (rbeg < rend) {
#pragma unroll
    for (int s2 = 0; s2 < NSET; ++s2) load_step(s2, rbeg + s2 * RS);
    // Steps past the end read zeros (outside the descriptors): harmless.
    for (int64_t r0 = rbeg; r0 < rend; r0 += NSET * RS) {
#pragma unroll
      for (int s2 = 0; s2 < NSET; ++s2) step(s2, r0 + s2 * RS);
    }
  }

  // ---- partials out (plain stores; every slot of ws is written) ----
  float* ws = p.ws + (int64_t)chunk * p.N * p.K;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const int k = k0 + wk * 64 + g * 32 + rl;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int n = n0 + wn * 64 + h * 32 + acc_row(i, slot);
        if (n < p.N && k < p.K) ws[(int64_t)n * p.K + k] = acc[h][g][i];
      }
    }
  }
  if (want_bias) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float v = bsum[h] + __shfl_xor(bsum[h], 32);
      const int n = n0 + wn * 64 + h * 32 + rl;
      if (slot == 0 && n < p.N) p.wsb[(int64_t)chunk * p.N + n] = v;
    }
  }
}

// dW / db = fixed-order sums of the chunk partials, rounded once.  A
// workgroup owns 64 consecutive outputs (16 groups of 4) and all chunks: lane
// t loads outputs 4*(t%16).. of chunks t/16, t/16 + 16, ... (16-byte loads,
// all issued together), sums them in chunk order, and a fixed LDS tree adds
// the 16 chunk residues -- the same order on every run.
template <class T>
__global__ __launch_bounds__(kBlock) void wgrad_reduce_kernel(WgradArgs p, void* dw0, void* dw1,
                                                              void* db0, void* db1) {
  __shared__ float4 red[kBlock];
  const int64_t nk = (int64_t)p.N * p.K;
  const int64_t total = nk + (p.wsb != nullptr ? p.N : 0);
  const int g = threadIdx.x & 15, cs = threadIdx.x >> 4;
  const int nper = (p.nchunks + 15) / 16;  // chunks per lane (some past the end)
  for (int64_t base = (int64_t)blockIdx.x * 64; base < total; base += (int64_t)gridDim.x * 64) {
    const int64_t i0 = base + 4 * g;  // this lane's 4 outputs: i0 .. i0+3
    float4 acc = {0.f, 0.f, 0.f, 0.f};
    if (base + 64 <= nk && (nk & 3) == 0 && nper == 1) {
      // At most 16 chunks: one partial per lane (cs), none past the end.
      if (cs < p.nchunks) {
        const float4 v = *reinterpret_cast<const float4*>(p.ws + (int64_t)cs * nk + i0);
        acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
      }
    } else if (base + 64 <= nk && (nk & 3) == 0) {
      for (int j0 = 0; j0 < nper; j0 += 4) {
        float4 v[4];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int c = cs + 16 * (j0 + jj);
          const int cc = c < p.nchunks ? c : p.nchunks - 1;
          v[jj] = *reinterpret_cast<const float4*>(p.ws + (int64_t)cc * nk + i0);
          if (c >= p.nchunks) v[jj] = float4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          acc.x += v[jj].x; acc.y += v[jj].y; acc.z += v[jj].z; acc.w += v[jj].w;
        }
      }
    } else {
      float t[4] = {0.f, 0.f, 0.f, 0.f};
      for (int e = 0; e < 4; ++e) {
        const int64_t i = i0 + e;
        if (i >= total) continue;
        for (int c = cs; c < p.nchunks; c += 16) {
          t[e] += i < nk ? p.ws[(int64_t)c * nk + i] : p.wsb[(int64_t)c * p.N + (i - nk)];
        }
      }
      acc = float4{t[0], t[1], t[2], t[3]};
    }
    red[threadIdx.x] = acc;
    __syncthreads();
#pragma unroll
    for (int h = 8; h >= 1; h >>= 1) {  // chunk groups cs, cs + h
      if (cs < h) {
        float4 o = red[threadIdx.x + 16 * h];
        float4 m = red[threadIdx.x];
        m.x += o.x; m.y += o.y; m.z += o.z; m.w += o.w;
        red[threadIdx.x] = m;
      }
      __syncthreads();
    }
    if (cs == 0) {
      const float sv[4] = {red[g].x, red[g].y, red[g].z, red[g].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t i = i0 + e;
        if (i >= total) continue;
        if (i < nk) {
          const int n = (int)(i / p.K);
          const int k = (int)(i - (int64_t)n * p.K);
          if (n < p.nsplit) {
            if (dw0 != nullptr) store1<T>(dw0, (uint64_t)n * p.K + k, sv[e]);
          } else if (dw1 != nullptr) {
            store1<T>(dw1, (uint64_t)(n - p.nsplit) * p.K + k, sv[e]);
          }
        } else {
          const int n = (int)(i - nk);
          if (n < p.nsplit) {
            if (db0 != nullptr) store1<T>(db0, (uint64_t)n, sv[e]);
          } else if (db1 != nullptr) {
            store1<T>(db1, (uint64_t)(n - p.nsplit), sv[e]);
          }
        }
      }
    }
    __syncthreads();
  }
}

int cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0) {
      n = 256;
    }
    cached[dev] = n;
  }
  return cached[dev];
}

template <class T, int NU, bool ACC, bool SPLITA, bool SPLITN>
hipError_t launch_proj_t(ProjArgs a, hipStream_t st) {
  const int gy = (a.N + 127) / 128;
  // Resident workgroups per CU = waves per SIMD (4 waves per workgroup).
  const int occ = proj_waves_per_eu<NU, SPLITA>();
  int want = cu_count() * occ / gy;
  want = (want + 7) / 8 * 8;  // keep gx a multiple of 8: same XCD across grid.y
  const int per = (a.nblocks + want - 1) / want;
  int gx = (a.nblocks + per - 1) / per;
  gx = (gx + 7) / 8 * 8;
  if (per <= 2) {
    hipLaunchKernelGGL((proj_kernel<T, NU, ACC, SPLITA, SPLITN, true>), dim3(gx, gy), dim3(kBlock),
                       0, st, a);
  } else {
    hipLaunchKernelGGL((proj_kernel<T, NU, ACC, SPLITA, SPLITN, false>), dim3(gx, gy), dim3(kBlock),
                       0, st, a);
  }
  return hipGetLastError();
}

template <class T, int NU, bool ACC>
hipError_t launch_proj_split(const ProjArgs& a, hipStream_t st) {
  const bool sa = a.ksplit < a.K, sn = a.nsplit < a.N;
  if (sa) return launch_proj_t<T, NU, ACC, true, false>(a, st);  // never both: callers
  if (sn) return launch_proj_t<T, NU, ACC, false, true>(a, st);  // split one side only
  return launch_proj_t<T, NU, ACC, false, false>(a, st);
}

template <class T>
hipError_t launch_proj_dtype(const ProjArgs& a, bool accumulate, hipStream_t st) {
  if constexpr (T::kBytes == 4) {
    if (accumulate) return launch_proj_split<T, 32, true>(a, st);
    return launch_proj_split<T, 32, false>(a, st);
  } else {
    if (a.K <= 256) return launch_proj_split<T, 16, false>(a, st);
    return launch_proj_split<T, 32, false>(a, st);
  }
}

template <class T, int NSET>
void launch_wgrad_nset(const WgradArgs& a, int nblk, hipStream_t st) {
  const bool m = a.mask != nullptr, sg = a.nsplit < a.N;
  if (m && sg) {
    hipLaunchKernelGGL((wgrad_kernel<T, true, true, NSET>), dim3(nblk), dim3(kBlock), 0, st, a);
  } else if (m) {
    hipLaunchKernelGGL((wgrad_kernel<T, true, false, NSET>), dim3(nblk), dim3(kBlock), 0, st, a);
  } else if (sg) {
    hipLaunchKernelGGL((wgrad_kernel<T, false, true, NSET>), dim3(nblk), dim3(kBlock), 0, st, a);
  } else {
    hipLaunchKernelGGL((wgrad_kernel<T, false, false, NSET>), dim3(nblk), dim3(kBlock), 0, st, a);
  }
}

template <class T>
hipError_t launch_wgrad_t(WgradArgs a, void* dw0, void* dw1, void* db0, void* db1,
                          hipStream_t st) {
  const int nblk = a.nchunks * a.ntile_n * a.ntile_k;
  if (a.nset == 4) {
    launch_wgrad_nset<T, 4>(a, nblk, st);
  } else {
    launch_wgrad_nset<T, 2>(a, nblk, st);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t total = (int64_t)a.N * a.K + a.N;
  int64_t g = (total + 63) / 64;
  if (g > 4096) g = 4096;
  hipLaunchKernelGGL(wgrad_reduce_kernel<T>, dim3((int)g), dim3(kBlock), 0, st, a, dw0, dw1,
                     db0, db1);
  return hipGetLastError();
}

}  // namespace

int proj_max_reduction(int dtype) { return dtype == kF32 ? 256 : 512; }

hipError_t launch_projection(int dtype, bool accumulate, const ProjArgs& args, hipStream_t st) {
  if (args.rows <= 0) return hipSuccess;
  if (args.ksplit < args.K && args.nsplit < args.N) return hipErrorInvalidValue;
  // Buffer offsets are 32-bit: slice the rows so every operand's slice stays
  // below 2^31 bytes.
  const int e = dtype == kF32 ? 4 : 2;
  int64_t widest = args.lda0;
  for (int64_t l : {args.lda1, args.ldy0, args.ldy1}) widest = l > widest ? l : widest;
  const int64_t cap = ((int64_t)1 << 31) - 1 - 1024 * (int64_t)e;
  int64_t slice = cap / (widest * e);
  slice = slice / 32 * 32;
  if (slice < 32) return hipErrorInvalidValue;
  for (int64_t r0 = 0; r0 < args.rows; r0 += slice) {
    ProjArgs a = args;
    a.rows = (int)(args.rows - r0 < slice ? args.rows - r0 : slice);
    a.a0 = static_cast<const char*>(args.a0) + r0 * args.lda0 * e;
    if (a.a1) a.a1 = static_cast<const char*>(args.a1) + r0 * args.lda1 * e;
    a.y0 = static_cast<char*>(args.y0) + r0 * args.ldy0 * e;
    if (a.y1) a.y1 = static_cast<char*>(args.y1) + r0 * args.ldy1 * e;
    if (a.mask) a.mask = args.mask + r0;
    a.abytes0 = (uint32_t)(a.rows * args.lda0 * e);
    a.abytes1 = a.a1 ? (uint32_t)(a.rows * args.lda1 * e) : 0u;
    a.ybytes0 = (uint32_t)(a.rows * args.ldy0 * e);
    a.ybytes1 = a.y1 ? (uint32_t)(a.rows * args.ldy1 * e) : 0u;
    a.nblocks = (a.rows + 31) / 32;
    hipError_t err;
    switch (dtype) {
      case kF32: err = launch_proj_dtype<F32>(a, accumulate, st); break;
      case kF16: err = launch_proj_dtype<F16>(a, false, st); break;
      default: err = launch_proj_dtype<BF16>(a, false, st); break;
    }
    if (err != hipSuccess) return err;
  }
  return hipSuccess;
}

hipError_t launch_transpose(int dtype, const void* w0, const void* w1, int ksplit, int K, int N,
                            void* wt, hipStream_t st) {
  const dim3 grid((K + 31) / 32, (N + 31) / 32);
  switch (dtype) {
    case kF32:
      hipLaunchKernelGGL(transpose_kernel<F32>, grid, dim3(kBlock), 0, st, w0, w1, ksplit, K, N, wt);
      break;
    case kF16:
      hipLaunchKernelGGL(transpose_kernel<F16>, grid, dim3(kBlock), 0, st, w0, w1, ksplit, K, N, wt);
      break;
    default:
      hipLaunchKernelGGL(transpose_kernel<BF16>, grid, dim3(kBlock), 0, st, w0, w1, ksplit, K, N,
                         wt);
  }
  return hipGetLastError();
}

void wgrad_plan(int64_t rows, int n, int k, int dtype, WgradArgs* a) {
  const int rs = dtype == kF32 ? 32 : 64;
  a->rows = rows;
  a->N = n;
  a->K = k;
  a->ntile_n = (n + 127) / 128;
  a->ntile_k = (k + 127) / 128;
  const int ntiles = a->ntile_n * a->ntile_k;
  // About two workgroups per CU; chunk count a multiple of 8 (one group per XCD).
  int want = 2 * cu_count() / ntiles;
  if (want < 8) want = 8;
  int64_t steps = (rows + rs - 1) / rs;
  if (steps < 1) steps = 1;
  int64_t per = (steps + want - 1) / want;  // steps per chunk
  // At least two steps: short calls keep few chunks (one-step chunks made
  // the partial reduction longer than the chains they saved); a multiple of
  // the steps in flight.
  per = per < 2 ? 2 : (per + 1) / 2 * 2;
  // Buffer descriptors cover one chunk: keep its rows under 2^31 bytes.
  const int64_t row_bytes = (int64_t)(n > k ? n : k) * (dtype == kF32 ? 4 : 2);
  const int64_t max_steps = (((int64_t)1 << 31) - 1) / (row_bytes * rs) / 4 * 4;
  if (per > max_steps) per = max_steps > 4 ? max_steps : 4;
  int64_t chunks = (steps + per - 1) / per;
  chunks = (chunks + 7) / 8 * 8;
  // One workgroup per CU or fewer and chunks of four steps or more: four
  // steps in flight (per a multiple of 4).
  a->nset = (chunks * ntiles <= cu_count() && per >= 4) ? 4 : 2;
  if (a->nset == 4 && per % 4 != 0) {
    per = (per + 3) / 4 * 4;
    if (per > max_steps) per = max_steps;
    chunks = ((steps + per - 1) / per + 7) / 8 * 8;
  }
  a->rows_per_chunk = per * rs;
  a->nchunks = (int)chunks;
}

int64_t wgrad_workspace_bytes(int64_t rows, int n, int k, int dtype) {
  WgradArgs a{};
  wgrad_plan(rows, n, k, dtype, &a);
  return (int64_t)a.nchunks * ((int64_t)n * k + n) * 4;
}

hipError_t launch_wgrad(int dtype, const WgradArgs& a, void* dw0, void* dw1, void* db0, void* db1,
                        hipStream_t st) {
  switch (dtype) {
    case kF32:
      return launch_wgrad_t<F32>(a, dw0, dw1, db0, db1, st);
    case kF16:
      return launch_wgrad_t<F16>(a, dw0, dw1, db0, db1, st);
    default:
      return launch_wgrad_t<BF16>(a, dw0, dw1, db0, db1, st);
  }
}

}  // namespace msda
