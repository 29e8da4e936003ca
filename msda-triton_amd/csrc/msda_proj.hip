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
// Persistent workgroups of 4 waves; a workgroup owns 4*32*TILES output columns
// (grid.y) and walks row blocks of 32 (grid.x stride).  Each wave keeps its
// 32*TILES weight columns x KP in registers for the whole kernel (KP = NU*UK,
// zero past K, so the MFMA loop has a fixed trip count).  The 32 x KP
// activation block is loaded with 16-byte row-contiguous buffer loads two
// blocks ahead (registers), parked in LDS (two buffers, one barrier per
// block) and read back as MFMA fragments.  Every load and store is a buffer
// access whose range check turns rows past the end into zero reads and
// dropped writes: the instruction stream is the same for every block, so the
// compiler's wait counts stay exact and the prefetch really overlaps.  The
// row mask of a block travels as one 32-bit word (wave 0's ballot).  Output:
// lanes 2m, 2m+1 hold columns c, c+1; one DPP swap per row pair lets each
// lane store two adjacent columns of one row (8 stores per 32x32 tile).
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

template <class T, int TILES, bool ACC, bool SPLITA, bool SPLITN>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(1, 1)))
void proj_kernel(ProjArgs p) {
  constexpr int E = T::kBytes;
  constexpr int EPU = 16 / E;    // elements per lane per unit
  constexpr int UK = 2 * EPU;    // k covered by one unit
  constexpr int NU = 32 / TILES; // units per row (K <= NU * UK)
  constexpr int KP = NU * UK;
  constexpr int PITCH = KP * E + 16;
  constexpr int CPR = KP * E / 16;           // 16-byte chunks per staged row
  constexpr int ROUNDS = 32 * CPR / kBlock;  // loads per thread per block
  constexpr int BUF = 32 * PITCH + 16;
  __shared__ __align__(16) unsigned char smem[2 * BUF];

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

  // ---- weights and bias -> registers ----
  const int col0 = (blockIdx.y * 4 + wave) * 32 * TILES;
  i32x4 w[TILES][NU];
  float bias[TILES];
#pragma unroll
  for (int t = 0; t < TILES; ++t) {
    const int c = col0 + 32 * t + rl;
    const bool hi = c >= p.nsplit;
    const int64_t cc = hi ? c - p.nsplit : c;
    const char* base = static_cast<const char*>(hi ? p.w1 : p.w0) + cc * p.ldw * E;
    const void* bp = hi ? p.b1 : p.b0;
    bias[t] = (c < p.N && bp != nullptr) ? load1<T>(bp, (uint64_t)cc) : 0.f;
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const int k = UK * u + EPU * slot;
      w[t][u] = (c < p.N && k < p.K) ? ld16(base + k * E) : i32x4{0, 0, 0, 0};
    }
  }

  // ---- activation staging (two blocks in flight) ----
  // Rows are clamped to p.rows, whose offsets lie at or past num_records.
  i32x4 pre[2][ROUNDS];
  uint32_t pre_mask[2] = {0u, 0u};
  auto load_block = [&](int pb, int blk) {
    const int r0 = blk * 32;
#pragma unroll
    for (int q = 0; q < ROUNDS; ++q) {
      const int idx = tid + kBlock * q;
      const int r = idx / CPR;
      const int k = (idx - r * CPR) * EPU;
      const uint32_t row = (uint32_t)min(r0 + r, nrows);
      if constexpr (SPLITA) {
        const uint32_t o0 = k < p.ksplit ? (row * lda0 + k) * E : kOob;
        const uint32_t o1 = (k >= p.ksplit && k < p.K) ? (row * lda1 + k - p.ksplit) * E : kOob;
        pre[pb][q] = __builtin_amdgcn_raw_buffer_load_b128(ra0, o0, 0, 0) |
                     __builtin_amdgcn_raw_buffer_load_b128(ra1, o1, 0, 0);
      } else {
        const uint32_t o0 = k < p.K ? (row * lda0 + k) * E : kOob;
        pre[pb][q] = __builtin_amdgcn_raw_buffer_load_b128(ra0, o0, 0, 0);
      }
    }
    pre_mask[pb] = (wave == 0 && lane < 32)
                       ? (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(
                             rmask, (uint32_t)min(r0 + lane, nrows), 0, 0)
                       : 0u;
  };

  // One block: park the prefetched rows (register buffer pb) in LDS buffer
  // pb, refill the register buffer with the block two ahead, MFMA, epilogue.
  auto process = [&](int pb, int blk) {
    unsigned char* b = smem + pb * BUF;
#pragma unroll
    for (int q = 0; q < ROUNDS; ++q) {
      const int idx = tid + kBlock * q;
      const int r = idx / CPR;
      const int ch = idx - r * CPR;
      *reinterpret_cast<i32x4*>(b + r * PITCH + ch * 16) = pre[pb][q];
    }
    if (wave == 0) {
      const uint64_t bits = __ballot(pre_mask[pb] != 0u);
      if (lane == 0) *reinterpret_cast<uint32_t*>(b + 32 * PITCH) = (uint32_t)bits;
    }
    __syncthreads();
    load_block(pb, blk + 2 * (int)gridDim.x);
    f32x16 acc[TILES];
#pragma unroll
    for (int t = 0; t < TILES; ++t) acc[t] = f32x16{};
    const unsigned char* arow = b + rl * PITCH + slot * 16;
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const i32x4 a = *reinterpret_cast<const i32x4*>(arow + u * 32);
#pragma unroll
      for (int t = 0; t < TILES; ++t) Mfma<T>::unit(a, w[t][u], acc[t]);
    }
    const uint32_t mword = *reinterpret_cast<const uint32_t*>(b + 32 * PITCH);
    const int r0 = blk * 32;
    const bool odd = rl & 1;
#pragma unroll
    for (int t = 0; t < TILES; ++t) {
      const int c = col0 + 32 * t + rl;
      const int cp = c - (odd ? 1 : 0);  // first column of this lane's pair
      const bool hi = SPLITN && cp >= p.nsplit;
      const int cc = hi ? cp - p.nsplit : cp;
      const uint32_t ldy = (uint32_t)(hi ? p.ldy1 : p.ldy0);
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
        const int i0 = 2 * jj, i1 = 2 * jj + 1;
        const int ra = acc_row(i0, slot), rb = acc_row(i1, slot);
        const float v0 = ((mword >> ra) & 1u) ? 0.f : acc[t][i0] + bias[t];
        const float v1 = ((mword >> rb) & 1u) ? 0.f : acc[t][i1] + bias[t];
        // even lane keeps row ra and takes the partner's (row ra, c+1);
        // odd lane keeps row rb and takes the partner's (row rb, c-1).
        const float x = swap_pair_lane(odd ? v0 : v1);
        const int rr = odd ? rb : ra;
        const int row = r0 + rr;
        PairT<T> pv = odd ? make_pair<T>(x, v1) : make_pair<T>(v0, x);
        const uint32_t off = (row < nrows && cp < p.N)
                                 ? ((uint32_t)row * ldy + (uint32_t)cc) * E
                                 : kOob;
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
  };

  const int blk0 = blockIdx.x;
  load_block(0, blk0);
  load_block(1, blk0 + gridDim.x);
  // Weights, bias and the first blocks in one round trip; the loop then has
  // only its own prefetch in flight.
  __builtin_amdgcn_s_waitcnt(0);
  // Blocks blk0 + j*G alternate between buffers 0 and 1 (a block past the end
  // reads zeros and stores nothing).  LDS buffer pb is rewritten two blocks
  // after it was read, behind the barrier of the block in between, which
  // every wave reaches only after finishing that read.
  for (int blk = blk0; blk < p.nblocks; blk += 2 * gridDim.x) {
    process(0, blk);
    process(1, blk + gridDim.x);
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
template <class T, bool MASKED>
__global__ __launch_bounds__(kBlock) void wgrad_kernel(WgradArgs p) {
  constexpr int E = T::kBytes;
  constexpr int EPU = 16 / E;
  constexpr int UK = 2 * EPU;
  constexpr int TW = 128;              // tile width in n and in k
  constexpr int RS = 128 / E;          // rows per step
  constexpr int RW = RS / 4;           // rows per wave per step
  constexpr int PITCH = RS * E + 8;    // LDS bytes per transposed column
  constexpr int TILE_BYTES = TW * PITCH;
  constexpr int GROUP = 8 / E;         // rows per 8-byte LDS piece
  using Pair = typename std::conditional<E == 4, uint2, uint32_t>::type;
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

  // This lane's two columns of the G and X tiles.
  const int gc0 = n0 + 2 * lane, xc0 = k0 + 2 * lane;
  const bool g_ok = gc0 < p.N, x_ok = xc0 < p.K;
  const int gc = g_ok ? gc0 : 0, xc = x_ok ? xc0 : 0;  // dead lanes read column 0
  const bool g_hi = gc >= p.nsplit;
  const char* gbase = g_hi ? static_cast<const char*>(p.g1) + (int64_t)(gc - p.nsplit) * E
                           : static_cast<const char*>(p.g0) + (int64_t)gc * E;
  const int64_t ldg = g_hi ? p.ldg1 : p.ldg0;
  const char* xbase = static_cast<const char*>(p.x) + (int64_t)xc * E;

  // Loads are unconditional (rows clamped into the chunk, so every address is
  // valid) and rows past the end or masked are zeroed when parked: the
  // instruction stream is the same every step and the compiler's wait counts
  // stay exact, so the next step's loads overlap this step's MFMAs.
  Pair gp[RW], xp[RW];
  uint32_t mk[RW];      // mask bytes, looked at only when parked
  uint32_t inrange = 0; // bit i: row i of this wave's share exists
  auto load_step = [&](int64_t r0) {
    inrange = 0;
#pragma unroll
    for (int i = 0; i < RW; ++i) {
      const int64_t row = r0 + wave * RW + i;
      const int64_t rc = row < rend ? row : rend - 1;
      gp[i] = *reinterpret_cast<const Pair*>(gbase + rc * ldg * E);
      xp[i] = *reinterpret_cast<const Pair*>(xbase + rc * p.ldx * E);
      if constexpr (MASKED) mk[i] = p.mask[rc];
      inrange |= (row < rend ? 1u : 0u) << i;
    }
  };
  auto park_step = [&](unsigned char* b) {
    unsigned char* tg = b + (2 * lane) * PITCH + wave * RW * E;
    unsigned char* tx = tg + TILE_BYTES;
#pragma unroll
    for (int i = 0; i < RW; ++i) {
      bool live = (inrange >> i) & 1u;
      if constexpr (MASKED) live = live && mk[i] == 0u;
      if (!g_ok || !live) gp[i] = Pair{};
      if (!x_ok || !live) xp[i] = Pair{};
    }
#pragma unroll
    for (int g = 0; g < RW; g += GROUP) {
      uint2 lo_g, hi_g, lo_x, hi_x;
      if constexpr (E == 4) {
        lo_g = uint2{gp[g].x, gp[g + 1].x};
        hi_g = uint2{gp[g].y, gp[g + 1].y};
        lo_x = uint2{xp[g].x, xp[g + 1].x};
        hi_x = uint2{xp[g].y, xp[g + 1].y};
      } else {
        // [r0.lo16 | r1.lo16] = perm(r1, r0, 0x05040100); hi halves 0x07060302.
        lo_g = uint2{__builtin_amdgcn_perm(gp[g + 1], gp[g], 0x05040100u),
                     __builtin_amdgcn_perm(gp[g + 3], gp[g + 2], 0x05040100u)};
        hi_g = uint2{__builtin_amdgcn_perm(gp[g + 1], gp[g], 0x07060302u),
                     __builtin_amdgcn_perm(gp[g + 3], gp[g + 2], 0x07060302u)};
        lo_x = uint2{__builtin_amdgcn_perm(xp[g + 1], xp[g], 0x05040100u),
                     __builtin_amdgcn_perm(xp[g + 3], xp[g + 2], 0x05040100u)};
        hi_x = uint2{__builtin_amdgcn_perm(xp[g + 1], xp[g], 0x07060302u),
                     __builtin_amdgcn_perm(xp[g + 3], xp[g + 2], 0x07060302u)};
      }
      *reinterpret_cast<uint2*>(tg + g * E) = lo_g;
      *reinterpret_cast<uint2*>(tg + PITCH + g * E) = hi_g;
      *reinterpret_cast<uint2*>(tx + g * E) = lo_x;
      *reinterpret_cast<uint2*>(tx + PITCH + g * E) = hi_x;
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
  int buf = 0;
  if (rbeg < rend) load_step(rbeg);
  for (int64_t r0 = rbeg; r0 < rend; r0 += RS) {
    unsigned char* b = lds[buf];
    park_step(b);
    __syncthreads();
    if (r0 + RS < rend) load_step(r0 + RS);
    const unsigned char* ta = b + (wn * 64 + rl) * PITCH + slot * 16;
    const unsigned char* tb = b + TILE_BYTES + (wk * 64 + rl) * PITCH + slot * 16;
#pragma unroll
    for (int u = 0; u < RS / UK; ++u) {
      i32x4 fa[2], fb[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        fa[h] = frag(ta + h * 32 * PITCH + u * 32);
        fb[h] = frag(tb + h * 32 * PITCH + u * 32);
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
    buf ^= 1;
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

// dW / db = fixed-order sums of the chunk partials, rounded once.
template <class T>
__global__ __launch_bounds__(kBlock) void wgrad_reduce_kernel(WgradArgs p, void* dw0, void* dw1,
                                                              void* db0, void* db1) {
  const int64_t nk = (int64_t)p.N * p.K;
  const int64_t total = nk + (p.wsb != nullptr ? p.N : 0);
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * kBlock) {
    float s = 0.f;
    if (i < nk) {
      // Fixed order c = 0, 1, ...; eight loads in flight at a time.
      int c = 0;
      for (; c + 8 <= p.nchunks; c += 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = p.ws[(int64_t)(c + u) * nk + i];
#pragma unroll
        for (int u = 0; u < 8; ++u) s += v[u];
      }
      for (; c < p.nchunks; ++c) s += p.ws[(int64_t)c * nk + i];
      const int n = (int)(i / p.K);
      const int k = (int)(i - (int64_t)n * p.K);
      if (n < p.nsplit) {
        if (dw0 != nullptr) store1<T>(dw0, (uint64_t)n * p.K + k, s);
      } else if (dw1 != nullptr) {
        store1<T>(dw1, (uint64_t)(n - p.nsplit) * p.K + k, s);
      }
    } else {
      const int n = (int)(i - nk);
      for (int c = 0; c < p.nchunks; ++c) s += p.wsb[(int64_t)c * p.N + n];
      if (n < p.nsplit) {
        if (db0 != nullptr) store1<T>(db0, (uint64_t)n, s);
      } else if (db1 != nullptr) {
        store1<T>(db1, (uint64_t)(n - p.nsplit), s);
      }
    }
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

template <class T, int TILES, bool ACC, bool SPLITA, bool SPLITN>
hipError_t launch_proj_t(ProjArgs a, hipStream_t st) {
  const int cols_per_wg = 4 * 32 * TILES;
  const int gy = (a.N + cols_per_wg - 1) / cols_per_wg;
  // One resident workgroup per CU (the weight registers take a whole SIMD
  // slot per wave); blocks split evenly over grid.x.
  int want = cu_count() / gy;
  if (want < 1) want = 1;
  const int per = (a.nblocks + want - 1) / want;
  const int gx = (a.nblocks + per - 1) / per;
  hipLaunchKernelGGL((proj_kernel<T, TILES, ACC, SPLITA, SPLITN>), dim3(gx, gy), dim3(kBlock), 0,
                     st, a);
  return hipGetLastError();
}

template <class T, int TILES, bool ACC>
hipError_t launch_proj_split(const ProjArgs& a, hipStream_t st) {
  const bool sa = a.ksplit < a.K, sn = a.nsplit < a.N;
  if (sa) return launch_proj_t<T, TILES, ACC, true, false>(a, st);  // never both: callers
  if (sn) return launch_proj_t<T, TILES, ACC, false, true>(a, st);  // split one side only
  return launch_proj_t<T, TILES, ACC, false, false>(a, st);
}

template <class T>
hipError_t launch_proj_dtype(const ProjArgs& a, bool accumulate, hipStream_t st) {
  if constexpr (T::kBytes == 4) {
    if (accumulate) return launch_proj_split<T, 1, true>(a, st);
    return launch_proj_split<T, 1, false>(a, st);
  } else {
    if (a.K <= 256) return launch_proj_split<T, 2, false>(a, st);
    return launch_proj_split<T, 1, false>(a, st);
  }
}

template <class T>
hipError_t launch_wgrad_t(WgradArgs a, void* dw0, void* dw1, void* db0, void* db1,
                          hipStream_t st) {
  const int nblk = a.nchunks * a.ntile_n * a.ntile_k;
  if (a.mask != nullptr) {
    hipLaunchKernelGGL((wgrad_kernel<T, true>), dim3(nblk), dim3(kBlock), 0, st, a);
  } else {
    hipLaunchKernelGGL((wgrad_kernel<T, false>), dim3(nblk), dim3(kBlock), 0, st, a);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t total = (int64_t)a.N * a.K + a.N;
  int64_t g = (total + kBlock - 1) / kBlock;
  if (g > 2048) g = 2048;
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
  // About one workgroup per CU; chunk count a multiple of 8 (one group per XCD).
  int want = cu_count() / ntiles;
  if (want < 8) want = 8;
  int64_t steps = (rows + rs - 1) / rs;
  if (steps < 1) steps = 1;
  int64_t per = (steps + want - 1) / want;  // steps per chunk
  int64_t chunks = (steps + per - 1) / per;
  chunks = (chunks + 7) / 8 * 8;
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
