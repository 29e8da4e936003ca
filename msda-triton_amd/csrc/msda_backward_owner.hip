// Owner-computes grad_value for gfx950: every element of grad_value is
// written exactly once, with plain stores -- no atomics, no zero-fill.
//
// The reference scatters grad_value[corner] += A * w_c * grad_out[pair] with
// atomics (src/msda_triton/kernels.py:278-291) into a zeroed buffer
// (src/msda_triton/ops.py:76-77).  Measured on MI355X, those buffer atomics
// are forwarded past L2 and complete at a fixed chip-wide rate of requests,
// and the zero-fill alone writes the whole tensor once; at decoder sizes the
// two make up ~85% of the backward.  When a (b, m, level) holds few samples
// (Q * K <= kOwnCap: decoder cross-attention, Q ~ 300-900), the same sums
// can be formed by the rows' owners instead:
//
//   one workgroup owns (batch b, head m, band [lo, hi) of the pixel axis);
//   it loads every sample of (b, m) on each level that meets the band (Q *
//   K samples, <= 8 per lane), keeps those whose corner rows meet the band's
//   pixel rows (packed into the first lanes, in sample order), evaluates
//   their bilinear geometry, counts the in-map corners that land in the band
//   per row (integer LDS atomics), turns the counts into CSR offsets (block
//   scan), stores zeros for rows no sample touches, fills the CSR with
//   (A * w_c, query) entries, and then gives each row to a team of G lanes
//   that sums its entries' grad_out chunks (staged once in LDS) in fp32
//   registers and stores the row.
//
// The sums are the reference's, accumulated in fp32 and rounded once, in
// every mode (the fp32_grad_accum choice is moot here).  Their order within a
// row follows the CSR, whose order is fixed by the inputs (each wave counts
// into its own row counters, so an entry's rank depends only on that wave's
// instructions in program order): grad_value is bitwise reproducible across
// runs, unlike the reference's atomics, and the deterministic entry points
// use this path unchanged.  grad_loc / grad_attn come from the direct
// backward kernel's body without its scatter.
//
// Bands: for a standard level table (start_0 = 0, start_{l+1} = start_l +
// H_l W_l, levels covering [0, S): what level_start_index = None gives) each
// level l is split into n_l = min(H_l W_l, max(ceil(H_l W_l / own_rows),
// own_split)) bands, so coarse levels -- few pixels, as many corner entries
// as the fine ones -- are shared by several workgroups.  Any other table
// gets uniform bands of own_rows pixels; a band then may meet several levels
// (handled one level per round: the first round stores every row, later
// rounds add into the rows they touch -- the workgroup is their only
// writer) or none (rows stored as zeros).
#include <algorithm>
#include <atomic>

#include "../../include/msda_hip.h"
#include "msda_bwd_body.h"
#include "msda_launch.h"

namespace msda {

namespace {

constexpr int kOwnRows = 8 * kBlock;       // pixels per band, at most (8 per lane in the scan)
constexpr int kOwnCap = 2048;              // CSR entries per sub-band; path needs Q * K <= it
constexpr int kOwnBandFill = kOwnCap * 4 / 5;  // corner entries per band, at most (level split)
constexpr int kOwnEntriesPerNs = 100;      // least entries per band per sample slot (level split)
constexpr int kOwnGBytes = 19456;          // staged grad_out rows (Q * D * elem), at most
// A second build of the kernel stages up to kOwnGBytesBig (fp32 decoders,
// Q * D * elem up to 40 KB) at two workgroups per CU instead of four.
constexpr int kOwnGBytesBig = 40960;

// Level l's (H, W, start) read from the caller's int64 tensors.  The index
// is uniform and nothing has been stored yet where this is called, so these
// are scalar loads: a workgroup learns its band before any vector load, and
// groups past the last band leave at once, freeing their slot.
struct OwnLevel {
  int h, w, start;
};
__device__ __forceinline__ OwnLevel own_level(const Params& p, int l) {
  return {(int)p.shapes[2 * l], (int)p.shapes[2 * l + 1], (int)p.starts[l]};
}

// Band [lo, hi) of group gi of a (b, m).  Returns 1 for a band of the
// cumulative level table (it lies in level lv, whose (H, W, start) is `lev`),
// 2 for a band of another table (every level that meets it is processed), 0
// for groups past the last band.  Same answer in every lane.
__device__ int own_band(const Params& p, int gi, int& lo, int& hi, int& lv, OwnLevel& lev) {
  // One pass: the table check and, assuming the table is the cumulative
  // one, the band's level (unrolled so that the scalar loads overlap).
  bool standard = true, found = false;
  int64_t acc = 0;
  int g = gi;
#pragma unroll 4
  for (int l = 0; l < p.L; ++l) {
    const OwnLevel v = own_level(p, l);
    if (v.h < 0 || v.w < 0 || (int64_t)v.start != acc) standard = false;
    acc += (int64_t)v.h * v.w;
    const int hw = v.h * v.w;
    if (!found && hw > 0) {
      int n = (hw + p.own_rows - 1) / p.own_rows;
      if (n < p.own_split) n = p.own_split;
      if (n > hw) n = hw;
      if (g < n) {
        const int size = (hw + n - 1) / n;
        lo = v.start + g * size;
        hi = min(lo + size, v.start + hw);
        lv = l;
        lev = v;
        found = true;
      }
      g -= n;
    }
  }
  if (acc != (int64_t)p.S) standard = false;
  if (standard) return found && lo < hi ? 1 : 0;
  lo = gi * p.own_rows;
  hi = min(lo + p.own_rows, p.S);
  return lo < hi ? 2 : 0;
}

// Maximum of v over the wave (every lane active): DPP within each row of 16
// lanes (swap neighbours, pairs, mirror the halves, mirror the row), then
// the four rows' maxima read as scalars.
__device__ __forceinline__ int own_wave_max(int v) {
  v = max(v, __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false));   // quad_perm [1,0,3,2]
  v = max(v, __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false));   // quad_perm [2,3,0,1]
  v = max(v, __builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, false));  // row_half_mirror
  v = max(v, __builtin_amdgcn_mov_dpp(v, 0x140, 0xF, 0xF, false));  // row_mirror
  return max(max(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
             max(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}

// Exclusive prefix sum of v over the workgroup; `tot` receives the total
// and `mx` the maximum of m.
__device__ __forceinline__ int own_scan(int v, int m, int* wsum, int* wmax, int* tot, int* mx) {
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int wm = own_wave_max(m);
  int x = v;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int y = __shfl_up(x, d);
    if (lane >= d) x += y;
  }
  if (lane == kWave - 1) {
    // The addresses are formed here: hoisted to the kernel's start they
    // would hold a register throughout (and be spilled).
    int w = wave;
    asm volatile("" : "+v"(w));
    wsum[w] = x;
    wmax[w] = wm;
  }
  __syncthreads();
  int base = 0;
  for (int w = 0; w < wave; ++w) base += wsum[w];
  *tot = wsum[0] + wsum[1] + wsum[2] + wsum[3];
  *mx = max(max(wmax[0], wmax[1]), max(wmax[2], wmax[3]));
  return base + x - v;
}

// Location (fused: the image coordinate ref_x * W + offset_x - 0.5, rounded
// as make_sample_at rounds it) and weight A (fused: exp(logit - lse)) of one
// sample; own_cell turns them into the cell.  Loads go through buffer
// descriptors: an out-of-range offset (a lane past the last sample) reads
// zeros, no branch.
struct OwnRsrc {
  __amdgpu_buffer_rsrc_t loc, attn, ref, lse;
};

template <class T, bool FUSED>
__device__ __forceinline__ void own_sample(const Params& p, const OwnRsrc& rs, uint32_t pair,
                                           uint32_t s, uint32_t bq, uint32_t l, bool valid,
                                           float fw, float fh, float& x, float& y, float& a) {
  const uint32_t pi = pair * (uint32_t)p.LK + s;
  const uint32_t dead = valid ? 0u : 0x80000000u;
  float u, v, w;
  if constexpr (T::kBytes == 4) {
    const i32x2 xy = __builtin_amdgcn_raw_buffer_load_b64(rs.loc, (pi * 8u) | dead, 0, 0);
    u = __int_as_float(xy[0]);
    v = __int_as_float(xy[1]);
    w = __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs.attn, (pi * 4u) | dead, 0, 0));
  } else {
    unpack2<T>((uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rs.loc, (pi * 4u) | dead, 0, 0), u, v);
    w = unpack1<T>((uint16_t)__builtin_amdgcn_raw_buffer_load_b16(rs.attn, (pi * 2u) | dead, 0, 0));
  }
  if constexpr (FUSED) {
    const uint32_t ri = p.ref_levels ? bq * (uint32_t)p.L + l : bq;
    float rx, ry;
    if constexpr (T::kBytes == 4) {
      const i32x2 r2 = __builtin_amdgcn_raw_buffer_load_b64(rs.ref, (ri * 8u) | dead, 0, 0);
      rx = __int_as_float(r2[0]);
      ry = __int_as_float(r2[1]);
    } else {
      unpack2<T>((uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rs.ref, (ri * 4u) | dead, 0, 0), rx,
                 ry);
    }
    const float lse =
        __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs.lse, (pair * 4u) | dead, 0, 0));
    x = __fsub_rn(__fmaf_rn(rx, fw, u), 0.5f);
    y = __fsub_rn(__fmaf_rn(ry, fh, v), 0.5f);
    a = expf(w - lse);
  } else {
    x = u;  // the location itself: own_cell forms the coordinate (split_coord)
    y = v;
    a = w;
  }
  if (!valid) x = y = FUSED ? -4.f : -1e6f;  // a cell outside every map
}

// Corner cell of a sample: pixel index of corner 00, fractions, and the
// bits of the corners that lie in the map and in [lo, hi) (bit c: corner c
// = 00, 01, 10, 11 at pixel pix + (c & 1) + (c >> 1) * W).  (x, y) is the
// image coordinate (FUSED) or the location (else); same floors, fractions
// and validity as make_sample_at.
template <class T, bool FUSED>
__device__ __forceinline__ uint32_t own_cell(float x, float y, int W, int H, int st, int lo, int hi,
                                             int& pix, float& lx, float& ly) {
  float x0f, y0f;
  if constexpr (FUSED) {
    x0f = floorf(x);
    y0f = floorf(y);
    lx = x - x0f;
    ly = y - y0f;
  } else {
    coord_cell<T>(x, (float)W, x0f, lx);
    coord_cell<T>(y, (float)H, y0f, ly);
  }
  x0f = fminf(fmaxf(x0f, -2.f), (float)W + 1.f);
  y0f = fminf(fmaxf(y0f, -2.f), (float)H + 1.f);
  const int x0 = (int)x0f, y0 = (int)y0f;
  const bool vx0 = (x0 >= 0) & (x0 < W), vx1 = (x0 >= -1) & (x0 < W - 1);
  const bool vy0 = (y0 >= 0) & (y0 < H), vy1 = (y0 >= -1) & (y0 < H - 1);
  pix = st + y0 * W + x0;
  const bool c0 = vy0 & vx0 & (pix >= lo) & (pix < hi);
  const bool c1 = vy0 & vx1 & (pix + 1 >= lo) & (pix + 1 < hi);
  const bool c2 = vy1 & vx0 & (pix + W >= lo) & (pix + W < hi);
  const bool c3 = vy1 & vx1 & (pix + W + 1 >= lo) & (pix + W + 1 < hi);
  return (uint32_t)c0 | (uint32_t)c1 << 1 | (uint32_t)c2 << 2 | (uint32_t)c3 << 3;
}

constexpr int kOwnQBits = 11;  // query index in a CSR entry (Q <= Q * K <= kOwnCap)
static_assert(kOwnCap <= (1 << kOwnQBits), "query index field");

constexpr int kOwnMaxNs = 8;      // samples per lane and level, at most (Q * K <= 8 * kBlock)
constexpr int kOwnQueue = 1280;   // compaction: samples moved between lanes per round

// LDS of an owner workgroup.
template <int kVec, int GB>
struct OwnLds {
  LevelTable lt;
  union {
    struct {
      uint16_t s_off[kOwnRows + 8];  // CSR offsets (exclusive prefix sum of the counts)
      // Entries per row counted per wave (count pass; 16-bit counters, rows
      // 2k and 2k + 1 in word k), then each wave's exclusive prefix over the
      // waves; then the CSR entries (A * w_c, query | local row <<
      // kOwnQBits), rows contiguous; then, after the entries are read, each
      // team's piece of the row it continues from the slice before.
      union {
        uint32_t cnt[kBlock / kWave][kOwnRows / 2];
        float2 csr[kOwnCap];
        float piece[kBlock * kVec];
      } u;
    } m;
    // Compaction staging (before the count): kept samples (x, y, A, j) in
    // their dense order.
    struct {
      float4 queue[kOwnQueue];
    } q;
  };
  int s_wsum[kBlock / kWave];
  int s_qc[kOwnMaxNs][kBlock / kWave];  // kept samples per iteration and wave
  alignas(16) uint8_t s_g[GB];  // grad_out rows of (b, m): Q x D * elem
};
static_assert(sizeof(float4) * kOwnQueue <= (kOwnRows + 8) * 2 + kOwnCap * 8,
              "the queue overlays the CSR offsets and counters");

// T: storage dtype; NS: samples per lane and level (NS * kBlock >= Q * K).
// p.g_rt lanes (a power of two, g_real of them live) cover a value row in
// 16-byte chunks.  ~40.7 KB of LDS and <= 128 VGPRs: four workgroups per CU.
//
// p.nblocks workgroups own bands of grad_value; pd.nblocks more compute
// grad_loc / grad_attn (the direct backward body without its scatter, launch
// shape pd).  Dispatched after the bands, they take the slots that finished
// band workgroups free up, so the two halves of the backward overlap instead
// of running as two launches (decoder preset: 28 us against 32 us).
// DG > 0: the gradient workgroups' shape is 16-byte chunks, DG lanes per
// row, 4 slots (compiled); 0: pd's runtime shape (16-byte chunks).
// GB: bytes of staged grad_out (kOwnGBytes or kOwnGBytesBig).
template <class T, int NS, bool FUSED, int DG, int GB>
__global__ __launch_bounds__(kBlock, 4) void owner_kernel(Params p, Params pd) {
  using C = Chunk<T, 16>;
  constexpr int kVec = C::kVec;
  constexpr int kGIt = (GB / 16 + kBlock - 1) / kBlock;  // staged 16-byte chunks per lane
  static_assert(kOwnRows == 8 * kBlock, "eight rows per lane in the scan");
  static_assert(GB % 16 == 0, "whole chunks");
  static_assert(4 * NS * kBlock < 65536, "16-bit CSR offsets");
  static_assert(NS <= kOwnMaxNs, "compaction counts");

  __shared__ union {
    OwnLds<kVec, GB> own;
    BwdLds grad;
  } smem;
  // Chunks of 8 consecutive workgroups (one per XCD): p.own_cut band
  // chunks, then the gradient chunks, then the other band chunks (groups
  // past the estimated last band, mostly idle).  The gradient workgroups so
  // take the slots the bands leave free from the start instead of waiting
  // behind the idle groups (decoder 23.2 -> 22.7 us, Q = 100 16.9 -> 15.6).
  const int x8 = blockIdx.x & 7, c8 = blockIdx.x >> 3;
  const int cg = (pd.nblocks + 7) >> 3;
  const int gc = c8 - p.own_cut;  // gradient chunk, if in [0, cg)
  if (gc >= 0 && gc < cg) {
    const int blk = gc * 8 + x8;
    if (blk < pd.nblocks)
      bwd_body<T, NoAcc, 16, DG, DG ? 4 : 0, FUSED>(pd, xcd_remap(blk, pd.nblocks), smem.grad);
    return;
  }
  LevelTable& lt = smem.own.lt;
  uint16_t* const s_off = smem.own.m.s_off;
  auto& u = smem.own.m.u;
  int* const s_wsum = smem.own.s_wsum;
  uint8_t* const s_g = smem.own.s_g;

  int tid = threadIdx.x;
  // Grid: bid = 8 k + x runs on XCD x (round-robin dispatch).  Band group
  // bg = (k / M) * 8 + x and head m = k % M: the heads of a band share an
  // XCD (whole 128-byte lines of grad_value meet in its L2), XCDs get
  // interleaved band groups, and bands past the last level (idle groups)
  // come last in dispatch order.
  const int k8 = c8 < p.own_cut ? c8 : c8 - cg;
  const int m = k8 % p.M;
  const int bg = (k8 / p.M) * 8 + x8;
  const int nb = p.npairs / (p.Q * p.M);
  const int b = bg % nb;
  const int gi = bg / nb;
  if (gi >= p.own_groups) return;  // grid padding

  int lo, hi, lv0 = 0;
  OwnLevel lev0 = {0, 0, 0};
  const int kind = own_band(p, gi, lo, hi, lv0, lev0);
  if (kind == 0) return;  // past the last band

  const int rowb = p.D * T::kBytes;  // g_real * 16 (path condition)
  const int nsmp = p.Q * p.K;
  // Stage grad_out[b, :, m, :] (chunk k of the stage is its byte k * 16)
  // with loads that write LDS directly (lane i of a wave's load lands at
  // the wave's base + 16 i): no registers held, and they complete while the
  // parameter loads are in flight -- the first barrier after those waits
  // for both.  Waves whose chunks all lie past the last one issue nothing;
  // the stage's size is a multiple of a wave's 64 chunks, so a wave that
  // issues stays inside it.
  static_assert(GB % (16 * kWave) == 0, "whole waves of chunks");
  const __amdgpu_buffer_rsrc_t rg = make_rsrc(p.grad_out, p.gout_bytes);
  const uint32_t gq0 = ((uint32_t)b * (uint32_t)p.Q * (uint32_t)p.M + (uint32_t)m) * (uint32_t)rowb;
  const uint32_t gqs = (uint32_t)p.M * (uint32_t)rowb;  // grad_out stride between queries
  const int nchunk = p.Q * p.g_real;
#pragma unroll
  for (int k = 0; k < kGIt; ++k) {
    const int kk = tid + k * kBlock;
    const int k0 = kk & ~(kWave - 1);  // the wave's first chunk (uniform)
    if (k0 < nchunk) {
      const int q = (int)fdiv((uint32_t)kk, p.div_g);
      const uint32_t off = kk < nchunk ? gq0 + (uint32_t)q * gqs + (uint32_t)(kk - q * p.g_real) * 16u
                                       : 0x80000000u;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rg, (__attribute__((address_space(3))) void*)(s_g + k0 * 16), 16, off, 0, 0, 0);
    }
  }
  if (kind == 2) {  // other level tables: an LDS copy
    load_levels(p, lt);
    __syncthreads();
  }
  const int l_begin = kind == 1 ? lv0 : 0, l_end = kind == 1 ? lv0 + 1 : p.L;

  const int G = p.g_rt, lg = p.own_lg;  // lanes per row and its log2
  const int kTeams = kBlock >> lg;
  const int team = tid >> lg, ch = tid & (G - 1);
  const bool live = ch < p.g_real;
  const int chg = live ? ch * 16 : 0;  // padding lanes read a live chunk, store nothing
  const int nrows = hi - lo;
  const int e = T::kBytes;
  const uint32_t nsp = (uint32_t)p.npairs * (uint32_t)p.LK;  // samples in the slice
  const OwnRsrc rs = {make_rsrc(p.loc, nsp * 2u * e), make_rsrc(p.attn, nsp * e),
                      make_rsrc(p.ref, FUSED ? p.ref_bytes : 0u),
                      make_rsrc(p.lse, FUSED ? (uint32_t)p.npairs * 4u : 0u)};
  // Row r of the band at byte rbase + r * rstride of grad_value (32-bit
  // buffer offsets; padding lanes get an offset past the buffer, so their
  // stores are dropped by the range check).
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(p.grad_acc, p.acc_bytes);
  const uint32_t rstride = (uint32_t)p.M * (uint32_t)rowb;
  const uint32_t rbase =
      live ? (((uint32_t)b * (uint32_t)p.S + (uint32_t)lo) * (uint32_t)p.M + (uint32_t)m) *
                     (uint32_t)rowb + (uint32_t)ch * 16u
           : 0x80000000u;
  // Store a finished row sum: plain in the first round, added to the row's
  // earlier value in later rounds (this workgroup is the row's only writer).
  auto put = [&](int r, const float (&acc)[kVec], bool written) {
    const uint32_t off = rbase + __umul24((uint32_t)r, rstride);  // both < 2^24
    float v[kVec];
#pragma unroll
    for (int k = 0; k < kVec; ++k) v[k] = acc[k];
    if (written) {
      const i32x4 raw = __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 0);
      const uint32_t w4[4] = {(uint32_t)raw[0], (uint32_t)raw[1], (uint32_t)raw[2], (uint32_t)raw[3]};
      float old[kVec];
      C::unpack(w4, old);
#pragma unroll
      for (int k = 0; k < kVec; ++k) v[k] += old[k];
    }
    __builtin_amdgcn_raw_buffer_store_b128(pack16<T>(v), rv, off, 0, 0);
  };

  bool written = false;
  for (int l = l_begin; l < l_end; ++l) {
    const int H = kind == 1 ? lev0.h : lt.h[l];
    const int W = kind == 1 ? lev0.w : lt.w[l];
    const int st = kind == 1 ? lev0.start : lt.start[l];
    if (H <= 0 || W <= 0) continue;
    // Addresses derived from tid are recomputed in each level round rather
    // than kept in registers across rounds (most calls have one round).
    asm volatile("" : "+v"(tid));
    if ((int64_t)st >= hi || (int64_t)st + (int64_t)H * W <= lo) continue;
    const float fw = (float)W, fh = (float)H;

    // Coordinates and weights of this lane's samples j = tid + i * kBlock of
    // (b, m, l), all parameter loads in flight together.
    float sx[NS], sy[NS], sa[NS];
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      const int j = tid + i * kBlock;
      const bool valid = j < nsmp;
      const uint32_t q = fdiv((uint32_t)(valid ? j : 0), p.div_k);
      const uint32_t bq = (uint32_t)b * (uint32_t)p.Q + q;
      own_sample<T, FUSED>(p, rs, bq * (uint32_t)p.M + m, (uint32_t)(l * p.K + j) - q * p.K, bq,
                           (uint32_t)l, valid, fw, fh, sx[i], sy[i], sa[i]);
    }

    // 0. Compaction.  A sample can put a corner in the band only if one of
    // its corner rows y0, y0 + 1 meets the band's pixel rows [ylo, yhi] of
    // the level -- typically 10-30% of the level's samples.  Those are
    // packed, in increasing j, into the first npass slots c = tid + i *
    // kBlock (through LDS), so the count, fill and rank work below runs
    // over ceil(npass / kBlock) slots instead of NS.  The order (and so
    // every rank and row sum) stays fixed by the inputs.
    const int lane = tid & (kWave - 1), wave = tid / kWave;
    const int ylo = (max(lo, st) - st) / W;
    const int yhi = (min(hi, st + H * W) - 1 - st) / W;
    bool keep[NS];
    uint32_t kpre[NS];
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      float y0f, ly;
      if constexpr (FUSED) {
        y0f = floorf(sy[i]);
      } else {
        coord_cell<T>(sy[i], fh, y0f, ly);
      }
      y0f = fminf(fmaxf(y0f, -2.f), fh + 1.f);
      const int y0 = (int)y0f;  // invalid samples: -2, never kept
      keep[i] = y0 <= yhi && y0 + 1 >= ylo;
      const uint64_t bal = __ballot(keep[i]);
      kpre[i] = __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                          __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
      if (lane == 0) smem.own.s_qc[i][wave] = (int)__popcll(bal);
    }
    __syncthreads();  // counts of kept samples (and, in later rounds, the last pieces read)
    int npass = 0;
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      // slot of this lane's kept sample i: kept samples of the iterations
      // before, then of the waves before in this iteration, then its lanes'
      int before_w = 0, all_w = 0;
#pragma unroll
      for (int w = 0; w < kBlock / kWave; ++w) {
        const int c = smem.own.s_qc[i][w];
        before_w += w < wave ? c : 0;
        all_w += c;
      }
      kpre[i] += (uint32_t)(npass + before_w);
      npass += all_w;
    }
    float cx[NS], cy[NS], ca[NS];
    uint32_t cj[NS];
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      cx[i] = cy[i] = -1e6f;
      ca[i] = 0.f;
      cj[i] = 0u;
    }
    for (int r0 = 0; r0 < npass; r0 += kOwnQueue) {  // one round unless npass > kOwnQueue
#pragma unroll
      for (int i = 0; i < NS; ++i) {
        const int pos = (int)kpre[i] - r0;
        if (keep[i] && pos >= 0 && pos < kOwnQueue)
          smem.own.q.queue[pos] = make_float4(sx[i], sy[i], sa[i], __int_as_float(tid + i * kBlock));
      }
      __syncthreads();
#pragma unroll
      for (int i = 0; i < NS; ++i) {
        const int c = tid + i * kBlock;
        if (c >= r0 && c < r0 + kOwnQueue && c < npass) {
          const float4 v = smem.own.q.queue[c - r0];
          cx[i] = v.x;
          cy[i] = v.y;
          ca[i] = v.z;
          cj[i] = (uint32_t)__float_as_int(v.w);
        }
      }
      __syncthreads();  // queue read: its LDS becomes the counters
    }
    const int ns_c = (npass + kBlock - 1) / kBlock;  // dense slots in use (uniform)

    if (npass == 0) {  // no sample reaches the band: zeros in the first round
      if (!written) {
        const float zero[kVec] = {};
        for (int r = team; r < nrows; r += kTeams) put(r, zero, false);
      }
      __builtin_amdgcn_s_waitcnt(0);
      written = true;
      continue;
    }

#pragma unroll
    for (int w = 0; w < kBlock / kWave; ++w)
      for (int r = tid; r < (nrows + 1) / 2; r += kBlock) u.cnt[w][r] = 0;
    __syncthreads();  // counts zeroed

    // 1. Entries per row.  Each wave counts into its own counters, so the
    // count an entry finds -- its rank among the wave's entries of the row
    // -- depends only on that wave's instructions, in program order; the
    // ranks (and so the CSR order and every row sum) are the same on every
    // run.  The cells (corner-00 pixel, fractions, in-band corner bits
    // 4i..4i+3) are kept for the fill.
    uint32_t rank[NS * 2];  // 16-bit ranks, corners 2h and 2h + 1 of a sample in word h
    int pix[NS];
    float slx[NS], sly[NS];
    uint32_t bits = 0;
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      rank[2 * i] = rank[2 * i + 1] = 0u;
      pix[i] = 0;
      slx[i] = sly[i] = 0.f;
      if (i < ns_c) {
        const uint32_t bi =
            own_cell<T, FUSED>(cx[i], cy[i], W, H, st, lo, hi, pix[i], slx[i], sly[i]);
        bits |= bi << (4 * i);
        uint32_t rk[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          rk[c] = 0;
          if (bi & (1u << c)) {
            // A wave adds at most 64 * NS < 2^16 to a row: no carry between halves.
            const int r = pix[i] + (c & 1) + (c >> 1) * W - lo;
            const uint32_t sh = (uint32_t)(r & 1) * 16u;
            rk[c] = (atomicAdd(&u.cnt[wave][r >> 1], 1u << sh) >> sh) & 0xffffu;
          }
        }
        rank[2 * i] = rk[0] | rk[1] << 16;
        rank[2 * i + 1] = rk[2] | rk[3] << 16;
      }
    }
    __syncthreads();

    // 2. CSR offsets of the rows' totals; each wave's counter becomes the
    // sum over the waves before it.  maxlen: the longest row's entries.
    int maxlen;
    {
      // Row totals < 2^16 (a row takes at most one corner per sample), so
      // two share a word here too.
      uint32_t c2[4];
      int sum = 0, mloc = 0;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int wd = tid * 4 + k;  // rows 2 wd, 2 wd + 1
        uint32_t c = 0;
        if (2 * wd < nrows) {
#pragma unroll
          for (int w = 0; w < kBlock / kWave; ++w) {
            const uint32_t n = u.cnt[w][wd];
            u.cnt[w][wd] = c;
            c += n;  // both halves at once: no half exceeds 2^16
          }
        }
        c2[k] = c;
        sum += (int)((c & 0xffffu) + (c >> 16));
        mloc = max(mloc, (int)max(c & 0xffffu, c >> 16));
      }
      int tot;
      int ex = own_scan(sum, mloc, s_wsum, smem.own.s_qc[1], &tot, &maxlen);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int r = tid * 8 + k;
        if (r < nrows) s_off[r] = (uint16_t)ex;
        ex += (int)((c2[k >> 1] >> ((k & 1) * 16)) & 0xffffu);
      }
      if (tid == 0) s_off[nrows] = (uint16_t)tot;
    }
    __syncthreads();

    // Rows without entries: zeros in the first round (untouched in later
    // ones), stored now so that the writes drain while the CSR is filled
    // and summed.  Four rows per team and step, their offsets read together.
    if (!written) {
      const float zero[kVec] = {};
      for (int rb = team * 4; rb < nrows; rb += kTeams * 4) {
        int o[5];
#pragma unroll
        for (int k = 0; k < 5; ++k) o[k] = s_off[min(rb + k, nrows)];
#pragma unroll
        for (int k = 0; k < 4; ++k)
          if (rb + k < nrows && o[k + 1] == o[k]) put(rb + k, zero, false);
      }
    }

    // An entry's rank in its row: the entries of the waves before it, then
    // its rank within its wave.
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      if (i < ns_c) {
        int before[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const bool in = (bits >> (4 * i + c)) & 1u;
          const int r = in ? pix[i] + (c & 1) + (c >> 1) * W - lo : 0;
          before[c] = (int)((u.cnt[wave][r >> 1] >> ((r & 1) * 16)) & 0xffffu);
          if (!in) before[c] = 0;
        }
        rank[2 * i] += (uint32_t)before[0] | (uint32_t)before[1] << 16;
        rank[2 * i + 1] += (uint32_t)before[2] | (uint32_t)before[3] << 16;
      }
    }
    __syncthreads();  // counters read: the CSR reuses them

    // 3. Sub-bands of at most kOwnCap entries: one unless many samples pile
    // onto the band.  A row alone never exceeds it: a sample puts at most one
    // corner on a row, and Q * K <= kOwnCap.
    for (int r0 = 0; r0 < nrows;) {
      const int base = s_off[r0];
      int a = nrows, z = nrows;
      if (s_off[nrows] - base > kOwnCap) {  // binary search for the sub-band's end
        a = r0 + 1;
        while (a < z) {
          const int mid = (a + z + 1) >> 1;
          if (s_off[mid] - base <= kOwnCap) {
            a = mid;
          } else {
            z = mid - 1;
          }
        }
      }
      const int r1 = a;
      const int ne = s_off[r1] - base;

      // Fill: entry slot = row offset + rank.  The per-corner values are
      // formed here rather than hoisted out of the sub-band loop by the
      // compiler: those of all NS samples would otherwise stay live (~100
      // registers).
#pragma unroll
      for (int i = 0; i < NS; ++i)
        asm volatile("" : "+v"(pix[i]), "+v"(slx[i]), "+v"(sly[i]), "+v"(ca[i]), "+v"(cj[i]));
#pragma unroll
      for (int i = 0; i < NS; ++i) {
        if (i >= ns_c) continue;
        const float lx = slx[i], ly = sly[i];
        const uint32_t q = fdiv(cj[i], p.div_k);
        const float mx = 1.f - lx, my = 1.f - ly;
        // The four row offsets are read unconditionally (row 0 stands in
        // for corners that add nothing) so that they share one LDS wait.
        int r[4], o[4];
        bool in[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          r[c] = pix[i] + (c & 1) + (c >> 1) * W - lo;
          in[c] = (bits & (1u << (4 * i + c))) && r[c] >= r0 && r[c] < r1;
          o[c] = s_off[in[c] ? r[c] : 0];
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          if (in[c]) {
            const float w = (c & 1 ? lx : mx) * (c >> 1 ? ly : my);
            const int slot = o[c] - base + (int)((rank[2 * i + (c >> 1)] >> (16 * (c & 1))) & 0xffffu);
            u.csr[slot] = make_float2(ca[i] * w, __int_as_float((int)q | r[c] << kOwnQBits));
          }
        }
      }
      __syncthreads();

      // Entries: team t sums slice [t * cs, (t + 1) * cs) of the CSR.  A row
      // whose entries all lie in the slice is stored by the team; the piece
      // of a row that started in an earlier slice waits in `first`, the
      // piece of a row that runs on into later slices in `tail`.
      const int cs = (ne + kTeams - 1) / kTeams;
      // Pieces are summed in groups of pg (pg^2 >= kTeams - 1: at most pg
      // groups per row); a row of len entries spans at most pg + 1 slices
      // when len <= pg * cs.
      constexpr int kPGMax = 16;
      const int pg = kTeams > 64 ? 16 : 8;
      const int e_lo = min(team * cs, ne), e_hi = min(e_lo + cs, ne);
      float first[kVec], acc[kVec];
      int prow = -1;  // the row of the piece in `first`, if any
      int tail_row = -1;
#pragma unroll
      for (int k = 0; k < kVec; ++k) first[k] = acc[k] = 0.f;
      if (e_lo < e_hi) {
        // The slice's first row may have begun in an earlier slice (then
        // its sum here is a piece, kept in `first`); every other row that
        // ends inside the slice is complete.  Only the last row can run on
        // past the slice.  So the row boundaries inside the loop need no
        // offset lookups.
        const int row0 = __float_as_int(u.csr[e_lo].y) >> kOwnQBits;
        const bool first_part = s_off[row0] - base < e_lo;
        int cur = row0;
        // g offsets: query < 2^11, row bytes <= 256 (24-bit multiply)
        const uint32_t gb = (uint32_t)chg;
        for (int e0 = e_lo; e0 < e_hi; e0 += 4) {
          float2 en[4];
#pragma unroll
          for (int k = 0; k < 4; ++k) en[k] = u.csr[min(e0 + k, e_hi - 1)];
          // The four entries' grad_out chunks, read together (their LDS
          // latencies overlap instead of one wait per entry).
          uint4 graw4[4];
#pragma unroll
          for (int k = 0; k < 4; ++k)
            graw4[k] = *reinterpret_cast<const uint4*>(
                s_g + (__umul24((uint32_t)__float_as_int(en[k].y) & ((1u << kOwnQBits) - 1),
                                (uint32_t)rowb) + gb));
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            if (e0 + k < e_hi) {
              const uint32_t bits = (uint32_t)__float_as_int(en[k].y);
              const int r = (int)(bits >> kOwnQBits);
              if (r != cur) {  // row cur ends here
                if (cur == row0 && first_part) {
#pragma unroll
                  for (int v = 0; v < kVec; ++v) first[v] = acc[v];
                  prow = row0;
                } else {
                  put(cur, acc, written);
                }
#pragma unroll
                for (int v = 0; v < kVec; ++v) acc[v] = 0.f;
                cur = r;
              }
              const uint32_t w4[4] = {graw4[k].x, graw4[k].y, graw4[k].z, graw4[k].w};
              float gv[kVec];
              C::unpack(w4, gv);
#pragma unroll
              for (int v = 0; v < kVec; ++v) acc[v] += en[k].x * gv[v];
            }
          }
        }
        if (cur == row0 && first_part) {  // a piece (the slice lies inside one row)
#pragma unroll
          for (int v = 0; v < kVec; ++v) first[v] = acc[v];
          prow = row0;
        } else if (s_off[cur + 1] - base > e_hi) {
          tail_row = cur;  // acc stays the tail
        } else {
          put(cur, acc, written);
        }
      }
      // The pieces of a row that spans slices t1 + 1 .. t2 (t1 holds its
      // tail) lie in consecutive teams.  The tail team adds them in order
      // when the row is at most pg slices long (at most pg pieces: the
      // common case).  A longer (deep) row -- heavy contention: dozens of
      // slices -- is summed in two steps: the group heads t1 + 1 + j pg add
      // the pieces of their group of pg, loads in flight together, and the
      // tail team adds the group sums.  The second step runs when the band's
      // longest row (maxlen, from the scan) could be deep.  Which step runs,
      // and every addition, follows from the CSR alone: the sums are the
      // same on every run.
      const bool grouped = maxlen > pg * cs;  // some row of the band is deep (uniform)
      __syncthreads();  // every entry read: the pieces may overwrite the CSR
      if (prow >= 0) {
#pragma unroll
        for (int k = 0; k < kVec; ++k) u.piece[(team * G + ch) * kVec + k] = first[k];
      }
      __syncthreads();
      if (grouped) {
        // Group heads t1 + 1 + j pg of the deep rows: the group's sum
        // replaces the head's piece (no other team reads that slot).
        const int p0 = prow >= 0 ? s_off[prow] - base : 0;
        const int p1 = prow >= 0 ? s_off[prow + 1] - base : 0;
        if (p1 - p0 > pg * cs) {  // a piece of a deep row
          const int t1 = p0 / cs, t2 = (p1 - 1) / cs;
          if (((team - t1 - 1) & (pg - 1)) == 0) {
            const int n = min(pg, t2 - team + 1);
            int th = team;  // addresses formed here (not hoisted: registers)
            asm volatile("" : "+v"(th));
#pragma unroll
            for (int j = 1; j < kPGMax; j += 4) {
              if (j >= n) break;
              float pc[4][kVec];
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                const int t = th + min(j + i, n - 1);
#pragma unroll
                for (int k = 0; k < kVec; ++k) pc[i][k] = u.piece[(t * G + ch) * kVec + k];
              }
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                if (j + i < n) {
#pragma unroll
                  for (int k = 0; k < kVec; ++k) first[k] += pc[i][k];
                }
              }
            }
#pragma unroll
            for (int k = 0; k < kVec; ++k) u.piece[(team * G + ch) * kVec + k] = first[k];
          }
        }
        __syncthreads();  // group sums stored
      }
      if (tail_row >= 0) {  // the tail, then the later pieces (or group sums) in order
        const int c0 = s_off[tail_row] - base, c1 = s_off[tail_row + 1] - base;
        const int te = (c1 - 1) / cs;  // the row's last team
        if (!grouped) {
#pragma unroll 4
          for (int t = team + 1; t <= te; ++t) {
#pragma unroll
            for (int k = 0; k < kVec; ++k) acc[k] += u.piece[(t * G + ch) * kVec + k];
          }
        } else {
          const int step = c1 - c0 > pg * cs ? pg : 1;
          const int cnt = (te - team - 1) / step + 1;  // 1 .. pg slots
          // Their addresses are formed here, not hoisted to the kernel's
          // start, where they would hold registers for the whole kernel.
          int t0 = team + 1;
          asm volatile("" : "+v"(t0));
#pragma unroll
          for (int j = 0; j < kPGMax; j += 4) {
            if (j >= cnt) break;
            float pc[4][kVec];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int t = t0 + min(j + i, cnt - 1) * step;
#pragma unroll
              for (int k = 0; k < kVec; ++k) pc[i][k] = u.piece[(t * G + ch) * kVec + k];
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              if (j + i < cnt) {
#pragma unroll
                for (int k = 0; k < kVec; ++k) acc[k] += pc[i][k];
              }
            }
          }
        }
        put(tail_row, acc, written);
      }
      __syncthreads();  // pieces read before the next sub-band's fill
      r0 = r1;
    }
    // Later rounds read back rows this workgroup stored: let the stores land.
    __builtin_amdgcn_s_waitcnt(0);
    written = true;
  }

  if (!written) {  // no level meets the band: its rows are zero
    const float zero[kVec] = {};
    for (int r = team; r < nrows; r += kTeams) put(r, zero, false);
  }
}

template <class T, int NS, bool FUSED>
hipError_t launch_ns(const Params& p, const Params& pd, hipStream_t st) {
  const int grid = p.nblocks + (pd.nblocks + 7) / 8 * 8;  // p.nblocks: a multiple of 8
  // Compiled gradient shape for 32-channel rows (2 * elem lanes of 16 bytes).
  constexpr int kDG = 2 * T::kBytes;
  const bool dg = pd.g_rt == kDG && pd.ts_rt == 4;
  if (p.own_big) {
    if (dg) {
      hipLaunchKernelGGL((owner_kernel<T, NS, FUSED, kDG, kOwnGBytesBig>), dim3(grid), dim3(kBlock),
                         0, st, p, pd);
    } else {
      hipLaunchKernelGGL((owner_kernel<T, NS, FUSED, 0, kOwnGBytesBig>), dim3(grid), dim3(kBlock),
                         0, st, p, pd);
    }
  } else if (dg) {
    hipLaunchKernelGGL((owner_kernel<T, NS, FUSED, kDG, kOwnGBytes>), dim3(grid), dim3(kBlock), 0,
                       st, p, pd);
  } else {
    hipLaunchKernelGGL((owner_kernel<T, NS, FUSED, 0, kOwnGBytes>), dim3(grid), dim3(kBlock), 0,
                       st, p, pd);
  }
  return hipGetLastError();
}

template <class T, bool FUSED>
hipError_t launch_t(const Params& p, const Params& pd, hipStream_t st) {
  switch ((p.Q * p.K + kBlock - 1) / kBlock) {
    case 1: return launch_ns<T, 1, FUSED>(p, pd, st);
    case 2: return launch_ns<T, 2, FUSED>(p, pd, st);
    case 3: return launch_ns<T, 3, FUSED>(p, pd, st);
    case 4: return launch_ns<T, 4, FUSED>(p, pd, st);
    case 5: return launch_ns<T, 5, FUSED>(p, pd, st);
    case 6: return launch_ns<T, 6, FUSED>(p, pd, st);
    case 7: return launch_ns<T, 7, FUSED>(p, pd, st);
    case 8: return launch_ns<T, 8, FUSED>(p, pd, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

// Band geometry overrides for sweeps: MSDA_KNOB_OWN_ROWS, the most rows per
// band (64..kOwnRows), and MSDA_KNOB_OWN_ENTRIES, the corner entries per
// band the level split aims at (>= 64).
static int64_t own_knob(int knob, int64_t dflt, int64_t lo, int64_t hi) {
  const int64_t x = launch_override(knob, (int)dflt);
  return x < lo ? lo : x > hi ? hi : x;
}

// Workgroup slots of the current device for this kernel: `per_cu` per CU.
static int64_t own_slots(int per_cu) {
  static std::atomic<int> cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 1024;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cus[dev].store(n, std::memory_order_relaxed);
  }
  return per_cu * (int64_t)n;
}

bool owner_plan(int64_t B, int64_t Q, int64_t K, int64_t D, int64_t S, int64_t L,
                int elem_bytes, Params* p) {
  const int64_t rowb = D * elem_bytes;
  if (rowb <= 0 || rowb % 16 != 0 || rowb / 16 > 16) return false;
  if (Q * K <= 0 || Q * K > kOwnCap || Q * rowb > kOwnGBytesBig) return false;
  const bool big = Q * rowb > kOwnGBytes;  // the 40 KB staging build, 2 per CU
  if (S <= 0 || L <= 0) return false;
  // Bands per level: at least ceil(H * W / rows), and at least `split`,
  // which spreads a level's corner entries (up to 4 Q K) over bands.  More
  // bands run in parallel but each scans all Q K samples of its level, so
  // the split is the least that (a) keeps a band's entries within one CSR
  // pass (kOwnBandFill) and (b) gives ~80% of a round of workgroups (the
  // gradient workgroups of the same launch fill the rest), but no more
  // than keeps kOwnEntriesPerNs entries per band per sample slot.  Measured
  // on MI355X (decoder pyramid, B=1/2/4/8, Q*K=400/1200; tiny): within 5%
  // of the best fixed split in every case, 1.2-1.6x faster than one split
  // for all.  The host does not see H and W (they live on the device), so
  // bands are estimated from S and L.  Rows per band: kOwnRows where the
  // grid still fills ~80% of a round with them (fewer bands scan the fine
  // level's samples: decoder B=4 23.9 against 24.6 us, B=8 37.5 against
  // 42.5), else half that (small grids: a band's own time is the kernel's).
  const int64_t ent = 4 * Q * K;
  const int64_t want = own_slots(big ? 2 : 4) * 4 / 5;
  const bool env_split = launch_override_set(MSDA_KNOB_OWN_ENTRIES);
  auto plan_split = [&](int64_t rows, bool* full) {
    const int64_t fine = (S + rows - 1) / rows;
    auto wgs = [&](int64_t s) { return B * p->M * (std::max(fine, s) + (L - 1) * s); };
    if (env_split) {
      const int64_t target = own_knob(MSDA_KNOB_OWN_ENTRIES, kOwnBandFill, 64, 1 << 20);
      *full = true;
      return (ent + target - 1) / target;
    }
    const int64_t ns = (Q * K + kBlock - 1) / kBlock;
    const int64_t lo = (ent + kOwnBandFill - 1) / kOwnBandFill;
    const int64_t hi = std::max(lo, ent / (kOwnEntriesPerNs * ns));
    int64_t s = lo;
    while (s < hi && wgs(s) < want) ++s;
    *full = wgs(s) >= want;
    return s;
  };
  int64_t rows = own_knob(MSDA_KNOB_OWN_ROWS, kOwnRows, 64, kOwnRows);
  bool full = true;
  int64_t split = plan_split(rows, &full);
  if (!full && !launch_override_set(MSDA_KNOB_OWN_ROWS)) {
    rows = kOwnRows / 2;
    split = plan_split(rows, &full);
  }
  const int64_t groups = (S + rows - 1) / rows + L * (1 + split);
  if (groups * (int64_t)p->M * 64 >= (1ll << 31)) return false;
  p->own_rows = (int32_t)rows;
  p->own_big = big ? 1 : 0;
  p->own_split = (int32_t)split;
  {
    const int64_t fine = (S + rows - 1) / rows;
    p->own_est = (int32_t)(std::max(fine, split) + (L - 1) * split);
  }
  p->own_groups = (int32_t)groups;
  p->g_real = (int32_t)(rowb / 16);
  int g = 1, lg = 0;
  while (g < p->g_real) {
    g <<= 1;
    ++lg;
  }
  p->g_rt = g;
  p->own_lg = lg;
  return true;
}

hipError_t launch_owner(int dtype, bool fused, const Params& p0, const Params& pd,
                        hipStream_t st) {
  Params p = p0;
  const int64_t nb = p.npairs / ((int64_t)p.Q * p.M);  // batch elements in the slice
  const int64_t groups = (nb * p.own_groups + 7) / 8 * 8;  // band groups, padded to the XCDs
  p.nblocks = (int32_t)(groups * p.M);
  if (p.nblocks + pd.nblocks == 0) return hipSuccess;
  // Band chunks before the gradient chunks: all (0), none (1), or those of
  // the groups up to the estimated last band (2; the groups after it are
  // mostly idle and would hold the gradient workgroups back).
  const int64_t cb = p.nblocks / 8;
  const int64_t cut_est = (int64_t)p.M * ((p.own_est * nb + 7) / 8);
  p.own_cut = (int32_t)(p.own_mix == 1 ? 0 : p.own_mix == 2 ? std::min(cb, cut_est) : cb);
  switch (dtype) {
    case kF32: return fused ? launch_t<F32, true>(p, pd, st) : launch_t<F32, false>(p, pd, st);
    case kF16: return fused ? launch_t<F16, true>(p, pd, st) : launch_t<F16, false>(p, pd, st);
    case kBF16:
      return fused ? launch_t<BF16, true>(p, pd, st) : launch_t<BF16, false>(p, pd, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace msda
