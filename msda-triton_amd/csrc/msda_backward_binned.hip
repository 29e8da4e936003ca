// Binned owner backward: grad_value for calls with many samples per (batch,
// head, level) -- encoder self-attention, pixel decoders -- formed by the
// owners of bands of value rows, with plain stores where one workgroup owns
// a band and few atomics where several share it.
//
// Computes the grad_value scatter of the reference's `_msda_backward_kernel`
// (src/msda_triton/kernels.py:278-291: every in-map corner c of a sample
// receives A * w_c * grad_out[b, q, m, :]); grad_sampling_locations and
// grad_attention_weights come from the direct backward kernel without its
// scatter (msda_backward.hip, NoAcc), launched after these kernels.
//
// Per (b, m, level) group, the level's pixels are cut into bands of P rows
// (P * D fp32 fit in 32 KB of LDS).  A sample's in-map corners lie in
// [pk, pk + W + 1], pk its first in-map corner, so keying each sample by the
// band of pk puts every sample that can touch band j in the keys
// band((j P - W - 1)+) .. j, which are contiguous once the samples are
// sorted by key.  Four launches:
//   bin_count_kernel   per block of 4096 samples, its count per key (LDS
//                      histogram), one row of a count matrix;
//   bin_scan_kernel    per group: each block's exclusive prefix within each
//                      key, the key cursors (exclusive prefix over the keys)
//                      and the work items: each band's entry range in chunks
//                      of at most `chunk` entries;
//   bin_fill_kernel    writes each sample's id (q * K + k) at a slot fixed
//                      by the inputs (cursor + earlier blocks + earlier
//                      waves + per-wave LDS rank): a key's entries are in
//                      sample order, so grouped by query;
//   bin_acc_kernel     per work item: the entries' corner contributions to
//                      the band's rows are summed in fp32 registers, then
//                      the band is stored (its only item) or added with
//                      buffer atomics (items of a band split in chunks, or
//                      any band when the level table lets levels share rows).
// No workspace: the entry lists live in grad_sampling_locations (4 bytes per
// sample, its size at least) and the cursors and items in
// grad_attention_weights, both written in full afterwards by the gradient
// kernel; the count matrix lives in the accumulator (grad_value or the fp32
// scratch), which is zero-filled after the binning.  Entry order and the
// order of every fp32 sum within a work item are fixed by the inputs; bands
// split over several items add their partial sums with float atomics, whose
// order varies.  The deterministic entry points accumulate in int64 fixed
// point instead (each item's fp32 sums converted, then stored or added
// exactly), so their grad_value is bitwise reproducible.
#include "msda_launch.h"

#include <atomic>

namespace msda {

namespace {

constexpr int kBinPerWave = 1024;                            // samples per wave (contiguous)
constexpr int kBinPerWg = kBinPerWave * (kBlock / kWave);    // samples per binning workgroup
constexpr int kBinIt = kBinPerWave / kWave;                  // samples per lane
constexpr int kBinXcds = 8;                                  // item counters (one per XCD)

// Cell of a sample, as make_sample_at forms it (same clamps): (x, y) is the
// location, or (FUSED) the offset in level pixels from reference point
// (rx, ry).
template <class T, bool FUSED>
__device__ __forceinline__ void bin_cell(float x, float y, float rx, float ry, float fw, float fh,
                                         int32_t& x0, int32_t& y0, float& lx, float& ly) {
  float x0f, y0f;
  if constexpr (FUSED) {
    const float xx = __fsub_rn(__fmaf_rn(rx, fw, x), 0.5f);
    const float yy = __fsub_rn(__fmaf_rn(ry, fh, y), 0.5f);
    x0f = floorf(xx);
    y0f = floorf(yy);
    lx = xx - x0f;
    ly = yy - y0f;
  } else {
    (void)rx;
    (void)ry;
    coord_cell<T>(x, fw, x0f, lx);
    coord_cell<T>(y, fh, y0f, ly);
  }
  x0f = fminf(fmaxf(x0f, -2.f), fw + 1.f);
  y0f = fminf(fmaxf(y0f, -2.f), fh + 1.f);
  x0 = (int32_t)x0f;
  y0 = (int32_t)y0f;
}

// Bit c set when corner c (00, 01, 10, 11) of cell (x0, y0) is in the map.
__device__ __forceinline__ uint32_t bin_vmask(int32_t x0, int32_t y0, int32_t H, int32_t W) {
  const bool vx0 = (x0 >= 0) & (x0 < W), vx1 = (x0 >= -1) & (x0 < W - 1);
  const bool vy0 = (y0 >= 0) & (y0 < H), vy1 = (y0 >= -1) & (y0 < H - 1);
  return (uint32_t)(vy0 & vx0) | (uint32_t)(vy0 & vx1) << 1 | (uint32_t)(vy1 & vx0) << 2 |
         (uint32_t)(vy1 & vx1) << 3;
}

// Buffer views of a call's sample inputs (out-of-range reads give zeros).
struct BinSrc {
  __amdgpu_buffer_rsrc_t loc, attn, ref, lse;
};

__device__ __forceinline__ BinSrc bin_src(const Params& p, const BinArgs& a) {
  return BinSrc{make_rsrc(p.loc, a.loc_bytes), make_rsrc(p.attn, a.attn_bytes),
                make_rsrc(p.ref, p.ref_bytes), make_rsrc(p.lse, (uint32_t)p.npairs * 4u)};
}

// `dead` (0 or 0x80000000) is OR-ed into the byte offset: a dead lane's
// load lies past num_records (< 2^31) and reads zeros, so callers issue the
// loads without a branch (a branch whose block also uses the value makes the
// compiler wait for each load before the next is issued).
template <class T>
__device__ __forceinline__ void bin_xy(__amdgpu_buffer_rsrc_t r, uint32_t i, float& x, float& y,
                                       uint32_t dead = 0u) {
  if constexpr (T::kBytes == 4) {
    const i32x2 xy = __builtin_amdgcn_raw_buffer_load_b64(r, (i * 8u) | dead, 0, 0);
    x = __int_as_float(xy[0]);
    y = __int_as_float(xy[1]);
  } else {
    unpack2<T>((uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (i * 4u) | dead, 0, 0), x, y);
  }
}

template <class T>
__device__ __forceinline__ float bin_one(__amdgpu_buffer_rsrc_t r, uint32_t i, uint32_t dead = 0u) {
  if constexpr (T::kBytes == 4) {
    return __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, (i * 4u) | dead, 0, 0));
  } else {
    return unpack1<T>((uint16_t)__builtin_amdgcn_raw_buffer_load_b16(r, (i * 2u) | dead, 0, 0));
  }
}

// Raw inputs of one sample: location (or offset), weight (or logit), and
// for FUSED the reference point and the pair's log-sum-exp.
struct BinIn {
  float x, y, a, rx, ry, lse;
};

template <class T, bool FUSED, bool kWeight>
__device__ __forceinline__ BinIn bin_load(const Params& p, const BinSrc& rs, uint32_t bq,
                                          uint32_t pair, uint32_t pi, uint32_t l,
                                          uint32_t dead = 0u) {
  BinIn r;
  bin_xy<T>(rs.loc, pi, r.x, r.y, dead);
  r.a = kWeight ? bin_one<T>(rs.attn, pi, dead) : 0.f;
  r.rx = r.ry = r.lse = 0.f;
  if constexpr (FUSED) {
    bin_xy<T>(rs.ref, p.ref_levels ? bq * (uint32_t)p.L + l : bq, r.rx, r.ry, dead);
    if constexpr (kWeight)
      r.lse = __int_as_float(
          __builtin_amdgcn_raw_buffer_load_b32(rs.lse, (pair * 4u) | dead, 0, 0));
  }
  return r;
}

// Exclusive prefix sum over the workgroup; `total` receives the sum.  A
// shuffle scan within each wave, then the waves' totals through `s` (one
// barrier, and one more so that `s` can be reused by the next call).  Every
// thread must call it.
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t* s, uint32_t& total) {
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  uint32_t x = v;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const uint32_t y = __shfl_up(x, d);
    if (lane >= d) x += y;
  }
  if (lane == kWave - 1) s[wave] = x;
  __syncthreads();
  uint32_t base = 0u, tot = 0u;
#pragma unroll
  for (int w = 0; w < kBlock / kWave; ++w) {
    const uint32_t t = s[w];
    base += w < wave ? t : 0u;
    tot += t;
  }
  total = tot;
  __syncthreads();
  return base + x - v;
}

struct GroupLevel {
  int32_t b, m, l, H, W, st, nb, nk;  // nb bands of 2^log2p pixels, nk keys of 2^log2k
};

__device__ __forceinline__ GroupLevel group_level(const Params& p, const BinArgs& a, int g) {
  GroupLevel r;
  r.l = g % p.L;
  const int bm = g / p.L;
  r.m = bm % p.M;
  r.b = bm / p.M;
  r.H = (int32_t)p.shapes[2 * r.l];
  r.W = (int32_t)p.shapes[2 * r.l + 1];
  r.st = (int32_t)p.starts[r.l];
  const int64_t hw = (int64_t)r.H * r.W;
  const int64_t nk = (hw + (1 << a.log2k) - 1) >> a.log2k;
  const bool bad = hw < 0 || nk > a.nbmax;  // the group is skipped
  r.nk = bad ? -1 : (int32_t)nk;
  r.nb = bad ? -1 : (int32_t)((hw + (1 << a.log2p) - 1) >> a.log2p);
  return r;
}

// Key of each of this lane's kBinIt samples of group g, sample block qb:
// sample li = qb * kBinPerWg + wave * kBinPerWave + u * kWave + lane (a
// wave's samples are one contiguous run, in sample order), key = 2^log2k
// pixel block of the first in-map corner, ~0 for a sample with no corner in
// the map (or past the last sample).
template <class T, bool FUSED>
__device__ __forceinline__ void bin_keys(const Params& p, const BinArgs& a, const GroupLevel& gl,
                                         int qb, uint32_t (&key)[kBinIt]) {
  const uint32_t qk = (uint32_t)(p.Q * p.K);
  const BinSrc rs = bin_src(p, a);
  const float fw = (float)gl.W, fh = (float)gl.H;
  const uint32_t li0 = (uint32_t)qb * kBinPerWg + (threadIdx.x / kWave) * kBinPerWave +
                       (threadIdx.x & (kWave - 1));
  BinIn in[kBinIt];
#pragma unroll
  for (int u = 0; u < kBinIt; ++u) {  // all loads in flight together (no branch)
    const uint32_t li = li0 + u * kWave;
    const bool ok = li < qk;
    const uint32_t lc = ok ? li : 0u;
    const uint32_t q = fdiv(lc, p.div_k), k = lc - q * (uint32_t)p.K;
    const uint32_t bq = (uint32_t)gl.b * p.Q + q;
    const uint32_t pair = bq * p.M + gl.m;
    const uint32_t pi = pair * (uint32_t)p.LK + (uint32_t)gl.l * p.K + k;
    in[u] = bin_load<T, FUSED, false>(p, rs, bq, pair, pi, gl.l, ok ? 0u : 0x80000000u);
  }
#pragma unroll
  for (int u = 0; u < kBinIt; ++u) {
    const uint32_t li = li0 + u * kWave;
    key[u] = ~0u;
    if (li < qk) {
      int32_t x0, y0;
      float lx, ly;
      bin_cell<T, FUSED>(in[u].x, in[u].y, in[u].rx, in[u].ry, fw, fh, x0, y0, lx, ly);
      const uint32_t vm = bin_vmask(x0, y0, gl.H, gl.W);
      if (vm) {
        const int32_t c = __builtin_ctz(vm);
        const int32_t pk = y0 * gl.W + x0 + ((c & 1) ? 1 : 0) + ((c & 2) ? gl.W : 0);
        key[u] = (uint32_t)pk >> a.log2k;
      }
    }
  }
}

// Group and sample block of a binning workgroup.  Each XCD takes a
// contiguous range of (b, m, sample block, level) with the level fastest:
// the L levels' samples of a query share the parameter lines its XCD's L2
// holds (a pair's L * K locations are one run).
__device__ __forceinline__ void bin_block(const Params& p, const BinArgs& a, int& g, int& qb) {
  const int lb = xcd_remap((int)blockIdx.x, (int)gridDim.x);
  const int l = lb % p.L;
  const int t = lb / p.L;
  qb = t % a.nqb;
  g = (t / a.nqb) * p.L + l;
}

// Per sample block: its samples' count per key, one row of the group's
// count matrix a.mat (every key written, so no zero-fill is needed).
template <class T, bool FUSED>
__global__ __launch_bounds__(kBlock) void bin_count_kernel(Params p, BinArgs a) {
  __shared__ uint32_t s_hist[kBinMaxBands];
  int g, qb;
  bin_block(p, a, g, qb);
  const GroupLevel gl = group_level(p, a, g);
  if (gl.nk <= 0) return;
  for (int j = threadIdx.x; j < gl.nk; j += kBlock) s_hist[j] = 0u;
  __syncthreads();
  uint32_t key[kBinIt];
  bin_keys<T, FUSED>(p, a, gl, qb, key);
  // Neighbouring lanes hold neighbouring samples (a query's K points, then
  // the next query's), which mostly share a key: each run of equal keys in
  // a wave instruction adds its length once, from its first lane (lanes
  // adding to one LDS word in one instruction are serialised).
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int u = 0; u < kBinIt; ++u) {
    const uint32_t k = key[u];
    // wave_shr:1 -- lane i receives lane i - 1's key; lane 0 keeps ~k.
    const uint32_t prev = __builtin_amdgcn_update_dpp(~k, k, 0x138, 0xF, 0xF, false);
    const bool head = prev != k;
    const uint64_t hm = __ballot(head);
    const uint64_t above = lane == kWave - 1 ? 0ull : hm >> (lane + 1);
    const int next = above ? lane + 1 + __builtin_ctzll(above) : kWave;
    if (head && k != ~0u) atomicAdd(&s_hist[k], (uint32_t)(next - lane));
  }
  __syncthreads();
  uint32_t* const row = a.mat + ((uint64_t)g * a.nqb + qb) * a.nbmax;
  for (int j = threadIdx.x; j < gl.nk; j += kBlock) row[j] = s_hist[j];
}

// Per sample block: each sample's entry id (q * K + k) at its slot.  The
// slot of a sample is fixed by the inputs: key cursor (entries of the
// group's earlier keys) + entries of the key from earlier sample blocks
// (a.mat after bin_scan_kernel) + entries of the key from earlier waves of
// the block + the sample's rank among its wave's samples of the key.  The
// last comes from per-wave LDS counters, whose returned values depend only
// on the wave's own instructions in program order.  So a key's entries are
// in sample order block by block, wave by wave: grouped by query, which
// the accumulation kernel's loads of grad_out rows and parameters rely on.
template <class T, bool FUSED>
__global__ __launch_bounds__(kBlock) void bin_fill_kernel(Params p, BinArgs a) {
  // 16-bit counters per wave, keys 2k and 2k + 1 in word k (a wave adds at
  // most kBinPerWave < 2^16 to a key), then each wave's exclusive prefix
  // over the waves before it.
  __shared__ uint32_t s_cnt[kBlock / kWave][kBinMaxBands / 2];
  __shared__ uint32_t s_base[kBinMaxBands];
  int g, qb;
  bin_block(p, a, g, qb);
  const GroupLevel gl = group_level(p, a, g);
  if (gl.nk <= 0) return;
  const int nwd = (gl.nk + 1) / 2;
  const int wave = threadIdx.x / kWave;
#pragma unroll
  for (int w = 0; w < kBlock / kWave; ++w)
    for (int j = threadIdx.x; j < nwd; j += kBlock) s_cnt[w][j] = 0u;
  // Every key's base: its cursor + its entries in earlier blocks.  All loads
  // issued before the first is used (buffer loads: past the last key they
  // read zeros); a loop that stored each pair before loading the next waited
  // out one memory round trip per 256 keys.
  {
    const __amdgpu_buffer_rsrc_t rrow = make_rsrc(
        a.mat + ((uint64_t)g * a.nqb + qb) * a.nbmax, (uint32_t)gl.nk * 4u);
    const __amdgpu_buffer_rsrc_t rcur = make_rsrc(a.cursors + (uint32_t)g * a.nbmax,
                                                  (uint32_t)gl.nk * 4u);
    constexpr int kIt = kBinMaxBands / kBlock;
    uint32_t v[kIt];
#pragma unroll
    for (int i = 0; i < kIt; ++i) {
      const uint32_t o = (uint32_t)(threadIdx.x + i * kBlock) * 4u;
      v[i] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rcur, o, 0, 0) +
             (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rrow, o, 0, 0);
    }
    // (The compiler would sink each load into its guarded store below.)
#pragma unroll
    for (int i = 0; i < kIt; ++i) asm volatile("" : "+v"(v[i]));
#pragma unroll
    for (int i = 0; i < kIt; ++i) {
      const int j = threadIdx.x + i * kBlock;
      if (j < gl.nk) s_base[j] = v[i];
    }
  }
  __syncthreads();
  uint32_t key[kBinIt], rank[kBinIt];
  bin_keys<T, FUSED>(p, a, gl, qb, key);
#pragma unroll
  for (int u = 0; u < kBinIt; ++u) {
    rank[u] = 0u;
    if (key[u] != ~0u) {
      const uint32_t sh = (key[u] & 1u) * 16u;
      rank[u] = (atomicAdd(&s_cnt[wave][key[u] >> 1], 1u << sh) >> sh) & 0xffffu;
    }
  }
  __syncthreads();
  for (int j = threadIdx.x; j < nwd; j += kBlock) {
    uint32_t c = 0u;  // both halves at once: no half exceeds 2^16
#pragma unroll
    for (int w = 0; w < kBlock / kWave; ++w) {
      const uint32_t n = s_cnt[w][j];
      s_cnt[w][j] = c;
      c += n;
    }
  }
  __syncthreads();
  const uint32_t qk = (uint32_t)(p.Q * p.K);
  uint32_t* const ent = a.entries + (uint64_t)g * qk;
  const uint32_t li0 = (uint32_t)qb * kBinPerWg + wave * kBinPerWave + (threadIdx.x & (kWave - 1));
#pragma unroll
  for (int u = 0; u < kBinIt; ++u) {
    if (key[u] != ~0u) {
      const uint32_t k = key[u];
      const uint32_t before = (s_cnt[wave][k >> 1] >> ((k & 1u) * 16u)) & 0xffffu;
      const uint32_t pos = s_base[k] + before + rank[u];
      if (pos < qk) ent[pos] = li0 + u * kWave;
    }
  }
}

// One workgroup per group: each key's total over the sample blocks, the
// count matrix turned into each block's exclusive prefix within the key,
// the key cursors (exclusive prefix of the totals over the keys), then the
// work items (band | several << 31, first entry, end entry, 0).
__global__ __launch_bounds__(kBlock) void bin_scan_kernel(Params p, BinArgs a) {
  __shared__ uint32_t s_off[kBinMaxBands + 1];
  __shared__ uint32_t s_scan[kBlock];
  const int g = blockIdx.x;
  if (g == 0 && threadIdx.x < kBinXcds) a.next[threadIdx.x] = 0u;
  const GroupLevel gl = group_level(p, a, g);
  if (gl.nk <= 0) {
    if (threadIdx.x == 0) a.nitems[g] = 0u;
    return;
  }
  uint32_t* const mat = a.mat + (uint64_t)g * a.nqb * a.nbmax;
  uint32_t* cursors = a.cursors + (uint32_t)g * a.nbmax;
  uint32_t carry = 0u, total = 0u;
  for (int j0 = 0; j0 < gl.nk; j0 += kBlock) {
    const int j = j0 + threadIdx.x;
    uint32_t v = 0u;
    if (j < gl.nk) {
      // The key's column, eight blocks' loads in flight at a time.
      for (int qb0 = 0; qb0 < a.nqb; qb0 += 8) {
        uint32_t n[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
          n[i] = qb0 + i < a.nqb ? mat[(uint64_t)(qb0 + i) * a.nbmax + j] : 0u;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          if (qb0 + i < a.nqb) mat[(uint64_t)(qb0 + i) * a.nbmax + j] = v;
          v += n[i];
        }
      }
    }
    const uint32_t ex = block_excl_scan(v, s_scan, total);
    if (j < gl.nk) {
      s_off[j] = carry + ex;
      cursors[j] = carry + ex;
    }
    carry += total;
  }
  if (threadIdx.x == 0) s_off[gl.nk] = carry;
  __syncthreads();

  // Band j (pixels [jP, jP + P)) takes the samples keyed from pixel
  // jP - W - 1 (their last corner is at most W + 1 past the key pixel) to
  // its last pixel: keys lo_key(j) .. hi_key(j), contiguous entries.
  const int64_t hw = (int64_t)gl.H * gl.W;
  auto range = [&](int j, uint32_t& lo, uint32_t& hi) {
    const int64_t p0 = ((int64_t)j << a.log2p) - (int64_t)gl.W - 1;
    const int64_t p1 = ((int64_t)(j + 1) << a.log2p) < hw ? ((int64_t)(j + 1) << a.log2p) : hw;
    lo = s_off[p0 <= 0 ? 0 : (int)(p0 >> a.log2k)];
    hi = s_off[(int)((p1 - 1) >> a.log2k) + 1];
  };
  uint32_t vis = 0u;
  for (int j = threadIdx.x; j < gl.nb; j += kBlock) {
    uint32_t lo, hi;
    range(j, lo, hi);
    vis += hi - lo;
  }
  uint32_t vtot = 0u;
  (void)block_excl_scan(vis, s_scan, vtot);
  const uint32_t room = (uint32_t)(a.cap - gl.nb);  // > 0 (host: cap > bands per level)
  uint32_t ceff = (vtot + room - 1u) / room;
  if (ceff < (uint32_t)a.chunk) ceff = (uint32_t)a.chunk;

  // A band is stored with plain stores only when it is one item and its
  // rows belong to its level alone: the level table must be the cumulative
  // one (start_l = sum of the H W before it, covering S), as
  // level_start_index = None gives.  Levels of any other table may share
  // rows, so every band then adds into the zeroed accumulator with atomics.
  bool shared = false;
  {
    int64_t acc = 0;
    for (int l = 0; l < p.L; ++l) {
      if (p.starts[l] != acc) shared = true;
      acc += p.shapes[2 * l] * p.shapes[2 * l + 1];
    }
    if (acc != (int64_t)p.S) shared = true;
  }
  uint4* items = a.items + (uint32_t)g * a.cap;
  uint32_t ibase = 0u;
  for (int j0 = 0; j0 < gl.nb; j0 += kBlock) {
    const int j = j0 + threadIdx.x;
    uint32_t lo = 0u, hi = 0u, nch = 0u;
    if (j < gl.nb) {
      range(j, lo, hi);
      nch = (hi - lo + ceff - 1u) / ceff;
    }
    const uint32_t ex = block_excl_scan(nch, s_scan, total);
    const uint32_t per = nch ? (hi - lo + nch - 1u) / nch : 0u;  // equal chunks
    for (uint32_t c = 0; c < nch; ++c) {
      const uint32_t e0 = lo + c * per;
      const uint32_t e1 = hi - e0 > per ? e0 + per : hi;
      const uint32_t idx = ibase + ex + c;
      if (idx < (uint32_t)a.cap)
        items[idx] = make_uint4((uint32_t)j | (nch > 1u || shared ? 0x80000000u : 0u), e0, e1, 0u);
    }
    ibase += total;
  }
  if (threadIdx.x == 0) a.nitems[g] = ibase < (uint32_t)a.cap ? ibase : (uint32_t)a.cap;
}

// Per work item: sum the entries' contributions to the band's rows in LDS,
// then store or add them.  Each round of 256 staged samples is sorted by
// band row in LDS (integer counts, prefix, fill); every thread owns 32
// fp32 accumulators (32 channels of one row, or all channels of several) in
// registers for the whole item and adds its rows' entries to them -- no
// float atomics, no read-modify-write of LDS.  The sums leave through LDS so
// that the stores (or atomics) cover whole rows.  RB = D * sizeof(T) bytes
// of a grad_out row.  A: the element type of the target (T, or F32 for the fp32
// scratch).  Persistent: workgroups take the items of the flattened list in
// order from a global counter until it passes the item count.
template <class T, class A, int RB, bool FUSED>
__global__ __launch_bounds__(kBlock, 3) void bin_acc_kernel(Params p, BinArgs a) {
  constexpr int kD = RB / T::kBytes;  // channels
  constexpr int kQ = RB / 16;         // 16-byte pieces of a grad_out row
  constexpr int kStride = kD + 1;     // LDS row stride (floats): spreads teams over banks
  static_assert(kD <= kWave && (kD & (kD - 1)) == 0, "team of D lanes");
  constexpr int kP = kBinAccFloats / kD;  // rows per band
  constexpr int kWPT = (kP / 2 + kBlock - 1) / kBlock;  // counter words per thread
  // Thread-owned accumulators: kChT channels of kRowsT rows (32 floats);
  // 8 channels each, so that the entries of a busy row are split over
  // several threads.
  constexpr int kChT = kD < 8 ? kD : 8;
  constexpr int kTpr = kD / kChT;                // threads per row
  constexpr int kRowsT = kP * kTpr / kBlock;     // rows per thread
  constexpr int kRowStep = kBlock / kTpr;
  static_assert(kRowsT * kChT == kBinAccFloats / kBlock, "32 accumulators per thread");
  // grad_out rows (raw) during the rounds; the band's sums at the end.
  constexpr int kUnion16 = (kP * kStride * 4 > kBlock * RB ? kP * kStride * 4 : kBlock * RB) / 16;
  __shared__ i32x4 s_u[kUnion16];
  i32x4* const s_g = s_u;
  float* const s_acc = reinterpret_cast<float*>(s_u);
  __shared__ float4 s_coef[kBlock];   // A * w_c
  // Corner entries per band row counted per wave (this round; 16-bit, rows
  // 2k and 2k + 1 in word k), then each wave's exclusive prefix over the
  // waves before it: an entry's rank in its row depends only on the
  // inputs, so the order of every fp32 sum is fixed.
  __shared__ uint32_t s_cnt[kBlock / kWave][kP / 2];
  __shared__ uint32_t s_off[kP + 1];  // row offsets: exclusive prefix of the row totals
  __shared__ uint16_t s_ent[4 * kBlock];  // entries by row: staged sample * 4 + corner
  __shared__ uint32_t s_wsum[kBlock / kWave];
  __shared__ uint32_t s_pre[kBinMaxGroups + 1];
  __shared__ uint32_t s_scan[kBlock];
  static_assert(kP % 2 == 0, "two rows per counter word");
#pragma unroll
  for (int w = 0; w < kBlock / kWave; ++w)
    for (int i = threadIdx.x; i < kP / 2; i += kBlock) s_cnt[w][i] = 0u;
  const int wave = threadIdx.x / kWave;

  // Item prefix over the groups.
  {
    constexpr int kPer = kBinMaxGroups / kBlock;
    uint32_t v[kPer], sum = 0u, total = 0u;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int gi = threadIdx.x * kPer + i;
      v[i] = gi < a.ngroups ? a.nitems[gi] : 0u;
      sum += v[i];
    }
    uint32_t ex = block_excl_scan(sum, s_scan, total);
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int gi = threadIdx.x * kPer + i;
      if (gi < a.ngroups) s_pre[gi] = ex;
      ex += v[i];
    }
    if (threadIdx.x == 0) s_pre[a.ngroups] = total;
    __syncthreads();
  }
  const uint32_t qk = (uint32_t)(p.Q * p.K);
  const uint32_t P = 1u << a.log2p;
  const BinSrc rs = bin_src(p, a);
  const __amdgpu_buffer_rsrc_t rg = make_rsrc(p.grad_out, p.gout_bytes);
  const __amdgpu_buffer_rsrc_t rc = make_rsrc(p.grad_acc, p.acc_bytes);
  const float det_s = A::kBytes == 8 ? det_scale(p) : 0.f;  // int64 fixed-point scale

  // Items by XCD: XCD x owns the items of groups [x ng / 8, (x + 1) ng / 8)
  // -- whole (b, m) runs of levels, whose items share grad_out rows and
  // parameter lines in that XCD's L2 -- and its workgroups (block ids x, x
  // + 8, ...) take them in order from counter x; then they help the other
  // XCDs' lists in turn.  Every workgroup's loop ends once all eight
  // counters have passed their lists' ends.
  __shared__ uint32_t s_w;
  const int xcd = (int)(blockIdx.x % kBinXcds);
  int src = 0;
  for (;;) {
    const int xs = (xcd + src) % kBinXcds;
    const int g0 = xs * a.ngroups / kBinXcds, g1 = (xs + 1) * a.ngroups / kBinXcds;
    const uint32_t end = s_pre[g1];
    if (threadIdx.x == 0) s_w = s_pre[g0] < end ? s_pre[g0] + atomicAdd(&a.next[xs], 1u) : end;
    __syncthreads();
    const uint32_t w = s_w;
    __syncthreads();
    if (w >= end) {
      if (++src == kBinXcds) break;
      continue;
    }
    int lo = g0, hi = g1;  // s_pre[lo] <= w < s_pre[hi]
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (s_pre[mid] <= w) lo = mid; else hi = mid;
    }
    const int g = lo;
    const uint4 it = a.items[(uint32_t)g * a.cap + (w - s_pre[g])];
    const GroupLevel gl = group_level(p, a, g);
    const uint32_t band = it.x & 0x7fffffffu;
    const bool several = (it.x >> 31) != 0u;
    const uint32_t e0 = it.y, e1 = it.z < qk ? it.z : qk;
    const int32_t r0 = (int32_t)(band << a.log2p);
    const int32_t hw = gl.H * gl.W;
    const int32_t nrow = hw - r0 < (int32_t)P ? hw - r0 : (int32_t)P;
    const float fw = (float)gl.W, fh = (float)gl.H;
    const uint32_t* ent = a.entries + (uint64_t)g * qk;
    float acc[kRowsT][kChT];
#pragma unroll
    for (int i = 0; i < kRowsT; ++i)
#pragma unroll
      for (int k = 0; k < kChT; ++k) acc[i][k] = 0.f;
    const int own_r0 = threadIdx.x / kTpr, own_c0 = (threadIdx.x % kTpr) * kChT;

    // Software pipeline: entry ids two rounds ahead, parameters and
    // grad_out rows one round ahead of the round being added.
    auto load_id = [&](uint32_t e) { return e < e1 ? ent[e] : ~0u; };
    struct Pre {
      uint32_t ok;
      BinIn in;
      i32x4 g[kQ];
    };
    auto load_pre = [&](uint32_t li, Pre& s) {
      s.ok = li < qk;
      s.in = BinIn{0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      if (s.ok) {
        const uint32_t q = fdiv(li, p.div_k), k = li - q * (uint32_t)p.K;
        const uint32_t bq = (uint32_t)gl.b * p.Q + q;
        const uint32_t pair = bq * p.M + gl.m;
        const uint32_t pi = pair * (uint32_t)p.LK + (uint32_t)gl.l * p.K + k;
        s.in = bin_load<T, FUSED, true>(p, rs, bq, pair, pi, gl.l);
#pragma unroll
        for (int i = 0; i < kQ; ++i)
          s.g[i] = __builtin_amdgcn_raw_buffer_load_b128(rg, pair * (uint32_t)RB + 16u * i, 0, 0);
      }
    };
    Pre cur;
    load_pre(load_id(e0 + threadIdx.x), cur);
    uint32_t id_next = load_id(e0 + kBlock + threadIdx.x);
    for (uint32_t rb = e0; rb < e1; rb += kBlock) {
      // Stage this round's samples; count their corner entries per row
      // (the returned count is the entry's rank in its row).
      uint32_t rw[4] = {0xffffu, 0xffffu, 0xffffu, 0xffffu}, rk[4] = {0u, 0u, 0u, 0u};
      float4 cf = make_float4(0.f, 0.f, 0.f, 0.f);
      if (cur.ok) {
        int32_t x0, y0;
        float lx, ly;
        bin_cell<T, FUSED>(cur.in.x, cur.in.y, cur.in.rx, cur.in.ry, fw, fh, x0, y0, lx, ly);
        const uint32_t vm = bin_vmask(x0, y0, gl.H, gl.W);
        const int32_t base = y0 * gl.W + x0 - r0;
        const int32_t rr[4] = {base, base + 1, base + gl.W, base + gl.W + 1};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          if (((vm >> c) & 1u) && rr[c] >= 0 && rr[c] < nrow) {
            rw[c] = (uint32_t)rr[c];
            const uint32_t sh = (rw[c] & 1u) * 16u;  // a wave adds at most 4 * 64 to a row
            rk[c] = (atomicAdd(&s_cnt[wave][rw[c] >> 1], 1u << sh) >> sh) & 0xffffu;
          }
        }
        const float mx = 1.f - lx, my = 1.f - ly;
        const float aw = FUSED ? expf(cur.in.a - cur.in.lse) : cur.in.a;
        cf = make_float4(aw * (mx * my), aw * (lx * my), aw * (mx * ly), aw * (lx * ly));
      }
      s_coef[threadIdx.x] = cf;
#pragma unroll
      for (int i = 0; i < kQ; ++i) s_g[threadIdx.x * kQ + i] = cur.g[i];
      // Next round's loads, in flight while this round is summed.
      load_pre(id_next, cur);
      id_next = load_id(rb + 2 * kBlock + threadIdx.x);
      __syncthreads();

      // Row offsets: exclusive prefix of the row totals; each wave's counter
      // becomes the entries of the waves before it.  A thread takes kWPT
      // counter words (rows 2 wd, 2 wd + 1), both halves summed at once: a
      // row takes at most one corner of each of the round's samples, so no
      // half exceeds 2^16.
      {
        uint32_t v[2 * kWPT], sum = 0u;
#pragma unroll
        for (int i = 0; i < kWPT; ++i) {
          const int wd = threadIdx.x * kWPT + i;
          uint32_t c = 0u;
          if (wd < kP / 2) {
#pragma unroll
            for (int w = 0; w < kBlock / kWave; ++w) {
              const uint32_t n = s_cnt[w][wd];
              s_cnt[w][wd] = c;
              c += n;
            }
          }
          v[2 * i] = c & 0xffffu;
          v[2 * i + 1] = c >> 16;
          sum += v[2 * i] + v[2 * i + 1];
        }
        const int lane = threadIdx.x & (kWave - 1), wv = threadIdx.x / kWave;
        uint32_t x = sum;
#pragma unroll
        for (int d = 1; d < kWave; d <<= 1) {
          const uint32_t y = (uint32_t)__shfl_up((int)x, d);
          if (lane >= d) x += y;
        }
        if (lane == kWave - 1) s_wsum[wv] = x;
        __syncthreads();
        uint32_t ex = x - sum, tot = 0u;
#pragma unroll
        for (int w2 = 0; w2 < kBlock / kWave; ++w2) {
          const uint32_t ws = s_wsum[w2];
          if (w2 < wv) ex += ws;
          tot += ws;
        }
#pragma unroll
        for (int i = 0; i < 2 * kWPT; ++i) {
          const int r = threadIdx.x * 2 * kWPT + i;
          if (r < kP) s_off[r] = ex;
          ex += v[i];
        }
        if (threadIdx.x == 0) s_off[kP] = tot;
        __syncthreads();
      }
#pragma unroll
      for (int c = 0; c < 4; ++c)
        if (rw[c] != 0xffffu) {
          const uint32_t before = (s_cnt[wave][rw[c] >> 1] >> ((rw[c] & 1u) * 16u)) & 0xffffu;
          s_ent[s_off[rw[c]] + before + rk[c]] = (uint16_t)(threadIdx.x * 4 + c);
        }
      __syncthreads();
      // Counters reset for the next round (it counts after this round's
      // closing barrier).
#pragma unroll
      for (int w = 0; w < kBlock / kWave; ++w)
        for (int i = threadIdx.x; i < kP / 2; i += kBlock) s_cnt[w][i] = 0u;

      // Each thread adds the entries of the rows it owns to its registers.
      const float* coefs = reinterpret_cast<const float*>(s_coef);
#pragma unroll
      for (int i = 0; i < kRowsT; ++i) {
        const int r = own_r0 + i * kRowStep;
        const uint32_t eb = s_off[r], ee = s_off[r + 1];
        constexpr int kW = kChT * T::kBytes / 16;  // 16-byte pieces of this thread's channels
        const int q0 = own_c0 * T::kBytes / 16;
        auto add = [&](float c, const i32x4 (&x)[kW]) {
#pragma unroll
          for (int w = 0; w < kW; ++w) {
            if constexpr (T::kBytes == 4) {
#pragma unroll
              for (int k = 0; k < 4; ++k) acc[i][4 * w + k] += c * __int_as_float(x[w][k]);
            } else {
#pragma unroll
              for (int k = 0; k < 4; ++k) {
                float lo, hi;
                unpack2<T>((uint32_t)x[w][k], lo, hi);
                acc[i][8 * w + 2 * k] += c * lo;
                acc[i][8 * w + 2 * k + 1] += c * hi;
              }
            }
          }
        };
        uint32_t e = eb;
        for (; e + 4 <= ee; e += 4) {  // four entries' loads in flight together
          uint32_t u[4];
          float c[4];
          i32x4 x[4][kW];
#pragma unroll
          for (int j = 0; j < 4; ++j) u[j] = s_ent[e + j];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            c[j] = coefs[u[j]];
#pragma unroll
            for (int w = 0; w < kW; ++w) x[j][w] = s_g[(u[j] >> 2) * kQ + q0 + w];
          }
#pragma unroll
          for (int j = 0; j < 4; ++j) add(c[j], x[j]);
        }
        for (; e < ee; ++e) {
          const uint32_t u = s_ent[e];
          i32x4 x[kW];
#pragma unroll
          for (int w = 0; w < kW; ++w) x[w] = s_g[(u >> 2) * kQ + q0 + w];
          add(coefs[u], x);
        }
      }
      __syncthreads();
    }

    // Accumulators to LDS (rows exclusive to their threads), then out.
#pragma unroll
    for (int i = 0; i < kRowsT; ++i)
#pragma unroll
      for (int k = 0; k < kChT; ++k) s_acc[(own_r0 + i * kRowStep) * kStride + own_c0 + k] = acc[i][k];
    __syncthreads();

    // The band's rows: value rows st + r0 + row of (b, m).
    const uint32_t vrow0 = (((uint32_t)gl.b * p.S + gl.st + r0) * p.M + gl.m) * (uint32_t)kD;
    const uint32_t vstep = (uint32_t)p.M * kD;
    for (int idx = 2 * threadIdx.x; idx < nrow * kD; idx += 2 * kBlock) {
      const int row = idx / kD, c0 = idx % kD;
      const float v0 = s_acc[row * kStride + c0], v1 = s_acc[row * kStride + c0 + 1];
      const uint32_t el = vrow0 + (uint32_t)row * vstep + c0;
      if constexpr (A::kBytes == 8) {
        // Deterministic: the item's fp32 sums (their order fixed by the
        // inputs) in int64 fixed point, stored, or added exactly when the
        // band is split over items; det_cast_kernel rounds them afterwards.
        const long long q0 = to_fixed(v0, det_s), q1 = to_fixed(v1, det_s);
        if (!several) {
          __builtin_amdgcn_raw_buffer_store_b128(
              i32x4{(int)(uint32_t)q0, (int)(q0 >> 32), (int)(uint32_t)q1, (int)(q1 >> 32)}, rc,
              el * 8u, 0, 0);
        } else {
          if (q0 != 0) raw_buffer_atomic_add_i64(q0, rc, (int)(el * 8u), 0, 0);
          if (q1 != 0) raw_buffer_atomic_add_i64(q1, rc, (int)(el * 8u + 8u), 0, 0);
        }
      } else if (!several) {
        if constexpr (A::kBytes == 4) {
          __builtin_amdgcn_raw_buffer_store_b64(i32x2{__float_as_int(v0), __float_as_int(v1)}, rc,
                                                el * 4u, 0, 0);
        } else {
          __builtin_amdgcn_raw_buffer_store_b32((int)pack2<A>(v0, v1), rc, el * 2u, 0, 0);
        }
      } else if (v0 != 0.f || v1 != 0.f) {
        if constexpr (A::kBytes == 4) {
          __builtin_amdgcn_raw_ptr_buffer_atomic_fadd_f32(v0, rc, (int)(el * 4u), 0, 0);
          __builtin_amdgcn_raw_ptr_buffer_atomic_fadd_f32(v1, rc, (int)(el * 4u + 4u), 0, 0);
        } else if constexpr (A::kCode == kBF16) {
          raw_buffer_atomic_fadd_v2bf16(bf16x2{(__bf16)v0, (__bf16)v1}, rc, (int)(el * 2u), 0, 0);
        } else {
          __builtin_amdgcn_raw_ptr_buffer_atomic_fadd_v2f16(f16x2{(_Float16)v0, (_Float16)v1}, rc,
                                                            (int)(el * 2u), 0, 0);
        }
      }
    }
    __syncthreads();
  }
}

int bin_cus() {
  static std::atomic<int> cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cus[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

template <class T, class A, bool FUSED>
hipError_t launch_acc(int rb, const Params& p, const BinArgs& a, hipStream_t st) {
  const int64_t slots = (int64_t)a.ngroups * a.cap;
  const int64_t want = 3 * (int64_t)bin_cus();
  const dim3 grid((unsigned)(slots < want ? slots : want));
  switch (rb) {
    case 32:
      hipLaunchKernelGGL((bin_acc_kernel<T, A, 32, FUSED>), grid, dim3(kBlock), 0, st, p, a);
      break;
    case 64:
      hipLaunchKernelGGL((bin_acc_kernel<T, A, 64, FUSED>), grid, dim3(kBlock), 0, st, p, a);
      break;
    case 128:
      hipLaunchKernelGGL((bin_acc_kernel<T, A, 128, FUSED>), grid, dim3(kBlock), 0, st, p, a);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <class T, bool FUSED>
hipError_t launch_t(bool f32acc, bool det, const Params& p, const BinArgs& a, hipStream_t st) {
  const int ng = a.ngroups;
  const dim3 gbin((unsigned)(ng * a.nqb));
  hipLaunchKernelGGL((bin_count_kernel<T, FUSED>), gbin, dim3(kBlock), 0, st, p, a);
  hipLaunchKernelGGL(bin_scan_kernel, dim3((unsigned)ng), dim3(kBlock), 0, st, p, a);
  hipLaunchKernelGGL((bin_fill_kernel<T, FUSED>), gbin, dim3(kBlock), 0, st, p, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  // The count matrix lived in the accumulator; now it is zeroed for the sums.
  e = launch_zero(p.grad_acc, p.acc_bytes, st);
  if (e != hipSuccess) return e;
  const int rb = p.D * T::kBytes;
  if (det) return launch_acc<T, I64, FUSED>(rb, p, a, st);
  if constexpr (T::kBytes == 4) {
    (void)f32acc;
    return launch_acc<T, F32, FUSED>(rb, p, a, st);
  } else {
    return f32acc ? launch_acc<T, F32, FUSED>(rb, p, a, st) : launch_acc<T, T, FUSED>(rb, p, a, st);
  }
}

}  // namespace

bool bin_plan(int64_t B, int64_t Q, int64_t M, int64_t K, int64_t D, int64_t S, int64_t L,
              int elem_bytes, void* grad_loc, void* grad_attn, void* acc, int acc_elem_bytes,
              BinArgs* a) {
  const int64_t rb = D * elem_bytes;
  if (rb != 32 && rb != 64 && rb != 128) return false;
  if (D > kWave || (D & (D - 1)) != 0) return false;
  const int64_t qk = Q * K;
  if (qk <= 0 || S <= 0 || L <= 0 || B <= 0 || M <= 0) return false;
  const int64_t ng = B * M * L;
  if (ng > kBinMaxGroups) return false;
  int log2p = 0;
  while ((int64_t)2 << log2p <= kBinAccFloats / D) ++log2p;  // P = 2^log2p <= 8192 / D
  const int64_t P = (int64_t)1 << log2p;
  // Keys of 32 pixels (coarser for very large maps): a band reads the keys
  // of its own pixels and of the W + 1 before it.
  int log2k = 5;
  while (log2k < log2p && (S >> log2k) + 2 > kBinMaxBands) ++log2k;
  const int64_t nbmax = (S >> log2k) + 2;  // keys per level, at most
  if (nbmax > kBinMaxBands) return false;
  const int64_t bands = (S + P - 1) / P + 1;
  const int64_t cap = bands + (2 * qk + kBinChunk - 1) / kBinChunk + 16;
  // Entries: 4 bytes per sample in grad_loc (2 * elem_bytes per sample).
  if ((reinterpret_cast<uintptr_t>(grad_loc) & 3u) != 0) return false;
  // Cursors, item counts, the item counter, then 16-byte aligned items in
  // grad_attn.
  uintptr_t base = reinterpret_cast<uintptr_t>(grad_attn);
  if ((base & 3u) != 0) return false;
  const uint64_t avail = (uint64_t)(ng * qk * elem_bytes);
  const uint64_t n_cur = (uint64_t)(ng * nbmax) * 4u;
  uint64_t off_items = n_cur + (uint64_t)ng * 4u + 4u * kBinXcds;
  off_items += (16u - ((base + off_items) & 15u)) & 15u;
  const uint64_t need = off_items + (uint64_t)(ng * cap) * 16u;
  if (need > avail || (uint64_t)(ng * qk * 2 * elem_bytes) > 0xffffffffull) return false;
  // The count matrix (one row of keys per sample block) in the accumulator,
  // which is zeroed after the binning.
  const int64_t nqb = (qk + kBinPerWg - 1) / kBinPerWg;
  if ((reinterpret_cast<uintptr_t>(acc) & 3u) != 0) return false;
  if ((uint64_t)(ng * nqb * nbmax) * 4u > (uint64_t)(B * S * M * D * acc_elem_bytes)) return false;
  char* ws = static_cast<char*>(grad_attn);
  a->entries = static_cast<uint32_t*>(grad_loc);
  a->cursors = reinterpret_cast<uint32_t*>(ws);
  a->nitems = reinterpret_cast<uint32_t*>(ws + n_cur);
  a->next = reinterpret_cast<uint32_t*>(ws + n_cur + (uint64_t)ng * 4u);
  a->items = reinterpret_cast<uint4*>(ws + off_items);
  a->mat = static_cast<uint32_t*>(acc);
  a->ngroups = (int32_t)ng;
  a->nbmax = (int32_t)nbmax;
  a->cap = (int32_t)cap;
  a->nqb = (int32_t)nqb;
  a->log2p = log2p;
  a->log2k = log2k;
  a->chunk = kBinChunk;
  a->loc_bytes = (uint32_t)(ng * qk * 2 * elem_bytes);
  a->attn_bytes = (uint32_t)(ng * qk * elem_bytes);
  return true;
}

hipError_t launch_binned(int dtype, bool fused, bool f32acc, bool det, const Params& p,
                         const BinArgs& a, hipStream_t st) {
  if (a.ngroups <= 0) return hipSuccess;
  switch (dtype) {
    case kF32:
      return fused ? launch_t<F32, true>(false, det, p, a, st)
                   : launch_t<F32, false>(false, det, p, a, st);
    case kF16:
      return fused ? launch_t<F16, true>(f32acc, det, p, a, st)
                   : launch_t<F16, false>(f32acc, det, p, a, st);
    case kBF16:
      return fused ? launch_t<BF16, true>(f32acc, det, p, a, st)
                   : launch_t<BF16, false>(f32acc, det, p, a, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace msda
