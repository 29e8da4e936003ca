// Atomic scatter of gradient rows into grad_value (or its fp32 scratch),
// shared by the direct and the LDS-privatised backward kernels.
#pragma once

#include "msda_device.h"

namespace msda {

// Add one 4-byte accumulator word: an fp32 element, or a packed pair of
// fp16 / bf16 elements (lo, hi), at byte offset `off` of buffer `r`.
// Out-of-range offsets are dropped by the buffer range check.
template <class A>
__device__ __forceinline__ void atomic_add_word(__amdgpu_buffer_rsrc_t r, uint32_t off, float lo,
                                                float hi) {
  if constexpr (A::kBytes == 4) {
    (void)hi;
    __builtin_amdgcn_raw_ptr_buffer_atomic_fadd_f32(lo, r, (int)off, 0, 0);
  } else if constexpr (A::kCode == kBF16) {
    bf16x2 x = {(__bf16)lo, (__bf16)hi};
    raw_buffer_atomic_fadd_v2bf16(x, r, (int)off, 0, 0);
  } else {
    f16x2 x = {(_Float16)lo, (_Float16)hi};
    __builtin_amdgcn_raw_ptr_buffer_atomic_fadd_v2f16(x, r, (int)off, 0, 0);
  }
}

// Scatter of one corner row.  The accumulator row holds D elements of A;
// seen as 4-byte words (one fp32 element, or a packed pair of fp16 / bf16
// elements), live chunk lane c of the g_real lanes owns the words
// c, c + g_real, c + 2 g_real, ...  One atomic instruction then covers
// g_real consecutive words of every row it touches: the hardware executes
// buffer atomics per 64-byte segment, so a full segment per instruction is
// four times faster than the 16-byte pieces a lane's own gather chunk would
// give.  `sg` holds this lane's grad_out values in that word order.
//
// A = I64 (deterministic backward): each element is one 8-byte word of
// int64 fixed point; contributions are converted with the call's scale
// (det_scale) and added with 64-bit integer atomics, so the result does not
// depend on their order.
template <class T, class A, int CB>
struct Scatter {
  static constexpr int kVec = CB / T::kBytes;
  static constexpr int kWordBytes = A::kBytes == 8 ? 8 : 4;
  static constexpr int kWordsPerLane = kVec * A::kBytes / kWordBytes;  // 0: odd-D half rows
  static constexpr int kElemsPerWord = A::kBytes > 0 ? kWordBytes / A::kBytes : 1;
  static constexpr int kSlots = kWordsPerLane > 0 ? kWordsPerLane * kElemsPerWord : 1;

  // grad_out values of the words this lane scatters.
  __device__ __forceinline__ static void load_g(const Params& p, int pair, int ch, bool live,
                                                float (&sg)[kSlots]) {
    for (int i = 0; i < kSlots; ++i) sg[i] = 0.f;
    if (!live || pair >= p.npairs) return;
    const uint64_t base = (uint64_t)pair * (uint32_t)p.D;
    if constexpr (kWordsPerLane == 0) {
      sg[0] = load1<T>(p.grad_out, base + ch);  // CB == 2: one element per lane
    } else {
#pragma unroll
      for (int i = 0; i < kWordsPerLane; ++i) {
        const uint64_t e0 = base + (uint64_t)(ch + p.g_real * i) * kElemsPerWord;
        if constexpr (kElemsPerWord == 2) {
          load_xy<T>(p.grad_out, e0 / 2, sg[2 * i], sg[2 * i + 1]);
        } else {
          sg[i] = load1<T>(p.grad_out, e0);
        }
      }
    }
  }

  // Add coef * sg into the row whose accumulator byte offset is `row`
  // (out-of-range rows are dropped by the buffer range check).
  __device__ __forceinline__ static void add(__amdgpu_buffer_rsrc_t r, uint32_t row, int ch,
                                             int g_real, float coef, const float (&sg)[kSlots],
                                             float det_s = 0.f) {
    if constexpr (A::kBytes == 8) {
#pragma unroll
      for (int i = 0; i < kWordsPerLane; ++i) {
        const uint32_t off = row + 8u * (uint32_t)(ch + g_real * i);
        raw_buffer_atomic_add_i64(to_fixed(coef * sg[i], det_s), r, (int)off, 0, 0);
      }
    } else if constexpr (kWordsPerLane == 0) {
      // Half storage with odd D: rows are not word aligned; add this lane's
      // element with the packed atomic on its enclosing word, zero in the
      // other half.
      const uint32_t off = row + (uint32_t)ch * A::kBytes;
      const float v = coef * sg[0];
      const bool hi = (off & 2u) != 0;
      if constexpr (A::kCode == kBF16) {
        bf16x2 x = {(__bf16)(hi ? 0.f : v), (__bf16)(hi ? v : 0.f)};
        raw_buffer_atomic_fadd_v2bf16(x, r, (int)(off & ~3u), 0, 0);
      } else {
        f16x2 x = {(_Float16)(hi ? 0.f : v), (_Float16)(hi ? v : 0.f)};
        __builtin_amdgcn_raw_ptr_buffer_atomic_fadd_v2f16(x, r, (int)(off & ~3u), 0, 0);
      }
    } else {
#pragma unroll
      for (int i = 0; i < kWordsPerLane; ++i) {
        const uint32_t off = row + 4u * (uint32_t)(ch + g_real * i);
        if constexpr (A::kBytes == 4) {
          atomic_add_word<A>(r, off, coef * sg[i], 0.f);
        } else {
          atomic_add_word<A>(r, off, coef * sg[2 * i], coef * sg[2 * i + 1]);
        }
      }
    }
  }
};

}  // namespace msda
