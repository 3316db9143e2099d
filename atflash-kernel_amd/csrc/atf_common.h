// Shared definitions for the gfx950 windowed-attention kernels.
//
// Head dim and the window rule
//   d = 128, P = d/2 = 64 RoPE pairs.  Pair r (standard order, r = 0 highest
//   frequency) sits in dims (r, r+P) of the half-split ("rotate_half") layout.
//   The window keeps the lowest-frequency pairs, a prefix in wavelength order, in
//   16-dim levels: level l (0 = always kept) holds pairs r in [P-8(l+1), P-8l),
//   i.e. dims [P-8(l+1), P-8l) and the same range + P.  In the sorted-pair
//   layout of the reference (atflash/window_table.py:13-21) level l is simply
//   dims [16l, 16l+16).
//   D_eff(z) = 16 * #{i : zhi[i] >= z} (microbench/b1_correctness.py:43-44), with
//   zhi the per-level table of window_tables/atflash_window.py:85-108; window OFF
//   is zhi[i] = INT32_MAX, i.e. D_eff = d everywhere.
//
//   The decode kernel also takes the finer table of the FlashInfer window port
//   (kernels/flashinfer_port/fiwin_common.py:35-47): 16 slices of 8 dims, slice s
//   = 4 pairs in wavelength order (pairs r in [P-4(s+1), P-4s)), read for key
//   ages z <= zhi8[s]; level l is slices 2l and 2l+1.
//
// Paged KV cache (one layer), page = 16 tokens.  One 8 KB block per (page, kv
// head), V half first, then the K half:
//   V half   [128 dims][16 token slots] bf16 = 4096 B (V transposed), token t of
//            the page stored in slot kVSlot(t); the slot order matches the lane
//            layout of the 32x32x16 and 16x16x16 MFMA accumulators so that P never
//            leaves registers.
//   K half   [16 slices][16 tokens][8 dims] bf16 = 4096 B, RoPE already applied.
//            The dims of slice s are stored as [first-half 4 | second-half 4]
//            (half-split: dims [P-4(s+1), P-4s) then the same + P) or
//            [8s .. 8s+7] (sorted pair).  Slices are contiguous 256 B runs in
//            wavelength order, so a page read for n slices (L levels = 2L
//            slices) is one contiguous 256*n-byte prefix of the K half.
//   kv_cache: [num_pages][num_kv_heads][8192 B].
// A decode read of a page is therefore one contiguous run, V and then the K
// slices in the window.  With K and V in two arrays (two runs per page) the
// memory system delivered the windowed reads 7-10% slower per byte: the
// decode's k=2 / OFF ratio at Qwen 128K was 1.15 against 1.23 here, same box.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace atf {

constexpr int kD = 128;
constexpr int kP = 64;
constexpr int kLevels = 8;
constexpr int kSlices = 16;    // 8-dim slices, two per level
constexpr int kSliceDims = 8;
constexpr int kPage = 16;
constexpr int kBlockElems = kSlices * kPage * kSliceDims;  // one half: 2048 bf16 = 4096 B
constexpr int kKvBlockElems = 2 * kBlockElems;            // a (page, kv head) block: 8192 B
constexpr int kKHalfElems = kBlockElems;                  // offset of the K half in a block
constexpr int kLayoutHalfSplit = 0;
constexpr int kLayoutSortedPair = 1;

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
typedef __attribute__((ext_vector_type(4))) short s16x4;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(2))) float f32x2;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;

// The per-level distance table, passed by value (kernel argument, lives in SGPRs).
struct LevelTable {
  int32_t zhi[kLevels];
};

// Number of 16-dim levels read at causal distance z (>= 1: D_eff is clamped to 16).
__device__ __forceinline__ int levels_of(const LevelTable& t, int z) {
  int n = 0;
#pragma unroll
  for (int i = 0; i < kLevels; ++i) n += (t.zhi[i] >= z) ? 1 : 0;
  return n < 1 ? 1 : n;
}

// Word 3 of a raw buffer resource (no format conversion, 32-bit data format
// field), as the raw buffer-load path of gfx9-family targets expects.
constexpr int kBufferWord3 = 0x00020000;

// Cache-policy operand of a buffer load that streams data read once: the
// non-temporal bit (`nt`).  On a decode-shaped probe (4 KB blocks in random
// order, 268 MB per call) it raises the read rate from 5.8 to 6.6 TB/s.
constexpr int kLoadStream = 2;

// The per-slice distance table of the decode kernel (kernel argument, SGPRs).
struct SliceTable {
  int32_t zhi[kSlices];
};

// First dim of the two 8-dim chunks of level l in the input row (half-split:
// the first-half and second-half dims of the level's 8 pairs).
__device__ __forceinline__ int level_chunk0(int layout, int l) {
  return layout == kLayoutHalfSplit ? kP - 8 * (l + 1) : 16 * l;
}
__device__ __forceinline__ int level_chunk1(int layout, int l) {
  return layout == kLayoutHalfSplit ? 2 * kP - 8 * (l + 1) : 16 * l + 8;
}

// First pair (half-split: first dim) of slice s: pairs r in [P-4(s+1), P-4s).
__device__ __forceinline__ int slice_pair0(int s) { return kP - 4 * (s + 1); }

// The 8 dims of slice s of an input row, in the order the cache stores them:
// half-split [x1 of the slice's 4 pairs | x2 of the same pairs] (two 8-byte
// loads), sorted pair dims [8s, 8s+8) (one 16-byte load).
__device__ __forceinline__ u32x4 load_slice(const uint16_t* row, int layout, int s) {
  if (layout == kLayoutHalfSplit) {
    const u32x2 x1 = *reinterpret_cast<const u32x2*>(row + slice_pair0(s));
    const u32x2 x2 = *reinterpret_cast<const u32x2*>(row + kP + slice_pair0(s));
    return u32x4{x1[0], x1[1], x2[0], x2[1]};
  }
  return *reinterpret_cast<const u32x4*>(row + 8 * s);
}

// Slices s0 + stride * i (i = 0..3) of an input row, as load_slice reads them,
// with the layout test outside the loads so that all of them are issued before
// any is waited for.
template <int kStride>
__device__ __forceinline__ void load_slices4(const uint16_t* row, int layout, int s0, u32x4 (&out)[4]) {
  if (layout == kLayoutHalfSplit) {
    u32x2 x1[4], x2[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x1[i] = *reinterpret_cast<const u32x2*>(row + slice_pair0(s0 + kStride * i));
      x2[i] = *reinterpret_cast<const u32x2*>(row + kP + slice_pair0(s0 + kStride * i));
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = u32x4{x1[i][0], x1[i][1], x2[i][0], x2[i][1]};
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = *reinterpret_cast<const u32x4*>(row + 8 * (s0 + kStride * i));
  }
}

// Slot of token t (0..15) inside a transposed V page: token groups of 4 are
// stored in the order {0, 2, 1, 3}.
__device__ __forceinline__ int v_slot(int t) {
  const int g = t >> 2;
  const int gs = (g == 1) ? 2 : (g == 2 ? 1 : g);
  return 4 * gs + (t & 3);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// fp32 -> bf16, round to nearest even (finite inputs; NaN stays NaN).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// Two floats -> packed bf16 pair (lo in bits 0-15), round to nearest even.  The
// two-element vector conversion selects one v_cvt_pk_bf16_f32; converting the
// halves separately and or-ing them costs four instructions.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// Unpack 8 bf16 (16 B) into floats.
__device__ __forceinline__ void unpack8(const u32x4& v, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(v[i] << 16);
    f[2 * i + 1] = __uint_as_float(v[i] & 0xffff0000u);
  }
}

__device__ __forceinline__ u32x4 pack8(const float* f) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = pack_bf16x2(f[2 * i], f[2 * i + 1]);
  return r;
}

// Rotate-half RoPE on one 8-pair chunk: lane keeps the first half
// (x1 c - x2 s) or the second half (x2 c + x1 s), times `scale`.  cs holds
// (cos, sin) per pair.
__device__ __forceinline__ u32x4 rope_half(const u32x4& x1v, const u32x4& x2v, const float* cs, bool second,
                                          float scale = 1.f) {
  float x1[8], x2[8], y[8];
  unpack8(x1v, x1);
  unpack8(x2v, x2);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float c = cs[2 * i], s = cs[2 * i + 1];
    y[i] = scale * (second ? (x2[i] * c + x1[i] * s) : (x1[i] * c - x2[i] * s));
  }
  return pack8(y);
}

// Rotate-half RoPE on one half-split slice x = [x1 of 4 pairs | x2 of the same
// pairs]: [x1 c - x2 s | x2 c + x1 s], times `scale`.  cs holds (cos, sin) per
// pair.
__device__ __forceinline__ u32x4 rope_slice(const u32x4& x, const float* cs, float scale = 1.f) {
  float v[8], y[8];
  unpack8(x, v);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float c = cs[2 * i], s = cs[2 * i + 1];
    y[i] = scale * (v[i] * c - v[4 + i] * s);
    y[4 + i] = scale * (v[4 + i] * c + v[i] * s);
  }
  return pack8(y);
}

__device__ __forceinline__ u32x4 ldg16(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

__device__ __forceinline__ void load_cs8(const float* rope_cs, int pos, int pair0, float* cs) {
  const u32x4* p = reinterpret_cast<const u32x4*>(rope_cs + (static_cast<size_t>(pos) * kP + pair0) * 2);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const u32x4 v = p[i];
    cs[4 * i + 0] = __uint_as_float(v[0]);
    cs[4 * i + 1] = __uint_as_float(v[1]);
    cs[4 * i + 2] = __uint_as_float(v[2]);
    cs[4 * i + 3] = __uint_as_float(v[3]);
  }
}

// (cos, sin) of the 4 pairs starting at pair0, at position pos.
__device__ __forceinline__ void load_cs4(const float* rope_cs, int pos, int pair0, float* cs) {
  const u32x4* p = reinterpret_cast<const u32x4*>(rope_cs + (static_cast<size_t>(pos) * kP + pair0) * 2);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const u32x4 v = p[i];
    cs[4 * i + 0] = __uint_as_float(v[0]);
    cs[4 * i + 1] = __uint_as_float(v[1]);
    cs[4 * i + 2] = __uint_as_float(v[2]);
    cs[4 * i + 3] = __uint_as_float(v[3]);
  }
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Exchange with lane ^ 32.
__device__ __forceinline__ float swap32(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]);
}

}  // namespace atf
