// Paged KV-cache writer: RoPE on K at write time, one block per (page, kv
// head) holding the transposed V page and then the slice-blocked K page (the
// cache format both attention kernels read).
//
// Replaces the reference's two steps around the cache: the RoPE + head-dim
// permutation patch (e2e_pipeline/atflash_e2e_fafi.py:186-192) and the HF cache
// append the kernels then read (e2e_pipeline/atflash_e2e_fafi.py:101-119).
// The permutation is not needed here: the cache stores the half-split dims of
// each 8-dim slice (4 pairs) contiguously, in wavelength order, so the window
// stays a prefix of every page.
#include "atf_launch.h"

namespace atf {

// One workgroup of 128 threads per (cache page, sequence): it writes the
// page's slots that the call covers, for every kv head, kKvwHeads heads per
// pass, so the RoPE (cos, sin) row of each position is read once for all of
// them.  K: thread (level l = tid/16, slot tid%16) loads its token's level l
// (slices 2l, 2l+1) of every head of the pass, then rotates it and writes the
// two 16 B slice rows, so a wave writes eight whole 256 B slice blocks per head.  V: the page's token rows of
// the pass's heads are staged in LDS with 16-byte loads, then thread d writes
// V^T row d of each head (32 B: 16 slots in the {0,2,1,3} group order) with
// two 16-byte stores.  A page the call covers only in part (the first and last
// page of a call, e.g. every single-token decode append) merges the covered
// slots into the row it reads back first, so slots outside the call keep their
// contents.  Tokens at negative positions, past max_pages, past the RoPE table
// or whose page-table entry is invalid are skipped, as one token at a time
// would be.
// grid: x = page index relative to the call's first page, y = sequence.
constexpr int kKvwHeads = 4;
__global__ __launch_bounds__(128) void kv_write_kernel(KvWriteArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t sv[kKvwHeads][kPage][kD];
  const int b = blockIdx.y;
  const int tid = threadIdx.x;
  const int start = a.start_pos[b];
  const int64_t end64 = static_cast<int64_t>(start) + a.n_tokens;  // exclusive
  const int first = max(start, 0) >> 4;
  const int pidx = first + static_cast<int>(blockIdx.x);
  const int64_t p0 = static_cast<int64_t>(pidx) * kPage;
  if (pidx >= a.max_pages || p0 >= end64) return;
  // covered slots [s0, s1) of this page
  int64_t lo = max(p0, static_cast<int64_t>(max(start, 0)));
  int64_t hi = min(p0 + kPage, end64);
  if (a.rope_cs != nullptr) hi = min(hi, static_cast<int64_t>(a.rope_max_pos));
  if (lo >= hi) return;
  const int s0 = static_cast<int>(lo - p0), s1 = static_cast<int>(hi - p0);
  const int pg = a.page_table[static_cast<int64_t>(b) * a.max_pages + pidx];
  if (pg < 0 || pg >= a.num_pages) return;
  const size_t blk0 = static_cast<size_t>(pg) * a.hkv * kKvBlockElems;  // the page's block of head 0
  const int t0 = static_cast<int>(p0 - start);  // source token of slot 0

  // K lane roles and the (cos, sin) of the lane's position and level, loaded once
  const int l = tid >> 4, slot = tid & 15;
  const bool k_on = slot >= s0 && slot < s1;
  const int c0 = level_chunk0(a.layout, l);
  const int c1 = level_chunk1(a.layout, l);
  float cs[16];
  if (k_on && a.rope_cs != nullptr) load_cs8(a.rope_cs, static_cast<int>(p0) + slot, c0, cs);

  for (int h0 = 0; h0 < a.hkv; h0 += kKvwHeads) {
    // ---- K: the pass's rows loaded first, then rotated and written ----
    if (k_on) {
      const uint16_t* krow = a.k_src + static_cast<int64_t>(b) * a.ks_b + static_cast<int64_t>(t0 + slot) * a.ks_t;
      u32x4 x1[kKvwHeads], x2[kKvwHeads];
#pragma unroll
      for (int j = 0; j < kKvwHeads; ++j) {
        if (h0 + j < a.hkv) {
          x1[j] = ldg16(krow + static_cast<int64_t>(h0 + j) * a.ks_h + c0);
          x2[j] = ldg16(krow + static_cast<int64_t>(h0 + j) * a.ks_h + c1);
        }
      }
#pragma unroll
      for (int j = 0; j < kKvwHeads; ++j) {
        if (h0 + j < a.hkv) {
          u32x4 y1 = x1[j], y2 = x2[j];
          if (a.rope_cs != nullptr) {
            y1 = rope_half(x1[j], x2[j], cs, false);
            y2 = rope_half(x1[j], x2[j], cs, true);
          }
          // half-split: y1 / y2 hold the first / second halves of the level's 8
          // pairs in ascending pair order; slice 2l is the upper 4 pairs (the
          // longer wavelengths), slice 2l+1 the lower 4.  Sorted pair: the two
          // 8-dim chunks are the slices.
          const bool hs = a.layout == kLayoutHalfSplit;
          const u32x4 sa = hs ? u32x4{y1[2], y1[3], y2[2], y2[3]} : y1;
          const u32x4 sb = hs ? u32x4{y1[0], y1[1], y2[0], y2[1]} : y2;
          uint16_t* kdst = a.kv_cache + blk0 + static_cast<size_t>(h0 + j) * kKvBlockElems + kKHalfElems +
                           (2 * l) * (kPage * kSliceDims) + slot * kSliceDims;
          *reinterpret_cast<u32x4*>(kdst) = sa;
          *reinterpret_cast<u32x4*>(kdst + kPage * kSliceDims) = sb;
        }
      }
    }

    // ---- V: stage the covered token rows of the pass's heads, then write
    // transposed rows ----
#pragma unroll
    for (int j = 0; j < kKvwHeads; ++j) {
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int idx = tid + 128 * r;  // token idx/16, 16-byte chunk idx%16
        const int tok = idx >> 4, ch = idx & 15;
        if (h0 + j < a.hkv && tok >= s0 && tok < s1) {
          const uint16_t* vrow = a.v_src + static_cast<int64_t>(b) * a.vs_b +
                                 static_cast<int64_t>(t0 + tok) * a.vs_t + static_cast<int64_t>(h0 + j) * a.vs_h;
          *reinterpret_cast<u32x4*>(&sv[j][tok][8 * ch]) = ldg16(vrow + 8 * ch);
        }
      }
    }
    __syncthreads();
    const int d = tid;
#pragma unroll
    for (int j = 0; j < kKvwHeads; ++j) {
      if (h0 + j >= a.hkv) break;
      uint16_t* vdst = a.kv_cache + blk0 + static_cast<size_t>(h0 + j) * kKvBlockElems + d * kPage;
      uint32_t w[8];  // the row's 16 slots as 8 packed pairs
      if (s0 == 0 && s1 == kPage) {
#pragma unroll
        for (int i = 0; i < 8; ++i) w[i] = 0u;
      } else {
        const u32x4 r0 = *reinterpret_cast<const u32x4*>(vdst);
        const u32x4 r1 = *reinterpret_cast<const u32x4*>(vdst + 8);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          w[i] = r0[i];
          w[4 + i] = r1[i];
        }
      }
#pragma unroll
      for (int tok = 0; tok < kPage; ++tok) {
        if (tok >= s0 && tok < s1) {
          const int sl = v_slot(tok);
          const uint32_t val = sv[j][tok][d];
          w[sl >> 1] = (sl & 1) ? ((w[sl >> 1] & 0x0000ffffu) | (val << 16)) : ((w[sl >> 1] & 0xffff0000u) | val);
        }
      }
      *reinterpret_cast<u32x4*>(vdst) = u32x4{w[0], w[1], w[2], w[3]};
      *reinterpret_cast<u32x4*>(vdst + 8) = u32x4{w[4], w[5], w[6], w[7]};
    }
    __syncthreads();  // sv is staged again by the next pass
  }
}

hipError_t launch_kv_write(const KvWriteArgs& a, hipStream_t s) {
  if (a.n_tokens <= 0 || a.batch <= 0) return hipSuccess;
  // a call of n tokens touches at most ceil(n / 16) + 1 pages per sequence
  dim3 grid((a.n_tokens + kPage - 1) / kPage + 1, a.batch);
  hipLaunchKernelGGL(kv_write_kernel, grid, dim3(128), 0, s, a);
  return hipGetLastError();
}

}  // namespace atf
