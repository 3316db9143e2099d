// Paged KV-cache writer: RoPE on K at write time, level-blocked K pages and
// transposed V pages (the cache format both attention kernels read).
//
// Replaces the reference's two steps around the cache: the RoPE + head-dim
// permutation patch (e2e_pipeline/atflash_e2e_fafi.py:186-192) and the HF cache
// append the kernels then read (e2e_pipeline/atflash_e2e_fafi.py:101-119).
// The permutation is not needed here: the cache stores the half-split dims of
// each 16-dim level contiguously, so the window stays a prefix of every page.
#include "atf_launch.h"

namespace atf {

// One workgroup of 128 threads per (cache page, sequence * kv head): it writes
// the page's slots that the call covers.  K: thread (level l = tid/16, slot
// tid%16) rotates and writes the 32 B of its token's level l, so a wave writes
// four whole 512 B level blocks.  V: the page's token rows are staged in LDS
// with 16-byte loads, then thread d writes V^T row d (32 B: 16 slots in the
// {0,2,1,3} group order) with two 16-byte stores.  A page the call covers only
// in part (the first and last page of a call, e.g. every single-token decode
// append) merges the covered slots into the row it reads back first, so slots
// outside the call keep their contents.  Tokens at negative positions, past
// max_pages, past the RoPE table or whose page-table entry is invalid are
// skipped, as one token at a time would be.
// grid: x = page index relative to the call's first page, y = batch * hkv.
__global__ __launch_bounds__(128) void kv_write_kernel(KvWriteArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t sv[kPage][kD];
  const int b = blockIdx.y / a.hkv;
  const int h = blockIdx.y - b * a.hkv;
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
  const size_t blk = (static_cast<size_t>(pg) * a.hkv + h) * kBlockElems;
  const int t0 = static_cast<int>(p0 - start);  // source token of slot 0

  // ---- K ----
  {
    const int l = tid >> 4, slot = tid & 15;
    if (slot >= s0 && slot < s1) {
      const int t = t0 + slot;
      const uint16_t* krow = a.k_src + static_cast<int64_t>(b) * a.ks_b + static_cast<int64_t>(t) * a.ks_t +
                             static_cast<int64_t>(h) * a.ks_h;
      const int c0 = level_chunk0(a.layout, l);
      const int c1 = level_chunk1(a.layout, l);
      u32x4 x1 = ldg16(krow + c0);
      u32x4 x2 = ldg16(krow + c1);
      if (a.rope_cs != nullptr) {
        float cs[16];
        load_cs8(a.rope_cs, static_cast<int>(p0) + slot, c0, cs);
        const u32x4 y1 = rope_half(x1, x2, cs, false);
        const u32x4 y2 = rope_half(x1, x2, cs, true);
        x1 = y1;
        x2 = y2;
      }
      uint16_t* kdst = a.k_cache + blk + l * 256 + slot * 16;
      *reinterpret_cast<u32x4*>(kdst) = x1;
      *reinterpret_cast<u32x4*>(kdst + 8) = x2;
    }
  }

  // ---- V: stage the covered token rows, then write transposed rows ----
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int idx = tid + 128 * r;  // token idx/16, 16-byte chunk idx%16
    const int tok = idx >> 4, ch = idx & 15;
    if (tok >= s0 && tok < s1) {
      const uint16_t* vrow = a.v_src + static_cast<int64_t>(b) * a.vs_b + static_cast<int64_t>(t0 + tok) * a.vs_t +
                             static_cast<int64_t>(h) * a.vs_h;
      *reinterpret_cast<u32x4*>(&sv[tok][8 * ch]) = ldg16(vrow + 8 * ch);
    }
  }
  __syncthreads();
  const int d = tid;
  uint16_t* vdst = a.v_cache + blk + d * kPage;
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
      const uint32_t val = sv[tok][d];
      w[sl >> 1] = (sl & 1) ? ((w[sl >> 1] & 0x0000ffffu) | (val << 16)) : ((w[sl >> 1] & 0xffff0000u) | val);
    }
  }
  *reinterpret_cast<u32x4*>(vdst) = u32x4{w[0], w[1], w[2], w[3]};
  *reinterpret_cast<u32x4*>(vdst + 8) = u32x4{w[4], w[5], w[6], w[7]};
}

hipError_t launch_kv_write(const KvWriteArgs& a, hipStream_t s) {
  if (a.n_tokens <= 0 || a.batch <= 0) return hipSuccess;
  // a call of n tokens touches at most ceil(n / 16) + 1 pages per sequence
  dim3 grid((a.n_tokens + kPage - 1) / kPage + 1, a.batch * a.hkv);
  hipLaunchKernelGGL(kv_write_kernel, grid, dim3(128), 0, s, a);
  return hipGetLastError();
}

}  // namespace atf
