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

// grid: x = token blocks of 64, y = level (0..7), z = batch * hkv.
// Thread (token t, level l) writes K level l of token t (32 B) and V dims
// 16l..16l+15 of token t (16 transposed slots).
__global__ __launch_bounds__(64) void kv_write_kernel(KvWriteArgs a) {
  const int t = blockIdx.x * 64 + threadIdx.x;
  const int l = blockIdx.y;
  const int b = blockIdx.z / a.hkv;
  const int h = blockIdx.z % a.hkv;
  if (t >= a.n_tokens) return;
  const int pos = a.start_pos[b] + t;
  const int pidx = pos / kPage, slot = pos % kPage;
  if (pos < 0 || pidx >= a.max_pages) return;
  if (a.rope_cs != nullptr && pos >= a.rope_max_pos) return;
  const int pg = a.page_table[static_cast<int64_t>(b) * a.max_pages + pidx];
  if (pg < 0 || pg >= a.num_pages) return;
  const size_t blk = (static_cast<size_t>(pg) * a.hkv + h) * kBlockElems;

  const uint16_t* krow = a.k_src + static_cast<int64_t>(b) * a.ks_b + static_cast<int64_t>(t) * a.ks_t +
                         static_cast<int64_t>(h) * a.ks_h;
  const int c0 = level_chunk0(a.layout, l);
  const int c1 = level_chunk1(a.layout, l);
  u32x4 x1 = ldg16(krow + c0);
  u32x4 x2 = ldg16(krow + c1);
  if (a.rope_cs != nullptr) {
    float cs[16];
    load_cs8(a.rope_cs, pos, c0, cs);
    const u32x4 y1 = rope_half(x1, x2, cs, false);
    const u32x4 y2 = rope_half(x1, x2, cs, true);
    x1 = y1;
    x2 = y2;
  }
  uint16_t* kdst = a.k_cache + blk + l * 256 + slot * 16;
  *reinterpret_cast<u32x4*>(kdst) = x1;
  *reinterpret_cast<u32x4*>(kdst + 8) = x2;

  const uint16_t* vrow = a.v_src + static_cast<int64_t>(b) * a.vs_b + static_cast<int64_t>(t) * a.vs_t +
                         static_cast<int64_t>(h) * a.vs_h + 16 * l;
  const u32x4 v0 = ldg16(vrow);
  const u32x4 v1 = ldg16(vrow + 8);
  uint16_t* vdst = a.v_cache + blk + v_slot(slot);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    vdst[(16 * l + 2 * i) * 16] = static_cast<uint16_t>(v0[i] & 0xffffu);
    vdst[(16 * l + 2 * i + 1) * 16] = static_cast<uint16_t>(v0[i] >> 16);
    vdst[(16 * l + 8 + 2 * i) * 16] = static_cast<uint16_t>(v1[i] & 0xffffu);
    vdst[(16 * l + 8 + 2 * i + 1) * 16] = static_cast<uint16_t>(v1[i] >> 16);
  }
}

hipError_t launch_kv_write(const KvWriteArgs& a, hipStream_t s) {
  if (a.n_tokens <= 0 || a.batch <= 0) return hipSuccess;
  dim3 grid((a.n_tokens + 63) / 64, kLevels, a.batch * a.hkv);
  hipLaunchKernelGGL(kv_write_kernel, grid, dim3(64), 0, s, a);
  return hipGetLastError();
}

}  // namespace atf
