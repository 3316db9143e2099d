// Windowed split-KV decode over the paged, level-blocked KV cache (gfx950).
//
// Replaces the FlashInfer window port's single-request decode
// (single_decode_with_kv_cache_with_jit_module(..., maybe_zhi_slice=...),
// kernels/flashinfer_port/fiwin_common.py:96-112, e2e_pipeline/atflash_e2e_fafi.py:106-109;
// window predicate: kernels/flashinfer_port/decode.cuh.diff:47-89).
//
// One wave per (sequence, kv head, split of pages).  The G = Hq/Hkv query heads
// of the kv head are the 16 columns of v_mfma_f32_16x16x32_bf16 (S^T = K Q^T,
// two 16-dim levels per instruction) and v_mfma_f32_16x16x16_bf16
// (O^T = V^T P^T, 16 tokens per instruction).  K and V are loaded straight into
// the MFMA operand registers (no LDS).  The window predicate is per page:
// page p is read for its first L(p) = D_eff/16 levels, where
// D_eff = 16 * #{i : zhi[i] >= (N-1) - (16p+15)}; the loads of the other levels
// are never issued, so out-of-window K bytes are not read from HBM.  Each split
// writes an unnormalised partial (m, l, o); a second kernel merges the partials
// by log-sum-exp.
#include "atf_launch.h"

namespace atf {

// max / sum over the 4 lanes {l, l^16, l^32, l^48} that hold one query head.
__device__ __forceinline__ float quad_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}
__device__ __forceinline__ float quad_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}

struct PageRegs {
  u32x4 k[4];  // level pairs
  u32x2 v[8];  // 16-row d blocks
  int L;
  int n0;
};

__device__ __forceinline__ void dec_load_page(const DecodeArgs& a, int b, int h, int p, int N, int lane,
                                              PageRegs& r) {
  r.n0 = p * kPage;
  r.L = levels_of(a.lt, max(0, (N - 1) - (r.n0 + kPage - 1)));
  int pg = a.page_table[static_cast<int64_t>(b) * a.max_pages + p];
  const bool ok = pg >= 0 && pg < a.num_pages;
  const size_t blk = (static_cast<size_t>(ok ? pg : 0) * a.hkv + h) * kBlockElems;
  const uint16_t* kb = a.k_cache + blk;
  const uint16_t* vb = a.v_cache + blk;
  const int lvl_hi = lane >> 5;
  const int half = (lane >> 4) & 1;
  const int tok = lane & 15;
#pragma unroll
  for (int lp = 0; lp < 4; ++lp) {
    u32x4 v = {0u, 0u, 0u, 0u};
    const int level = 2 * lp + lvl_hi;
    if (ok && level < r.L) v = ldg16(kb + level * 256 + tok * 16 + half * 8);
    r.k[lp] = v;
  }
  // V^T operand: d row 16*db + lane%16, tokens 4*(lane/16)..+3 -> stored slots.
  const int grp = lane >> 4;
  const int slot0 = 4 * ((grp == 1) ? 2 : (grp == 2 ? 1 : grp));
#pragma unroll
  for (int db = 0; db < 8; ++db) {
    u32x2 v = {0u, 0u};
    if (ok) v = *reinterpret_cast<const u32x2*>(vb + (16 * db + tok) * 16 + slot0);
    r.v[db] = v;
  }
}

__global__ __launch_bounds__(64) void decode_split_kernel(DecodeArgs a) {
  const int s = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int lane = threadIdx.x;
  const int g = lane & 15;
  const int N = max(0, min(a.seq_lens[b], a.max_seq_len));
  const int n_pages = (N + kPage - 1) / kPage;
  const int p_begin = s * a.pages_per_split;
  const int p_end = min(n_pages, p_begin + a.pages_per_split);
  const float NEG_INF = -__builtin_huge_valf();
  const float c = a.scale_log2;

  // ---- Q^T fragments: lane holds q head g, level 2lp + lane/32, half (lane/16)%2 ----
  u32x4 Qf[4];
  {
    const int qh = h * a.group + g;
    const bool valid = g < a.group && N > 0;
    const uint16_t* qrow = a.q + static_cast<int64_t>(b) * a.q_sb + static_cast<int64_t>(qh) * a.q_sh;
    const bool second = ((lane >> 4) & 1) != 0;
#pragma unroll
    for (int lp = 0; lp < 4; ++lp) {
      u32x4 v = {0u, 0u, 0u, 0u};
      const int level = 2 * lp + (lane >> 5);
      if (valid) {
        const int c0 = level_chunk0(a.layout, level);
        const int c1 = level_chunk1(a.layout, level);
        if (a.rope_cs != nullptr) {
          float cs[16];
          load_cs8(a.rope_cs, N - 1, c0, cs);
          v = rope_half(ldg16(qrow + c0), ldg16(qrow + c1), cs, second);
        } else {
          v = ldg16(qrow + (second ? c1 : c0));
        }
      }
      Qf[lp] = v;
    }
  }

  f32x4 O[8];
#pragma unroll
  for (int db = 0; db < 8; ++db) O[db] = f32x4{};
  float m_run = NEG_INF, l_run = 0.f;

  for (int p0 = p_begin; p0 < p_end; p0 += kDecUnroll) {
    PageRegs pr[kDecUnroll];
#pragma unroll
    for (int u = 0; u < kDecUnroll; ++u) {
      if (p0 + u < p_end) dec_load_page(a, b, h, p0 + u, N, lane, pr[u]);
    }
#pragma unroll
    for (int u = 0; u < kDecUnroll; ++u) {
      if (p0 + u >= p_end) break;
      PageRegs& r = pr[u];
      f32x4 S = f32x4{};
#pragma unroll
      for (int lp = 0; lp < 4; ++lp) {
        if (2 * lp < r.L)
          S = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, r.k[lp]),
                                                      __builtin_bit_cast(bf16x8, Qf[lp]), S, 0, 0, 0);
      }
      // S lane layout: q head g, tokens 4*(lane/16) + i.
      const int tok0 = r.n0 + 4 * (lane >> 4);
      const bool tail = r.n0 + kPage > N;
      float mx = NEG_INF;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (tail && tok0 + i >= N) S[i] = NEG_INF;
        mx = fmaxf(mx, S[i]);
      }
      if (tail) {
        // zero V of tokens past N so that 0 * V stays 0
#pragma unroll
        for (int db = 0; db < 8; ++db) {
          if (tok0 + 0 >= N) r.v[db][0] &= 0xffff0000u;
          if (tok0 + 1 >= N) r.v[db][0] &= 0x0000ffffu;
          if (tok0 + 2 >= N) r.v[db][1] &= 0xffff0000u;
          if (tok0 + 3 >= N) r.v[db][1] &= 0x0000ffffu;
        }
      }
      mx = quad_max(mx);
      const float m_new = fmaxf(m_run, mx);
      float alpha, msc;
      if (m_new == NEG_INF) {
        alpha = 1.f;
        msc = 0.f;
      } else {
        alpha = fast_exp2((m_run - m_new) * c);
        msc = m_new * c;
      }
      m_run = m_new;
      float pv[4];
      float ls = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pv[i] = fast_exp2(__builtin_fmaf(S[i], c, -msc));
        ls += pv[i];
      }
      l_run = l_run * alpha + ls;
      u32x2 pk;
      pk[0] = pack_bf16x2(pv[0], pv[1]);
      pk[1] = pack_bf16x2(pv[2], pv[3]);
      const s16x4 pb = __builtin_bit_cast(s16x4, pk);
#pragma unroll
      for (int db = 0; db < 8; ++db) {
        O[db] *= alpha;
        O[db] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, r.v[db]), pb, O[db], 0, 0, 0);
      }
    }
  }

  const float l_tot = quad_sum(l_run);
  const int64_t part = ((static_cast<int64_t>(b) * a.hkv + h) * a.n_splits + s) * kDecMaxGroup;
  if (g < a.group) {
    float* o = a.ws_o + (part + g) * kD;
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      const int d = 16 * db + 4 * (lane >> 4);
      *reinterpret_cast<f32x4*>(o + d) = O[db];
    }
    if (lane < 16) {
      a.ws_ml[(part + g) * 2 + 0] = m_run;
      a.ws_ml[(part + g) * 2 + 1] = l_tot;
    }
  }
}

// One workgroup of 256 threads per (q head, sequence).  The split weights
// w_s = exp2((m_s - M) c) go to LDS once; the weighted sum over splits is then
// read as coalesced 128-float rows, two splits in flight per thread pair.
__device__ __forceinline__ float block_reduce(float v, float* red, bool is_max) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float o = __shfl_xor(v, off);
    v = is_max ? fmaxf(v, o) : v + o;
  }
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  v = red[0];
#pragma unroll
  for (int i = 1; i < 4; ++i) v = is_max ? fmaxf(v, red[i]) : v + red[i];
  return v;
}

__global__ __launch_bounds__(256) void decode_merge_kernel(MergeArgs a) {
  __shared__ float wsh[kDecMaxSplits];
  __shared__ float red[4];
  __shared__ float half_acc[kD];
  const int qh = blockIdx.x, b = blockIdx.y;
  const int tid = threadIdx.x;
  const int h = qh / a.group, g = qh % a.group;
  const int64_t base = (static_cast<int64_t>(b) * a.hkv + h) * a.n_splits;
  const float NEG_INF = -__builtin_huge_valf();
  float M = NEG_INF;
  for (int s = tid; s < a.n_splits; s += 256) M = fmaxf(M, a.ws_ml[((base + s) * kDecMaxGroup + g) * 2]);
  M = block_reduce(M, red, true);
  float L = 0.f;
  for (int s = tid; s < a.n_splits; s += 256) {
    const int64_t pi = (base + s) * kDecMaxGroup + g;
    const float m = a.ws_ml[pi * 2];
    const float w = (M == NEG_INF) ? 0.f : fast_exp2((m - M) * a.scale_log2);  // m = -inf -> 0
    wsh[s] = w;
    L += w * a.ws_ml[pi * 2 + 1];
  }
  L = block_reduce(L, red, false);  // also orders the wsh writes before the reads below
  const int d = tid & (kD - 1);
  const int part = tid >> 7;
  float acc = 0.f;
#pragma unroll 8
  for (int s = part; s < a.n_splits; s += 2) acc += wsh[s] * a.ws_o[((base + s) * kDecMaxGroup + g) * kD + d];
  if (part == 1) half_acc[d] = acc;
  __syncthreads();
  if (part == 0) {
    acc += half_acc[d];
    const float o = L > 0.f ? acc / L : 0.f;
    a.out[static_cast<int64_t>(b) * a.o_sb + static_cast<int64_t>(qh) * a.o_sh + d] = f32_to_bf16(o);
  }
}

// Level count per page for one sequence of length N (decode rule, block_n = 16).
__global__ void decode_page_levels_kernel(int32_t* out, int n_pages, int N, LevelTable lt) {
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= n_pages) return;
  out[p] = levels_of(lt, max(0, (N - 1) - (p * kPage + kPage - 1)));
}

hipError_t launch_decode(const DecodeArgs& a, const MergeArgs& m, hipStream_t s) {
  if (a.batch <= 0) return hipSuccess;
  hipLaunchKernelGGL(decode_split_kernel, dim3(a.n_splits, a.hkv, a.batch), dim3(64), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(decode_merge_kernel, dim3(m.hq, m.batch), dim3(256), 0, s, m);
  return hipGetLastError();
}

hipError_t launch_decode_page_levels(int32_t* out, int n_pages, int seq_len, const LevelTable& lt,
                                     hipStream_t s) {
  if (n_pages <= 0) return hipSuccess;
  hipLaunchKernelGGL(decode_page_levels_kernel, dim3((n_pages + 255) / 256), dim3(256), 0, s, out, n_pages,
                     seq_len, lt);
  return hipGetLastError();
}

}  // namespace atf
