// Windowed split-KV decode over the paged, level-blocked KV cache (gfx950).
//
// Replaces the FlashInfer window port's single-request decode
// (single_decode_with_kv_cache_with_jit_module(..., maybe_zhi_slice=...),
// kernels/flashinfer_port/fiwin_common.py:96-112, e2e_pipeline/atflash_e2e_fafi.py:106-109;
// window predicate: kernels/flashinfer_port/decode.cuh.diff:47-89).
//
// One workgroup of 8 waves per (sequence, kv head, split of pages); each wave
// streams its own pages.  The G = Hq/Hkv query heads of the kv head are the 16
// columns of v_mfma_f32_16x16x32_bf16 (S^T = K Q^T, two 16-dim levels per
// instruction) and v_mfma_f32_16x16x16_bf16 (O^T = V^T P^T, 16 tokens per
// instruction).  K and V are loaded straight into the MFMA operand registers.
// The window predicate is per page: page p is read for its first
// L(p) = D_eff/16 levels, D_eff = 16 * #{i : zhi[i] >= (N-1) - (16p+15)}; the
// loads of the other levels are never issued, so out-of-window K bytes are not
// read from HBM.
//
// Merging, all in the one launch: the 8 wave partials (m, l, o) of a split are
// combined in LDS and written to the workspace; the last workgroup to finish
// for a (sequence, kv head) -- it sees the device-scope arrival counter reach
// n_splits - 1 -- merges the split partials by log-sum-exp, writes the output
// and resets the counter to zero for the next call.
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

// two waves per SIMD: at most 256 registers per wave
__global__ __launch_bounds__(kDecWaves * 64) __attribute__((amdgpu_waves_per_eu(2)))
void decode_kernel(DecodeArgs a) {
  // wave partials; in the merging workgroup, afterwards, the split weights
  __shared__ __attribute__((aligned(16))) float sh_o[kDecWaves * kDecMaxGroup * kD];
  __shared__ float sh_m[kDecWaves * kDecMaxGroup], sh_l[kDecWaves * kDecMaxGroup];
  __shared__ float red[kDecWaves * 64];
  __shared__ float sh_M[kDecMaxGroup], sh_L[kDecMaxGroup];
  __shared__ int sh_last;
  static_assert(kDecMaxSplits * kDecMaxGroup <= kDecWaves * kDecMaxGroup * kD, "split weights must fit sh_o");

  const int s = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
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

  // wave w takes the groups of kDecUnroll pages that start at p_begin + kDecUnroll * (w + kDecWaves * i)
  for (int p0 = p_begin + kDecUnroll * wave; p0 < p_end; p0 += kDecUnroll * kDecWaves) {
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

  // ---- the split's partial: combine the wave partials in LDS ----
  const float l_tot = quad_sum(l_run);
  if (g < a.group) {
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      const int d = 16 * db + 4 * (lane >> 4);
      *reinterpret_cast<f32x4*>(&sh_o[(wave * kDecMaxGroup + g) * kD + d]) = O[db];
    }
    if (lane < 16) {
      sh_m[wave * kDecMaxGroup + g] = m_run;
      sh_l[wave * kDecMaxGroup + g] = l_tot;
    }
  }
  __syncthreads();
  // thread t owns query head t / 32, dims 4 (t % 32) .. +3 (group <= 16: 512 tasks)
  const int gq = tid >> 5, d4 = 4 * (tid & 31);
  const bool owner = gq < a.group;
  const int64_t pbase = (static_cast<int64_t>(b) * a.hkv + h) * a.n_splits * kDecMaxGroup;  // split 0, head 0
  if (owner) {
    float M = NEG_INF;
#pragma unroll
    for (int w = 0; w < kDecWaves; ++w) M = fmaxf(M, sh_m[w * kDecMaxGroup + gq]);
    float L = 0.f;
    f32x4 acc = f32x4{};
    if (M != NEG_INF) {
#pragma unroll
      for (int w = 0; w < kDecWaves; ++w) {
        const float wt = fast_exp2((sh_m[w * kDecMaxGroup + gq] - M) * c);  // empty wave: m = -inf -> 0
        L += wt * sh_l[w * kDecMaxGroup + gq];
        acc += wt * *reinterpret_cast<const f32x4*>(&sh_o[(w * kDecMaxGroup + gq) * kD + d4]);
      }
    }
    const int64_t pi = pbase + static_cast<int64_t>(s) * kDecMaxGroup + gq;
    *reinterpret_cast<f32x4*>(a.ws_o + pi * kD + d4) = acc;
    if (d4 == 0) {
      a.ws_ml[pi * 2 + 0] = M;
      a.ws_ml[pi * 2 + 1] = L;
    }
  }

  // ---- arrival: the last split of (b, h) to finish merges all splits ----
  // One release per workgroup: the barrier orders every wave's partial stores
  // before thread 0's agent-scope release increment (each device-scope fence
  // writes back the XCD's L2, so it is issued once, not per wave).
  __syncthreads();
  uint32_t* cnt = a.counters + (static_cast<int64_t>(b) * a.hkv + h);
  if (tid == 0) {
    const uint32_t old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    const int last = (old == static_cast<uint32_t>(a.n_splits - 1)) ? 1 : 0;
    if (last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");  // the other splits' partials are visible
    sh_last = last;
  }
  __syncthreads();
  if (!sh_last) return;

  // split weights w_s = exp2((m_s - M) c) and L = sum_s w_s l_s per query head;
  // thread (gi, part) holds the (m, l) of splits part, part + 32, ... in registers
  constexpr int kParts = kDecWaves * 64 / kDecMaxGroup;
  constexpr int kPerPart = (kDecMaxSplits + kParts - 1) / kParts;
  const int gi = tid & (kDecMaxGroup - 1), part = tid >> 4;
  float ml[kPerPart][2];
  float M = NEG_INF;
#pragma unroll
  for (int j = 0; j < kPerPart; ++j) {
    const int sp = part + kParts * j;
    ml[j][0] = NEG_INF;
    ml[j][1] = 0.f;
    if (gi < a.group && sp < a.n_splits) {
      const int64_t pi = pbase + static_cast<int64_t>(sp) * kDecMaxGroup + gi;
      ml[j][0] = a.ws_ml[pi * 2];
      ml[j][1] = a.ws_ml[pi * 2 + 1];
    }
    M = fmaxf(M, ml[j][0]);
  }
  red[part * kDecMaxGroup + gi] = M;
  __syncthreads();
  if (tid < kDecMaxGroup) {
    float mm = NEG_INF;
    for (int p2 = 0; p2 < kParts; ++p2) mm = fmaxf(mm, red[p2 * kDecMaxGroup + tid]);
    sh_M[tid] = mm;
  }
  __syncthreads();
  float* wts = sh_o;  // [n_splits][16]
  {
    const float Mg = sh_M[gi];
    float L = 0.f;
#pragma unroll
    for (int j = 0; j < kPerPart; ++j) {
      const int sp = part + kParts * j;
      const float wt = (Mg == NEG_INF) ? 0.f : fast_exp2((ml[j][0] - Mg) * c);  // m = -inf -> 0
      if (sp < a.n_splits) wts[sp * kDecMaxGroup + gi] = wt;
      L += wt * ml[j][1];
    }
    __syncthreads();  // every read of sh_M / red above is done
    red[part * kDecMaxGroup + gi] = L;
  }
  __syncthreads();
  if (tid < kDecMaxGroup) {
    float ll = 0.f;
    for (int p2 = 0; p2 < kParts; ++p2) ll += red[p2 * kDecMaxGroup + tid];
    sh_L[tid] = ll;
  }
  __syncthreads();
  if (owner) {
    // out = sum_s w_s o_s / L, kBatch independent 16-byte loads in flight per thread
    constexpr int kBatch = 32;
    const float* po = a.ws_o + (pbase + gq) * kD + d4;
    const int64_t sstride = static_cast<int64_t>(kDecMaxGroup) * kD;
    f32x4 acc = f32x4{};
    for (int s0 = 0; s0 < a.n_splits; s0 += kBatch) {
      f32x4 buf[kBatch];
#pragma unroll
      for (int j = 0; j < kBatch; ++j)
        buf[j] = (s0 + j < a.n_splits) ? *reinterpret_cast<const f32x4*>(po + (s0 + j) * sstride) : f32x4{};
#pragma unroll
      for (int j = 0; j < kBatch; ++j)
        if (s0 + j < a.n_splits) acc += wts[(s0 + j) * kDecMaxGroup + gq] * buf[j];
    }
    const float Lg = sh_L[gq];
    const float inv = Lg > 0.f ? 1.f / Lg : 0.f;
    uint16_t* o = a.out + static_cast<int64_t>(b) * a.o_sb + static_cast<int64_t>(h * a.group + gq) * a.o_sh + d4;
    u32x2 pk;
    pk[0] = pack_bf16x2(acc[0] * inv, acc[1] * inv);
    pk[1] = pack_bf16x2(acc[2] * inv, acc[3] * inv);
    *reinterpret_cast<u32x2*>(o) = pk;
  }
  if (tid == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Level count per page for one sequence of length N (decode rule, block_n = 16).
__global__ void decode_page_levels_kernel(int32_t* out, int n_pages, int N, LevelTable lt) {
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= n_pages) return;
  out[p] = levels_of(lt, max(0, (N - 1) - (p * kPage + kPage - 1)));
}

hipError_t launch_decode(const DecodeArgs& a, hipStream_t s) {
  if (a.batch <= 0) return hipSuccess;
  hipLaunchKernelGGL(decode_kernel, dim3(a.n_splits, a.hkv, a.batch), dim3(kDecWaves * 64), 0, s, a);
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
