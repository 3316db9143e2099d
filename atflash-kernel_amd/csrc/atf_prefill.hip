// Windowed causal GQA prefill attention for gfx950 (CDNA4).
//
// Replaces the FA4 window port's forward (called as
// _flash_attn_fwd(q, k, v, causal=True, atflash_window_zhi=zhi),
// microbench/b1_correctness.py:84-85, e2e_pipeline/atflash_e2e_fafi.py:118-119).
//
// Work decomposition
//   workgroup = 8 waves = 256 consecutive query positions of one q head;
//   wave      = 32 positions (one MFMA row block); two waves share each SIMD, so
//               the softmax VALU work of one overlaps the MFMAs of the other;
//   k-tile    = 64 keys = 4 cache pages, staged through LDS (double buffered) with
//               direct global->LDS loads; the window is quantized per 32-key block
//               ("kb"), i.e. the oracle tile is (block_m, block_n) = (32, 32).
//   S^T = K Q^T and O^T = V^T P^T on v_mfma_f32_32x32x16_bf16: the accumulator
//   lane l always holds query row l%32, so the online-softmax max/sum stay in the
//   lane except one exchange with lane l^32 (v_permlane32_swap).
//   Per (wave, kb) the QK contraction runs over the first L = D_eff/16 levels
//   only, and the workgroup copies only the levels its first wave needs, so the
//   out-of-window K levels never enter LDS.  Q is rotated (RoPE) at load.
//   Online softmax with a lazily updated reference max: O and l are rescaled only
//   when a row's max grows by more than 2^8 in exp2 units, so P <= 256.
#include "atf_launch.h"

namespace atf {

typedef __attribute__((address_space(3))) uint8_t lds_u8;

constexpr float kLazyRescaleLog2 = 8.0f;

__device__ __forceinline__ float pair_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// acc + x.lo + x.hi for a packed bf16 pair (row sums of the bf16 P used in PV).
// Written as the VOP3P instruction: the clang builtin for the bf16 dot2 lowers
// to the VOP2 form with the same source register for every element of a
// vector (ROCm 7.2), which sums the wrong values.
__device__ __forceinline__ float dot2_ones(uint32_t x, float acc) {
  asm("v_dot2_f32_bf16 %0, %1, %2, %0" : "+v"(acc) : "v"(x), "v"(0x3f803f80u));
  return acc;
}

__device__ __forceinline__ bf16x8 lds_frag(const lds_u8* p) {
  return *reinterpret_cast<const __attribute__((address_space(3))) bf16x8*>(p);
}

// Stage one 64-key tile (4 pages) into LDS: waves 0-3 copy K (first L levels)
// of page w, waves 4-7 copy V of page w-4.  Missing pages are zero-filled.
__device__ __forceinline__ void pf_load_tile(const PrefillArgs& a, int b, int kvh, int t, int L,
                                             lds_u8* stage, int wave, int lane) {
  const int page = wave & 3;
  const bool is_v = wave >= 4;
  const int pidx = 4 * t + page;
  const int n_pages_k = (a.nk + kPage - 1) / kPage;
  int pg = -1;
  if (pidx < n_pages_k) {
    pg = a.page_table[static_cast<int64_t>(b) * a.max_pages + pidx];
    if (pg < 0 || pg >= a.num_pages) pg = -1;
  }
  lds_u8* dst = stage + (is_v ? 4 * 4096 : 0) + page * 4096;
  if (pg < 0) {
    const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<__attribute__((address_space(3))) u32x4*>(dst + i * 1024 + lane * 16) = z;
    return;
  }
  const size_t blk = (static_cast<size_t>(pg) * a.hkv + kvh) * 4096;
  if (is_v) {
    const uint8_t* src = reinterpret_cast<const uint8_t*>(a.v_cache) + blk;
#pragma unroll
    for (int i = 0; i < 4; ++i) __builtin_amdgcn_global_load_lds(src + i * 1024 + lane * 16, dst + i * 1024, 16, 0, 0);
  } else {
    const uint8_t* src = reinterpret_cast<const uint8_t*>(a.k_cache) + blk;
    const int npairs = (L + 1) >> 1;
    for (int lp = 0; lp < npairs; ++lp) {
      if (lane < 32 || 2 * lp + 1 < L)
        __builtin_amdgcn_global_load_lds(src + lp * 1024 + lane * 16, dst + lp * 1024, 16, 0, 0);
    }
  }
}

// S^T (32 keys x 32 rows) over the first L levels, highest level first.
__device__ __forceinline__ f32x16 qk_levels(const bf16x8 (&kf)[kLevels], const u32x4 (&Qf)[kLevels], int L) {
  f32x16 S = f32x16{};
#define ATF_QK(l) S = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[l], __builtin_bit_cast(bf16x8, Qf[l]), S, 0, 0, 0)
  switch (L) {
    case 8: ATF_QK(7); [[fallthrough]];
    case 7: ATF_QK(6); [[fallthrough]];
    case 6: ATF_QK(5); [[fallthrough]];
    case 5: ATF_QK(4); [[fallthrough]];
    case 4: ATF_QK(3); [[fallthrough]];
    case 3: ATF_QK(2); [[fallthrough]];
    case 2: ATF_QK(1); [[fallthrough]];
    default: ATF_QK(0);
  }
#undef ATF_QK
  return S;
}

__global__ __launch_bounds__(kPfWaves * 64, 1) void prefill_kernel(PrefillArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem_raw[];
  lds_u8* smem = (lds_u8*)(smem_raw);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

  // XCD-aware block mapping: block i runs on XCD i % 8.  Each XCD walks the q
  // heads of one q-tile in order (so the heads sharing a kv head share its K/V
  // tiles in that XCD's L2), and the 8 XCDs take 8 neighbouring q-tiles, the
  // heaviest (last) tiles first.
  const int bid = blockIdx.x;
  const int xcd = bid & 7;
  const int j = bid >> 3;
  const int per_b = a.n_qgroups * a.hq;
  const int b = j / per_b;
  const int jr = j - b * per_b;
  const int h = jr % a.hq;
  const int qrank = (jr / a.hq) * 8 + xcd;
  const int qt = a.n_qtiles - 1 - qrank;
  if (qt < 0 || b >= a.batch) return;
  const int kvh = h / a.group;

  const int lr0_wg = qt * kPfRowsWg;
  const int lr0 = lr0_wg + wave * kPfRowsWave;
  const int pos0_wg = a.q_offset + lr0_wg;
  const int pos0 = a.q_offset + lr0;
  const int n_ktiles = (a.nk + kPfTileN - 1) / kPfTileN;
  const int last_wg = a.q_offset + min(a.nq, lr0_wg + kPfRowsWg) - 1;
  const int t_end_wg = min(n_ktiles, last_wg / kPfTileN + 1);
  const int t_end =
      (lr0 < a.nq) ? min(n_ktiles, (a.q_offset + min(a.nq, lr0 + kPfRowsWave) - 1) / kPfTileN + 1) : 0;

  // ---- Q fragments (B operand of S^T = K Q^T), RoPE applied at load ----
  u32x4 Qf[kLevels];
  const bool second = lane >= 32;
  const int row = lr0 + (lane & 31);
  {
    const uint16_t* qrow = a.q + static_cast<int64_t>(b) * a.q_sb + static_cast<int64_t>(row) * a.q_st +
                           static_cast<int64_t>(h) * a.q_sh;
#pragma unroll
    for (int l = 0; l < kLevels; ++l) {
      u32x4 v = {0u, 0u, 0u, 0u};
      if (row < a.nq) {
        const int c0 = level_chunk0(a.layout, l);
        const int c1 = level_chunk1(a.layout, l);
        if (a.rope_cs != nullptr) {
          float cs[16];
          load_cs8(a.rope_cs, a.q_offset + row, c0, cs);
          v = rope_half(ldg16(qrow + c0), ldg16(qrow + c1), cs, second);
        } else {
          v = ldg16(qrow + (second ? c1 : c0));
        }
      }
      Qf[l] = v;
    }
  }

  f32x16 O[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) O[db] = f32x16{};
  const float NEG_INF = -__builtin_huge_valf();
  float m_ref = NEG_INF;  // reference max of the exponentials (raw score units)
  float l_run = 0.f;      // this lane's partial row sum relative to m_ref
  const float c = a.scale_log2;

  // ---- prologue: stage tile 0 (levels of its nearest key for the first row) ----
  if (t_end_wg > 0) pf_load_tile(a, b, kvh, 0, levels_of(a.lt, max(0, pos0_wg - (kPfTileN - 1))), smem, wave, lane);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  for (int t = 0; t < t_end_wg; ++t) {
    lds_u8* cur = smem + (t & 1) * kPfStageBytes;
    const int n0 = t * kPfTileN;
    // Keys past nk in the last tile: zero their V so that 0 * V stays 0.
    if (n0 + kPfTileN > a.nk) {
      const int page = threadIdx.x >> 7;
      __attribute__((address_space(3))) uint16_t* vrow = reinterpret_cast<__attribute__((address_space(3))) uint16_t*>(
          cur + 4 * 4096 + page * 4096 + (threadIdx.x & 127) * 32);
#pragma unroll
      for (int tk = 0; tk < kPage; ++tk)
        if (n0 + page * kPage + tk >= a.nk) vrow[v_slot(tk)] = 0;
      __syncthreads();
    }
    if (t + 1 < t_end_wg) {
      const int L1 = levels_of(a.lt, max(0, pos0_wg - ((t + 1) * kPfTileN + kPfTileN - 1)));
      pf_load_tile(a, b, kvh, t + 1, L1, smem + ((t + 1) & 1) * kPfStageBytes, wave, lane);
    }

    if (t < t_end) {
      // ---- S^T = K Q^T over the surviving levels of each 32-key block ----
      f32x16 S[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const int L = levels_of(a.lt, max(0, pos0 - (n0 + 32 * kb + 31)));
        const lds_u8* kbase = cur + (2 * kb + ((lane & 31) >> 4)) * 4096 + (lane & 15) * 32 + (lane >> 5) * 16;
        bf16x8 kf[kLevels];
#pragma unroll
        for (int l = 0; l < kLevels; ++l) kf[l] = lds_frag(kbase + l * 512);  // unread levels stay unused
        S[kb] = qk_levels(kf, Qf, L);
      }

      // ---- online softmax (lane = query row) ----
      const bool need_mask = (n0 + kPfTileN - 1 > pos0) || (n0 + kPfTileN > a.nk);
      const int row_pos = pos0 + (lane & 31);
      float mx = NEG_INF;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          if (need_mask) {
            const int key = n0 + 32 * kb + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            if (key > row_pos || key >= a.nk) S[kb][r] = NEG_INF;
          }
          mx = fmaxf(mx, S[kb][r]);
        }
      }
      mx = pair_max(mx);
      const bool grow = mx * c > m_ref * c + kLazyRescaleLog2;
      if (__builtin_amdgcn_ballot_w64(grow) != 0) {
        const float alpha = grow ? fast_exp2((m_ref - mx) * c) : 1.f;  // m_ref = -inf -> 0
        if (grow) m_ref = mx;
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < 4; ++db) O[db] *= alpha;
      }
      const float msc = (m_ref == NEG_INF) ? 0.f : m_ref * c;
      bf16x8 Pf[4];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int hs = 0; hs < 2; ++hs) {
          u32x4 pk;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float p0 = fast_exp2(__builtin_fmaf(S[kb][8 * hs + 2 * i], c, -msc));
            const float p1 = fast_exp2(__builtin_fmaf(S[kb][8 * hs + 2 * i + 1], c, -msc));
            pk[i] = pack_bf16x2(p0, p1);
            l_run = dot2_ones(pk[i], l_run);
          }
          Pf[2 * kb + hs] = __builtin_bit_cast(bf16x8, pk);
        }
      }

      // ---- O^T += V^T P^T ----
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        bf16x8 vf[4];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
          vf[ks] = lds_frag(cur + 4 * 4096 + ks * 4096 + (32 * db + (lane & 31)) * 32 + (lane >> 5) * 16);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) O[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[ks], Pf[ks], O[db], 0, 0, 0);
      }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  }

  // ---- epilogue: normalise and store ----
  const float l = pair_sum(l_run);
  const float inv = l > 0.f ? 1.f / l : 0.f;
  if (row < a.nq) {
    uint16_t* orow = a.out + static_cast<int64_t>(b) * a.o_sb + static_cast<int64_t>(row) * a.o_st +
                     static_cast<int64_t>(h) * a.o_sh;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = 32 * db + 8 * g + 4 * (lane >> 5);
        u32x2 w;
        w[0] = pack_bf16x2(O[db][4 * g + 0] * inv, O[db][4 * g + 1] * inv);
        w[1] = pack_bf16x2(O[db][4 * g + 2] * inv, O[db][4 * g + 3] * inv);
        *reinterpret_cast<u32x2*>(orow + d) = w;
      }
    }
    if (a.lse != nullptr && lane < 32) {
      a.lse[(static_cast<int64_t>(b) * a.hq + h) * a.nq + row] =
          (l > 0.f) ? m_ref * a.sm_scale + __logf(l) : NEG_INF;
    }
  }
}

// Level count per (32-row tile, 32-key block), from the same device rule the
// kernel uses; out is [n_row_tiles][n_kblocks].
__global__ void prefill_tile_levels_kernel(int32_t* out, int n_row_tiles, int n_kblocks, int q_offset,
                                           LevelTable lt) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_row_tiles * n_kblocks) return;
  const int rt = i / n_kblocks, kb = i % n_kblocks;
  const int pos0 = q_offset + rt * kPfRowsWave;
  out[i] = levels_of(lt, max(0, pos0 - (32 * kb + 31)));
}

hipError_t launch_prefill(const PrefillArgs& a, hipStream_t s) {
  if (a.nq <= 0 || a.batch <= 0) return hipSuccess;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(prefill_kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, kPfLdsBytes);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  const int blocks = a.batch * a.n_qgroups * a.hq * 8;
  hipLaunchKernelGGL(prefill_kernel, dim3(blocks), dim3(kPfWaves * 64), kPfLdsBytes, s, a);
  return hipGetLastError();
}

hipError_t launch_prefill_tile_levels(int32_t* out, int n_row_tiles, int n_kblocks, int q_offset,
                                      const LevelTable& lt, hipStream_t s) {
  const int n = n_row_tiles * n_kblocks;
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(prefill_tile_levels_kernel, dim3((n + 255) / 256), dim3(256), 0, s, out, n_row_tiles,
                     n_kblocks, q_offset, lt);
  return hipGetLastError();
}

}  // namespace atf
