// Windowed causal GQA prefill attention for gfx950 (CDNA4).
//
// Replaces the FA4 window port's forward (called as
// _flash_attn_fwd(q, k, v, causal=True, atflash_window_zhi=zhi),
// microbench/b1_correctness.py:84-85, e2e_pipeline/atflash_e2e_fafi.py:118-119).
//
// Work decomposition
//   workgroup = 8 waves = 256 consecutive query positions of one q head;
//   wave      = 32 positions (one MFMA row block).  Waves w and w+4 share a SIMD
//               and run one phase apart ("ping-pong"): at every step one of them
//               issues MFMAs (PV of tile t-1, then QK of tile t) while the other
//               runs the softmax of its current tile, so the matrix pipe and the
//               VALU work at the same time;
//   k-tile    = 64 keys = 4 cache pages, staged through a 3-deep LDS ring with
//               direct global->LDS loads; the window is quantized per 32-key block
//               ("kb"), i.e. the oracle tile is (block_m, block_n) = (32, 32).
//   S^T = K Q^T and O^T = V^T P^T on v_mfma_f32_32x32x16_bf16: the accumulator
//   lane l always holds query row l%32, so the online-softmax max/sum stay in the
//   lane except one exchange with lane l^32 (v_permlane32_swap).
//   Per (wave, kb) the QK contraction runs over the first L = D_eff/16 levels
//   only, and the workgroup copies only the levels its first wave needs, so the
//   out-of-window K levels never enter LDS.  Q is rotated (RoPE) at load.
//   Online softmax in log2 units with a lazily updated reference max m_ref: Q is
//   scaled by sm_scale*log2(e) when it is loaded (rounded to bf16 once, as it is
//   anyway after RoPE), and every QK chain starts from -m_ref (a register tuple
//   used as the C operand of its first MFMA), so the MFMAs return S - m_ref and
//   P = exp2 of the accumulator directly.  O and l are rescaled only when a
//   row's max grows past m_ref by more than 8, so P <= 256.
#include "atf_launch.h"

namespace atf {

typedef __attribute__((address_space(3))) uint8_t lds_u8;

constexpr float kLazyRescaleLog2 = 8.0f;
constexpr float kLn2 = 0.6931471805599453f;

// s_waitcnt immediate for vmcnt(0) alone (gfx9 encoding: vmcnt bits 3:0 and
// 15:14, expcnt 6:4, lgkmcnt 11:8), issued through the builtin so the
// compiler's own wait insertion accounts for it.
constexpr int kWaitVm = 0x0F70;

// Barrier inside the tile loop.  __syncthreads() carries a workgroup release
// fence, for which the compiler waits until every pending global->LDS copy of
// the wave has landed (vmcnt(0)) before the s_barrier; a copy requested during
// a phase would then stall the barrier that ends that same phase.  This
// barrier waits only for the wave's LDS instructions (lgkmcnt(0): zero fills
// written with ds_write); each copy is waited for explicitly (vmcnt(0)) by the
// wave that issued it, before the barrier that precedes its first reader.  The
// memory clobber keeps the compiler from moving LDS accesses across it.
__device__ __forceinline__ void pf_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__device__ __forceinline__ float pair_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Level count of tile t for a fixed (query anchor, key offset) pair as t walks
// up: level i is read from tile T_i = ceil((anchor - off - zhi[i]) / 64) on, so
// L(t) = #{i : T_i <= t} (the D_eff rule at distance anchor - (64 t + off)).
// advance(t) costs one compare per tile except when a level boundary is crossed.
struct LevelWalker {
  int L;
  int next;
  int anchor;
  __device__ __forceinline__ int start_tile(const LevelTable& lt, int i) const {
    const int z = min(lt.zhi[i], 1 << 30);
    return (anchor - z + kPfTileN - 1) >> 6;  // ceil((anchor - zhi) / 64), arithmetic shift
  }
  __device__ __forceinline__ void init(const LevelTable& lt, int anchor_minus_off) {
    anchor = anchor_minus_off;
    L = 0;
    next = start_tile(lt, 0);
  }
  __device__ __forceinline__ int advance(const LevelTable& lt, int t) {
    while (t >= next) {
      ++L;
      next = (L < kLevels) ? start_tile(lt, L) : 0x7fffffff;
    }
    return L < 1 ? 1 : L;  // D_eff >= 16
  }
};

__device__ __forceinline__ bf16x8 lds_frag(const lds_u8* p) {
  return *reinterpret_cast<const __attribute__((address_space(3))) bf16x8*>(p);
}

// Raw page-table entry of page `pidx` of sequence b (-1 past the keys), in a
// vector register (every lane holds the same value).  Each wave fetches the
// entry of its next page one tile ahead, so the table read is never waited for
// at the start of a phase.  The load is kept a vector load on purpose: a scalar
// load inside the tile loop shares the LDS wait counter and, since scalar loads
// return out of order, would force every LDS wait behind it to drain fully.
__device__ __forceinline__ int fetch_page(const PrefillArgs& a, int b, int pidx) {
  int lane_zero;
  asm volatile("v_mov_b32 %0, 0" : "=v"(lane_zero));  // a value the compiler cannot prove uniform
  const int n_pages_k = (a.nk + kPage - 1) / kPage;
  int pg = -1;
  if (pidx < n_pages_k) pg = a.page_table[static_cast<int64_t>(b) * a.max_pages + pidx + lane_zero];
  return pg;
}

// The wave-uniform page id of a fetched entry; -1 for an invalid entry.  Read
// on every path before the register is fetched into again (otherwise the
// compiler guards the refetch with a wait for every outstanding load).
__device__ __forceinline__ int page_id(const PrefillArgs& a, int raw) {
  const int pg = __builtin_amdgcn_readfirstlane(raw);
  return (pg < 0 || pg >= a.num_pages) ? -1 : pg;
}

// LDS layout of a staged page.  An MFMA A operand is read with ds_read_b128,
// lane l taking 16 bytes of row l%32 (half l/32 of the 16-element k slice).
// The cache rows are 32 bytes long (16 keys of a V^T row, 16 dims of a K level
// row), so reading them in place puts lanes j and j+4 of every 8-lane group on
// the same LDS banks.  The staging copy therefore permutes the 16-byte chunks
// of each 1 KB copy (its source address is per lane): LDS chunk i of a copy
// holds half (i/16)%2 of K row i%16 of level i/32, resp. half i/32 of V^T row
// i%32.  Every operand read is then 64 consecutive 16-byte chunks per half:
//   K   level lv, token tk, half hf:  lv*512 + hf*256 + tk*16
//   V^T row d (1 KB block d/32), half hf:  (d/32)*1024 + hf*512 + (d%32)*16
__device__ __forceinline__ int k_copy_src(int lane) {
  return ((lane >> 5) << 9) + ((lane & 15) << 5) + (((lane >> 4) & 1) << 4);
}
__device__ __forceinline__ int v_copy_src(int lane) { return ((lane & 31) << 5) + ((lane >> 5) << 4); }
// Byte offset of V^T element (dim d, slot s) in a staged page.
__device__ __forceinline__ int v_lds_elem(int d, int s) {
  return ((d >> 5) << 10) + ((s >> 3) << 9) + ((d & 31) << 4) + ((s & 7) << 1);
}

// Direct global->LDS copies (16 bytes per lane, a 1 KB row per wave, to LDS
// address dst + 16 * lane), written as inline assembly.  When the compiler
// sees a global->LDS copy anywhere in a loop, its wait insertion no longer
// counts LDS reads in order and waits for all of them (lgkmcnt(0)) before
// every use of one, which exposes the full LDS latency in front of each MFMA
// of the operand ring.  The copies are therefore invisible to it: every copy
// is waited for explicitly (vmcnt(0)) before the barrier that publishes it,
// and a vector-load wait the compiler computes for its own loads only becomes
// stricter when copies it does not count are in flight.  M0 holds the LDS
// address for the copies (one wait state after it is written) and is restored.
//
// lds_copy_rows<N> copies N consecutive 1 KB rows: lane l reads 16 bytes at
// base + voff(l) + 1024 i (a wave-uniform base in scalar registers plus a
// per-lane offset) and writes LDS dst + 16 l + 1024 i.  The instruction's
// immediate offset moves the global and the LDS address alike, so one M0
// setting serves all N rows.
template <int N>
__device__ __forceinline__ void lds_copy_rows(const uint8_t* base, uint32_t voff, lds_u8* dst) {
  static_assert(N >= 1 && N <= 4, "1 to 4 rows");
  const uint32_t la = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(dst)));
  uint32_t saved;
#define ATF_LDS_ROW(off) "global_load_lds_dwordx4 %1, %2 offset:" #off "\n\t"
  if constexpr (N == 1)
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\t" ATF_LDS_ROW(0) "s_mov_b32 m0, %0"
                 : "=&s"(saved) : "v"(voff), "s"(base), "s"(la) : "memory");
  else if constexpr (N == 2)
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\t" ATF_LDS_ROW(0) ATF_LDS_ROW(1024)
                 "s_mov_b32 m0, %0"
                 : "=&s"(saved) : "v"(voff), "s"(base), "s"(la) : "memory");
  else if constexpr (N == 3)
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\t" ATF_LDS_ROW(0) ATF_LDS_ROW(1024)
                 ATF_LDS_ROW(2048) "s_mov_b32 m0, %0"
                 : "=&s"(saved) : "v"(voff), "s"(base), "s"(la) : "memory");
  else
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\t" ATF_LDS_ROW(0) ATF_LDS_ROW(1024)
                 ATF_LDS_ROW(2048) ATF_LDS_ROW(3072) "s_mov_b32 m0, %0"
                 : "=&s"(saved) : "v"(voff), "s"(base), "s"(la) : "memory");
#undef ATF_LDS_ROW
}

// Stage one 64-key tile (4 pages) into LDS: waves 0-3 copy K (first L levels)
// of page w, waves 4-7 copy V of page w-4; `pg` is the page id (-1: missing
// page, zero-filled).
// `voff` is the lane's chunk offset within a copied 1 KB row (k_copy_src or
// v_copy_src for the wave's half).
__device__ __forceinline__ void pf_load_tile(const PrefillArgs& a, int kvh, int pg, int L, lds_u8* stage,
                                             int wave, int lane, uint32_t voff) {
  const int page = wave & 3;
  const bool is_v = wave >= 4;
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
    lds_copy_rows<4>(reinterpret_cast<const uint8_t*>(a.v_cache) + blk, voff, dst);
  } else {
    // whole 1 KB level pairs (an odd L also copies level L, which is not read)
    const uint8_t* src = reinterpret_cast<const uint8_t*>(a.k_cache) + blk;
    switch ((L + 1) >> 1) {
      case 4: lds_copy_rows<4>(src, voff, dst); break;
      case 3: lds_copy_rows<3>(src, voff, dst); break;
      case 2: lds_copy_rows<2>(src, voff, dst); break;
      default: lds_copy_rows<1>(src, voff, dst); break;
    }
  }
}

// S^T (32 keys x 32 rows) of one 32-key block over its first L levels: one MFMA
// chain, the operand of level l+1 read from LDS while level l's MFMA runs.  `a`
// holds the level-0 operand on entry.
template <int L>
__device__ __forceinline__ f32x16 qk_chain(const lds_u8* kbase, const u32x4 (&Qf)[kLevels], bf16x8 a,
                                          const f32x16& C) {
  f32x16 S = C;
#pragma unroll
  for (int l = 0; l < L; ++l) {
    bf16x8 an = a;
    if (l + 1 < L) an = lds_frag(kbase + (l + 1) * 512);
    S = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, __builtin_bit_cast(bf16x8, Qf[l]), S, 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    a = an;
  }
  return S;
}

// Both 32-key blocks with the same level count: two interleaved chains,
// operands one level ahead.
template <int L>
__device__ __forceinline__ void qk_pair(const lds_u8* k0, const lds_u8* k1, const u32x4 (&Qf)[kLevels], bf16x8 a,
                                        bf16x8 b, const f32x16& C, f32x16& S0, f32x16& S1) {
  S0 = C;
  S1 = C;
#pragma unroll
  for (int l = 0; l < L; ++l) {
    bf16x8 an = a, bn = b;
    if (l + 1 < L) {
      an = lds_frag(k0 + (l + 1) * 512);
      bn = lds_frag(k1 + (l + 1) * 512);
    }
    S0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, __builtin_bit_cast(bf16x8, Qf[l]), S0, 0, 0, 0);
    S1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b, __builtin_bit_cast(bf16x8, Qf[l]), S1, 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    a = an;
    b = bn;
  }
}

__device__ __forceinline__ f32x16 qk_one(int L, const lds_u8* kbase, const u32x4 (&Qf)[kLevels], bf16x8 a,
                                        const f32x16& C) {
  switch (L) {
    case 8: return qk_chain<8>(kbase, Qf, a, C);
    case 7: return qk_chain<7>(kbase, Qf, a, C);
    case 6: return qk_chain<6>(kbase, Qf, a, C);
    case 5: return qk_chain<5>(kbase, Qf, a, C);
    case 4: return qk_chain<4>(kbase, Qf, a, C);
    case 3: return qk_chain<3>(kbase, Qf, a, C);
    case 2: return qk_chain<2>(kbase, Qf, a, C);
    default: return qk_chain<1>(kbase, Qf, a, C);
  }
}

// S^T + C for the two 32-key blocks of a tile with level counts L0 (far) and
// L1 (near); a0/a1 hold their level-0 operands.
__device__ __forceinline__ void qk_tile(int L0, int L1, const lds_u8* k0, const lds_u8* k1,
                                        const u32x4 (&Qf)[kLevels], bf16x8 a0, bf16x8 a1, const f32x16& C,
                                        f32x16& S0, f32x16& S1) {
  if (L0 == L1) {
    switch (L0) {
      case 8: qk_pair<8>(k0, k1, Qf, a0, a1, C, S0, S1); break;
      case 7: qk_pair<7>(k0, k1, Qf, a0, a1, C, S0, S1); break;
      case 6: qk_pair<6>(k0, k1, Qf, a0, a1, C, S0, S1); break;
      case 5: qk_pair<5>(k0, k1, Qf, a0, a1, C, S0, S1); break;
      case 4: qk_pair<4>(k0, k1, Qf, a0, a1, C, S0, S1); break;
      case 3: qk_pair<3>(k0, k1, Qf, a0, a1, C, S0, S1); break;
      case 2: qk_pair<2>(k0, k1, Qf, a0, a1, C, S0, S1); break;
      default: qk_pair<1>(k0, k1, Qf, a0, a1, C, S0, S1); break;
    }
  } else {
    S0 = qk_one(L0, k0, Qf, a0, C);
    S1 = qk_one(L1, k1, Qf, a1, C);
  }
}

// The MFMA phase as one stream of MFMAs, each taking one 1 KB A operand from
// LDS: stream i < 16 is PV step (ks, db) = (i/4, i%4), O[db] += V^T[db,ks] P^T[ks];
// stream 16 + j is QK level j/2 of 32-key block j%2 (the first level starts
// from C), 16 + 2L MFMAs in all when both blocks have L levels.  The operands
// go through a ring of kRing registers: the read of operand i + kRing - 1 is
// issued before MFMA i (scheduling barriers keep that order), so each read has
// kRing - 1 MFMAs (32 cycles each) to arrive; the LDS latency under four SIMDs'
// operand traffic is longer than one or two.  The PV part is shared by every
// level count: it reads the first QK operands ahead in this order, which is
// the same for any L (an operand past 2L is read and not used; its address is
// still inside the staged tile).
#ifndef ATF_PF_RING
#define ATF_PF_RING 6
#endif
constexpr int kRing = ATF_PF_RING;
static_assert(kRing >= 2 && kRing - 1 <= 16, "ring depth");

__device__ __forceinline__ const lds_u8* stream_src(const lds_u8* vb, const lds_u8* kb, int i) {
  if (i < 16) return vb + (i >> 2) * 4096 + (i & 3) * 1024;
  const int j = i - 16;
  return kb + (j & 1) * (2 * 4096) + (j >> 1) * 512;
}

// The first kRing - 1 operands of the stream (V^T only).
static_assert(kRing - 1 <= 16, "ring prefetch must stay within the PV operands");
__device__ __forceinline__ void pv_prefetch(const lds_u8* vb, bf16x8 (&f)[kRing]) {
#pragma unroll
  for (int i = 0; i < kRing - 1; ++i) {
    f[i] = lds_frag(stream_src(vb, vb, i));
    __builtin_amdgcn_sched_barrier(0);
  }
}

__device__ __forceinline__ void pv_stream(const lds_u8* vb, const lds_u8* kb, const bf16x8 (&Pf)[4], f32x16 (&O)[4],
                                          bf16x8 (&f)[kRing]) {
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    f[(i + kRing - 1) % kRing] = lds_frag(stream_src(vb, kb, i + kRing - 1));
    __builtin_amdgcn_sched_barrier(0);
    O[i & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f[i % kRing], Pf[i >> 2], O[i & 3], 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
  }
}

template <int L>
__device__ __forceinline__ void qk_stream(const lds_u8* kb, bf16x8 (&f)[kRing], const u32x4 (&Qf)[kLevels],
                                          const f32x16& C, f32x16 (&S)[2]) {
  constexpr int NS = 16 + 2 * L;
#pragma unroll
  for (int i = 16; i < NS; ++i) {
    if (i + kRing - 1 < NS) f[(i + kRing - 1) % kRing] = lds_frag(stream_src(kb, kb, i + kRing - 1));
    __builtin_amdgcn_sched_barrier(0);
    const int j = i - 16;
    S[j & 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f[i % kRing], __builtin_bit_cast(bf16x8, Qf[j >> 1]),
                                                       (j >> 1) == 0 ? C : S[j & 1], 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// P = exp2(S) of a tile packed to bf16 (the B operands of the next PV steps),
// and the lane's partial row sum of P.
__device__ __forceinline__ float exp_tile(const f32x16 (&S)[2], bf16x8 (&Pf)[4]) {
  float lt = 0.f;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
    for (int hs = 0; hs < 2; ++hs) {
      u32x4 pk;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p0 = fast_exp2(S[kb][8 * hs + 2 * i]);
        const float p1 = fast_exp2(S[kb][8 * hs + 2 * i + 1]);
        pk[i] = pack_bf16x2(p0, p1);
        lt += p0 + p1;
      }
      Pf[2 * kb + hs] = __builtin_bit_cast(bf16x8, pk);
    }
  }
  return lt;
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

  // ---- Q fragments (B operand of S^T = K Q^T), with RoPE and the log2-unit
  // softmax scale applied at load ----
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
          v = rope_half(ldg16(qrow + c0), ldg16(qrow + c1), cs, second, a.scale_log2);
        } else {
          v = scale8(ldg16(qrow + (second ? c1 : c0)), a.scale_log2);
        }
      }
      Qf[l] = v;
    }
  }

  f32x16 O[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) O[db] = f32x16{};
  const float NEG_INF = -__builtin_huge_valf();
  float m_ref = 0.f;      // reference max (log2 units), set by the first tile
  float l_run = 0.f;      // this lane's partial row sum relative to m_ref
  f32x16 Cm = f32x16{};   // -m_ref in every element
  const int T = t_end_wg;
#ifndef ATF_PF_GROUP
#define ATF_PF_GROUP(w) ((w) >> 2)
#define ATF_PF_RANK(w) ((w) & 3)
#endif
  const int grp = ATF_PF_GROUP(wave);  // ping-pong group (waves w and w+4 share a SIMD)
  const int rank = ATF_PF_RANK(wave);  // 0..3 within the group

  // Level walkers: far (keys n0..n0+31) and near (n0+32..n0+63) blocks of this
  // wave, and the workgroup's staging count (nearest key, first row).
  LevelWalker w_far, w_near, w_ld;
  w_far.init(a.lt, pos0 - 31);
  w_near.init(a.lt, pos0 - 63);
  w_ld.init(a.lt, pos0_wg - 63);

  // LDS ring: byte offsets of the stages holding tiles t-1, t and t+1.
  int o_prev = 2 * kPfStageBytes, o_cur = 0, o_next = kPfStageBytes;

  // ---- prologue: stage tile 0 ----
  const int page_w = wave & 3;  // this wave's page within a tile
  const uint32_t copy_off = static_cast<uint32_t>(wave >= 4 ? v_copy_src(lane) : k_copy_src(lane));
  if (T > 0) pf_load_tile(a, kvh, page_id(a, fetch_page(a, b, page_w)), w_ld.advance(a.lt, 0), smem + o_cur, wave, lane, copy_off);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (T > 0 && kPfTileN > a.nk) {  // zero V of keys past nk (0 * V must stay 0)
    const int page = threadIdx.x >> 7;
    const int d = threadIdx.x & 127;
    lds_u8* vpage = smem + o_cur + 4 * 4096 + page * 4096;
#pragma unroll
    for (int tk = 0; tk < kPage; ++tk)
      if (page * kPage + tk >= a.nk)
        *reinterpret_cast<__attribute__((address_space(3))) uint16_t*>(vpage + v_lds_elem(d, v_slot(tk))) = 0;
    __syncthreads();
  }

  f32x16 S[2];
  bf16x8 Pf[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) Pf[i] = bf16x8{};
  // Global step k: group g runs phase k - g.  Phase 2t is the MFMA phase of
  // tile t (PV of tile t-1, QK of tile t), phase 2t+1 its softmax.  Copies are
  // issued in softmax phases only, so an MFMA phase never waits behind them:
  // K of tile t+2 by group 0 in its softmax of tile t (step 2t+1), V of tile
  // t+2 by group 1 in its softmax of tile t (step 2t+2).  Each wave waits for
  // its copies before the barrier ending its next MFMA phase (steps 2t+2 and
  // 2t+3); tile t+2 is first read at step 2t+4.  Tile 1 is requested before
  // the loop.  The MFMA phase runs unconditionally (P = 0 when there is
  // nothing to add) so the accumulators stay in place.
  const int v_lane = 4 * 4096 + (lane >> 5) * 512 + (lane & 31) * 16;
  // next page-table entry of this wave: tile 1 for group 0, tile 2 for group 1
  int pg_next;
  if (grp == 1) {
    if (1 < T)
      pf_load_tile(a, kvh, page_id(a, fetch_page(a, b, 4 + page_w)), w_ld.advance(a.lt, 1), smem + o_next, wave,
                   lane, copy_off);
    pg_next = fetch_page(a, b, 8 + page_w);
    pf_barrier();  // group 1 starts one step late
  } else {
    if (1 < T)
      pf_load_tile(a, kvh, page_id(a, fetch_page(a, b, 4 + page_w)), w_ld.advance(a.lt, 1), smem + o_next, wave,
                   lane, copy_off);
    pg_next = fetch_page(a, b, 8 + page_w);
  }
  for (int t = 0; t <= T; ++t) {
    // ---- MFMA phase of tile t ----
#ifndef ATF_PF_NO_PRIO
    __builtin_amdgcn_s_setprio(1);
#endif
    {
      const lds_u8* kbase = smem + o_cur + ((lane & 31) >> 4) * 4096 + (lane >> 5) * 256 + (lane & 15) * 16;
      // O^T += V^T P^T for tile t-1 (P = 0 at t = 0), then S^T = K Q^T over the
      // surviving levels of each 32-key block of tile t (unused when the wave
      // has no tile t).
      const lds_u8* vb = smem + (t == 0 ? o_cur : o_prev) + v_lane;
      const int L0 = w_far.advance(a.lt, t);
      const int L1 = w_near.advance(a.lt, t);
      bf16x8 f[kRing];
      pv_prefetch(vb, f);
      pv_stream(vb, kbase, Pf, O, f);
      if (L0 == L1) {
        switch (L0) {
          case 8: qk_stream<8>(kbase, f, Qf, Cm, S); break;
          case 7: qk_stream<7>(kbase, f, Qf, Cm, S); break;
          case 6: qk_stream<6>(kbase, f, Qf, Cm, S); break;
          case 5: qk_stream<5>(kbase, f, Qf, Cm, S); break;
          case 4: qk_stream<4>(kbase, f, Qf, Cm, S); break;
          case 3: qk_stream<3>(kbase, f, Qf, Cm, S); break;
          case 2: qk_stream<2>(kbase, f, Qf, Cm, S); break;
          default: qk_stream<1>(kbase, f, Qf, Cm, S); break;
        }
      } else {  // a level boundary between the two blocks: two chains
        qk_tile(L0, L1, kbase, kbase + 2 * 4096, Qf, f[16 % kRing], f[17 % kRing], Cm, S[0], S[1]);
      }
    }
#ifndef ATF_PF_NO_PRIO
    __builtin_amdgcn_s_setprio(0);
#endif
    // this wave's copies of tile t+1 (requested in its previous phase) land
    // before the barrier after which tile t+1 is first read
    __builtin_amdgcn_s_waitcnt(kWaitVm);
    pf_barrier();
    {
      // K (group 0) or V (group 1) of tile t+2 into the stage of tile t-1:
      // both groups have read that tile's K, and its V is read only by the
      // MFMA phases of tile t, which end before the copy into V starts
      const int pg = page_id(a, pg_next);
      if (t + 2 < T) pf_load_tile(a, kvh, pg, w_ld.advance(a.lt, t + 2), smem + o_prev, wave, lane, copy_off);
      pg_next = fetch_page(a, b, 4 * (t + 3) + page_w);
    }
    // ---- softmax phase of tile t (lane = query row) ----
    if (t < t_end) {
      const int n0 = t * kPfTileN;
      const bool need_mask = (n0 + kPfTileN - 1 > pos0) || (n0 + kPfTileN > a.nk);
      if (need_mask) {
        // element (kb, r) holds key n0 + 4*(lane/32) + c with c = 32kb + 8(r/4) + r%4;
        // masked when key > min(row position, nk - 1).  Selects, no branches.
        const int thr = min(pos0 + (lane & 31), a.nk - 1) - n0 - 4 * (lane >> 5);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            S[kb][r] = (32 * kb + 8 * (r >> 2) + (r & 3) > thr) ? NEG_INF : S[kb][r];
      }
      // S holds score - m_ref, so every P = exp2(S) is at most 256 unless a
      // score exceeds m_ref by more than 8; P >= 0, so that shows as a partial
      // row sum above 256 (or an infinite one).  Only then, and on the first
      // tile (key 0 is visible to every row, so its max is finite), is the row
      // max taken: where it exceeds m_ref by more than 8 (always on the first
      // tile), m_ref moves up to it, O and l are rescaled, and the tile's P is
      // computed again from the shifted scores (shift 0 for the other lanes).
      float lt = exp_tile(S, Pf);
      if (__builtin_amdgcn_ballot_w64((t == 0) || !(lt <= 256.f)) != 0) {
        float mx = NEG_INF;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) mx = fmaxf(mx, S[kb][r]);
        mx = pair_max(mx);
        const bool grow = (t == 0) || mx > kLazyRescaleLog2;
        if (__builtin_amdgcn_ballot_w64(grow) != 0) {
          const float delta = grow ? mx : 0.f;
          if (t > 0) {
            const float alpha = fast_exp2(-delta);
            l_run *= alpha;
#pragma unroll
            for (int db = 0; db < 4; ++db) O[db] *= alpha;
          }
          m_ref += delta;
#pragma unroll
          for (int i = 0; i < 16; ++i) Cm[i] = -m_ref;
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) S[kb][r] -= delta;
          lt = exp_tile(S, Pf);
        }
      }
      l_run += lt;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) Pf[i] = bf16x8{};
    }
    pf_barrier();
    // Tile t+1 has landed; group 0 zeroes the V of keys past nk in a partial
    // last tile (read no earlier than two barriers later).
    if (grp == 0 && t + 1 < T && (t + 1) * kPfTileN + kPfTileN > a.nk) {
      const int n0 = (t + 1) * kPfTileN;
      lds_u8* vpage = smem + o_next + 4 * 4096 + rank * 4096;
#pragma unroll
      for (int rr = 0; rr < 2; ++rr) {
#pragma unroll
        for (int tk = 0; tk < kPage; ++tk)
          if (n0 + rank * kPage + tk >= a.nk)
            *reinterpret_cast<__attribute__((address_space(3))) uint16_t*>(vpage + v_lds_elem(lane * 2 + rr, v_slot(tk))) =
                0;
      }
    }
    // rotate the ring: tile t+1 becomes current
    const int o_old = o_prev;
    o_prev = o_cur;
    o_cur = o_next;
    o_next = o_old;
  }
  if (grp == 0) __syncthreads();  // group 0 ends one step late

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
          (l > 0.f) ? m_ref * kLn2 + __logf(l) : NEG_INF;
    }
  }
}

// Level count per (32-row tile, 32-key block) through the LevelWalker the
// attention kernel uses (even blocks are the far half of a 64-key tile, odd
// blocks the near half); out is [n_row_tiles][n_kblocks].
__global__ void prefill_tile_levels_kernel(int32_t* out, int n_row_tiles, int n_kblocks, int q_offset,
                                           LevelTable lt) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_row_tiles * n_kblocks) return;
  const int rt = i / n_kblocks, kb = i % n_kblocks;
  const int pos0 = q_offset + rt * kPfRowsWave;
  LevelWalker w;
  w.init(lt, pos0 - ((kb & 1) ? 63 : 31));
  out[i] = w.advance(lt, kb >> 1);
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
