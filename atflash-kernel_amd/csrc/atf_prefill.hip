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
//               issues MFMAs (PV of the previous tile pair, then QK of the
//               current pair) while the other runs the softmax of its current
//               pair, so the matrix pipe and the VALU work at the same time;
//   k-tile    = 64 keys = 4 cache pages; a phase covers a pair of tiles (128
//               keys, 64 MFMAs with the window off), so the per-phase barrier
//               and pipeline ramp are paid once per 128 keys.  K and V are
//               staged through LDS rings (3 K pairs, 2 V pairs: 160 KB) with
//               direct global->LDS loads; the window is quantized per 32-key
//               block ("kb"), i.e. the oracle tile is (block_m, block_n) = (32, 32).
//   S^T = K Q^T and O^T = V^T P^T on v_mfma_f32_32x32x16_bf16: the accumulator
//   lane l always holds query row l%32, so the online-softmax max/sum stay in the
//   lane except one exchange with lane l^32 (v_permlane32_swap).
//   Per (wave, kb) the QK contraction runs over the first L = D_eff/16 levels
//   only, and the workgroup copies only the levels its first wave needs, so the
//   out-of-window K levels never enter LDS.  Q is rotated (RoPE) at load.
//   Online softmax in log2 units with a lazily updated reference max m_ref.
//   With RoPE at load, Q is scaled by sm_scale*log2(e) as it is rotated (rounded
//   to bf16 once, as it is anyway after RoPE), and every QK chain starts from
//   -m_ref (a register tuple used as the C operand of its first MFMA), so the
//   MFMAs return S - m_ref and P = exp2 of the accumulator directly.  A
//   pre-rotated bf16 Q is used unscaled and the scale multiplies the fp32
//   scores instead (kernel template kRaw).  O and l are rescaled only when a
//   row's max grows past m_ref by more than 8, so P <= 256.
#include <mutex>

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
// advance(t) costs one compare per tile except when a level boundary is crossed
// (at most kLevels times per walker), which is laid out as the unlikely path.
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
    while (__builtin_expect(t >= next, 0)) {
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
// Read in place, rows 32 bytes long would put lanes j and j+4 of every 8-lane
// group on the same LDS banks; every operand read is instead 64 consecutive
// 16-byte chunks per half:
//   K   level lv, token tk, half hf:  lv*512 + hf*256 + tk*16
//   V^T row d (1 KB block d/32), half hf:  (d/32)*1024 + hf*512 + (d%32)*16
// For K this is the cache's own page layout (slice 2lv + hf, token tk), so a
// copy is contiguous.  The V^T rows of the cache are 32 bytes long (16 keys),
// so the V copy permutes the 16-byte chunks of each 1 KB copy (its source
// address is per lane): LDS chunk i holds half i/32 of V^T row i%32.
__device__ __forceinline__ int k_copy_src(int lane) { return lane << 4; }
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
// lds_copy_page copies the first `nbytes` (a multiple of 1 KB, at most 4 KB)
// of a page through a raw buffer resource whose range is nbytes: it always
// issues the four row loads, and the hardware range check turns the rows
// past the range into zeros without a memory request.  Lane l reads 16 bytes
// at base + voff(l) + 1024 i and writes LDS dst + 16 l + 1024 i (the
// instruction's immediate offset moves the memory and the LDS address alike,
// so one M0 setting serves all four rows).  One straight-line sequence serves
// every row count: a switch over the count cost about 400 cycles of branching
// per copying step, on the wave whose softmax sets the step when the window
// trims the QK work.
__device__ __forceinline__ void lds_copy_page(const uint8_t* base, uint32_t nbytes, uint32_t voff, lds_u8* dst) {
  const uint32_t la = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(dst)));
  const uint64_t ad = reinterpret_cast<uint64_t>(base);
  u32x4 rs;  // raw buffer resource: base, stride 0, num_records = nbytes
  rs[0] = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(ad)));
  rs[1] = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(ad >> 32))) & 0xffffu;
  rs[2] = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(nbytes));
  rs[3] = static_cast<uint32_t>(kBufferWord3);
  uint32_t saved;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\t"
               "buffer_load_dwordx4 %1, %2, 0 offen lds\n\t"
               "buffer_load_dwordx4 %1, %2, 0 offen offset:1024 lds\n\t"
               "buffer_load_dwordx4 %1, %2, 0 offen offset:2048 lds\n\t"
               "buffer_load_dwordx4 %1, %2, 0 offen offset:3072 lds\n\t"
               "s_mov_b32 m0, %0"
               : "=&s"(saved) : "v"(voff), "s"(rs), "s"(la) : "memory");
}

__device__ __forceinline__ void zero_page(lds_u8* dst, int lane) {
  const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int i = 0; i < 4; ++i) *reinterpret_cast<__attribute__((address_space(3))) u32x4*>(dst + i * 1024 + lane * 16) = z;
}

// Stage one 4 KB page half into LDS at `dst`: K (whole 1 KB level pairs
// covering the first L levels; an odd L also copies level L, which is not
// read) or V.
// `pg` is the page id (-1: missing page, zero-filled); `voff` is the lane's
// chunk offset within a copied 1 KB row (k_copy_src or v_copy_src).
__device__ __forceinline__ void pf_load_page(const PrefillArgs& a, int kvh, int pg, int L, bool is_v, lds_u8* dst,
                                             int lane, uint32_t voff) {
  if (pg < 0) {
    zero_page(dst, lane);
    return;
  }
  const size_t blk = (static_cast<size_t>(pg) * a.hkv + kvh) * (kKvBlockElems * 2);
  const uint8_t* src = reinterpret_cast<const uint8_t*>(a.kv_cache) + blk + (is_v ? 0 : kKHalfElems * 2);
  lds_copy_page(src, is_v ? 4096u : static_cast<uint32_t>((L + 1) >> 1) * 1024u, voff, dst);
}

// pf_load_page for the tile loop: the page's source is cbase + pg * pstride,
// with the cache base (offset to the kv head) and the page stride computed once
// before the loop, so the copy does not reload kernel arguments; `rows` 1 KB
// rows are copied.
__device__ __forceinline__ void stage_page(const uint8_t* cbase, uint32_t pstride, int pg, int rows, lds_u8* dst,
                                           int lane, uint32_t voff) {
  if (pg < 0) {
    zero_page(dst, lane);
    return;
  }
  lds_copy_page(cbase + static_cast<size_t>(static_cast<uint32_t>(pg)) * pstride, static_cast<uint32_t>(rows) * 1024u,
                voff, dst);
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

// LDS ring.  A K slot holds the K pages of one 64-key tile, a V slot its V
// pages (4 pages of 4 KB).  Phase u reads the K of tiles 2u and 2u+1 and the V
// of tiles 2u-2 and 2u-1, so tiles are staged in pairs: K pair u % 3 holds
// tiles 2u, 2u+1 (three pairs: read, landing, being copied), V pair u % 2
// holds tiles 2u, 2u+1 (two pairs: read, being copied).
constexpr int kPfSlotBytes = 4 * 4096;
constexpr int kPfPairBytes = 2 * kPfSlotBytes;
constexpr int kPfKPairs = 3;
constexpr int kPfVPairs = 2;
constexpr int kPfVRegion = kPfKPairs * kPfPairBytes;
constexpr int kPfLdsTotal = (kPfKPairs + kPfVPairs) * kPfPairBytes;  // 160 KB
static_assert(kPfLdsTotal <= 160 * 1024, "gfx950 LDS");

// The MFMA phase as one stream of MFMAs, each taking one 1 KB A operand from
// LDS.  Stream i < 32 is PV step (page p, dim block db) = (i/4, i%4) over the
// tile pair's 8 pages, O[db] += V^T[db, p] P^T[p]; stream 32 + j is QK level
// j/4 of 32-key block j%4 (blocks 0, 1: first tile of the pair, 2, 3: second;
// the first level starts from C), 32 + 4L MFMAs in all when the four blocks
// have L levels.  The operands go through a ring of kRing registers: the read
// of operand i + kRing - 1 is issued before MFMA i (scheduling barriers keep
// that order), so each read has kRing - 1 MFMAs (32 cycles each) to arrive;
// the LDS latency under four SIMDs' operand traffic is longer than one or
// two.  The PV part is shared by every level count: it reads the first QK
// operands ahead in this order, which is the same for any L (an operand past
// 4L is read and not used; its address is still inside the staged pair).
constexpr int kRing = 6;  // 5 measures the same, 7 about 1% slower
static_assert(kRing - 1 >= 4 && kRing - 1 <= 32, "ring depth: the level-0 operands of all four blocks are read ahead");

__device__ __forceinline__ const lds_u8* stream_src(const lds_u8* vb, const lds_u8* kb, int i) {
  if (i < 32) return vb + (i >> 2) * 4096 + (i & 3) * 1024;
  const int j = i - 32;
  return kb + (j & 3) * 8192 + (j >> 2) * 512;
}

// The first kRing - 1 operands of the stream (V^T only).
__device__ __forceinline__ void pv_prefetch(const lds_u8* vb, bf16x8 (&f)[kRing]) {
#pragma unroll
  for (int i = 0; i < kRing - 1; ++i) {
    f[i] = lds_frag(stream_src(vb, vb, i));
    __builtin_amdgcn_sched_barrier(0);
  }
}

__device__ __forceinline__ void pv_stream(const lds_u8* vb, const lds_u8* kb, const bf16x8 (&Pf)[8], f32x16 (&O)[4],
                                          bf16x8 (&f)[kRing]) {
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    f[(i + kRing - 1) % kRing] = lds_frag(stream_src(vb, kb, i + kRing - 1));
    __builtin_amdgcn_sched_barrier(0);
    O[i & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f[i % kRing], Pf[i >> 2], O[i & 3], 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// QK of the four blocks with one level count L: four interleaved chains.
template <int L>
__device__ __forceinline__ void qk_stream(const lds_u8* kb, bf16x8 (&f)[kRing], const u32x4 (&Qf)[kLevels],
                                          const f32x16& C, f32x16 (&S)[4]) {
  constexpr int NS = 32 + 4 * L;
#pragma unroll
  for (int i = 32; i < NS; ++i) {
    if (i + kRing - 1 < NS) f[(i + kRing - 1) % kRing] = lds_frag(stream_src(kb, kb, i + kRing - 1));
    __builtin_amdgcn_sched_barrier(0);
    const int j = i - 32;
    S[j & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f[i % kRing], __builtin_bit_cast(bf16x8, Qf[j >> 2]),
                                                       (j >> 2) == 0 ? C : S[j & 3], 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// The MFMA phase of tile pair u with one level count L for its four 32-key
// blocks: PV of the previous pair, then QK of this pair, as one straight-line
// stream (the level counts are known before the phase starts, so nothing
// branches between its first LDS read and its last MFMA).
template <int L>
__device__ __forceinline__ void mfma_phase(const lds_u8* vb, const lds_u8* kb, const bf16x8 (&Pf)[8],
                                           f32x16 (&O)[4], const u32x4 (&Qf)[kLevels], const f32x16& C,
                                           f32x16 (&S)[4]) {
  bf16x8 f[kRing];
  pv_prefetch(vb, f);
  pv_stream(vb, kb, Pf, O, f);
  qk_stream<L>(kb, f, Qf, C, S);
}

// The MFMA phase of a pair with a level boundary inside it (L0 <= L1 <= L2 <= L3,
// not all equal): PV as above, then per-tile chains.
__device__ __forceinline__ void mfma_phase_mixed(int L0, int L1, int L2, int L3, const lds_u8* vb,
                                                 const lds_u8* kb, const bf16x8 (&Pf)[8], f32x16 (&O)[4],
                                                 const u32x4 (&Qf)[kLevels], const f32x16& C, f32x16 (&S)[4]) {
  bf16x8 f[kRing];
  pv_prefetch(vb, f);
  pv_stream(vb, kb, Pf, O, f);
  qk_tile(L0, L1, kb, kb + 8192, Qf, f[32 % kRing], f[33 % kRing], C, S[0], S[1]);
  qk_tile(L2, L3, kb + 16384, kb + 24576, Qf, f[34 % kRing], f[35 % kRing], C, S[2], S[3]);
}

// P = exp2(S) of one 32-key block (S[kb]) packed to bf16 (Pf[2kb], Pf[2kb+1]
// are the B operands of the PV steps of its two pages), added to the lane's
// partial row sum lt.  kRaw: S is in raw score units (Q was not scaled) and
// P = exp2(S * c).
template <bool kRaw>
__device__ __forceinline__ void exp_block(const f32x16& Sk, bf16x8& P0, bf16x8& P1, float c, float& lt) {
#pragma unroll
  for (int hs = 0; hs < 2; ++hs) {
    u32x4 pk;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float s0 = Sk[8 * hs + 2 * i], s1 = Sk[8 * hs + 2 * i + 1];
      const float p0 = fast_exp2(kRaw ? s0 * c : s0);
      const float p1 = fast_exp2(kRaw ? s1 * c : s1);
      pk[i] = pack_bf16x2(p0, p1);
      lt += p0 + p1;
    }
    (hs == 0 ? P0 : P1) = __builtin_bit_cast(bf16x8, pk);
  }
}

// P of the whole tile pair and its partial row sum.
template <bool kRaw>
__device__ __forceinline__ float exp_tiles(const f32x16 (&S)[4], bf16x8 (&Pf)[8], float c) {
  float lt = 0.f;
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) exp_block<kRaw>(S[kb], Pf[2 * kb], Pf[2 * kb + 1], c, lt);
  return lt;
}

// kRaw selects how the softmax scale c = sm_scale * log2(e) is applied.
//   false (RoPE at load): Q is rotated and multiplied by c in fp32 and rounded
//         to bf16 once, so the MFMAs return scores in log2 units directly;
//   true  (pre-rotated bf16 Q): Q is used exactly as given and c multiplies the
//         fp32 scores in the softmax (one multiply per score).  Scaling an
//         already-rounded bf16 Q and rounding it again would add a second
//         rounding error to every score, which grows with the score magnitude.
template <bool kRaw>
__global__ __launch_bounds__(kPfWaves * 64, 1) void prefill_kernel(PrefillArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem_raw[];
  lds_u8* smem = (lds_u8*)(smem_raw);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

  // XCD-aware block mapping: block i runs on XCD i % 8.  Each XCD walks the q
  // heads of one q-tile in order (so the heads sharing a kv head share its K/V
  // tiles in that XCD's L2), and the 8 XCDs take 8 neighbouring q-tiles, the
  // heaviest (last) tiles first.  With a.xcd_alt the XCD order alternates from
  // one round of 8 tiles to the next (serpentine), so that every XCD gets the
  // same causal work over two rounds; with the same order in every round the
  // first XCD takes the heaviest tile of every round (prefill_xcd_alternate
  // decides per launch).
  const int bid = blockIdx.x;
  const int xcd = bid & 7;
  const int j = bid >> 3;
  const int per_b = a.n_qgroups * a.hq;
  const int b = j / per_b;
  const int jr = j - b * per_b;
  const int h = jr % a.hq;
  const int rnd = jr / a.hq;
  const int qrank = rnd * 8 + ((rnd & a.xcd_alt & 1) ? 7 - xcd : xcd);
  const int qt = a.n_qtiles - 1 - qrank;
  if (qt < 0 || b >= a.batch) return;
  const int kvh = h / a.group;

  const int lr0_wg = qt * kPfRowsWg;
  const int lr0 = lr0_wg + wave * kPfRowsWave;
  const int pos0_wg = a.q_offset + lr0_wg;
  const int pos0 = a.q_offset + lr0;
  const int n_ktiles = (a.nk + kPfTileN - 1) / kPfTileN;
  const int last_wg = a.q_offset + min(a.nq, lr0_wg + kPfRowsWg) - 1;
  const int T = min(n_ktiles, last_wg / kPfTileN + 1);  // tiles of the workgroup
  const int T2 = (T + 1) & ~1;                          // rounded up to whole pairs
  const int t_end =
      (lr0 < a.nq) ? min(n_ktiles, (a.q_offset + min(a.nq, lr0 + kPfRowsWave) - 1) / kPfTileN + 1) : 0;

  // ---- Q fragments (B operand of S^T = K Q^T), with RoPE and the log2-unit
  // softmax scale applied at load ----
  // Every Q and (cos, sin) load is issued before any is used, four levels at a
  // time (one memory round trip per four levels instead of one per level):
  // rows past nq read row nq - 1, in bounds, and are zeroed afterwards.
  u32x4 Qf[kLevels];
  const bool second = lane >= 32;
  const int row = lr0 + (lane & 31);
  {
    const int row_c = min(row, a.nq - 1);
    const uint16_t* qrow = a.q + static_cast<int64_t>(b) * a.q_sb + static_cast<int64_t>(row_c) * a.q_st +
                           static_cast<int64_t>(h) * a.q_sh;
    // k half h of level l is slice 2l + h, as in the cache's K pages
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      u32x4 v[4];
      const int s0 = 8 * j + (second ? 1 : 0);  // levels 4j .. 4j+3: slices s0, s0+2, s0+4, s0+6
      load_slices4<2>(qrow, a.layout, s0, v);
      if (a.rope_cs != nullptr) {
        float cs[4][8];
#pragma unroll
        for (int i = 0; i < 4; ++i) load_cs4(a.rope_cs, a.q_offset + row_c, slice_pair0(s0 + 2 * i), cs[i]);
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = rope_slice(v[i], cs[i], a.scale_log2);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) Qf[4 * j + i] = (row < a.nq) ? v[i] : u32x4{0u, 0u, 0u, 0u};
    }
  }

  f32x16 O[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) O[db] = f32x16{};
  const float NEG_INF = -__builtin_huge_valf();
  float m_ref = 0.f;      // reference max (log2 units), set by the first tile
  float l_run = 0.f;      // this lane's partial row sum relative to m_ref
  f32x16 Cm = f32x16{};   // -m_ref in every element (-m_ref / c with kRaw)
  const float c = a.scale_log2;
  const float inv_c = 1.f / c;
  const int grp = wave >> 2;   // ping-pong group (waves w and w+4 share a SIMD)
  const int rank = wave & 3;   // 0..3 within the group: the page of a tile this wave copies
  const bool copies_v = grp == 1;

  // Level walkers: the four 32-key blocks of a phase are the far (keys
  // n0..n0+31) and near (n0+32..n0+63) halves of its two tiles; w_ld is the
  // workgroup's staging count (nearest key, first row).
  LevelWalker w_far, w_near, w_ld;
  w_far.init(a.lt, pos0 - 31);
  w_near.init(a.lt, pos0 - 63);
  w_ld.init(a.lt, pos0_wg - 63);

  const uint32_t copy_off = static_cast<uint32_t>(copies_v ? v_copy_src(lane) : k_copy_src(lane));
  const int k_lane = ((lane & 31) >> 4) * 4096 + (lane >> 5) * 256 + (lane & 15) * 16;
  const int v_lane = (lane >> 5) * 512 + (lane & 31) * 16;

  // ---- prologue ----
  // Group 0 copies K, group 1 copies V, each wave page `rank` of a tile.  Group
  // 0 stages the K of tiles 0 and 1 (waited for here) and requests tiles 2 and
  // 3; group 1 zeroes V pair 1 (read with P = 0 by phase 0) and requests the V
  // of tiles 0 and 1.  pg_a / pg_b: page-table entries of the wave's next two
  // copies, fetched one phase ahead.
  int pg_a, pg_b;
  if (!copies_v) {
    const int e0 = fetch_page(a, b, rank), e1 = fetch_page(a, b, 4 + rank);
    const int p0 = page_id(a, e0), p1 = page_id(a, e1);
    if (0 < T) pf_load_page(a, kvh, p0, w_ld.advance(a.lt, 0), false, smem + rank * 4096, lane, copy_off);
    if (1 < T) pf_load_page(a, kvh, p1, w_ld.advance(a.lt, 1), false, smem + kPfSlotBytes + rank * 4096, lane, copy_off);
  } else {
    const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        *reinterpret_cast<__attribute__((address_space(3))) u32x4*>(
            smem + kPfVRegion + kPfPairBytes + s * kPfSlotBytes + rank * 4096 + i * 1024 + lane * 16) = z;
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (!copies_v) {
    const int e2 = fetch_page(a, b, 8 + rank), e3 = fetch_page(a, b, 12 + rank);
    const int p2 = page_id(a, e2), p3 = page_id(a, e3);
    if (2 < T) pf_load_page(a, kvh, p2, w_ld.advance(a.lt, 2), false, smem + kPfPairBytes + rank * 4096, lane, copy_off);
    if (3 < T)
      pf_load_page(a, kvh, p3, w_ld.advance(a.lt, 3), false, smem + kPfPairBytes + kPfSlotBytes + rank * 4096, lane,
                   copy_off);
    pg_a = fetch_page(a, b, 16 + rank);
    pg_b = fetch_page(a, b, 20 + rank);
  } else {
    const int e0 = fetch_page(a, b, rank), e1 = fetch_page(a, b, 4 + rank);
    const int p0 = page_id(a, e0), p1 = page_id(a, e1);
    if (0 < T2) pf_load_page(a, kvh, p0, kLevels, true, smem + kPfVRegion + rank * 4096, lane, copy_off);
    if (1 < T2) pf_load_page(a, kvh, p1, kLevels, true, smem + kPfVRegion + kPfSlotBytes + rank * 4096, lane, copy_off);
    pg_a = fetch_page(a, b, 8 + rank);
    pg_b = fetch_page(a, b, 12 + rank);
    pf_barrier();  // group 1 starts one step late
  }

  f32x16 S[4];
  bf16x8 Pf[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) Pf[i] = bf16x8{};
  // Global step k: group g runs phase k - g.  Phase 2u is the MFMA phase of
  // tile pair u (PV of tiles 2u-2 and 2u-1, QK of tiles 2u and 2u+1), phase
  // 2u+1 its softmax.  Copies are issued in softmax phases only, so an MFMA
  // phase never waits behind them: K of tiles 2u+4, 2u+5 by group 0 in its
  // softmax of pair u (step 2u+1), V of tiles 2u+2, 2u+3 by group 1 in its
  // softmax of pair u (step 2u+2).  Each wave waits for its copies before the
  // barrier ending its next MFMA phase (steps 2u+2 and 2u+3); both are first
  // read at step 2u+4.  The MFMA phase runs unconditionally (P = 0 when there
  // is nothing to add) so the accumulators stay in place.
  // The copying group's half (V or K) of page 0's block at this kv head and
  // the page stride, computed once (loop invariants).
  const uint8_t* cbase = reinterpret_cast<const uint8_t*>(a.kv_cache) +
                         static_cast<size_t>(kvh) * (kKvBlockElems * 2) + (copies_v ? 0 : kKHalfElems * 2);
  const uint32_t pstride = static_cast<uint32_t>(a.hkv) * (kKvBlockElems * 2u);
  const int U = T2 >> 1;
  // Every load issued so far has landed before the loop, so the compiler's
  // wait counting inside the loop starts from nothing outstanding (it would
  // otherwise keep a full vector-memory wait in front of the QK stream).
  __builtin_amdgcn_s_waitcnt(0);
  // Level counts of the four 32-key blocks of the next MFMA phase, computed in
  // the softmax phase before it (pair 0: here).
  int L0 = w_far.advance(a.lt, 0), L1 = w_near.advance(a.lt, 0);
  int L2 = w_far.advance(a.lt, 1), L3 = w_near.advance(a.lt, 1);
  for (int u = 0; u <= U; ++u) {
    // ---- MFMA phase of pair u ----
    __builtin_amdgcn_s_setprio(1);
    {
      const lds_u8* kb = smem + (u % kPfKPairs) * kPfPairBytes + k_lane;
      const lds_u8* vb = smem + kPfVRegion + ((u + 1) & 1) * kPfPairBytes + v_lane;
      bf16x8 f[kRing];
      pv_prefetch(vb, f);
      pv_stream(vb, kb, Pf, O, f);
      if (__builtin_expect(L0 == L3, 1)) {  // L0 <= L1 <= L2 <= L3: one level count
        switch (L0) {
          case 8: qk_stream<8>(kb, f, Qf, Cm, S); break;
          case 7: qk_stream<7>(kb, f, Qf, Cm, S); break;
          case 6: qk_stream<6>(kb, f, Qf, Cm, S); break;
          case 5: qk_stream<5>(kb, f, Qf, Cm, S); break;
          case 4: qk_stream<4>(kb, f, Qf, Cm, S); break;
          case 3: qk_stream<3>(kb, f, Qf, Cm, S); break;
          case 2: qk_stream<2>(kb, f, Qf, Cm, S); break;
          default: qk_stream<1>(kb, f, Qf, Cm, S); break;
        }
      } else {  // a level boundary inside the pair: per-tile chains
        qk_tile(L0, L1, kb, kb + 8192, Qf, f[32 % kRing], f[33 % kRing], Cm, S[0], S[1]);
        qk_tile(L2, L3, kb + 16384, kb + 24576, Qf, f[34 % kRing], f[35 % kRing], Cm, S[2], S[3]);
      }
    }
    __builtin_amdgcn_s_setprio(0);
    // this wave's copies requested in its previous phase land before the
    // barrier after which they are first read
    __builtin_amdgcn_s_waitcnt(kWaitVm);
    if (copies_v && 2 * u < T2 && (2 * u + 2) * kPfTileN > a.nk) {
      // the V of tiles 2u, 2u+1 (pair u % 2) has landed: zero the slots of keys
      // past nk in this wave's pages (0 * V must stay 0); first read next phase
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int n0 = (2 * u + hh) * kPfTileN + rank * kPage;
        lds_u8* vpage = smem + kPfVRegion + (u & 1) * kPfPairBytes + hh * kPfSlotBytes + rank * 4096;
#pragma unroll
        for (int rr = 0; rr < 2; ++rr)
#pragma unroll
          for (int tk = 0; tk < kPage; ++tk)
            if (n0 + tk >= a.nk)
              *reinterpret_cast<__attribute__((address_space(3))) uint16_t*>(vpage + v_lds_elem(lane * 2 + rr, v_slot(tk))) =
                  0;
      }
    }
    pf_barrier();
    // ---- softmax phase of pair u (lane = query row), with this wave's copies ----
    // K (group 0) of tiles 2u+4, 2u+5 into the pair of tiles 2u-2, 2u-1 (read
    // by both groups in phase u-1), or V (group 1) of tiles 2u+2, 2u+3 into
    // the pair of tiles 2u-2, 2u-1 (read by both groups' PV in phase u).
    const int ct = 2 * u + (copies_v ? 2 : 4);
    const int lim = copies_v ? T2 : T;
    lds_u8* cdst = (copies_v ? smem + kPfVRegion + ((u + 1) & 1) * kPfPairBytes
                             : smem + ((u + 2) % kPfKPairs) * kPfPairBytes) + rank * 4096;
    // whole 1 KB level pairs for K (an odd L also copies level L, which is not read)
    const int rows_a = copies_v ? 4 : (w_ld.advance(a.lt, ct) + 1) >> 1;
    const int rows_b = copies_v ? 4 : (w_ld.advance(a.lt, ct + 1) + 1) >> 1;
    const int pa = page_id(a, pg_a), pb = page_id(a, pg_b);
    // The wave's two pages are copied in two batches, the first here and the
    // second halfway through the softmax: the four waves of the group issue
    // their copies together, and a wave issuing all eight 1 KB rows at once
    // waits for the CU's texture path to take them (k=2 -0.4 to -0.9%, OFF
    // unchanged against issuing both pages here).
    if (ct < lim) stage_page(cbase, pstride, pa, rows_a, cdst, lane, copy_off);
    if (2 * u < t_end) {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int tau = 2 * u + hh;
        const int n0 = tau * kPfTileN;
        if (tau >= t_end) {  // past this wave's last tile: P = 0
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) S[2 * hh + kb][r] = NEG_INF;
        } else if ((n0 + kPfTileN - 1 > pos0) || (n0 + kPfTileN > a.nk)) {
          // element (kb, r) holds key n0 + 4*(lane/32) + c with c = 32kb + 8(r/4) + r%4;
          // masked when key > min(row position, nk - 1).  Selects, no branches.
          const int thr = min(pos0 + (lane & 31), a.nk - 1) - n0 - 4 * (lane >> 5);
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r)
              S[2 * hh + kb][r] = (32 * kb + 8 * (r >> 2) + (r & 3) > thr) ? NEG_INF : S[2 * hh + kb][r];
        }
      }
      // S holds score - m_ref, so every P = exp2(S) is at most 256 unless a
      // score exceeds m_ref by more than 8; P >= 0, so that shows as a partial
      // row sum above 256 (or an infinite one).  Only then, and on the first
      // pair (key 0 is visible to every row, so its max is finite), is the row
      // max taken: where it exceeds m_ref by more than 8 (always on the first
      // pair), m_ref moves up to it, O and l are rescaled, and the pair's P is
      // computed again from the shifted scores (shift 0 for the other lanes).
      float lt = 0.f;
      exp_block<kRaw>(S[0], Pf[0], Pf[1], c, lt);
      exp_block<kRaw>(S[1], Pf[2], Pf[3], c, lt);
      __builtin_amdgcn_sched_barrier(0);
      if (ct + 1 < lim) stage_page(cbase, pstride, pb, rows_b, cdst + kPfSlotBytes, lane, copy_off);
      __builtin_amdgcn_sched_barrier(0);
      exp_block<kRaw>(S[2], Pf[4], Pf[5], c, lt);
      exp_block<kRaw>(S[3], Pf[6], Pf[7], c, lt);
      if (__builtin_amdgcn_ballot_w64((u == 0) || !(lt <= 256.f)) != 0) {
        float mx = NEG_INF;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) mx = fmaxf(mx, S[kb][r]);
        mx = pair_max(mx);
        if (kRaw) mx *= c;  // log2 units
        const bool grow = (u == 0) || mx > kLazyRescaleLog2;
        if (__builtin_amdgcn_ballot_w64(grow) != 0) {
          const float delta = grow ? mx : 0.f;
          if (u > 0) {
            const float alpha = fast_exp2(-delta);
            l_run *= alpha;
#pragma unroll
            for (int db = 0; db < 4; ++db) O[db] *= alpha;
          }
          m_ref += delta;
#pragma unroll
          for (int i = 0; i < 16; ++i) Cm[i] = kRaw ? -m_ref * inv_c : -m_ref;
          const float dS = kRaw ? delta * inv_c : delta;
#pragma unroll
          for (int kb = 0; kb < 4; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) S[kb][r] -= dS;
          lt = exp_tiles<kRaw>(S, Pf, c);
        }
      }
      l_run += lt;
    } else {
      if (ct + 1 < lim) stage_page(cbase, pstride, pb, rows_b, cdst + kPfSlotBytes, lane, copy_off);
#pragma unroll
      for (int i = 0; i < 8; ++i) Pf[i] = bf16x8{};
    }
    pg_a = fetch_page(a, b, 4 * (ct + 2) + rank);
    pg_b = fetch_page(a, b, 4 * (ct + 3) + rank);
    L0 = w_far.advance(a.lt, 2 * u + 2);
    L1 = w_near.advance(a.lt, 2 * u + 2);
    L2 = w_far.advance(a.lt, 2 * u + 3);
    L3 = w_near.advance(a.lt, 2 * u + 3);
    pf_barrier();
  }
  if (!copies_v) __syncthreads();  // group 0 ends one step late

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

// ---- measurement probe: the MFMA ceiling of this kernel's structure ----
// A pseudo-random bf16 value in about [-2, 2] (or [0, 1] for P), from a hash,
// so that the matrix core switches as much as on real data (the part's power
// limit, and with it the clock, depends on operand activity).
__device__ __forceinline__ uint32_t probe_hash(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352dU;
  x ^= x >> 15;
  x *= 0x846ca68bU;
  x ^= x >> 16;
  return x;
}
__device__ __forceinline__ uint32_t probe_bf16x2(uint32_t h, bool unit) {
  // sign (unless unit), exponent 126..128 (126..126 for unit), random mantissa, per half
  uint32_t r = 0;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const uint32_t b = h >> (16 * k);
    const uint32_t sign = unit ? 0u : (b & 1u);
    const uint32_t ex = unit ? 126u : 126u + ((b >> 1) % 3u);
    const uint32_t mant = (b >> 4) & 0x7fu;
    r |= ((sign << 15) | (ex << 7) | mant) << (16 * k);
  }
  return r;
}
__device__ __forceinline__ u32x4 probe_vec(uint32_t seed, bool unit) {
  return u32x4{probe_bf16x2(probe_hash(seed * 4 + 0), unit), probe_bf16x2(probe_hash(seed * 4 + 1), unit),
               probe_bf16x2(probe_hash(seed * 4 + 2), unit), probe_bf16x2(probe_hash(seed * 4 + 3), unit)};
}

// The prefill kernel's MFMA work with nothing else: the same grid, block
// mapping, waves, tile-pair count per workgroup (causal, nk = nq, window OFF),
// LDS operand ring and stream order (PV of 8 pages then QK of 8 levels over
// four 32-key blocks, 64 MFMAs per pair), s_setprio and the two barriers per
// pair with the two wave groups one phase apart -- but no softmax, no K/V
// copies (LDS holds random bf16 written once) and no masks.  Its time against
// prefill_kernel's at the same shape is the cost of the softmax side and the
// staging; its rate against the 2.5 PFLOP/s peak is the ceiling of the
// structure at the clock the part's power limit allows.  The accumulators are
// kept live by an empty asm statement and one store per lane at the end.
__global__ __launch_bounds__(kPfWaves * 64, 1) void prefill_mfma_probe_kernel(int nq, int hq, int n_qtiles,
                                                                               int xcd_alt, float* sink) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem_raw[];
  lds_u8* smem = (lds_u8*)(smem_raw);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int bid = blockIdx.x;
  const int xcd = bid & 7;
  const int j = bid >> 3;
  const int h = j % hq;
  const int rnd = j / hq;
  const int qrank = rnd * 8 + ((rnd & xcd_alt & 1) ? 7 - xcd : xcd);  // prefill_kernel's order
  const int qt = n_qtiles - 1 - qrank;
  if (qt < 0) return;
  const int last_wg = min(nq, qt * kPfRowsWg + kPfRowsWg) - 1;
  const int T = min((nq + kPfTileN - 1) / kPfTileN, last_wg / kPfTileN + 1);
  const int U = ((T + 1) & ~1) >> 1;
  // random operands: LDS once, Q and P in registers
  for (int i = tid; i < kPfLdsTotal / 16; i += kPfWaves * 64)
    *reinterpret_cast<__attribute__((address_space(3))) u32x4*>(smem + i * 16) =
        probe_vec(static_cast<uint32_t>(i) * 977u + static_cast<uint32_t>(h), false);
  u32x4 Qf[kLevels];
  bf16x8 Pf[8];
#pragma unroll
  for (int l = 0; l < kLevels; ++l) Qf[l] = probe_vec(static_cast<uint32_t>((bid * 512 + tid) * 16 + l), false);
#pragma unroll
  for (int i = 0; i < 8; ++i)
    Pf[i] = __builtin_bit_cast(bf16x8, probe_vec(static_cast<uint32_t>((bid * 512 + tid) * 16 + 8 + i), true));
  __syncthreads();
  f32x16 O[4], S[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    O[i] = f32x16{};
    S[i] = f32x16{};
  }
  const f32x16 C = f32x16{};
  const int grp = wave >> 2;
  const int k_lane = ((lane & 31) >> 4) * 4096 + (lane >> 5) * 256 + (lane & 15) * 16;
  const int v_lane = (lane >> 5) * 512 + (lane & 31) * 16;
  if (grp == 1) pf_barrier();  // group 1 starts one step late
  for (int u = 0; u <= U; ++u) {
    __builtin_amdgcn_s_setprio(1);
    {
      const lds_u8* kb = smem + (u % kPfKPairs) * kPfPairBytes + k_lane;
      const lds_u8* vb = smem + kPfVRegion + ((u + 1) & 1) * kPfPairBytes + v_lane;
      bf16x8 f[kRing];
      pv_prefetch(vb, f);
      pv_stream(vb, kb, Pf, O, f);
      qk_stream<kLevels>(kb, f, Qf, C, S);
    }
    __builtin_amdgcn_s_setprio(0);
#pragma unroll
    for (int i = 0; i < 4; ++i) asm volatile("" ::"v"(S[i]));  // the QK results stay live
    pf_barrier();
    pf_barrier();  // the other group's MFMA phase
  }
  if (grp == 0) pf_barrier();  // group 0 ends one step late
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) acc += O[i][0] + S[i][0];
  sink[static_cast<int64_t>(bid) * (kPfWaves * 64) + tid] = acc;
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

namespace {
constexpr int kPfMaxDevices = 64;
std::mutex g_attr_mu;
bool g_attr_set[kPfMaxDevices];  // the 160 KB dynamic-LDS attribute is set on this device

// The prefill kernels (and the probe) may use all 160 KB of LDS: the attribute
// is set once per device (the current one), under a lock, before the first
// launch there.
hipError_t ensure_lds_attribute() {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kPfMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_attr_mu);
  if (g_attr_set[dev]) return hipSuccess;
  for (const void* f : {reinterpret_cast<const void*>(prefill_kernel<false>),
                        reinterpret_cast<const void*>(prefill_kernel<true>),
                        reinterpret_cast<const void*>(prefill_mfma_probe_kernel)}) {
    e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, kPfLdsTotal);
    if (e != hipSuccess) return e;
  }
  g_attr_set[dev] = true;
  return hipSuccess;
}
}  // namespace

// Whether a launch takes the serpentine XCD order.  With the same order in
// every round of 8 q-tiles, XCD x gets tiles n-1-x, n-9-x, ...: the first XCD
// holds the heaviest tile of every round and finishes last.  Where that puts
// the busiest XCD's causal work (the k-tiles of its workgroups) more than 1%
// above the mean, the order alternates (same-box A/B, outputs bitwise equal:
// Llama-3.2-3B shape single shot, 8K -9 to -11%, 32K -2 to -3.6%; Qwen2.5-7B
// shape 32K in 8K chunks -1 to -1.5%; 128K single shot OFF -0.4 to -0.5%,
// k=2 -0.2 to +0.1% over 11 to 15 interleaved repetitions).  Where
// the tiles' work is nearly equal (a late chunk of a chunked prefill, whose
// keys are mostly the cached prefix) the plain order is kept: there the
// serpentine one measured 0 to 1% slower (Qwen2.5-7B shape, 256K in 8K chunks).
int prefill_xcd_alternate(int n_qtiles, int nq, int nk, int q_offset) {
  const int n_ktiles = (nk + kPfTileN - 1) / kPfTileN;
  double tot[8] = {};
  for (int qrank = 0; qrank < n_qtiles; ++qrank) {
    const int qt = n_qtiles - 1 - qrank;
    const int last = q_offset + std::min(nq, (qt + 1) * kPfRowsWg) - 1;
    tot[qrank & 7] += std::min(n_ktiles, last / kPfTileN + 1);
  }
  double mx = 0.0, sum = 0.0;
  for (double t : tot) {
    mx = std::max(mx, t);
    sum += t;
  }
  return (sum > 0.0 && 8.0 * mx > 1.01 * sum) ? 1 : 0;
}

hipError_t launch_prefill(const PrefillArgs& a, hipStream_t s) {
  if (a.nq <= 0 || a.batch <= 0) return hipSuccess;
  if (hipError_t e = ensure_lds_attribute(); e != hipSuccess) return e;
  const int blocks = a.batch * a.n_qgroups * a.hq * 8;
  PrefillArgs k = a;
  k.xcd_alt = prefill_xcd_alternate(a.n_qtiles, a.nq, a.nk, a.q_offset);
  if (a.rope_cs != nullptr)
    hipLaunchKernelGGL(prefill_kernel<false>, dim3(blocks), dim3(kPfWaves * 64), kPfLdsTotal, s, k);
  else
    hipLaunchKernelGGL(prefill_kernel<true>, dim3(blocks), dim3(kPfWaves * 64), kPfLdsTotal, s, k);
  return hipGetLastError();
}

hipError_t launch_prefill_mfma_probe(float* sink, int nq, int hq, hipStream_t s) {
  if (nq <= 0 || hq <= 0) return hipSuccess;
  if (hipError_t e = ensure_lds_attribute(); e != hipSuccess) return e;
  const int n_qtiles = (nq + kPfRowsWg - 1) / kPfRowsWg;
  const int blocks = ((n_qtiles + 7) / 8) * hq * 8;
  hipLaunchKernelGGL(prefill_mfma_probe_kernel, dim3(blocks), dim3(kPfWaves * 64), kPfLdsTotal, s, nq, hq, n_qtiles,
                     prefill_xcd_alternate(n_qtiles, nq, nq, 0), sink);
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
