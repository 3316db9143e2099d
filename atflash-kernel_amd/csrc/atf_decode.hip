// Windowed split-KV decode over the paged KV cache (gfx950): one block per
// (page, kv head), the transposed V page and then the slice-blocked K page.
//
// Replaces the FlashInfer window port's single-request decode
// (single_decode_with_kv_cache_with_jit_module(..., maybe_zhi_slice=...),
// kernels/flashinfer_port/fiwin_common.py:96-112, e2e_pipeline/atflash_e2e_fafi.py:106-109;
// window predicate: kernels/flashinfer_port/decode.cuh.diff:47-89).
//
// One workgroup of 8 waves per (sequence, kv head, split of pages); each wave
// streams its own pages.  The G = Hq/Hkv query heads of the kv head are the 16
// columns of v_mfma_f32_16x16x32_bf16 (S^T = K Q^T, four 8-dim slices per
// instruction) and v_mfma_f32_16x16x16_bf16 (O^T = V^T P^T, 16 tokens per
// instruction).  K and V are loaded straight into the MFMA operand registers.
// The window table is per 8-dim slice (16 entries; a 16-dim level table is
// passed as each level's value for its two slices).  Page p is read for the
// first n(p) = #{s : zhi8[s] >= (N-1) - (16p+15)} slices, those its youngest
// key reads: the page's K buffer range covers those slices only, so the loads
// of the other slices return zeros without a memory request and out-of-window
// K bytes are not read from HBM.  Page rule (level table, block_n = 16): every
// key of the page uses those slices.  Per-key rule (vec8 table, as the
// FlashInfer port's decode, kernels/flashinfer_port/decode.cuh.diff:47-89):
// on a page with a slice boundary inside it, an older key's out-of-window
// slices are zeroed in registers before the MFMA.
//
// Merging: the 8 wave partials (m, l, o) of a split are combined in LDS.  With
// one split per (sequence, kv head) the workgroup writes the output itself.
// Otherwise it stores the split's partial in the workspace and ends, and a
// second kernel (decode_merge_kernel, eight workgroups per (sequence, kv head))
// merges the split partials by log-sum-exp and writes the output.  The kernel
// boundary orders the partial stores before the merge loads, so no workgroup
// waits on another inside a launch: no arrival counters, atomics or fences.
// (Measured against merging in the last-arriving workgroup of one launch: the
// chain store -> wait -> arrival atomic -> acquire -> loads there kept a single
// workgroup busy for about 7 us after the last split finished.)
#include <mutex>

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
  u32x4 k[4];  // slice quads (32 dims each)
  u32x2 v[8];  // 16-row d blocks
  int n0;
  bool mask;   // per-key rule with a slice boundary inside the page
};

// Page order of a split: the split's local page j (0 <= j < its page count)
// is page po + pm * j of the sequence.  Splits of at least kDecIlvMinPages
// pages (one 4-page group per wave of an 8-wave workgroup) interleave
// (po = s, pm = n_splits: split s takes pages s, s + n_splits, ...), so that
// the workgroups of a call sweep the sequence from its oldest to its youngest
// page together and each split holds pages of every age.  Shorter splits (the
// 4-wave workgroups of short contexts) take contiguous runs
// (po = s * pages_per_split, pm = 1).  Measured per call against contiguous
// runs for every split (same box, graph-replayed; pools rotated past the
// last-level cache): with a page table in allocation order (the cache's own
// allocators) Qwen 128K OFF -2 to -4%, k=2 -8 to -10% (three runs), Llama 32K
// OFF -2.5 to -8.5%, k=2 -8.5 to -9.5%, Llama 128K OFF -2.5%, k=2 -5.5%,
// Llama 16K OFF -6.5%, k=2 -12%, Qwen 32K -2%; with randomly permuted pages
// +0.3 to +1.3% at those shapes; at 8K with 4-wave workgroups interleaving lost
// up to 4-6%.  po and pm are known before the sequence length is; count is set
// once it is.
constexpr int kDecIlvMinPages = kDecUnroll * kDecWaves;
struct PageOrder {
  int po, pm;
  int count;  // the split's pages for this sequence
};
__device__ __forceinline__ PageOrder page_order(int s, int n_splits, int pages_per_split) {
  const bool ilv = pages_per_split >= kDecIlvMinPages;
  return PageOrder{ilv ? s : s * pages_per_split, ilv ? n_splits : 1, 0};
}
__device__ __forceinline__ void set_page_count(PageOrder& o, int s, int n_splits, int pages_per_split,
                                               int n_pages) {
  o.count = o.pm != 1 ? (n_pages > s ? (n_pages - s + n_splits - 1) / n_splits : 0)
                      : max(0, min(n_pages - o.po, pages_per_split));  // (n_splits 1: the same count)
}

// Page-table entry of local page j (a vector register; every lane holds the
// same value).  The load is unconditional, its index clamped into the split:
// an entry for a page past the split is fetched but never used (its page is
// not loaded), and a split without pages reads entry po, inside the table
// row.  A load guarded by a branch with a default value would make the
// compiler wait for every outstanding load before the register's next use.
// A wave fetches a page's entry one stride ahead of its use, so the page loads
// are issued without waiting for the table.
__device__ __forceinline__ int dec_fetch_entry(const int32_t* row, const PageOrder& o, int j) {
  return row[o.po + o.pm * max(0, min(j, o.count - 1))];
}

// The fields of the call that the first page loads need, passed as leading
// scalar kernel arguments so that they arrive preloaded in SGPRs (kernarg
// preloading): the page-table and sequence-length loads are issued without
// first waiting for the argument block to be read from memory.
struct DecHot {
  const int32_t* page_table;
  const int32_t* seq_lens;
  const uint16_t* kv_cache;
  int max_pages, pages_per_split, max_seq_len, hkv, num_pages, n_splits;
};

// The slices page p reads and whether an older key of it reads fewer.  Page
// rule (level table): 2 L(p) slices, L(p) = levels of the youngest key's age.
// Per-key rule: the youngest key's slices, #{s : zhi8[s] >= age}; a slice
// boundary falls inside the page when the oldest key's count differs.  Lane
// s < 16 holds zhi8[s] (zc; the other lanes a limit no age meets), so each
// count is one vector compare and the popcount of its ballot (the caller keeps
// every lane active): against 16 scalar compares per count, -0.3 to -1.0 us per
// call at 32K-128K (+0.5 us at Llama 32K), and those in turn were 0.4 us per
// call faster at 128K than walking the slice boundaries page by page with a
// loop, whose branches sat in front of every page load.
template <bool kPerKey>
__device__ __forceinline__ void page_slices(const DecodeArgs& a, int zc, int p, int N, int& ns, bool& mask) {
  const int z_young = (N - 1) - (p * kPage + kPage - 1);
  if constexpr (kPerKey) {
    const int z_old = z_young + kPage - 1;
    const int cy = __builtin_popcountll(__builtin_amdgcn_ballot_w64(zc >= z_young));
    const int co = __builtin_popcountll(__builtin_amdgcn_ballot_w64(zc >= z_old));
    ns = cy;
    mask = co != cy;
  } else {
    ns = 2 * levels_of(a.lt, max(0, z_young));
    mask = false;
  }
}

// K and V operands of page p whose page-table entry is `raw`, reading its first
// ns slices of K; a page outside the split (in_split false) reads nothing.
// The page's V and K halves are range-checked buffer resources: a load at or
// past the range returns zeros without a memory request.  K's slices are a
// contiguous prefix of its half, so a range of ns * 256 bytes reads the
// in-window slices and yields zeros for the others, and what the page reads is
// one contiguous run (V, then those slices); an invalid page entry gets an
// empty range.  The loads are therefore unconditional: wave-uniform base,
// 32-bit lane offset, immediate row offset, no per-load address arithmetic.
// Every page is read once per call, so the loads are non-temporal.
// (The range goes through readfirstlane: the level count is uniform, but the
// compiler may count it in a vector register, and a resource built from one
// becomes a loop over lanes around every load.)
struct PageRef {
  size_t blk_elems;  // offset of the (page, kv head) block in the cache, in elements
  bool ok;
};
__device__ __forceinline__ PageRef page_ref(const DecHot& a, int h, int raw, bool in_split) {
  const int pg = __builtin_amdgcn_readfirstlane(raw);
  const bool ok = in_split && pg >= 0 && pg < a.num_pages;
  return PageRef{(static_cast<size_t>(ok ? pg : 0) * a.hkv + h) * kKvBlockElems, ok};
}
// K: slice 4 lp + lane/16, token lane%16: quad lp is the 1 KB run at lp * 1024
__device__ __forceinline__ void dec_load_k(const DecHot& a, const PageRef& pr, int ns, int lane, u32x4 (&k)[4]) {
  const int k_range = __builtin_amdgcn_readfirstlane(pr.ok ? ns * (kPage * kSliceDims * 2) : 0);
  const __amdgpu_buffer_rsrc_t rk =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.kv_cache) + pr.blk_elems + kKHalfElems, 0, k_range,
                                        kBufferWord3);
  const uint32_t koff = static_cast<uint32_t>(lane) << 4;
#pragma unroll
  for (int lp = 0; lp < 4; ++lp)
    k[lp] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rk, koff + lp * 1024u, 0, kLoadStream));
}
// V^T operand: d row 16*db + lane%16, tokens 4*(lane/16)..+3 -> stored slots.
__device__ __forceinline__ void dec_load_v(const DecHot& a, const PageRef& pr, int lane, u32x2 (&v)[8]) {
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(a.kv_cache) + pr.blk_elems, 0, pr.ok ? kBlockElems * 2 : 0, kBufferWord3);
  const int grp = lane >> 4;
  const int slot0 = 4 * ((grp == 1) ? 2 : (grp == 2 ? 1 : grp));
  const uint32_t voff = (static_cast<uint32_t>(lane & 15) << 5) + static_cast<uint32_t>(slot0) * 2u;
#pragma unroll
  for (int db = 0; db < 8; ++db)
    v[db] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rv, voff + db * 512u, 0, kLoadStream));
}
__device__ __forceinline__ void dec_load_page(const DecHot& a, int h, int raw, bool in_split, int p, int ns,
                                              bool mask, int lane, PageRegs& r) {
  r.n0 = p * kPage;
  r.mask = mask;
  const PageRef ref = page_ref(a, h, raw, in_split);
  dec_load_k(a, ref, ns, lane, r.k);
  dec_load_v(a, ref, lane, r.v);
}

// two waves per SIMD: at most 256 registers per wave.  kWaves = 8 (one
// workgroup per CU) or 4 (short contexts: smaller splits over more CUs).
template <bool kPerKey, int kWaves>
__global__ __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(2)))
void decode_kernel(const int32_t* page_table, const int32_t* seq_lens, const uint16_t* kv_cache, int max_pages,
                   int pages_per_split, int max_seq_len, int hkv, int num_pages, int n_splits, DecodeArgs a) {
  const DecHot hot{page_table, seq_lens, kv_cache, max_pages, pages_per_split, max_seq_len, hkv, num_pages, n_splits};
  // wave partials
  __shared__ __attribute__((aligned(16))) float sh_o[kWaves * kDecMaxGroup * kD];
  __shared__ float sh_m[kWaves * kDecMaxGroup], sh_l[kWaves * kDecMaxGroup];

  const int s = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int g = lane & 15;
  // Local page indices: wave w takes the groups of kDecUnroll local pages that
  // start at kDecUnroll * (w + kWaves * i); local page j is page po + pm * j.
  constexpr int kStride = kDecUnroll * kWaves;
  const int p_first = kDecUnroll * __builtin_amdgcn_readfirstlane(wave);
  PageOrder ord = page_order(s, hot.n_splits, hot.pages_per_split);
  const int po = ord.po, pm = ord.pm;
  // The first group's page-table entries are fetched together with the
  // sequence length, their index clamped into the table row only (an entry
  // past the split is never used), so the first page loads wait for two
  // memory round trips after the kernel arguments, not three.
  int ent[kDecUnroll];
  const int32_t* row = hot.page_table + static_cast<int64_t>(b) * hot.max_pages;
#pragma unroll
  for (int u = 0; u < kDecUnroll; ++u) ent[u] = row[min(po + pm * (p_first + u), hot.max_pages - 1)];
  const int N = max(0, min(hot.seq_lens[b], hot.max_seq_len));
  const int n_pages = (N + kPage - 1) / kPage;
  set_page_count(ord, s, hot.n_splits, hot.pages_per_split, n_pages);
  const int p_end = ord.count;
  const float NEG_INF = -__builtin_huge_valf();
  const float c = a.scale_log2;

  // The first group's page loads are issued before Q is loaded and rotated, so
  // the wave's first memory round trip overlaps the Q work.  Each page's
  // registers are reloaded with the page one stride on right after the page is
  // used, so the next group's loads go out while the rest of the group is
  // computed.  (A group still starts with a wait for all of its loads: the
  // reloads are conditional on the split's end.  Issuing every load on every
  // path, so that each page is waited for with the later pages' loads still in
  // flight, measured slower.)
  PageRegs pr[kDecUnroll];
  // per-key rule: lane s < 16 holds zhi8[s], the others a limit no age meets,
  // so a page's slice counts are one compare and a ballot popcount each
  int zc = INT32_MIN;
#pragma unroll
  for (int s = 0; s < kSlices && kPerKey; ++s)
    if (lane == s) zc = a.st.zhi[s];
  // Straight-line code up to the first page loads (a page past the split gets
  // an empty buffer range: its loads return zeros without a memory request), so
  // the compiler reads every kernel argument they need in the first batch.
#pragma unroll
  for (int u = 0; u < kDecUnroll; ++u) {
    int ns;
    bool mask;
    page_slices<kPerKey>(a, zc, po + pm * (p_first + u), N, ns, mask);
    dec_load_page(hot, h, ent[u], p_first + u < p_end, po + pm * (p_first + u), ns, mask, lane, pr[u]);
  }
#pragma unroll
  for (int u = 0; u < kDecUnroll; ++u) ent[u] = dec_fetch_entry(row, ord, p_first + kStride + u);

  // ---- Q^T fragments: lane holds q head g, slice 4 lp + lane/16 ----
  // Every Q and (cos, sin) load is issued before any is used (one memory round
  // trip, not one per slice): lanes past the group read the group's last head
  // and a sequence of length 0 reads position 0, both in bounds, and are
  // zeroed afterwards.
  u32x4 Qf[4];
  {
    const int qh = h * a.group + min(g, a.group - 1);
    const bool valid = g < a.group && N > 0;
    const uint16_t* qrow = a.q + static_cast<int64_t>(b) * a.q_sb + static_cast<int64_t>(qh) * a.q_sh;
    load_slices4<4>(qrow, a.layout, lane >> 4, Qf);
    if (a.rope_cs != nullptr) {
      float cs[4][8];
#pragma unroll
      for (int lp = 0; lp < 4; ++lp) load_cs4(a.rope_cs, max(N - 1, 0), slice_pair0(4 * lp + (lane >> 4)), cs[lp]);
#pragma unroll
      for (int lp = 0; lp < 4; ++lp) Qf[lp] = rope_slice(Qf[lp], cs[lp]);
    }
#pragma unroll
    for (int lp = 0; lp < 4; ++lp)
      if (!valid) Qf[lp] = u32x4{0u, 0u, 0u, 0u};
  }
  // per-key rule: the distance limit of this lane's slice in each quad
  int zl[4] = {0, 0, 0, 0};
#pragma unroll
  for (int lp = 0; lp < 4 && kPerKey; ++lp) {
    const int sg = lane >> 4;
    const int z0 = a.st.zhi[4 * lp], z1 = a.st.zhi[4 * lp + 1], z2 = a.st.zhi[4 * lp + 2], z3 = a.st.zhi[4 * lp + 3];
    zl[lp] = sg == 0 ? z0 : (sg == 1 ? z1 : (sg == 2 ? z2 : z3));
  }

  f32x4 O[8];
#pragma unroll
  for (int db = 0; db < 8; ++db) O[db] = f32x4{};
  float m_run = NEG_INF, l_run = 0.f;

  for (int p0 = p_first; p0 < p_end; p0 += kStride) {
#pragma unroll
    for (int u = 0; u < kDecUnroll; ++u) {
      if (p0 + u >= p_end) break;
      PageRegs& r = pr[u];
      if (kPerKey && r.mask) {
        // a slice boundary inside the page: a key older than its slice's limit
        // (age > zhi8[slice]) drops that slice (lane: key lane%16, slice 4 lp + lane/16)
        const int age = (N - 1) - (r.n0 + (lane & 15));
#pragma unroll
        for (int lp = 0; lp < 4; ++lp)
          if (age > zl[lp]) r.k[lp] = u32x4{0u, 0u, 0u, 0u};
      }
      // all four slice quads: the out-of-window slices were loaded as zeros and
      // add exact zeros (cheaper than branching around their MFMAs)
      f32x4 S = f32x4{};
#pragma unroll
      for (int lp = 0; lp < 4; ++lp)
        S = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, r.k[lp]),
                                                    __builtin_bit_cast(bf16x8, Qf[lp]), S, 0, 0, 0);
      // S lane layout: q head g, tokens 4*(lane/16) + i.
      const int tok0 = r.n0 + 4 * (lane >> 4);
      const bool tail = r.n0 + kPage > N;
      // This page's registers take the page one stride on: K as soon as the QK
      // MFMAs have read it, V after the PV MFMAs (-0.46 us per call at 128K
      // against reloading both after the page, same box; outputs bitwise equal).
      const int pn = p0 + kStride + u;
      const bool reload = pn < p_end;
      bool mask_n = false;
      PageRef ref_n{0, false};
      if (reload) {
        int ns;
        page_slices<kPerKey>(a, zc, po + pm * pn, N, ns, mask_n);
        ref_n = page_ref(hot, h, ent[u], true);
        dec_load_k(hot, ref_n, ns, lane, r.k);
      }
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
      // Lazy reference max: m_run moves only where a score exceeds it by more
      // than 8 (log2 units; the first finite score always does), so P <= 256
      // and O and l are rescaled on few pages.
      const bool grow = (mx - m_run) * c > 8.f;  // -inf - -inf = NaN: no
      if (__builtin_amdgcn_ballot_w64(grow) != 0) {
        const float alpha = !grow ? 1.f : (m_run == NEG_INF ? 0.f : fast_exp2((m_run - mx) * c));
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < 8; ++db) O[db] *= alpha;
        m_run = grow ? mx : m_run;
      }
      const float msc = (m_run == NEG_INF) ? 0.f : m_run * c;
      float pv[4];
      float ls = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pv[i] = fast_exp2(__builtin_fmaf(S[i], c, -msc));
        ls += pv[i];
      }
      l_run += ls;
      u32x2 pk;
      pk[0] = pack_bf16x2(pv[0], pv[1]);
      pk[1] = pack_bf16x2(pv[2], pv[3]);
      const s16x4 pb = __builtin_bit_cast(s16x4, pk);
#pragma unroll
      for (int db = 0; db < 8; ++db)
        O[db] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, r.v[db]), pb, O[db], 0, 0, 0);
      if (reload) {
        dec_load_v(hot, ref_n, lane, r.v);
        r.n0 = (po + pm * pn) * kPage;
        r.mask = mask_n;
        ent[u] = dec_fetch_entry(row, ord, pn + kStride);
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
  // thread t owns query heads t / 32 + 2 kWaves j, dims 4 (t % 32) .. +3
  const int d4 = 4 * (tid & 31);
  const int64_t pbase = (static_cast<int64_t>(b) * hot.hkv + h) * a.n_splits * kDecMaxGroup;  // split 0, head 0
  for (int gq = tid >> 5; gq < a.group; gq += 2 * kWaves) {
    float M = NEG_INF;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, sh_m[w * kDecMaxGroup + gq]);
    float L = 0.f;
    f32x4 acc = f32x4{};
    if (M != NEG_INF) {
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float wt = fast_exp2((sh_m[w * kDecMaxGroup + gq] - M) * c);  // empty wave: m = -inf -> 0
        L += wt * sh_l[w * kDecMaxGroup + gq];
        acc += wt * *reinterpret_cast<const f32x4*>(&sh_o[(w * kDecMaxGroup + gq) * kD + d4]);
      }
    }
    if (a.n_splits == 1) {  // the split is the whole sequence: write the output
      const float inv = L > 0.f ? 1.f / L : 0.f;
      uint16_t* out = a.out + static_cast<int64_t>(b) * a.o_sb + static_cast<int64_t>(h * a.group + gq) * a.o_sh + d4;
      u32x2 pk;
      pk[0] = pack_bf16x2(acc[0] * inv, acc[1] * inv);
      pk[1] = pack_bf16x2(acc[2] * inv, acc[3] * inv);
      *reinterpret_cast<u32x2*>(out) = pk;
    } else {  // the split's partial, merged by decode_merge_kernel
      const int64_t pi = pbase + static_cast<int64_t>(s) * kDecMaxGroup + gq;
      *reinterpret_cast<f32x4*>(a.ws_o + pi * kD + d4) = acc;
      if (d4 == 0) *reinterpret_cast<f32x2*>(a.ws_ml + pi * 2) = f32x2{M, L};
    }
  }
}

// ---- measurement probe: the streaming ceiling of the decode's page loads ----
// decode_kernel's grid, waves, split rule, page-table fetches and page loads
// (the same range-checked, non-temporal buffer loads of V and of the K slices
// the page's youngest key reads under a.st, the same 4-page groups with the
// rolling reload), with the compute replaced by an XOR of the loaded words, no
// LDS combine and no merge: what the memory system delivers to this access
// pattern.  One word per wave goes to
// sink[((b * hkv + h) * n_splits + s) * kDecWaves + wave].
__global__ __launch_bounds__(kDecWaves * 64) __attribute__((amdgpu_waves_per_eu(2)))
void decode_stream_probe_kernel(const int32_t* page_table, const int32_t* seq_lens, const uint16_t* kv_cache,
                                int max_pages, int pages_per_split, int max_seq_len, int hkv, int num_pages,
                                int n_splits, uint32_t* sink, DecodeArgs a) {
  const DecHot hot{page_table, seq_lens, kv_cache, max_pages, pages_per_split, max_seq_len, hkv, num_pages, n_splits};
  const int s = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  constexpr int kStride = kDecUnroll * kDecWaves;
  const int p_first = kDecUnroll * __builtin_amdgcn_readfirstlane(wave);
  PageOrder ord = page_order(s, hot.n_splits, hot.pages_per_split);
  const int po = ord.po, pm = ord.pm;
  int ent[kDecUnroll];
  const int32_t* row = hot.page_table + static_cast<int64_t>(b) * hot.max_pages;
#pragma unroll
  for (int u = 0; u < kDecUnroll; ++u) ent[u] = row[min(po + pm * (p_first + u), hot.max_pages - 1)];
  const int N = max(0, min(hot.seq_lens[b], hot.max_seq_len));
  const int n_pages = (N + kPage - 1) / kPage;
  set_page_count(ord, s, hot.n_splits, hot.pages_per_split, n_pages);
  const int p_end = ord.count;
  PageRegs pr[kDecUnroll];
  int zc = INT32_MIN;
#pragma unroll
  for (int sl = 0; sl < kSlices; ++sl)
    if (lane == sl) zc = a.st.zhi[sl];
#pragma unroll
  for (int u = 0; u < kDecUnroll; ++u) {
    int ns;
    bool mask;
    page_slices<true>(a, zc, po + pm * (p_first + u), N, ns, mask);
    dec_load_page(hot, h, ent[u], p_first + u < p_end, po + pm * (p_first + u), ns, false, lane, pr[u]);
  }
#pragma unroll
  for (int u = 0; u < kDecUnroll; ++u) ent[u] = dec_fetch_entry(row, ord, p_first + kStride + u);
  uint32_t acc = 0;
  for (int p0 = p_first; p0 < p_end; p0 += kStride) {
#pragma unroll
    for (int u = 0; u < kDecUnroll; ++u) {
      if (p0 + u >= p_end) break;
      PageRegs& r = pr[u];
#pragma unroll
      for (int lp = 0; lp < 4; ++lp) acc ^= r.k[lp][0] ^ r.k[lp][1] ^ r.k[lp][2] ^ r.k[lp][3];
#pragma unroll
      for (int db = 0; db < 8; ++db) acc ^= r.v[db][0] ^ r.v[db][1];
      const int pn = p0 + kStride + u;
      if (pn < p_end) {
        int ns;
        bool mask;
        page_slices<true>(a, zc, po + pm * pn, N, ns, mask);
        dec_load_page(hot, h, ent[u], true, po + pm * pn, ns, false, lane, pr[u]);
        ent[u] = dec_fetch_entry(row, ord, pn + kStride);
      }
    }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) acc ^= static_cast<uint32_t>(__shfl_xor(static_cast<int>(acc), m));
  if (lane == 0) sink[((static_cast<int64_t>(b) * hkv + h) * n_splits + s) * kDecWaves + wave] = acc;
}

// Log-sum-exp merge of the split partials, launched after decode_kernel when
// n_splits > 1.  One workgroup per (16-dim chunk, kv head, sequence), so that
// the merge's loads spread over 8 CUs per (sequence, kv head) (4 chunks of 32
// dims were 0.6-0.75 us slower per call, 16 chunks of 8 dims 0.2 us).  Thread
// t takes 4 dims of its chunk and, for query head mg, every H-th split
// starting at hh (H = 16 for G <= 8, 8 for larger groups).  It loads the
// (m, l) and o of up to kMergeBatch splits before using any of them, so with
// up to 64 splits (32 for G > 8) the merge costs one memory round trip; more
// splits are folded in batch by batch with a running max.  The H partial
// merges of a (head, dims) sit in lanes 4k + (t % 4) of one wave (half wave
// for G > 8) and are combined by DPP row rotations and permlane swaps, VALU
// moves without LDS or a workgroup barrier.
constexpr int kMergeChunks = 8;
constexpr int kMergeDims = kD / kMergeChunks;          // dims per workgroup
constexpr int kMergeLanes = kMergeDims / 4;            // lanes per (head, split group), 4 dims each
constexpr int kMergeRowsPerWave = 64 / kMergeLanes;    // (head, split group) rows per wave
constexpr int kMergeBatch = 4;                         // splits loaded per thread before use
static_assert(kMergeChunks * kMergeDims == kD && kMergeLanes == 4 && kDecMaxGroup <= 16,
              "merge layout: 4 lanes per (head, split group), one or two heads per wave (8 waves: 8 heads for "
              "G <= 8, 16 for larger groups)");

// The merge kernel's arguments are scalars (14 dwords), preloaded into SGPRs
// with the dispatch, so the partial loads are issued at once instead of after
// a read of an argument block.
struct MergeArgs {
  const float* ws_ml;
  const float* ws_o;
  uint16_t* out;
  int64_t o_sb, o_sh;
  int n_splits, group, hkv;
  float scale_log2;
};

// Two (m, l, o) partials merged by log-sum-exp.
__device__ __forceinline__ void merge_pair(float& m, float& l, f32x4& o, float mp, float lp, const f32x4& op,
                                           float c) {
  const float NEG_INF = -__builtin_huge_valf();
  const float M = fmaxf(m, mp);
  if (M != NEG_INF) {
    const float w = fast_exp2((m - M) * c), wp = fast_exp2((mp - M) * c);  // an empty side: m = -inf -> 0
    l = w * l + wp * lp;
    o = w * o + wp * op;
    m = M;
  }
}

// Lane (l + n) % 16 of l's 16-lane row (DPP row rotation: a VALU move, no LDS).
template <int kN>
__device__ __forceinline__ float row_ror(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x120 + kN, 0xF, 0xF, false));
}

// The partial of lane l merged with those of lanes l + 4, l + 8, l + 12 of its
// row (two row rotations), then with the rows l ^ 16 (and l ^ 32 when
// `whole_wave`) by the gfx950 permlane swaps, which hand each lane the value of
// the lane one row (two rows) away: afterwards every lane of a group {4h + q}
// holds the merge of the group's partials.  Every lane takes part; the caller
// keeps control flow uniform around it.
__device__ __forceinline__ void merge_lane_groups(float& m, float& l, f32x4& o, bool whole_wave, float c) {
  {
    f32x4 op;
#pragma unroll
    for (int i = 0; i < 4; ++i) op[i] = row_ror<8>(o[i]);
    merge_pair(m, l, o, row_ror<8>(m), row_ror<8>(l), op, c);
  }
  {
    f32x4 op;
#pragma unroll
    for (int i = 0; i < 4; ++i) op[i] = row_ror<4>(o[i]);
    merge_pair(m, l, o, row_ror<4>(m), row_ror<4>(l), op, c);
  }
  // a swap of a register with itself: result [0] holds rows (0, 0, 2, 2) and
  // result [1] rows (1, 1, 3, 3) of the value (32-lane swap: halves (0, 0) and
  // (1, 1)), so merging [0] with [1] merges each lane with its partner lane
  auto swap16 = [](float x) {
    return __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  };
  auto swap32 = [](float x) {
    return __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  };
  {
    const auto sm = swap16(m), sl = swap16(l);
    f32x4 o0, o1;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const auto so = swap16(o[i]);
      o0[i] = __uint_as_float(so[0]);
      o1[i] = __uint_as_float(so[1]);
    }
    m = __uint_as_float(sm[0]);
    l = __uint_as_float(sl[0]);
    o = o0;
    merge_pair(m, l, o, __uint_as_float(sm[1]), __uint_as_float(sl[1]), o1, c);
  }
  if (whole_wave) {  // uniform over the launch
    const auto sm = swap32(m), sl = swap32(l);
    f32x4 o0, o1;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const auto so = swap32(o[i]);
      o0[i] = __uint_as_float(so[0]);
      o1[i] = __uint_as_float(so[1]);
    }
    m = __uint_as_float(sm[0]);
    l = __uint_as_float(sl[0]);
    o = o0;
    merge_pair(m, l, o, __uint_as_float(sm[1]), __uint_as_float(sl[1]), o1, c);
  }
}

__global__ __launch_bounds__(512) void decode_merge_kernel(const float* ws_ml, const float* ws_o, uint16_t* out,
                                                            int64_t o_sb, int64_t o_sh, int n_splits, int group,
                                                            int hkv, float scale_log2) {
  const MergeArgs a{ws_ml, ws_o, out, o_sb, o_sh, n_splits, group, hkv, scale_log2};
  const int chunk = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x;
  const float NEG_INF = -__builtin_huge_valf();
  const float c = a.scale_log2;
  const int64_t pbase = (static_cast<int64_t>(b) * a.hkv + h) * a.n_splits * kDecMaxGroup;  // split 0, head 0
  const int H = (a.group <= 8) ? kMergeRowsPerWave : kMergeRowsPerWave / 2;
  const int row = tid / kMergeLanes;  // (head, split group)
  const int mg = row / H, hh = row - (row / H) * H;
  const int q4 = 4 * (tid % kMergeLanes);
  const int md4 = chunk * kMergeDims + q4;
  const bool mact = mg < a.group;
  float m_t = NEG_INF, L_t = 0.f;
  f32x4 acc_t = f32x4{};
  if (mact) {
    for (int j0 = hh; j0 < a.n_splits; j0 += kMergeBatch * H) {
      f32x2 mlv[kMergeBatch];
      f32x4 ov[kMergeBatch];
#pragma unroll
      for (int j = 0; j < kMergeBatch; ++j) {
        const int sp = j0 + j * H;
        mlv[j] = f32x2{NEG_INF, 0.f};
        ov[j] = f32x4{};
        if (sp < a.n_splits) {
          const int64_t pi = pbase + static_cast<int64_t>(sp) * kDecMaxGroup + mg;
          mlv[j] = *reinterpret_cast<const f32x2*>(a.ws_ml + pi * 2);
          ov[j] = *reinterpret_cast<const f32x4*>(a.ws_o + pi * kD + md4);
        }
      }
      float mb = m_t;
#pragma unroll
      for (int j = 0; j < kMergeBatch; ++j) mb = fmaxf(mb, mlv[j][0]);
      if (mb != NEG_INF) {
        const float r = fast_exp2((m_t - mb) * c);  // m_t = -inf -> 0
        L_t *= r;
        acc_t *= r;
#pragma unroll
        for (int j = 0; j < kMergeBatch; ++j) {
          const float wt = fast_exp2((mlv[j][0] - mb) * c);  // empty split: m = -inf -> 0
          L_t += wt * mlv[j][1];
          acc_t += wt * ov[j];
        }
        m_t = mb;
      }
    }
  }
  // every lane of the wave takes part in the exchanges (inactive rows hold an
  // empty partial); lanes 4k + (t % 4), k < H, hold one (head, dims): 16
  // groups per wave for G <= 8, 8 per half wave above
  merge_lane_groups(m_t, L_t, acc_t, H == 16, c);
  if (mact && hh == 0) {
    const float inv = L_t > 0.f ? 1.f / L_t : 0.f;
    uint16_t* out = a.out + static_cast<int64_t>(b) * a.o_sb + static_cast<int64_t>(h * a.group + mg) * a.o_sh + md4;
    u32x2 pk;
    pk[0] = pack_bf16x2(acc_t[0] * inv, acc_t[1] * inv);
    pk[1] = pack_bf16x2(acc_t[2] * inv, acc_t[3] * inv);
    *reinterpret_cast<u32x2*>(out) = pk;
  }
}

// Level count per page for one sequence of length N under the page rule
// (block_n = 16), as page_slices<false> computes it (the kernel reads twice as
// many 8-dim slices).
__global__ void decode_page_levels_kernel(int32_t* out, int n_pages, int N, LevelTable lt) {
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= n_pages) return;
  out[p] = levels_of(lt, max(0, (N - 1) - (p * kPage + kPage - 1)));
}

hipError_t launch_decode(const DecodeArgs& a, hipStream_t s) {
  if (a.batch <= 0) return hipSuccess;
  const dim3 grid(a.n_splits, a.hkv, a.batch);
#define ATF_DEC_LAUNCH(PK, W)                                                                                   \
  hipLaunchKernelGGL((decode_kernel<PK, W>), grid, dim3(W * 64), 0, s, a.page_table, a.seq_lens, a.kv_cache,    \
                     a.max_pages, a.pages_per_split, a.max_seq_len, a.hkv, a.num_pages, a.n_splits, a)
  if (a.waves == 8) {
    if (a.per_key) ATF_DEC_LAUNCH(true, 8); else ATF_DEC_LAUNCH(false, 8);
  } else {
    if (a.per_key) ATF_DEC_LAUNCH(true, 4); else ATF_DEC_LAUNCH(false, 4);
  }
#undef ATF_DEC_LAUNCH
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || a.n_splits == 1) return e;
  hipLaunchKernelGGL(decode_merge_kernel, dim3(kMergeChunks, a.hkv, a.batch), dim3(512), 0, s,
                     static_cast<const float*>(a.ws_ml), static_cast<const float*>(a.ws_o), a.out, a.o_sb, a.o_sh,
                     a.n_splits, a.group, a.hkv, a.scale_log2);
  return hipGetLastError();
}

// ---- fixed scratch for the entry point that allocates nothing ----
// One copy per GPU, held until the process ends.  In host code `scratch` is a
// stand-in for the symbol, not a device address: kernels and copies take the
// address hipGetSymbolAddress returns for the current device, kept per device.
// It holds split partials only; nothing in it has to start at any value.
static __device__ __align__(256) uint8_t scratch[kDecScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
uint8_t* g_scratch_ptr[kMaxDevices];  // device address of `scratch` per device, null until looked up

// The current device's scratch, looked up on its first use on that device.
// That first use must not be under stream capture on `s` (the lookup is not a
// stream operation and may load the code object): it fails with
// hipErrorStreamCaptureUnsupported instead.
hipError_t device_scratch(uint8_t** out, hipStream_t s) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(s, &cs);
    if (e != hipSuccess) return e;
    if (cs != hipStreamCaptureStatusNone) return hipErrorStreamCaptureUnsupported;
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (p == nullptr) return hipErrorInvalidSymbol;
    g_scratch_ptr[dev] = static_cast<uint8_t*>(p);
  }
  *out = g_scratch_ptr[dev];
  return hipSuccess;
}
}  // namespace

hipError_t launch_decode_noalloc(DecodeArgs a, hipStream_t s) {
  if (a.batch <= 0) return hipSuccess;
  uint8_t* base = nullptr;
  hipError_t e = device_scratch(&base, s);
  if (e != hipSuccess) return e;
  a.ws_ml = reinterpret_cast<float*>(base);
  a.ws_o = a.ws_ml + static_cast<size_t>(a.batch) * a.hkv * a.n_splits * kDecMaxGroup * 2;
  return launch_decode(a, s);
}

hipError_t launch_decode_stream_probe(const DecodeArgs& a, uint32_t* sink, hipStream_t s) {
  if (a.batch <= 0) return hipSuccess;
  hipLaunchKernelGGL(decode_stream_probe_kernel, dim3(a.n_splits, a.hkv, a.batch), dim3(kDecWaves * 64), 0, s,
                     a.page_table, a.seq_lens, a.kv_cache, a.max_pages, a.pages_per_split, a.max_seq_len, a.hkv,
                     a.num_pages, a.n_splits, sink, a);
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
