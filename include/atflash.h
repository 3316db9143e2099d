/*
 * atflash C ABI: per-RoPE-wavelength windowed attention on AMD MI355X (gfx950).
 *
 * Plain pointers and sizes only.  Every tensor pointer is a device pointer
 * (HIP), allocated and owned by the caller; `stream` is a hipStream_t passed as
 * void* (NULL = default stream).  All work is enqueued asynchronously on
 * `stream`; no entry point synchronises the device.  Every entry point returns
 * ATF_OK (0) or an ATF_ERR_* code; atf_last_error() then describes the failure
 * (per calling thread).
 *
 * Window tables.  `zhi` is a HOST array of ATF_LEVELS int32 entries: zhi[i] is
 * the largest causal key distance at which 16-dim level i is still read
 * (window_tables/atflash_window.py:85-108).  zhi[0] is the table's cap and must
 * be >= the longest causal distance of the call (prefill nk - 1, decode
 * max_seq_len - 1); a smaller cap is refused with ATF_ERR_INVALID, since it
 * would drop levels the rule keeps.  NULL means window OFF: plain causal attention,
 * every level read at every distance.  Level l holds RoPE pairs
 * r in [64-8(l+1), 64-8l) (dims r and r+64 of the half-split layout).
 * The decode also takes the FlashInfer window port's finer table `zhi_slice`
 * (atf_decode_paged_slices_bf16): ATF_SLICES int32 entries, zhi_slice[s] the
 * largest key age (seq_len - 1 - position) at which 8-dim slice s (RoPE pairs
 * r in [64-4(s+1), 64-4s), four pairs in wavelength order) is still read
 * (kernels/flashinfer_port/fiwin_common.py:35-47); level l is slices 2l, 2l+1.
 *
 * Paged KV cache (one layer): pages of ATF_PAGE_SIZE = 16 tokens.
 *   kv_cache  bf16 [num_pages][num_kv_heads][2][2048]: one 8 KB block per
 *             (page, kv head), 16-byte aligned,
 *     [0]  V half: [128 dims][16 token slots] (V transposed)
 *     [1]  K half: [16 slices][16 tokens][8 dims] (slice s: half-split dims
 *          [64-4(s+1), 64-4s) then the same + 64; sorted pair dims [8s, 8s+8))
 * written by atf_kv_write_bf16 (RoPE applied to K there); page_table is int32
 * [batch][max_pages] of page ids.  Token slots of a page that were never written
 * may hold any finite value.  A windowed read of a page is one contiguous run:
 * the V half and the in-window prefix of the K half.
 *
 * RoPE.  rope_cs, when not NULL, is fp32 [rope_max_pos][64][2] holding
 * (cos, sin) of position * inv_freq[r] (HF rotate-half convention); NULL means
 * the inputs are already rotated.  Layout ATF_LAYOUT_SORTED_PAIR (the
 * reference's wavelength-sorted layout) requires rope_cs == NULL.
 */
#ifndef ATFLASH_H_
#define ATFLASH_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ATF_ABI_VERSION 3
#define ATF_HEAD_DIM 128
#define ATF_LEVELS 8
#define ATF_SLICES 16
#define ATF_PAGE_SIZE 16
#define ATF_LAYOUT_HALF_SPLIT 0
#define ATF_LAYOUT_SORTED_PAIR 1
/* Tile quantization of the window (the block_m/block_n the oracle must use). */
#define ATF_PREFILL_BLOCK_M 32
#define ATF_PREFILL_BLOCK_N 32
#define ATF_DECODE_BLOCK_N 16
#define ATF_MAX_GQA_GROUP 16

enum {
  ATF_OK = 0,
  ATF_ERR_INVALID = 1,     /* bad argument (shape, stride, alignment, table) */
  ATF_ERR_UNSUPPORTED = 2, /* valid request this build does not support */
  ATF_ERR_LAUNCH = 3,      /* HIP launch or runtime error */
  ATF_ERR_WORKSPACE = 4    /* workspace missing or too small */
};

int atf_abi_version(void);
const char* atf_last_error(void);

/*
 * Write n_tokens tokens of each of `batch` sequences into the paged cache.
 * Source token t of sequence b sits at absolute position start_pos[b] + t
 * (start_pos: device int32 [batch]) and goes to page
 * page_table[b][pos / 16], slot pos % 16.  K is rotated with rope_cs at that
 * position.  Source strides are in elements; the last dim is contiguous.
 *
 * Positions live in device memory (start_pos), so they are checked in the
 * kernel, not here, and a token that cannot be placed is SKIPPED without an
 * error: a negative position, a position at or past rope_max_pos (when rope_cs
 * is given), a page index pos / 16 at or past max_pages, or a page-table entry
 * outside [0, num_pages).  Attention over such a token would read whatever the
 * slot held before, so callers must keep positions inside the page table and
 * the RoPE table (atflash.cache.PagedKVCache checks this on the host).
 *
 * Replaces the reference's RoPE + head-dim permutation patch and HF cache append
 * (e2e_pipeline/atflash_e2e_fafi.py:186-192, 101-119).
 */
int atf_kv_write_bf16(void* kv_cache, int num_pages, int num_kv_heads,
                      const void* k_src, int64_t ks_b, int64_t ks_t, int64_t ks_h,
                      const void* v_src, int64_t vs_b, int64_t vs_t, int64_t vs_h,
                      int batch, int n_tokens, const int32_t* start_pos,
                      const int32_t* page_table, int max_pages,
                      const float* rope_cs, int rope_max_pos, int layout, void* stream);

/*
 * Windowed causal GQA prefill: out[b, i, h, :] = attention of query row i
 * (absolute position q_offset + i) over keys 0..q_offset+i of sequence b read
 * from the paged cache (nk keys present, q_offset + nq <= nk).  q/out are bf16
 * [batch][nq][num_q_heads][128] with element strides (last dim contiguous;
 * q 16-byte aligned with strides multiples of 8, out 8-byte aligned with
 * strides multiples of 4).  lse (nullable) receives fp32 [batch][num_q_heads][nq] natural-log
 * log-sum-exp of the scaled scores.  Q is rotated with rope_cs at load.
 *
 * Replaces flash_attn.cute.interface._flash_attn_fwd(q, k, v, causal=True,
 * atflash_window_zhi=zhi) of the FA4 window port (call sites
 * microbench/b1_correctness.py:84-85, e2e_pipeline/atflash_e2e_fafi.py:118-119).
 */
int atf_prefill_bf16(void* out, int64_t o_sb, int64_t o_st, int64_t o_sh, float* lse,
                     const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh,
                     const void* kv_cache, int num_pages,
                     const int32_t* page_table, int max_pages,
                     int batch, int nq, int nk, int q_offset, int num_q_heads, int num_kv_heads,
                     const int32_t* zhi, float sm_scale, const float* rope_cs, int rope_max_pos,
                     int layout, void* stream);

/*
 * Bytes of device workspace atf_decode_paged_bf16 needs for these sizes: the
 * fp32 split partials (m, l, o) of every (sequence, kv head, split), 0 when the
 * call runs one split per (sequence, kv head).  The workspace needs no
 * initialisation: each call writes the partials it reads back.  Calls that
 * share a workspace must be ordered on one stream (concurrent calls race).
 */
size_t atf_decode_workspace_bytes(int batch, int num_q_heads, int num_kv_heads, int max_seq_len);

/*
 * Windowed split-KV decode: one query token per sequence at position
 * seq_lens[b] - 1 attending to keys 0..seq_lens[b]-1 of the paged cache.  It
 * enqueues one kernel, plus a second that merges the split partials when a
 * sequence is split (long contexts, small batches).
 * q/out are bf16 [batch][num_q_heads][128] with element strides (q: 16-byte
 * aligned, strides multiples of 8; out: 8-byte aligned, strides multiples of 4); seq_lens is a
 * device int32 [batch] whose entries must not exceed max_seq_len.  The window
 * is quantized per page (block_n = 16): page p reads its first L(p) levels only
 * (2 L(p) slices of its K half).
 *
 * Replaces flashinfer.decode.single_decode_with_kv_cache_with_jit_module(...,
 * maybe_zhi_slice=...) of the FlashInfer window port
 * (kernels/flashinfer_port/fiwin_common.py:96-112, e2e_pipeline/atflash_e2e_fafi.py:106-109).
 */
int atf_decode_paged_bf16(void* out, int64_t o_sb, int64_t o_sh,
                          const void* q, int64_t q_sb, int64_t q_sh,
                          const void* kv_cache, int num_pages,
                          const int32_t* page_table, int max_pages, const int32_t* seq_lens,
                          int batch, int num_q_heads, int num_kv_heads, int max_seq_len,
                          const int32_t* zhi, float sm_scale, const float* rope_cs, int rope_max_pos,
                          int layout, void* workspace, size_t workspace_bytes, void* stream);

/*
 * atf_decode_paged_bf16 with the per-slice (vec8) window table of the
 * FlashInfer port and its per-key rule: slice s of the key at position pos is
 * read iff seq_len - 1 - pos <= zhi_slice[s] (kernels/flashinfer_port/
 * decode.cuh.diff:47-89, gates/g2_correctness.py:37-70), with no minimum (a key
 * past every slice scores 0).  zhi_slice is a HOST int32 [ATF_SLICES],
 * non-negative and non-increasing, or NULL (window OFF).  Each page reads the
 * slices of its youngest key; an older key's slices past its limit are masked.
 * Same workspace as atf_decode_paged_bf16.
 *
 * Replaces single_decode_with_kv_cache_with_jit_module(mod, q, k, v, None,
 * zhi_slice, ...) (kernels/flashinfer_port/fiwin_common.py:96-112), whose
 * zhi_slice is fiwin_common.zhi_slice_vec8 (fiwin_common.py:35-47).
 */
int atf_decode_paged_slices_bf16(void* out, int64_t o_sb, int64_t o_sh,
                                 const void* q, int64_t q_sb, int64_t q_sh,
                                 const void* kv_cache, int num_pages,
                                 const int32_t* page_table, int max_pages, const int32_t* seq_lens,
                                 int batch, int num_q_heads, int num_kv_heads, int max_seq_len,
                                 const int32_t* zhi_slice, float sm_scale, const float* rope_cs,
                                 int rope_max_pos, int layout, void* workspace, size_t workspace_bytes,
                                 void* stream);

/*
 * atf_decode_paged_bf16 for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  It has no counterpart in the reference.  Same arguments and
 * result as atf_decode_paged_bf16 without the workspace: the split partials
 * live in a fixed 8 MiB scratch array in device memory, one per GPU the library
 * runs on, held until the process ends.  No call allocates or frees anything.
 * Limit: atf_decode_workspace_bytes(...) <= 8 MiB, otherwise
 * ATF_ERR_UNSUPPORTED; the split rule keeps every request within about 4.1 MiB
 * (fewer than 512 sequence x kv head x split triples).  The first call on a
 * device looks up the array's address there, so it must be made outside stream
 * capture (under capture it returns ATF_ERR_INVALID and launches nothing);
 * later calls may be captured.  The current device must be the stream's
 * (ATF_ERR_INVALID otherwise).  Every call on a GPU shares that GPU's scratch:
 * calls that overlap on one GPU (different streams, other threads) race.
 */
int atf_decode_paged_bf16_noalloc(void* out, int64_t o_sb, int64_t o_sh,
                                  const void* q, int64_t q_sb, int64_t q_sh,
                                  const void* kv_cache, int num_pages,
                                  const int32_t* page_table, int max_pages, const int32_t* seq_lens,
                                  int batch, int num_q_heads, int num_kv_heads, int max_seq_len,
                                  const int32_t* zhi, float sm_scale, const float* rope_cs, int rope_max_pos,
                                  int layout, void* stream);

/*
 * Measurement only; no counterpart in the reference.  Runs the prefill
 * kernel's matrix-core work for a causal window-OFF prefill of nq tokens and
 * num_q_heads q heads (one sequence) with nothing else: the same grid, waves,
 * LDS operand ring, MFMA order, priorities and barriers, but no softmax, no
 * K/V staging and random operands.  Its time beside atf_prefill_bf16's at the
 * same shape measures the ceiling of the kernel's structure at the clock the
 * part runs it at.  sink: device fp32 of ceil(ceil(nq / 256) / 8) * 8 *
 * num_q_heads * 512 elements (overwritten).
 */
int atf_prefill_mfma_probe(float* sink, int nq, int num_q_heads, void* stream);

/*
 * Measurement only; no counterpart in the reference.  Streams the bytes a
 * decode of this shape reads (the same split grid as atf_decode_paged_bf16,
 * always as 8-wave workgroups -- the decode's own shape wherever its splits
 * hold 32 pages or more, as at 128K -- the same page-table fetches and
 * range-checked non-temporal page loads in 4-page groups: V and the K slices
 * that each page's youngest key reads under zhi_slice, a HOST int32
 * [ATF_SLICES] table as in atf_decode_paged_slices_bf16, or NULL for window
 * OFF; a level table reads the same bytes as the slice table holding each
 * level's entry twice) with the compute replaced by an XOR of the loaded
 * words, and no merge: the rate the memory system gives this access pattern,
 * for comparison with the decode call.  sink: device uint32, at least
 * batch x num_kv_heads x n_splits x 8 words (n_splits <= 256);
 * ATF_ERR_WORKSPACE if sink_bytes is smaller.
 */
int atf_decode_stream_probe(uint32_t* sink, size_t sink_bytes, const void* kv_cache,
                            int num_pages, const int32_t* page_table, int max_pages, const int32_t* seq_lens,
                            int batch, int num_kv_heads, int max_seq_len, const int32_t* zhi_slice,
                            void* stream);

/*
 * Per-tile level counts (D_eff / 16) as the kernels compute them, for tests of
 * the integer window path.  prefill: out int32 [n_row_tiles][n_kblocks] for
 * 32-row query tiles starting at q_offset + 32*i and 32-key blocks;
 * decode: out int32 [n_pages] for a sequence of length seq_len.
 * Mirror atflash/window_table.py deff_segments (79-102) at these tiles.
 */
int atf_prefill_tile_levels(int32_t* out, int n_row_tiles, int n_kblocks, int q_offset,
                            const int32_t* zhi, void* stream);
int atf_decode_page_levels(int32_t* out, int n_pages, int seq_len, const int32_t* zhi, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ATFLASH_H_ */
