// C ABI of the atflash HIP library: argument validation, table packing and
// kernel launches.  Declarations and documentation: include/atflash.h.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <string>

#include "../../include/atflash.h"
#include "atf_launch.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int ok() {
  g_last_error.clear();
  return ATF_OK;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(ATF_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
}

bool aligned(const void* p, size_t n) { return (reinterpret_cast<uintptr_t>(p) % n) == 0; }

// Window table -> kernel argument.  NULL = window OFF (every level at every
// distance).  Entries must be >= 0 and non-increasing, as zhi_table produces them.
// zhi[0] is the table's cap (D_eff >= 16 at every distance, so level 0 always
// reaches it, window_tables/atflash_window.py:85-108): a level whose true width
// exceeds the cap carries the cap instead, and would be dropped past it.  The
// cap must therefore cover the longest causal distance of the call
// (`longest`; the reference sets WIN_ZHI_CAP above every context it runs,
// e2e_pipeline/atflash_e2e_fafi.py:55-58); a shorter cap is refused rather than
// trimming levels the rule keeps.  longest < 0 skips the check.
int make_table(const int32_t* zhi, atf::LevelTable* t, int64_t longest) {
  for (int i = 0; i < atf::kLevels; ++i) t->zhi[i] = zhi ? zhi[i] : INT32_MAX;
  if (!zhi) return ATF_OK;
  for (int i = 0; i < atf::kLevels; ++i) {
    if (zhi[i] < 0) return fail(ATF_ERR_INVALID, "zhi[%d] = %d is negative", i, zhi[i]);
    if (i > 0 && zhi[i] > zhi[i - 1])
      return fail(ATF_ERR_INVALID, "zhi must be non-increasing (zhi[%d]=%d > zhi[%d]=%d)", i, zhi[i], i - 1,
                  zhi[i - 1]);
  }
  if (longest >= 0 && zhi[0] < longest)
    return fail(ATF_ERR_INVALID,
                "window table cap zhi[0] = %d is below the longest causal distance %lld of this call; build the "
                "table with n_ctx >= the context length",
                zhi[0], static_cast<long long>(longest));
  return ATF_OK;
}

// Level table -> the decode kernel's arguments (page rule); the slice table
// holds each level's entry on its two 8-dim slices.
int make_decode_table_levels(const int32_t* zhi, atf::DecodeArgs* a, int64_t longest) {
  if (int r = make_table(zhi, &a->lt, longest)) return r;
  for (int s = 0; s < atf::kSlices; ++s) a->st.zhi[s] = a->lt.zhi[s / 2];
  a->per_key = 0;
  return ATF_OK;
}

// Per-slice (vec8) table of the FlashInfer window port -> kernel argument,
// per-key rule (kernels/flashinfer_port/decode.cuh.diff:47-89).  NULL = window
// OFF.  Entries must be >= 0 and non-increasing (slices in wavelength order, as
// zhi_slice_vec8 produces them), so that a page's slices are a prefix.  No
// slice is always read: a key past every slice scores 0, as in the port.
int make_decode_table_slices(const int32_t* zhi8, atf::DecodeArgs* a) {
  for (int s = 0; s < atf::kSlices; ++s) a->st.zhi[s] = zhi8 ? zhi8[s] : INT32_MAX;
  for (int l = 0; l < atf::kLevels; ++l) a->lt.zhi[l] = INT32_MAX;
  a->per_key = zhi8 ? 1 : 0;  // window OFF runs the level path with every level
  if (!zhi8) return ATF_OK;
  for (int s = 0; s < atf::kSlices; ++s) {
    if (zhi8[s] < 0) return fail(ATF_ERR_INVALID, "zhi_slice[%d] = %d is negative", s, zhi8[s]);
    if (s > 0 && zhi8[s] > zhi8[s - 1])
      return fail(ATF_ERR_INVALID, "zhi_slice must be non-increasing (zhi_slice[%d]=%d > zhi_slice[%d]=%d)", s,
                  zhi8[s], s - 1, zhi8[s - 1]);
  }
  return ATF_OK;
}

int check_layout(int layout, const float* rope_cs, int rope_max_pos) {
  if (layout != ATF_LAYOUT_HALF_SPLIT && layout != ATF_LAYOUT_SORTED_PAIR)
    return fail(ATF_ERR_INVALID, "unknown layout %d", layout);
  if (layout == ATF_LAYOUT_SORTED_PAIR && rope_cs)
    return fail(ATF_ERR_INVALID, "RoPE at load needs the half-split layout (sorted-pair inputs are pre-rotated)");
  if (rope_cs && !aligned(rope_cs, 16)) return fail(ATF_ERR_INVALID, "rope_cs must be 16-byte aligned");
  if (rope_cs && rope_max_pos <= 0) return fail(ATF_ERR_INVALID, "rope_max_pos must be positive");
  return ATF_OK;
}

void decode_split(int batch, int hkv, int max_seq_len, int* n_splits, int* pages_per_split, int* waves) {
  const int pages = max_seq_len > 0 ? (max_seq_len + atf::kPage - 1) / atf::kPage : 1;
  // one workgroup per CU over 256 CUs; at least one 4-page group per wave.
  // Workgroups of 8 waves, unless their 32-page minimum leaves fewer splits
  // than the target while there are several anyway: then 4 waves, whose
  // 16-page minimum spreads the context over up to twice as many CUs
  // (Llama-3.2-3B shape at 8K: 128 -> 256 workgroups, -12% per call).  A
  // context that fits one 8-wave split keeps it (a second split would add the
  // merge kernel).
  const int target_wgs = 256;
  int ns = (target_wgs + batch * hkv - 1) / (batch * hkv);
  if (ns < 1) ns = 1;
  const int splits8 = (pages + atf::kDecUnroll * atf::kDecWaves - 1) / (atf::kDecUnroll * atf::kDecWaves);
  const int w = (splits8 < ns && splits8 >= 2) ? atf::kDecWavesShort : atf::kDecWaves;
  const int min_pps = atf::kDecUnroll * w;
  *waves = w;
  int pps = (pages + ns - 1) / ns;
  if (pps < min_pps) pps = min_pps;
  if ((pages + pps - 1) / pps > atf::kDecMaxSplits) pps = (pages + atf::kDecMaxSplits - 1) / atf::kDecMaxSplits;
  *pages_per_split = pps;
  *n_splits = (pages + pps - 1) / pps;
}

// Bytes of split partials ([ws_ml][ws_o], fp32): none with one split.
size_t partial_bytes(int batch, int hkv, int ns) {
  if (ns <= 1) return 0;
  return static_cast<size_t>(batch) * hkv * ns * atf::kDecMaxGroup * (atf::kD + 2) * sizeof(float);
}

}  // namespace

extern "C" {

int atf_abi_version(void) { return ATF_ABI_VERSION; }

const char* atf_last_error(void) { return g_last_error.c_str(); }

int atf_kv_write_bf16(void* kv_cache, int num_pages, int num_kv_heads, const void* k_src,
                      int64_t ks_b, int64_t ks_t, int64_t ks_h, const void* v_src, int64_t vs_b, int64_t vs_t,
                      int64_t vs_h, int batch, int n_tokens, const int32_t* start_pos, const int32_t* page_table,
                      int max_pages, const float* rope_cs, int rope_max_pos, int layout, void* stream) {
  if (batch < 0 || n_tokens < 0) return fail(ATF_ERR_INVALID, "batch and n_tokens must be >= 0");
  if (batch == 0 || n_tokens == 0) return ok();
  if (!kv_cache || !k_src || !v_src || !start_pos || !page_table)
    return fail(ATF_ERR_INVALID, "null pointer argument");
  if (num_pages <= 0 || num_kv_heads <= 0 || max_pages <= 0)
    return fail(ATF_ERR_INVALID, "num_pages, num_kv_heads and max_pages must be positive");
  if (int r = check_layout(layout, rope_cs, rope_max_pos)) return r;
  if (!aligned(k_src, 16) || !aligned(v_src, 16) || !aligned(kv_cache, 16))
    return fail(ATF_ERR_INVALID, "k/v sources and kv_cache must be 16-byte aligned");
  const int64_t strides[6] = {ks_b, ks_t, ks_h, vs_b, vs_t, vs_h};
  for (int64_t s : strides)
    if (s % 8 != 0) return fail(ATF_ERR_INVALID, "source strides must be multiples of 8 elements");
  atf::KvWriteArgs a{};
  a.kv_cache = static_cast<uint16_t*>(kv_cache);
  a.num_pages = num_pages;
  a.hkv = num_kv_heads;
  a.k_src = static_cast<const uint16_t*>(k_src);
  a.v_src = static_cast<const uint16_t*>(v_src);
  a.ks_b = ks_b; a.ks_t = ks_t; a.ks_h = ks_h;
  a.vs_b = vs_b; a.vs_t = vs_t; a.vs_h = vs_h;
  a.batch = batch;
  a.n_tokens = n_tokens;
  a.start_pos = start_pos;
  a.page_table = page_table;
  a.max_pages = max_pages;
  a.rope_cs = rope_cs;
  a.rope_max_pos = rope_max_pos;
  a.layout = layout;
  hipError_t e = atf::launch_kv_write(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "kv_write launch");
  return ok();
}

int atf_prefill_bf16(void* out, int64_t o_sb, int64_t o_st, int64_t o_sh, float* lse, const void* q,
                     int64_t q_sb, int64_t q_st, int64_t q_sh, const void* kv_cache,
                     int num_pages, const int32_t* page_table, int max_pages, int batch, int nq, int nk,
                     int q_offset, int num_q_heads, int num_kv_heads, const int32_t* zhi, float sm_scale,
                     const float* rope_cs, int rope_max_pos, int layout, void* stream) {
  if (batch < 0 || nq < 0) return fail(ATF_ERR_INVALID, "batch and nq must be >= 0");
  if (batch == 0 || nq == 0) return ok();
  if (!out || !q || !kv_cache || !page_table) return fail(ATF_ERR_INVALID, "null pointer argument");
  if (num_q_heads <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads != 0)
    return fail(ATF_ERR_INVALID, "num_q_heads (%d) must be a positive multiple of num_kv_heads (%d)", num_q_heads,
                num_kv_heads);
  if (q_offset < 0 || nk < q_offset + nq)
    return fail(ATF_ERR_INVALID, "need 0 <= q_offset and q_offset + nq <= nk (q_offset=%d nq=%d nk=%d)", q_offset,
                nq, nk);
  if (nk >= (1 << 24)) return fail(ATF_ERR_UNSUPPORTED, "nk must be < 2^24");
  if (num_pages <= 0 || max_pages <= 0 || static_cast<int64_t>(max_pages) * atf::kPage < nk)
    return fail(ATF_ERR_INVALID, "page table too small for nk=%d (max_pages=%d)", nk, max_pages);
  if (!(sm_scale > 0.f) || !std::isfinite(sm_scale)) return fail(ATF_ERR_INVALID, "sm_scale must be positive");
  if (int r = check_layout(layout, rope_cs, rope_max_pos)) return r;
  if (rope_cs && q_offset + nq > rope_max_pos)
    return fail(ATF_ERR_INVALID, "rope table has %d positions, need %d", rope_max_pos, q_offset + nq);
  if (!aligned(q, 16) || !aligned(out, 8) || !aligned(kv_cache, 16))
    return fail(ATF_ERR_INVALID, "q and kv_cache must be 16-byte and out 8-byte aligned");
  if (q_sb % 8 || q_st % 8 || q_sh % 8) return fail(ATF_ERR_INVALID, "q strides must be multiples of 8 elements");
  if (o_sb % 4 || o_st % 4 || o_sh % 4) return fail(ATF_ERR_INVALID, "out strides must be multiples of 4 elements");
  atf::PrefillArgs a{};
  if (int r = make_table(zhi, &a.lt, static_cast<int64_t>(nk) - 1)) return r;
  a.q = static_cast<const uint16_t*>(q);
  a.q_sb = q_sb; a.q_st = q_st; a.q_sh = q_sh;
  a.out = static_cast<uint16_t*>(out);
  a.o_sb = o_sb; a.o_st = o_st; a.o_sh = o_sh;
  a.lse = lse;
  a.kv_cache = static_cast<const uint16_t*>(kv_cache);
  a.num_pages = num_pages;
  a.page_table = page_table;
  a.max_pages = max_pages;
  a.batch = batch;
  a.nq = nq;
  a.nk = nk;
  a.q_offset = q_offset;
  a.hq = num_q_heads;
  a.hkv = num_kv_heads;
  a.group = num_q_heads / num_kv_heads;
  a.n_qtiles = (nq + atf::kPfRowsWg - 1) / atf::kPfRowsWg;
  a.n_qgroups = (a.n_qtiles + 7) / 8;
  a.sm_scale = sm_scale;
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  a.rope_cs = rope_cs;
  a.layout = layout;
  hipError_t e = atf::launch_prefill(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "prefill launch");
  return ok();
}

size_t atf_decode_workspace_bytes(int batch, int num_q_heads, int num_kv_heads, int max_seq_len) {
  (void)num_q_heads;
  if (batch <= 0 || num_kv_heads <= 0) return 0;
  int ns = 1, pps = 1, waves = 0;
  decode_split(batch, num_kv_heads, max_seq_len, &ns, &pps, &waves);
  return partial_bytes(batch, num_kv_heads, ns);
}

}  // extern "C"

namespace {

// Validation and argument packing shared by the two decode entry points
// (everything except the workspace).
int decode_prepare(void* out, int64_t o_sb, int64_t o_sh, const void* q, int64_t q_sb, int64_t q_sh,
                   const void* kv_cache, int num_pages, const int32_t* page_table, int max_pages,
                   const int32_t* seq_lens, int batch, int num_q_heads, int num_kv_heads, int max_seq_len,
                   const int32_t* zhi, bool slice_table, float sm_scale, const float* rope_cs, int rope_max_pos,
                   int layout, atf::DecodeArgs* a) {
  if (!out || !q || !kv_cache || !page_table || !seq_lens)
    return fail(ATF_ERR_INVALID, "null pointer argument");
  if (num_q_heads <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads != 0)
    return fail(ATF_ERR_INVALID, "num_q_heads (%d) must be a positive multiple of num_kv_heads (%d)", num_q_heads,
                num_kv_heads);
  if (num_q_heads / num_kv_heads > atf::kDecMaxGroup)
    return fail(ATF_ERR_UNSUPPORTED, "GQA group %d > %d", num_q_heads / num_kv_heads, atf::kDecMaxGroup);
  if (max_seq_len <= 0 || max_seq_len >= (1 << 24)) return fail(ATF_ERR_INVALID, "max_seq_len out of range");
  if (num_pages <= 0 || max_pages <= 0 || static_cast<int64_t>(max_pages) * atf::kPage < max_seq_len)
    return fail(ATF_ERR_INVALID, "page table too small for max_seq_len=%d (max_pages=%d)", max_seq_len, max_pages);
  if (!(sm_scale > 0.f) || !std::isfinite(sm_scale)) return fail(ATF_ERR_INVALID, "sm_scale must be positive");
  if (int r = check_layout(layout, rope_cs, rope_max_pos)) return r;
  if (rope_cs && max_seq_len > rope_max_pos)
    return fail(ATF_ERR_INVALID, "rope table has %d positions, need %d", rope_max_pos, max_seq_len);
  if (!aligned(q, 16) || !aligned(out, 8) || !aligned(kv_cache, 16))
    return fail(ATF_ERR_INVALID, "q and kv_cache must be 16-byte and out 8-byte aligned");
  if (q_sb % 8 || q_sh % 8) return fail(ATF_ERR_INVALID, "q strides must be multiples of 8 elements");
  if (o_sb % 4 || o_sh % 4) return fail(ATF_ERR_INVALID, "out strides must be multiples of 4 elements");
  if (int r = slice_table ? make_decode_table_slices(zhi, a)
                          : make_decode_table_levels(zhi, a, static_cast<int64_t>(max_seq_len) - 1))
    return r;
  int ns = 1, pps = 1, waves = 0;
  decode_split(batch, num_kv_heads, max_seq_len, &ns, &pps, &waves);
  a->waves = waves;
  a->q = static_cast<const uint16_t*>(q);
  a->q_sb = q_sb;
  a->q_sh = q_sh;
  a->kv_cache = static_cast<const uint16_t*>(kv_cache);
  a->num_pages = num_pages;
  a->page_table = page_table;
  a->max_pages = max_pages;
  a->seq_lens = seq_lens;
  a->max_seq_len = max_seq_len;
  a->batch = batch;
  a->hq = num_q_heads;
  a->hkv = num_kv_heads;
  a->group = num_q_heads / num_kv_heads;
  a->n_splits = ns;
  a->pages_per_split = pps;
  a->scale_log2 = sm_scale * 1.4426950408889634f;
  a->rope_cs = rope_cs;
  a->layout = layout;
  a->out = static_cast<uint16_t*>(out);
  a->o_sb = o_sb;
  a->o_sh = o_sh;
  return ATF_OK;
}

}  // namespace

namespace {

// Decode with a caller-provided workspace, either table kind.
int decode_with_workspace(void* out, int64_t o_sb, int64_t o_sh, const void* q, int64_t q_sb, int64_t q_sh,
                          const void* kv_cache, int num_pages, const int32_t* page_table,
                          int max_pages, const int32_t* seq_lens, int batch, int num_q_heads, int num_kv_heads,
                          int max_seq_len, const int32_t* zhi, bool slice_table, float sm_scale,
                          const float* rope_cs, int rope_max_pos, int layout, void* workspace,
                          size_t workspace_bytes, void* stream) {
  if (batch < 0) return fail(ATF_ERR_INVALID, "batch must be >= 0");
  if (batch == 0) return ok();
  atf::DecodeArgs a{};
  if (int r = decode_prepare(out, o_sb, o_sh, q, q_sb, q_sh, kv_cache, num_pages, page_table, max_pages,
                             seq_lens, batch, num_q_heads, num_kv_heads, max_seq_len, zhi, slice_table, sm_scale,
                             rope_cs, rope_max_pos, layout, &a))
    return r;
  const size_t need = partial_bytes(batch, num_kv_heads, a.n_splits);
  if (need > 0 && (!workspace || workspace_bytes < need || !aligned(workspace, 16)))
    return fail(ATF_ERR_WORKSPACE, "workspace of %zu bytes (16-byte aligned) required, got %zu", need,
                workspace ? workspace_bytes : 0);
  a.ws_ml = static_cast<float*>(workspace);
  a.ws_o = need > 0 ? a.ws_ml + static_cast<size_t>(batch) * num_kv_heads * a.n_splits * atf::kDecMaxGroup * 2
                    : nullptr;
  hipError_t e = atf::launch_decode(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "decode launch");
  return ok();
}

}  // namespace

extern "C" {

int atf_decode_paged_bf16(void* out, int64_t o_sb, int64_t o_sh, const void* q, int64_t q_sb, int64_t q_sh,
                          const void* kv_cache, int num_pages, const int32_t* page_table,
                          int max_pages, const int32_t* seq_lens, int batch, int num_q_heads, int num_kv_heads,
                          int max_seq_len, const int32_t* zhi, float sm_scale, const float* rope_cs,
                          int rope_max_pos, int layout, void* workspace, size_t workspace_bytes, void* stream) {
  return decode_with_workspace(out, o_sb, o_sh, q, q_sb, q_sh, kv_cache, num_pages, page_table, max_pages,
                               seq_lens, batch, num_q_heads, num_kv_heads, max_seq_len, zhi, false, sm_scale,
                               rope_cs, rope_max_pos, layout, workspace, workspace_bytes, stream);
}

int atf_decode_paged_slices_bf16(void* out, int64_t o_sb, int64_t o_sh, const void* q, int64_t q_sb, int64_t q_sh,
                                 const void* kv_cache, int num_pages, const int32_t* page_table,
                                 int max_pages, const int32_t* seq_lens, int batch, int num_q_heads,
                                 int num_kv_heads, int max_seq_len, const int32_t* zhi_slice, float sm_scale,
                                 const float* rope_cs, int rope_max_pos, int layout, void* workspace,
                                 size_t workspace_bytes, void* stream) {
  return decode_with_workspace(out, o_sb, o_sh, q, q_sb, q_sh, kv_cache, num_pages, page_table, max_pages,
                               seq_lens, batch, num_q_heads, num_kv_heads, max_seq_len, zhi_slice, true, sm_scale,
                               rope_cs, rope_max_pos, layout, workspace, workspace_bytes, stream);
}

int atf_decode_paged_bf16_noalloc(void* out, int64_t o_sb, int64_t o_sh, const void* q, int64_t q_sb, int64_t q_sh,
                                  const void* kv_cache, int num_pages,
                                  const int32_t* page_table, int max_pages, const int32_t* seq_lens, int batch,
                                  int num_q_heads, int num_kv_heads, int max_seq_len, const int32_t* zhi,
                                  float sm_scale, const float* rope_cs, int rope_max_pos, int layout, void* stream) {
  if (batch < 0) return fail(ATF_ERR_INVALID, "batch must be >= 0");
  if (batch == 0) return ok();
  atf::DecodeArgs a{};
  if (int r = decode_prepare(out, o_sb, o_sh, q, q_sb, q_sh, kv_cache, num_pages, page_table, max_pages,
                             seq_lens, batch, num_q_heads, num_kv_heads, max_seq_len, zhi, false, sm_scale,
                             rope_cs, rope_max_pos, layout, &a))
    return r;
  const size_t partial = partial_bytes(batch, num_kv_heads, a.n_splits);
  if (partial > atf::kDecScratchBytes)
    return fail(ATF_ERR_UNSUPPORTED,
                "decode without allocation: %d x %d sequence x kv head pairs need %zu bytes of split partials; the "
                "fixed scratch holds %zu (use atf_decode_paged_bf16 with a workspace)",
                batch, num_kv_heads, partial, atf::kDecScratchBytes);
  // The scratch used is the current device's: the stream must belong to it.
  int dev = 0;
  if (hipError_t e = hipGetDevice(&dev); e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (stream != nullptr) {
    hipDevice_t sdev = 0;
    if (hipError_t e = hipStreamGetDevice(static_cast<hipStream_t>(stream), &sdev); e != hipSuccess)
      return hip_fail(e, "hipStreamGetDevice");
    if (sdev != dev)
      return fail(ATF_ERR_INVALID,
                  "decode without allocation: the stream belongs to device %d but device %d is current; make the "
                  "stream's device current first",
                  static_cast<int>(sdev), dev);
  }
  hipError_t e = atf::launch_decode_noalloc(a, static_cast<hipStream_t>(stream));
  if (e == hipErrorStreamCaptureUnsupported)
    return fail(ATF_ERR_INVALID,
                "decode without allocation: the first call on device %d was made under stream capture; make one "
                "call on each device outside capture first (it looks up the device's scratch address)",
                dev);
  if (e != hipSuccess) return hip_fail(e, "decode (no allocation) launch");
  return ok();
}

int atf_prefill_mfma_probe(float* sink, int nq, int num_q_heads, void* stream) {
  if (!sink || nq <= 0 || nq >= (1 << 24) || num_q_heads <= 0) return fail(ATF_ERR_INVALID, "bad arguments");
  hipError_t e = atf::launch_prefill_mfma_probe(sink, nq, num_q_heads, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "probe launch");
  return ok();
}

int atf_decode_stream_probe(uint32_t* sink, size_t sink_bytes, const void* kv_cache,
                            int num_pages, const int32_t* page_table, int max_pages, const int32_t* seq_lens,
                            int batch, int num_kv_heads, int max_seq_len, const int32_t* zhi_slice, void* stream) {
  if (!sink || !kv_cache || !page_table || !seq_lens) return fail(ATF_ERR_INVALID, "null pointer argument");
  if (batch <= 0 || num_kv_heads <= 0 || max_seq_len <= 0 || max_seq_len >= (1 << 24) || num_pages <= 0 ||
      max_pages <= 0 || static_cast<int64_t>(max_pages) * atf::kPage < max_seq_len)
    return fail(ATF_ERR_INVALID, "bad arguments");
  if (!aligned(kv_cache, 16)) return fail(ATF_ERR_INVALID, "kv_cache must be 16-byte aligned");
  atf::DecodeArgs a{};
  if (int r = make_decode_table_slices(zhi_slice, &a)) return r;
  int ns = 1, pps = 1, waves = 0;
  decode_split(batch, num_kv_heads, max_seq_len, &ns, &pps, &waves);
  const size_t need = static_cast<size_t>(batch) * num_kv_heads * ns * atf::kDecWaves * sizeof(uint32_t);
  if (sink_bytes < need) return fail(ATF_ERR_WORKSPACE, "probe sink of %zu bytes required, got %zu", need, sink_bytes);
  a.kv_cache = static_cast<const uint16_t*>(kv_cache);
  a.num_pages = num_pages;
  a.page_table = page_table;
  a.max_pages = max_pages;
  a.seq_lens = seq_lens;
  a.max_seq_len = max_seq_len;
  a.batch = batch;
  a.hkv = num_kv_heads;
  a.n_splits = ns;
  a.pages_per_split = pps;
  hipError_t e = atf::launch_decode_stream_probe(a, sink, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "probe launch");
  return ok();
}

int atf_prefill_tile_levels(int32_t* out, int n_row_tiles, int n_kblocks, int q_offset, const int32_t* zhi,
                            void* stream) {
  if (!out || n_row_tiles < 0 || n_kblocks < 0 || q_offset < 0) return fail(ATF_ERR_INVALID, "bad arguments");
  atf::LevelTable t{};
  if (int r = make_table(zhi, &t, -1)) return r;
  hipError_t e = atf::launch_prefill_tile_levels(out, n_row_tiles, n_kblocks, q_offset, t,
                                                 static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "tile levels launch");
  return ok();
}

int atf_decode_page_levels(int32_t* out, int n_pages, int seq_len, const int32_t* zhi, void* stream) {
  if (!out || n_pages < 0 || seq_len < 0) return fail(ATF_ERR_INVALID, "bad arguments");
  atf::LevelTable t{};
  if (int r = make_table(zhi, &t, -1)) return r;
  hipError_t e = atf::launch_decode_page_levels(out, n_pages, seq_len, t, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "page levels launch");
  return ok();
}

}  // extern "C"
