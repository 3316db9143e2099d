// Kernel argument blocks and host-side launchers (one per kernel file).
#pragma once
#include "atf_common.h"

namespace atf {

// Prefill geometry (the oracle's tile quantization is block_m = kPfRowsWave
// query positions by block_n = kPfWinN keys).  8 waves of 32 rows: at most 256
// registers per wave, so two waves share each SIMD and one wave's softmax
// overlaps the other's MFMAs.
constexpr int kPfWaves = 8;
constexpr int kPfRowsWave = 32;
constexpr int kPfRowsWg = kPfWaves * kPfRowsWave;
constexpr int kPfTileN = 64;
constexpr int kPfWinN = 32;

// Decode geometry (block_n = one page).
constexpr int kDecMaxGroup = 16;
constexpr int kDecUnroll = 4;      // pages in flight per wave
constexpr int kDecWaves = 8;       // waves per workgroup (one split), 2 per SIMD
constexpr int kDecWavesShort = 4;  // the same for contexts too short to give 256 splits of 8 waves
constexpr int kDecMaxSplits = 256;
// Fixed device scratch of the entry point that allocates nothing
// (atf_decode_paged_bf16_noalloc): split partials, laid out as in a workspace.
constexpr size_t kDecScratchBytes = size_t(8) << 20;

struct KvWriteArgs {
  uint16_t* kv_cache;  // [num_pages][hkv][V half | K half]
  int num_pages, hkv;
  const uint16_t* k_src;
  const uint16_t* v_src;
  int64_t ks_b, ks_t, ks_h, vs_b, vs_t, vs_h;
  int batch, n_tokens;
  const int32_t* start_pos;  // [batch], absolute position of source token 0
  const int32_t* page_table;
  int max_pages;
  const float* rope_cs;
  int rope_max_pos;
  int layout;
};

struct PrefillArgs {
  const uint16_t* q;
  int64_t q_sb, q_st, q_sh;
  uint16_t* out;
  int64_t o_sb, o_st, o_sh;
  float* lse;  // [B][Hq][nq] natural-log LSE, or null
  const uint16_t* kv_cache;  // [num_pages][hkv][V half | K half]
  int num_pages;
  int xcd_alt;  // serpentine XCD order (set by launch_prefill; fills the padding before page_table)
  const int32_t* page_table;
  int max_pages;
  int batch, nq, nk, q_offset, hq, hkv, group;
  int n_qtiles, n_qgroups;
  float scale_log2;
  float sm_scale;
  const float* rope_cs;
  int layout;
  LevelTable lt;
};

struct DecodeArgs {
  const uint16_t* q;  // [B][Hq][128] (strided)
  int64_t q_sb, q_sh;
  uint16_t* out;  // [B][Hq][128] (strided)
  int64_t o_sb, o_sh;
  const uint16_t* kv_cache;  // [num_pages][hkv][V half | K half]
  int num_pages;
  const int32_t* page_table;
  int max_pages;
  const int32_t* seq_lens;
  int max_seq_len;
  int batch, hq, hkv, group;
  int n_splits, pages_per_split;
  int waves;  // kDecWaves or kDecWavesShort per workgroup
  float scale_log2;
  const float* rope_cs;
  int layout;
  // Window.  per_key = 0: the level table lt, page rule (block_n = 16): every
  // key of a page reads the 2 L levels' slices of its youngest key, L >= 1.
  // per_key = 1: the per-slice (vec8) table st, slice s of a key at age z read
  // iff z <= st.zhi[s] (the FlashInfer port's rule, no minimum).
  LevelTable lt;
  SliceTable st;
  int per_key;
  float* ws_ml;        // [B][Hkv][n_splits][16][2]   split partials (n_splits > 1)
  float* ws_o;         // [B][Hkv][n_splits][16][128]
};

hipError_t launch_kv_write(const KvWriteArgs& a, hipStream_t s);
int prefill_xcd_alternate(int n_qtiles, int nq, int nk, int q_offset);
hipError_t launch_prefill(const PrefillArgs& a, hipStream_t s);
// The MFMA-ceiling probe of the prefill (measurement only): sink holds
// ceil(ceil(nq / 256) / 8) * 8 * hq * 512 floats.
hipError_t launch_prefill_mfma_probe(float* sink, int nq, int hq, hipStream_t s);
hipError_t launch_prefill_tile_levels(int32_t* out, int n_row_tiles, int n_kblocks, int q_offset,
                                      const LevelTable& lt, hipStream_t s);
hipError_t launch_decode(const DecodeArgs& a, hipStream_t s);
// launch_decode with the workspace pointers taken from the device's fixed
// scratch (a.ws_ml and a.ws_o are set here).
hipError_t launch_decode_noalloc(DecodeArgs a, hipStream_t s);
// The streaming probe of the decode (measurement only): 8-wave workgroups
// over a.n_splits x a.hkv x a.batch; sink holds one word per wave.
hipError_t launch_decode_stream_probe(const DecodeArgs& a, uint32_t* sink, hipStream_t s);
hipError_t launch_decode_page_levels(int32_t* out, int n_pages, int seq_len, const LevelTable& lt,
                                     hipStream_t s);

}  // namespace atf
