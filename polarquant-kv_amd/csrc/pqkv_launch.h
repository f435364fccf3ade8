// Host-side launcher declarations shared by the C-ABI layer (pqkv_api.cpp)
// and the kernel translation units. Arguments reaching these functions have
// already been validated.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/pqkv.h"
#include "pqkv_layout.h"

namespace pqkv {

constexpr int kMaxListHeads = PQKV_MAX_HEADS;  // kv heads per launch when heads are listed
constexpr int kMaxSplits = 1024;   // split-K partitions per (batch, kv head)
constexpr int kMergeHeads = 4;     // query heads per merge workgroup
constexpr int kMfmaBlocksPerCU = 2;  // decode_mfma_kernel workgroups resident per CU
constexpr int kMaxGroup = 8;         // query heads per kv head in one decode launch
// The prefill kernel's rotated queries and codebook planes carry this factor
// (fp16 hi / lo parts stay normal numbers); it divides out exactly.
constexpr float kPrefillPlaneScale = 64.0f;

struct EncodeArgs {
  const void *x;
  int64_t x_outer_stride;      // elements
  const float *R;
  const float *codebook;
  int bits;
  uint8_t *blocks;
  int64_t blocks_outer_stride; // bytes
  int64_t n_outer, n_inner;
  int d;
  const float *p_rot;          // [m][d] or null
  int m;
  uint8_t *qjl;                // or null
  int64_t qjl_outer_stride;    // bytes
  // Paged output (pages != null; blocks and the outer strides unused): vector
  // (o, i) is position page_start + i of stream o, stored as vector
  // (pos & (2^page_shift - 1)) of page pages[o * max_pages + (pos >> page_shift)];
  // its signs likewise in qjl_pages.
  uint8_t *const *pages;
  uint8_t *const *qjl_pages;
  int page_shift, max_pages;
  int64_t page_start;
};

// Output address of vector (o, i) of an encode: row o of the blocks (or
// signs) `stride` bytes apart, or (paged) its page slot; vb bytes per vector.
__device__ __forceinline__ uint8_t *encode_out_addr(const EncodeArgs &a, uint8_t *base, uint8_t *const *pages,
                                                    int64_t stride, int64_t o, int64_t i, int vb) {
  if (a.pages == nullptr) return base + o * stride + i * vb;
  const int64_t pos = a.page_start + i;
  return pages[o * a.max_pages + (pos >> a.page_shift)] + (pos & ((1 << a.page_shift) - 1)) * vb;
}

// One launch of the split-K decode kernel covers B x n_heads (batch, kv-head)
// streams with the same K and V bit widths.
struct DecodeArgs {
  const float *q;                // [B][Hq][d] fp32, rotated, times scale*log2(e)
  const uint8_t *k_cache, *v_cache;
  int64_t k_batch_stride, v_batch_stride;   // bytes between batches
  int64_t k_head_stride, v_head_stride;     // bytes between heads (uniform mode)
  const float *k_cb, *v_cb;      // codebook(s)
  int cb_head_stride;            // 0: one table; 16: per-head tables
  int cb_levels;                 // entries of each table (16, or fewer in the SoA layout)
  const float *k_rad, *v_rad;    // SoA layout only: fp32 radii, [B][Hkv][S_max]
  const uint8_t *qjl;            // [B][Hkv][S_max][m/8] or null
  const float *p_rot;            // [m][d] (QJL only)
  const float *pq;               // [B][Hq][m] = P_rot q / m (QJL only)
  float *part;                   // [B][Hq][split_stride][d + 2]
  int B, Hq, Hkv, S, S_max, d;
  int gq;                        // query heads per kv head (Hq / Hkv)
  int q_off, g;                  // this launch: query heads q_off .. q_off + g - 1 of each kv head (g <= kMaxGroup)
  int splits, tokens_per_split;
  int split_base, split_stride;  // this launch's splits are partials split_base .. of split_stride per query head
  int n_heads;                   // heads in this launch
  int listed;                    // 1: heads / offsets below are used
  // ggml layout (launch_decode_mfma_ggml only): bytes between consecutive
  // tokens of a stream; batch rows per key / value sequence (the sequence
  // of row b is b / rows_per_seq, k_batch_stride apart); fp16 additive mask
  // [seq][row][S] with element strides, or null.
  int64_t k_tok_stride, v_tok_stride;
  int rows_per_seq;
  const uint16_t *mask;
  int64_t mask_row_stride, mask_seq_stride;
  // Paged caches (the kernels' PG mode; k_cache / v_cache / qjl unused):
  // position t of stream s = b * Hkv + h is vector t & (2^page_shift - 1) of
  // page k_pages[s * max_pages + (t >> page_shift)] (v_pages, and the sign
  // pages s_pages, alike); page_shift >= 6, so a 64-token chunk lies in one page.
  const uint8_t *const *k_pages, *const *v_pages, *const *s_pages;
  int page_shift, max_pages;
  int16_t heads[kMaxListHeads];
  int64_t k_head_off[kMaxListHeads], v_head_off[kMaxListHeads];
};

// One launch of the chunked-prefill kernel: workgroups of prefill_rows(qjl)
// query rows (qt tokens x G heads) of one (batch, kv-head) with the same key
// and value widths; with listed = 1 the kv heads and their byte offsets
// come from the tables below (mixed widths), as in DecodeArgs.
struct PrefillArgs {
  const float *q;                // [B][Hq][Sq][d] fp32, rotated, times scale*log2(e)*kPrefillPlaneScale
  const uint8_t *k_cache, *v_cache;
  int64_t k_batch_stride, v_batch_stride;   // bytes between batches
  int64_t k_head_stride, v_head_stride;     // bytes between heads (listed = 0)
  const float *k_cb, *v_cb;      // [16], or per-head [Hkv][16] with cb_head_stride 16
  int cb_head_stride;
  const uint8_t *qjl;            // [B][Hkv][S_max][d/8] or null
  const float *pq;               // [B][Hq][Sq][d] = P_rot q_rot / m (QJL only)
  float *o;                      // [B][Hq][Sq][d] fp32, rotated, normalised
  int B, Hq, Hkv, G, Sq, q_start, S, S_max, d, causal;
  int qt;                        // query tokens per workgroup (rows / G)
  int n_heads, listed;
  // Paged caches (k_pages != null; k_cache / v_cache / qjl unused), as in
  // DecodeArgs: a 64-token tile lies in one page.
  const uint8_t *const *k_pages, *const *v_pages, *const *s_pages;
  int page_shift, max_pages;
  int16_t heads[kMaxListHeads];
  int64_t k_head_off[kMaxListHeads], v_head_off[kMaxListHeads];
};

// Workspace of one decode call whose plan has `splits` partitions per stream
// (rotated queries, split partials, QJL projections); returns the total
// bytes, the nullable pointers receive the three offsets.
size_t decode_workspace_layout(int B, int Hq, int splits, int d, size_t *q_off, size_t *part_off, size_t *pq_off);
// A 4-bit cache in the reference kernels' SoA layout: k_cache / v_cache hold
// the packed codes [B][Hkv][S_max][d/2], these the fp32 radii
// [B][Hkv][S_max]; the codebook has `levels` (<= 16) entries.
struct SoaCache {
  const float *k_rad, *v_rad;
  int levels;
};
// A paged cache (pqkv_*_paged): page address tables of B * Hkv * max_pages
// entries for keys, values and (nullable) QJL signs; pages of 2^page_shift
// tokens.
struct PagedCache {
  const uint8_t *const *k_pages, *const *v_pages, *const *s_pages;
  int page_shift, max_pages;
};
// The validated decode call behind pqkv_decode_attn (plan_sized = false: the
// workspace must hold pqkv_decode_workspace_bytes) and the allocation-free
// entry point (plan_sized = true: the workspace must hold this call's plan).
// soa (nullable): the caches are SoA; R may then be nullptr, meaning queries
// that are already rotated and a rotated output.
int decode_attn_run(const void *q, int q_dtype, const float *R, const uint8_t *k_cache, const uint8_t *v_cache,
                    const float *k_codebooks, const float *v_codebooks, int k_bits, int v_bits,
                    const int *k_head_bits, const int *v_head_bits, const uint8_t *qjl_signs, const float *p_rot,
                    int m, int B, int Hq, int Hkv, int S, int S_max, int d, float scale, void *out, int out_dtype,
                    void *workspace, size_t workspace_bytes, bool plan_sized, const SoaCache *soa,
                    void *stream, const PagedCache *pg = nullptr);
// The validated call behind pqkv_prefill_attn (pg: pqkv_prefill_attn_paged).
int prefill_attn_run(const void *q, int q_dtype, const float *R, const uint8_t *k_cache, const uint8_t *v_cache,
                     const float *k_codebooks, const float *v_codebooks, int k_bits, int v_bits,
                     const int *k_head_bits, const int *v_head_bits, const uint8_t *qjl_signs, const float *p_rot,
                     int m, int B, int Hq, int Hkv, int Sq, int q_start, int S, int S_max, int d, float scale,
                     int causal, void *out, int out_dtype, void *workspace, size_t workspace_bytes, void *stream,
                     const PagedCache *pg);
// The validated call behind pqkv_decode_attn_segments, and the split plans
// it makes (one per segment, sharing one partials layout; returns their
// total).
int segment_plans(int B, int Hkv, int n_seg, const int *S, int target, int *splits, int *tps);
int decode_segments_run(const void *q, int q_dtype, const float *R, int n_seg, const uint8_t *const *k_caches,
                        const uint8_t *const *v_caches, const float *const *k_codebooks,
                        const float *const *v_codebooks, const int *k_bits, const int *v_bits, const int *S,
                        const int *S_max, int B, int Hq, int Hkv, int d, float scale, void *out, int out_dtype,
                        void *workspace, size_t workspace_bytes, void *stream);

// Sets the thread's error message from a HIP error; returns PQKV_ERR_HIP
// (PQKV_OK for hipSuccess).
int report_hip_error(hipError_t e, const char *what);
// Sets the thread's error message (printf format); returns code.
int fail_status(int code, const char *fmt, ...);
// The matrix-core decode kernel's split plan for `streams` (batch, kv-head)
// streams of S tokens: one balanced round of workgroups.
void mfma_split_plan(int64_t streams, int S, int *splits, int *tps);

// Event brackets for the measurement hook (pqkv_profile_*): returns a token
// for prof_end, or -1 when profiling is off.
// repeated: the bracket holds prof_repeats() launches of the kernel.
int prof_begin(const char *name, hipStream_t s, bool repeated = false);
void prof_end(int token, hipStream_t s);
// Launches of a profiled kernel per event bracket: the pqkv_profile_repeat
// count while profiling is on, else 1. The kernels bracketed this way are
// idempotent (each repeat rewrites the same outputs from the same inputs).
int prof_repeats();

hipError_t launch_quantize_rotated(const float *x_rot, const float *codebook, int bits, uint8_t *blocks,
                                   float *radius_out, int64_t n, int d, hipStream_t s);
// y = (R x) sy and z = (M y) sz for n vectors in one launch (fp32 outputs).
hipError_t launch_rotate2(const void *x, int x_dtype, const float *R, const float *M, float *y, float *z, int64_t n,
                          int d, float sy, float sz, hipStream_t s);
// R == nullptr: y = x * out_scale (an identity rotation, exactly).
hipError_t launch_rotate(const void *x, int x_dtype, const float *R, void *y, int y_dtype, int64_t n, int d,
                         int inverse, float out_scale, hipStream_t s);
// fp32 rows gathered from a strided [n_seq][Hq][n_q] arrangement (element
// strides: s_q between query rows, s_h between heads, s_s between
// sequences) into y [n_seq][n_q][Hq][d] fp32, y = (R x) out_scale: the FMA
// chains of launch_rotate.
hipError_t launch_rotate_rows(const float *x, int64_t s_q, int64_t s_h, int64_t s_s, int n_q, int Hq, int n_seq,
                              const float *R, float *y, int d, float out_scale, hipStream_t s);
// y = (r16 c[code]) R for n block-encoded vectors (inverse rotation, one
// FMA chain per output as in launch_rotate); fp16 output saturates.
hipError_t launch_dequantize(const uint8_t *blocks, const float *codebook, int bits, const float *R, void *y,
                             int y_dtype, int64_t n, int d, hipStream_t s);
hipError_t launch_encode_exact(const EncodeArgs &a, int x_dtype, hipStream_t s);
// Register-blocked form of the exact encoder (same rotation, same indices)
// for inputs it reads in 16-byte pieces, without QJL signs; the exact
// launchers take it where tiled_encode_ok / tiled_soa_ok hold.
bool tiled_encode_ok(const EncodeArgs &a, int x_dtype);
hipError_t launch_encode_tiled(const EncodeArgs &a, int x_dtype, hipStream_t s);
bool tiled_soa_ok(const float *x, const float *R, const uint8_t *packed, int64_t n, int d);
hipError_t launch_encode_soa_tiled(const float *x, const float *R, const float *codebook, int n_levels,
                                   float *radius, uint8_t *packed, int64_t n, int d, hipStream_t s);
// Matrix-core encoder for fp16 input (with the QJL signs when a.qjl is set;
// rot_out and radius_out are for keys without them); rot_out and radius_out
// (nullable) receive the fp32 rotated vectors the quantiser saw, [n][d], and
// their fp32 radii, [n].
// One round of workgroups (two per compute unit) loops over the vectors.
hipError_t launch_encode_mfma(const EncodeArgs &a, float *rot_out, float *radius_out, int cus, hipStream_t s);
hipError_t launch_encode_soa(const float *x, const float *R, const float *codebook, int n_levels, float *radius,
                             uint8_t *packed, int64_t n, int d, hipStream_t s);
hipError_t launch_soa_to_blocks(const uint8_t *packed, const float *radius, uint8_t *blocks, int64_t n, int d,
                                hipStream_t s);
hipError_t launch_blocks_to_soa(const uint8_t *blocks, uint8_t *packed, float *radius, int64_t n, int d,
                                hipStream_t s);

hipError_t launch_decode_split(const DecodeArgs &a, int k_bits, int v_bits, hipStream_t s);
// Matrix-core variant for 2- and 4-bit keys and values, with or without QJL
// (same workspace).
hipError_t launch_decode_mfma(const DecodeArgs &a, int k_bits, int v_bits, hipStream_t s);
// Paged caches (a.k_pages, a.v_pages, a.s_pages; uniform widths, keys and
// values of `bits` each).
hipError_t launch_decode_mfma_paged(const DecodeArgs &a, int bits, hipStream_t s);
// Mixed widths with kv heads of exactly two kinds, 4-bit K and V sharing one
// codebook (a4) and 2-bit K and V (a2): one launch over both head lists.
hipError_t launch_decode_mfma_pair(const DecodeArgs &a4, const DecodeArgs &a2, hipStream_t s);
// 4-bit keys and values in the SoA layout (packed codes [stream][S_max][d/2]
// in k_cache / v_cache, fp32 radii in k_rad / v_rad), codebooks of cb_levels
// entries (one shared table when k_cb == v_cb), no QJL.
hipError_t launch_decode_mfma_soa(const DecodeArgs &a, hipStream_t s);
// 4-bit keys and values with one codebook in the ggml flash-attn-ext layout
// (a.k_tok_stride, a.rows_per_seq, a.mask), no QJL, unlisted heads. With
// ggml_heads_per_wave(n_heads) the grid's rows are B * n_heads / 4 (a
// workgroup takes four kv heads of the same tokens), so the split plan is
// made for that many rows.
hipError_t launch_decode_mfma_ggml(const DecodeArgs &a, hipStream_t s);
inline bool ggml_heads_per_wave(int n_heads) { return n_heads % 4 == 0; }
// R == nullptr: the normalised rotated output, not rotated back.
hipError_t launch_decode_merge(const float *part, const float *R, void *out, int out_dtype, int BHq, int splits,
                               int d, hipStream_t s);
hipError_t launch_fill_zero(void *p, size_t bytes, hipStream_t s);

// Group (min / scale) format of the reference's CPU quantizer: d <= 256,
// 1 <= gs <= d; codes [n][ceil(d/gs) gs], mins / scales [n][ceil(d/gs)].
hipError_t launch_group_compress(const void *x, int x_dtype, const double *R, int64_t n, int d, int bits, int gs,
                                 float *radius, uint8_t *codes, float *mins, float *scales, hipStream_t s);
hipError_t launch_group_decompress(const float *radius, const uint8_t *codes, const float *mins, const float *scales,
                                   const double *R, int64_t n, int d, int gs, float *out, hipStream_t s);
// The reference's GPU group format (CompressedKVCacheGPU): d <= 256, any
// 1 <= gs <= d; radius, lo and s in pdt (fp16 or fp32); codes packed 4-bit,
// 2-bit, or one byte per code for the other widths, [n][d_pad * sb / 8].
// Rt = R^T; resid (nullable) receives the QJL residual e [n][d] fp32.
hipError_t launch_group_gpu_compress(const void *x, int x_dtype, const float *Rt, const float *R, int64_t n, int d,
                                     int bits, int gs, void *radius, uint8_t *codes, void *mins, void *scales,
                                     int pdt, float *resid, hipStream_t s);
hipError_t launch_group_gpu_decompress(const void *radius, const uint8_t *codes, const void *mins,
                                       const void *scales, int pdt, const float *R, int64_t n, int d, int bits,
                                       int gs, void *out, int out_dtype, hipStream_t s);
// QJL signs of e = x - x_hat (x_hat nullable) against P given as Pt [d][m]
// fp64, and |e| in norm_dtype.
hipError_t launch_qjl_sketch(const void *x, int x_dtype, const float *x_hat, const double *Pt, int64_t n, int d,
                             int m, uint8_t *signs, void *norms, int norm_dtype, hipStream_t s);
// Fused attention on the group format: query rows rotated (q_rot [rows][dpad],
// x qs, zero-padded) with P q x qs / m beside them, the split kernel, the merge.
hipError_t launch_group_qprep(const void *q, int q_dtype, const float *R, const float *P, int64_t rows, int d,
                              int dpad, int m, float qs, float *q_rot, float *pq, hipStream_t s);
struct GroupAttnArgsHost {
  const float *q, *pq;
  const uint8_t *k_codes, *v_codes;
  const void *k_rad, *v_rad, *k_lo, *k_sc, *v_lo, *v_sc;
  const uint8_t *qjl;
  const void *res_norm;
  const float *cb;               // codebook mode (SoA caches): c[code], one group of dpad, no lo / s
  int cb_levels;
  float *part;
  int B, Hq, Hkv, S, S_max, d, dpad, gs, bits, pdt, m;
  int splits, tps;
};
hipError_t launch_group_attn(const GroupAttnArgsHost &a, hipStream_t s);
hipError_t launch_group_merge(const float *part, const float *R, void *out, int out_dtype, int64_t rows, int splits,
                              int d, hipStream_t s);
// The reference kernels' SoA encoder and fp32 rotations at any head dim
// (even d <= 256 / d <= 256), for the compat entry points.
hipError_t launch_encode_soa_generic(const float *x, const float *R, const float *codebook, int n_levels,
                                     float *radius, uint8_t *packed, int64_t n, int d, hipStream_t s);
hipError_t launch_rotate_generic(const float *x, const float *R, float *y, int64_t n, int d, int inverse,
                                 hipStream_t s);
// The split plan of the decode kernels (splits of tps tokens, a multiple of
// 64) for `streams` streams of S tokens and `target` workgroups.
void decode_plan_for(int64_t streams, int S, int target, int *splits, int *tps);
int device_compute_units();
// Measurement: read `bytes` (a multiple of 16) from p once, XOR into sink[block].
hipError_t launch_stream_read(const void *p, size_t bytes, uint32_t *sink, int blocks, hipStream_t s);
hipError_t launch_prefill(const PrefillArgs &a, int k_bits, int v_bits, hipStream_t s);
// Query rows per prefill workgroup (the QJL kernel holds 16 rows per wave
// instead of 32, to make room for the projection operands).
int prefill_rows_per_block(bool qjl);

}  // namespace pqkv
