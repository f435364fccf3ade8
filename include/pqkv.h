/*
 * pqkv.h - C ABI of the MI355X (gfx950) PolarQuant-KV hot path.
 *
 * One shared library, libpqkv_hip.so, exports every function below. All
 * tensor arguments are device pointers owned by the caller; `stream` is a
 * hipStream_t passed as void* (NULL = the null stream). Work is enqueued on
 * that stream and the call returns without synchronising. Every function
 * validates its arguments in host code before any HIP call and returns a
 * status (PQKV_OK = 0, negative on error); pqkv_last_error() gives the
 * message of the last failure on the calling thread. No function keeps state
 * between calls or allocates device memory, except the reference-compatible
 * polarquant_* entry points, which mirror the reference's own ownership
 * rules, pqkv_decode_attn_noalloc's scratch array and the host copy of the
 * ggml type's default rotation.
 *
 * Storage format (README.md:73-78 of the reference, "block_pq4"):
 *   one head vector of d coordinates = d/32 blocks; block = {fp16 radius;
 *   uint8 qs[16]} (18 B) for 4-bit codes, {fp16 radius; uint8 qs[8]} (10 B)
 *   for 2-bit codes. The radius is the fp16 (RNE) norm of the whole rotated
 *   vector, repeated in each block. Code of coordinate 32b+2i sits in the
 *   low nibble of qs[i], 32b+2i+1 in the high nibble; 2-bit codes pack
 *   v0 | v1<<2 | v2<<4 | v3<<6.
 * A KV cache is [B][H][S_max][d/32 blocks], i.e. each (batch, head) owns a
 * contiguous run of S_max vectors.
 */
#ifndef PQKV_H
#define PQKV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status and dtypes ------------------------------------------------ */
#define PQKV_OK               0
#define PQKV_ERR_INVALID     -1  /* null pointer, negative or inconsistent size   */
#define PQKV_ERR_UNSUPPORTED -2  /* head dim, bit width, dtype or group size       */
#define PQKV_ERR_WORKSPACE   -3  /* workspace smaller than the *_workspace_bytes  */
#define PQKV_ERR_HIP         -4  /* a HIP launch or runtime call failed            */

#define PQKV_F32  0
#define PQKV_F16  1
#define PQKV_BF16 2

#define PQKV_MAX_HEADS 64        /* kv heads per call with per-head (mixed) widths */

int         pqkv_version(void);
const char *pqkv_status_string(int status);
const char *pqkv_last_error(void);

/* Bytes of one block (18 for 4-bit, 10 for 2-bit) and of one d-vector.
 * Pure host functions; return <= 0 for unsupported arguments. */
int     pqkv_block_bytes(int n_bits);
int64_t pqkv_vector_bytes(int d, int n_bits);

/* Lloyd-Max codebook for one rotated unit-vector coordinate, computed on the
 * host (Beta((d-1)/2,(d-1)/2) on a grid over +-6/sqrt(d), midpoint/centroid
 * iterations). Replaces build_lloyd_max_codebook,
 * src/polarquant_kv_cuda/lloyd_max.py:12-79. centroids has 2^n_bits floats,
 * boundaries (nullable) 2^n_bits+1. Pure host function. */
int pqkv_lloyd_max_codebook(int d, int n_bits, int n_iterations, int grid_size,
                            float *centroids, float *boundaries);

/* ---- rotation ----------------------------------------------------------
 * y = x R^T (inverse = 0) or y = x R (inverse = 1) for n vectors of d.
 * x_dtype / y_dtype in {PQKV_F32, PQKV_F16}. Each output is one fp32 FMA
 * chain over j in increasing order, the arithmetic of the reference's
 * rotate kernels (integration/polarquant-kv.patch:395-437,
 * csrc/polarquant_full.cu:25-40,125-140) and of its encode kernel
 * (csrc/flash_turboquant.cu:132-137). d in {64, 128}; R is device fp32
 * [d][d], 16-byte aligned. */
int pqkv_rotate(const void *x, int x_dtype, const float *R, void *y, int y_dtype,
                int64_t n, int d, int inverse, void *stream);

/* ---- encode ------------------------------------------------------------
 * Bit-exact quantiser on fp32 rotated input (the parity surface):
 * radius by the reference's 128-slot tree of squares and sqrtf, direction by
 * IEEE divide, nearest centroid by a strict '<' scan, codes packed to blocks.
 * Replaces the quantise half of turboquant_compress_kernel
 * (csrc/flash_turboquant.cu:141-173). radius_out (nullable) receives the fp32
 * radius. d in {64, 128}, n_bits in {2, 4}. */
int pqkv_quantize_rotated(const float *x_rot, const float *codebook, int n_bits,
                          uint8_t *blocks_out, float *radius_out,
                          int64_t n, int d, void *stream);

/* Fused encoder: rotate, quantise and pack n_outer x n_inner vectors.
 * x: fp16, fp32 or bf16 (PQKV_BF16, widened exactly to fp32, as the
 * reference's kv.float()), vector (o, i) at x + (o * x_outer_stride + i * d)
 * elements.
 * blocks: vector (o, i) at blocks + o * blocks_outer_stride + i * vector_bytes.
 * Optional QJL sign sketch of the key residual (p_rot = P R^T, [m][d] fp32,
 * m = d): signs at qjl + o * qjl_outer_stride + i * (m/8), bit i of the
 * sketch = (p_rot[i] . (x_rot - r c[idx]) >= 0), LSB first
 * (src/polarquant_kv_cuda/compress_kernel.py:166-175, qjl_kernel.py:6-37).
 * fp16 input (x rows and R 16-byte aligned, blocks 4-byte aligned; with QJL
 * also p_rot 16-byte and the signs 4-byte aligned) runs on the matrix-core
 * encoder of pqkv_encode_mfma, signs included; PQKV_ENCODE_KERNEL=exact in
 * the environment forces the FMA-chain rotation of pqkv_rotate everywhere.
 * Replaces turboquant_compress (csrc/flash_turboquant.cu:213-225) and
 * polarquant_compress_cuda (patch:443-467). */
int pqkv_encode(const void *x, int x_dtype, int64_t x_outer_stride,
                const float *R, const float *codebook, int n_bits,
                uint8_t *blocks, int64_t blocks_outer_stride,
                int64_t n_outer, int64_t n_inner, int d,
                const float *p_rot, int m, uint8_t *qjl, int64_t qjl_outer_stride,
                void *stream);

/* Matrix-core encoder (no counterpart in the reference: a second, faster
 * implementation of pqkv_encode for fp16 input, which pqkv_encode uses with
 * or without QJL signs whenever its conditions hold unless the environment
 * sets PQKV_ENCODE_KERNEL=exact; this entry point takes keys without QJL and
 * exposes the rotation). x must be 16-byte aligned with a row stride that
 * is a multiple of 8 elements, R 16-byte aligned; otherwise
 * PQKV_ERR_UNSUPPORTED. The rotation runs on the matrix cores with fp32-grade
 * products but not the reference's FMA-chain rounding; the quantiser is
 * bit-exact on the rotated values it computes, which rot_out (nullable,
 * fp32 [n_outer * n_inner][d]) receives, together with their fp32 radii
 * (radius_out, nullable, [n_outer * n_inner]). */
int pqkv_encode_mfma(const void *x, int x_dtype, int64_t x_outer_stride,
                     const float *R, const float *codebook, int n_bits,
                     uint8_t *blocks, int64_t blocks_outer_stride,
                     int64_t n_outer, int64_t n_inner, int d,
                     float *rot_out, float *radius_out, void *stream);

/* ---- decode attention ----------------------------------------------------
 * One query token per sequence against a block-encoded cache:
 *   q_rot = q R^T; s_t = scale * r_k,t * q_rot . c_k[idx_t]
 *           (+ scale * (1/m) sum_i (2 sign_i - 1) (p_rot q_rot)_i if qjl)
 *   w = softmax(s);  out = (sum_t w_t r_v,t c_v[vidx_t]) R
 * q [B][Hq][d] (fp16/fp32), out [B][Hq][d] (fp16/fp32), caches
 * [B][Hkv][S_max] vectors, first S valid. q-head h reads kv-head
 * h / (Hq/Hkv). k_head_bits / v_head_bits: host arrays of Hkv widths (2 or 4)
 * for mixed-width heads, or NULL for uniform k_bits / v_bits; with mixed
 * widths each (b, h) run still holds S_max vectors of its own width, runs laid
 * out in (b, h) order. k_codebooks / v_codebooks: device [Hkv][16] fp32
 * per-head tables, or one table when the *_head_bits pointer is NULL.
 * Passing the same pointer for k_codebooks and v_codebooks with 4-bit keys
 * and values lets one LDS table serve both (faster); distinct pointers are
 * always correct.
 * Replaces turboquant_full_attention (csrc/flash_turboquant.cu:180-211),
 * polarquant_fused_attention_cuda (patch:469-506) plus the query and output
 * rotations around them (patch:395-437). R (and p_rot) are device fp32
 * [d][d], 16-byte aligned. S = 0 writes zeros. */
size_t pqkv_decode_workspace_bytes(int B, int Hq, int Hkv, int S, int d);

int pqkv_decode_attn(const void *q, int q_dtype, const float *R,
                     const uint8_t *k_cache, const uint8_t *v_cache,
                     const float *k_codebooks, const float *v_codebooks,
                     int k_bits, int v_bits,
                     const int *k_head_bits, const int *v_head_bits,
                     const uint8_t *qjl_signs, const float *p_rot, int m,
                     int B, int Hq, int Hkv, int S, int S_max, int d, float scale,
                     void *out, int out_dtype,
                     void *workspace, size_t workspace_bytes, void *stream);

/* Allocation-free variant of pqkv_decode_attn (no counterpart in the
 * reference): for callers that cannot allocate device memory (code under
 * stream or graph capture, serving loops that forbid it). Same arguments and
 * results as pqkv_decode_attn without the workspace: the library keeps one
 * PQKV_NOALLOC_SCRATCH_BYTES device array per GPU for the whole process and
 * uses it instead. A call whose split plan needs more (rotated queries,
 * split partials, QJL projections: about B*Hq*(2d + splits*(d+2))*4 bytes)
 * returns PQKV_ERR_WORKSPACE. The call allocates nothing. Every call on one
 * GPU shares that GPU's array: calls that overlap on one GPU (different
 * streams, or threads without ordering) race. */
#define PQKV_NOALLOC_SCRATCH_BYTES (16u << 20)
int pqkv_decode_attn_noalloc(const void *q, int q_dtype, const float *R,
                             const uint8_t *k_cache, const uint8_t *v_cache,
                             const float *k_codebooks, const float *v_codebooks,
                             int k_bits, int v_bits,
                             const int *k_head_bits, const int *v_head_bits,
                             const uint8_t *qjl_signs, const float *p_rot, int m,
                             int B, int Hq, int Hkv, int S, int S_max, int d, float scale,
                             void *out, int out_dtype, void *stream);

/* Decode attention over a cache split into segments of different widths
 * (per-token mixed precision, e.g. sink and recent-window tokens at 4 bits,
 * the rest at 2 bits; src/polarquant_kv_cuda/token_importance.py:17-40 of the
 * reference computes such widths but attends on no such cache). Segment i
 * holds caches k_caches[i] / v_caches[i] ([B][Hkv][S_max[i]] vectors of
 * k_bits[i] / v_bits[i], first S[i] valid) with device codebooks
 * k_codebooks[i] / v_codebooks[i]. The softmax runs over the tokens of all
 * segments together (token order does not matter to decode attention): every
 * segment's split-K partials land in one workspace and one merge combines
 * them. Otherwise as pqkv_decode_attn with uniform widths and no QJL.
 * At most PQKV_MAX_SEGMENTS segments; the pointer and size arrays are host
 * memory. */
#define PQKV_MAX_SEGMENTS 8
size_t pqkv_decode_segments_workspace_bytes(int B, int Hq, int Hkv, int n_seg, const int *S, int d);

int pqkv_decode_attn_segments(const void *q, int q_dtype, const float *R, int n_seg,
                              const uint8_t *const *k_caches, const uint8_t *const *v_caches,
                              const float *const *k_codebooks, const float *const *v_codebooks,
                              const int *k_bits, const int *v_bits, const int *S, const int *S_max,
                              int B, int Hq, int Hkv, int d, float scale,
                              void *out, int out_dtype,
                              void *workspace, size_t workspace_bytes, void *stream);

/* ---- paged caches --------------------------------------------------------
 * A paged cache keeps each (batch, kv-head) stream s = b * Hkv + h in pages
 * of page_tokens vectors (a power of two, 64 <= page_tokens <= 65536):
 * position t of stream s is vector t % page_tokens of the page whose device
 * address is pages[s * max_pages + t / page_tokens]. k_pages, v_pages and
 * (QJL keys) qjl_pages are device arrays of B * Hkv * max_pages addresses; a
 * key page and its sign page share an index. A page holds page_tokens
 * vectors of the cache's width (block_pq4 / block_pq2) or of m/8 sign bytes
 * and is 16-byte aligned; pages may sit anywhere in device memory, so a cache
 * grows by adding pages and writing their addresses, with no copy of what it
 * holds. Entries for pages that no valid position reaches are not read.
 * Replace the reference cache's grow-by-concatenation, which copies the
 * whole cache on every append (src/polarquant_kv_cuda/inference/kv_cache.py:
 * 93-112), and the attention on it (inference/attention.py:59-61). */

/* pqkv_encode into a paged cache: x as in pqkv_encode with n_streams rows
 * (x + o * x_outer_stride elements) of n_tokens vectors; vector (o, i) is
 * written to position start + i of stream o (blocks, and with p_rot its QJL
 * signs in qjl_pages). Same encoders and results as pqkv_encode. */
int pqkv_encode_paged(const void *x, int x_dtype, int64_t x_outer_stride,
                      const float *R, const float *codebook, int n_bits,
                      uint8_t *const *pages, int page_tokens, int max_pages, int64_t start,
                      int64_t n_streams, int64_t n_tokens, int d,
                      const float *p_rot, int m, uint8_t *const *qjl_pages, void *stream);

/* pqkv_decode_attn on a paged cache of S valid positions per stream, keys and
 * values of n_bits each (one codebook each; the same pointer for both lets
 * one LDS table serve them), QJL when qjl_pages and p_rot are given. The
 * workspace is pqkv_decode_workspace_bytes(B, Hq, Hkv, S, d). */
int pqkv_decode_attn_paged(const void *q, int q_dtype, const float *R,
                           const uint8_t *const *k_pages, const uint8_t *const *v_pages,
                           int page_tokens, int max_pages,
                           const float *k_codebook, const float *v_codebook, int n_bits,
                           const uint8_t *const *qjl_pages, const float *p_rot, int m,
                           int B, int Hq, int Hkv, int S, int d, float scale,
                           void *out, int out_dtype, void *workspace, size_t workspace_bytes, void *stream);

/* pqkv_prefill_attn on a paged cache (as pqkv_decode_attn_paged); the
 * workspace is pqkv_prefill_workspace_bytes(B, Hq, Hkv, Sq, S, d). */
int pqkv_prefill_attn_paged(const void *q, int q_dtype, const float *R,
                            const uint8_t *const *k_pages, const uint8_t *const *v_pages,
                            int page_tokens, int max_pages,
                            const float *k_codebook, const float *v_codebook, int n_bits,
                            const uint8_t *const *qjl_pages, const float *p_rot, int m,
                            int B, int Hq, int Hkv, int Sq, int q_start, int S, int d, float scale, int causal,
                            void *out, int out_dtype, void *workspace, size_t workspace_bytes, void *stream);

/* ---- group (min / scale) format ------------------------------------------
 * The reference's CPU quantizer format (python/polarquant_kv/quantizer.py:
 * 25-158, behind polarquant_kv.quantizer.compress / decompress /
 * compress_batch / decompress_batch) on the GPU: rotate with an fp64 R
 * (device [d][d] float64, the reference's rotation matrix), fp32 radius and
 * direction, then per group of group_size coordinates (the last group
 * zero-padded) min, scale = (max - min) / (2^n_bits - 1) (1 for a flat
 * group) and codes rint((u - min) / scale) clipped to [0, 2^n_bits - 1]
 * (0 for a flat group), one uint8 per coordinate. x [n][d] fp32 / fp16;
 * radius [n] fp32; codes [n][ng * group_size] uint8; mins, scales [n][ng]
 * fp32 with ng = ceil(d / group_size). 1 <= d <= 256, 2 <= n_bits <= 8,
 * 1 <= group_size <= d. decompress writes out [n][d] fp32 (zeros where the
 * radius is below 1e-30). Replaces compress / decompress
 * (python/polarquant_kv/quantizer.py:88-158). */
int pqkv_group_compress(const void *x, int x_dtype, const double *R, int64_t n, int d, int n_bits, int group_size,
                        float *radius, uint8_t *codes, float *mins, float *scales, void *stream);
int pqkv_group_decompress(const float *radius, const uint8_t *codes, const float *mins, const float *scales,
                          const double *R, int64_t n, int d, int group_size, float *out, void *stream);

/* ---- the reference's GPU group format (CompressedKVCacheGPU) -------------
 * The format of src/polarquant_kv_cuda/compress_kernel.py:100-189: per
 * vector y = clamp(x, +-65000) R^T (fp32), r = |y|, u = y / max(r, 1e-30)
 * (0 where r < 1e-30) zero-padded to d_pad = ceil(d / group_size) *
 * group_size, per group lo = min, s = (max - lo) / (2^n_bits - 1) (1 for a
 * flat group), code = round_half_even(clamp((u - lo) / s, 0, 2^n_bits - 1)).
 * Stored: radius [n] (saturated at 65504), mins / scales [n][ng] in
 * param_dtype (PQKV_F16 as the reference, or PQKV_F32), codes [n][row]
 * packed as the reference packs them: 4-bit d_pad/2 bytes (coordinate 2i
 * low nibble), 2-bit d_pad/4 bytes (v0 | v1<<2 | v2<<4 | v3<<6), every
 * other width one byte per code. x fp32 / fp16 / bf16 [n][d]; R [d][d] fp32
 * and Rt = R^T (both device); 1 <= d <= 256, 2 <= n_bits <= 8. residual
 * (nullable, needs R) receives the QJL residual e = (y - (code s + lo)
 * max(r, 1e-30)) R [n][d] fp32 with the unrounded lo and s
 * (compress_kernel.py:166-175). Replaces compress_gpu. */
int pqkv_group_gpu_compress(const void *x, int x_dtype, const float *R, const float *Rt, int64_t n, int d,
                            int n_bits, int group_size, void *radius, uint8_t *codes, void *mins, void *scales,
                            int param_dtype, float *residual, void *stream);
/* x^ = clamp(((code s + lo) r) R, +-65504) [n][d] in out_dtype (fp16 as the
 * reference's decompress_gpu, src/polarquant_kv_cuda/decompress_kernel.py:
 * 10-51, or fp32). */
int pqkv_group_gpu_decompress(const void *radius, const uint8_t *codes, const void *mins, const void *scales,
                              int param_dtype, const float *R, int64_t n, int d, int n_bits, int group_size,
                              void *out, int out_dtype, void *stream);
/* QJL sketch (compute_signatures_gpu, src/polarquant_kv_cuda/qjl_kernel.py:
 * 6-37; compute_signatures, python/polarquant_kv/qjl.py:25-35): e = x - x_hat
 * (x_hat nullable: e = x) in fp32, signs (P e >= 0) summed in fp64 against
 * Pt = P^T [d][m] fp64, packed LSB first into ceil(m/8) bytes per vector
 * (bits past m zero), and |e| in norm_dtype. */
int pqkv_qjl_sketch(const void *x, int x_dtype, const float *x_hat, const double *Pt, int64_t n, int d, int m,
                    uint8_t *signs, void *norms, int norm_dtype, void *stream);
/* Attention straight on group-format caches (compressed_attention_gpu,
 * src/polarquant_kv_cuda/attention_kernel.py:11-113, whose fallback
 * decompresses both caches; the reference's fused kernels,
 * csrc/polarquant_full.cu:45-111, read the same fields): q [B][Hq][d]
 * (original space; several query tokens per head are Hq*Sq rows ordered
 * [B][Hq][Sq], each attending to all S positions), caches [B][Hkv][S_max][..]
 * as pqkv_group_gpu_compress writes them with S valid positions; row h of a
 * batch reads kv head h / (Hq / Hkv). s_t = scale r_t sum_g (s_tg q_rot.c_tg
 * + lo_tg sum_{j in g} q_rot_j), plus, with qjl_signs ([B][Hkv][S_max][m/8])
 * and P ([m][d] fp32), scale (1/m) sum_i (2 sign_i - 1) (P q)_i, which is 0
 * where residual_norms ([B][Hkv][S_max] in param_dtype, nullable) is 0, or,
 * without norms, where the sketch is all ones (the reference's zero-residual
 * guard, python/polarquant_kv/qjl.py:50-51). out [B][Hq][d] = softmax(s)
 * (code s + lo) r, rotated back. The fused kernel needs group_size a
 * multiple of 8 (16 for 2-bit codes), d_pad <= 256 and, with QJL, m a
 * multiple of 32 up to 256 (PQKV_ERR_UNSUPPORTED otherwise). */
size_t pqkv_group_attn_workspace_bytes(int B, int Hq, int Hkv, int S, int d, int group_size, int m);
int pqkv_group_attn(const void *q, int q_dtype, const float *R, const float *P, int m, const uint8_t *k_codes,
                    const void *k_radius, const void *k_mins, const void *k_scales, const uint8_t *v_codes,
                    const void *v_radius, const void *v_mins, const void *v_scales, const uint8_t *qjl_signs,
                    const void *residual_norms, int n_bits, int param_dtype, int B, int Hq, int Hkv, int S,
                    int S_max, int d, int group_size, float scale, void *out, int out_dtype, void *workspace,
                    size_t workspace_bytes, void *stream);
/* Codebook attention on the reference kernels' SoA cache (packed 4-bit codes
 * [Hkv][S][d/2], fp32 radii [Hkv][S], a table of `levels` <= 16 entries;
 * csrc/flash_turboquant.cu:27-105, patch:277-389) at any d that is a
 * multiple of 8 up to 256, by the group kernel in its codebook mode: q_rot
 * [Hq][d] already rotated, out [Hq][d] rotated. The compat entry points use
 * it for the head dims the matrix-core kernels are not built for. */
size_t pqkv_soa_attn_generic_workspace_bytes(int Hq, int Hkv, int S, int d);
int pqkv_soa_attn_generic(const float *q_rot, const uint8_t *k_codes, const float *k_radius, const uint8_t *v_codes,
                          const float *v_radius, const float *codebook, int levels, int Hq, int Hkv, int S, int d,
                          float scale, float *out, void *workspace, size_t workspace_bytes, void *stream);

/* ---- chunked prefill attention -------------------------------------------
 * Sq query tokens per sequence (absolute positions q_start .. q_start+Sq-1)
 * against a cache that already holds them (append-then-attend,
 * src/polarquant_kv_cuda/inference/attention.py:59-61). With causal = 1
 * query i attends to cache positions <= q_start + i; with causal = 0 to all
 * S positions. q / out [B][Hq][Sq][d]. Widths, per-head tables and the QJL
 * correction (applied to every query token, as the reference's
 * attention_kernel.py:95-107 does) take the same arguments as
 * pqkv_decode_attn. */
size_t pqkv_prefill_workspace_bytes(int B, int Hq, int Hkv, int Sq, int S, int d);

int pqkv_prefill_attn(const void *q, int q_dtype, const float *R,
                      const uint8_t *k_cache, const uint8_t *v_cache,
                      const float *k_codebooks, const float *v_codebooks,
                      int k_bits, int v_bits,
                      const int *k_head_bits, const int *v_head_bits,
                      const uint8_t *qjl_signs, const float *p_rot, int m,
                      int B, int Hq, int Hkv, int Sq, int q_start, int S, int S_max,
                      int d, float scale, int causal,
                      void *out, int out_dtype,
                      void *workspace, size_t workspace_bytes, void *stream);

/* ---- dequantise -----------------------------------------------------------
 * out = (r16 c[code]) R for n block-encoded vectors: the stored radius times
 * the centroids, rotated back to the original space, each output one fp32
 * FMA chain over k ascending (as pqkv_rotate with inverse = 1). fp16 output
 * saturates at +-65504. Replaces the decompression of decompress_gpu
 * (src/polarquant_kv_cuda/decompress_kernel.py:10-55) for the codebook
 * format. blocks [n][vector bytes], codebook [16] fp32 (zero-padded),
 * R [d][d] fp32 16-byte aligned, out [n][d] fp32/fp16. */
int pqkv_dequantize(const uint8_t *blocks, const float *codebook, int n_bits, const float *R,
                    void *out, int out_dtype, int64_t n, int d, void *stream);

/* ---- layout converters ---------------------------------------------------
 * SoA (the reference kernels' format: packed u8 [n][d/2] + fp32 radius [n],
 * csrc/flash_turboquant.cu:29-32) <-> block_pq4. 4-bit codes only. */
int pqkv_soa_to_blocks(const uint8_t *packed, const float *radius,
                       uint8_t *blocks, int64_t n, int d, void *stream);
int pqkv_blocks_to_soa(const uint8_t *blocks, uint8_t *packed, float *radius,
                       int64_t n, int d, void *stream);

/* ---- measurement hook (no counterpart in the reference) -----------------
 * With profiling on, the library brackets each launch of its main kernels
 * with hipEvents recorded on the launch stream. pqkv_profile_collect waits
 * for those events and returns, for kernels whose name contains `name`
 * ("decode_split", "decode_merge", "encode", "rotate", ...), the summed
 * duration in ms and the number of launches, then forgets them. Used by
 * bench.py; off by default, and costs nothing when off. */
int pqkv_profile_enable(int on);
int pqkv_profile_collect(const char *name, double *total_ms, int64_t *launches);
/* While profiling is on, each bracketed kernel (decode rotation, split and
 * merge; the encoders; prefill; the ggml ops) is launched n times back to
 * back between its two events (1 <= n <= 1000; default 1), so that the
 * per-launch mean pqkv_profile_collect gives carries the events' dispatch
 * latency once per n launches. Those kernels are idempotent: a repeat
 * rewrites the same outputs from the same inputs. */
int pqkv_profile_repeat(int n);
/* A plain streaming read of `bytes` (a multiple of 16) at p with 16-byte
 * loads by `blocks` workgroups (the data is XOR-folded; sink, of `blocks`
 * words, is written only on a fold that never occurs in practice): the
 * most a read-only kernel draws from HBM on the device, which bench.py
 * reports beside the decode kernel's rate. */
int pqkv_profile_stream_read(const void *p, size_t bytes, uint32_t *sink, int blocks, void *stream);

/* ---- reference-compatible entry points -------------------------------------
 * Same names, arguments and return types as the extern "C" exports of the
 * reference's ggml CUDA backend (integration/polarquant-kv.patch:695-763),
 * which llama.cpp resolves with dlsym (patch:1508-1557). SoA layout (packed
 * u8 [N][D/2] + fp32 radius [N]); errors print to stderr and return, like
 * the reference's silent early returns (patch:452,481,515,534). */
typedef struct polarquant_kv_layer {
    uint8_t *k_packed;  /* [n_kv_heads][n_kv_max][head_dim/2] */
    float   *k_radius;  /* [n_kv_heads][n_kv_max]             */
    uint8_t *v_packed;
    float   *v_radius;
} polarquant_kv_layer;

typedef struct polarquant_state {
    int    enabled;     /* bool in the reference (patch:958); int here for a C ABI */
    int    n_bits;
    int    n_levels;
    int    head_dim;
    int    n_kv_heads;
    int    n_q_heads;
    int    n_layers;
    int    n_kv_max;
    float *codebook;    /* device [n_levels]            */
    float *rotation;    /* device [head_dim][head_dim]  */
    polarquant_kv_layer *layers;  /* host array of n_layers */
} polarquant_state;

polarquant_state *polarquant_init_c(int head_dim, int n_kv_heads, int n_q_heads,
                                    int n_layers, int n_kv_max, int n_bits);
void polarquant_free_c(polarquant_state *state);
void polarquant_compress_cuda_c(const float *input, const float *rotation,
                                const float *codebook, float *radius_out,
                                uint8_t *packed_out, int N, int D, int n_levels,
                                void *stream);
void polarquant_rotate_query_cuda_c(const float *q_input, const float *rotation,
                                    float *q_rotated, int total_q_heads, int D,
                                    void *stream);
void polarquant_fused_attention_cuda_c(const float *q_rotated, const uint8_t *packed_k,
                                       const float *k_radius, const uint8_t *packed_v,
                                       const float *v_radius, const float *codebook,
                                       float *output, int total_q_heads,
                                       int total_kv_heads, int S, int D, int n_levels,
                                       float scale, void *stream);
void polarquant_inverse_rotate_cuda_c(const float *input, const float *rotation,
                                      float *output, int total_q_heads, int D,
                                      void *stream);

/* ---- the reference's raw-pointer Python binding -----------------------------
 * Same names, argument order and meaning as the pybind module
 * polarquant_turboquant (csrc/flash_turboquant.cu:180-230), which callers
 * reach with device pointers passed as Python ints
 * (scripts/benchmark_turboquant.py:88-114): SoA layout (packed u8 [N][D/2],
 * coordinate 2i in the low nibble, + fp32 radius [N]), null stream,
 * asynchronous, no status (errors print to stderr).
 * turboquant_compress: rotate, quantise and pack N vectors of fp32 input,
 *   bit-exact to the reference kernel's arithmetic (:111-175).
 * turboquant_full_attention: attention of the rotated queries at q_rot over
 *   [total_kv][S] SoA keys and values, rotated fp32 output to attn_out; q, R
 *   and out are not read, as in the reference (:188-209); score
 *   ([total_heads][S] fp32) is used as scratch. k_cb / v_cb: n_levels fp32
 *   centroids each. */
void turboquant_compress(int64_t input_ptr, int64_t R_ptr, int64_t cb_ptr,
                         int64_t radius_ptr, int64_t packed_ptr, int N, int D, int n_levels);
void turboquant_full_attention(int64_t q_ptr, int64_t R_ptr, int64_t pk_ptr, int64_t kr_ptr,
                               int64_t pv_ptr, int64_t vr_ptr, int64_t k_cb_ptr, int64_t v_cb_ptr,
                               int64_t out_ptr, int64_t q_rot_ptr, int64_t score_ptr,
                               int64_t attn_out_ptr, int total_heads, int total_kv, int S, int D,
                               int n_levels, float scale);
/* The reference's pybind module polarquant_full
 * (csrc/polarquant_full.cu:142-186, called by
 * scripts/benchmark_turboquant.py:63-69): q [total_heads][D] fp32 in the
 * original space, group-format keys and values with 4-bit packed codes
 * [total_kv][S][D/2], fp32 group minima and scales [total_kv][S][num_groups]
 * and fp32 radii [total_kv][S]; out [total_heads][D] fp32, rotated back.
 * q_rot and attn_out are not needed; score ([total_heads][S] fp32) is used
 * as scratch when large enough. Runs pqkv_group_attn on the null stream. */
void full_compressed_attention(int64_t q_ptr, int64_t R_ptr, int64_t pk_ptr, int64_t km_ptr, int64_t ks_ptr,
                               int64_t kr_ptr, int64_t pv_ptr, int64_t vm_ptr, int64_t vs_ptr, int64_t vr_ptr,
                               int64_t out_ptr, int64_t q_rot_ptr, int64_t score_ptr, int64_t attn_out_ptr,
                               int total_heads, int total_kv, int S, int D, int group_size, int num_groups,
                               float scale);

/* ---- GGML_TYPE_PQ4: a ggml type and its HIP backend ops -------------------
 * No counterpart exists in the reference: its llama.cpp integration keeps the
 * cache as Q4_0 and never calls its kernels from the graph
 * (integration/polarquant-kv.patch:1130-1137,1303-1362,1385-1404). These are
 * the pieces a ggml type and backend would register for a cache in the block
 * format: blocks of PQKV_GGML_QK_PQ4 elements, PQKV_GGML_PQ4_TYPE_SIZE bytes
 * ({fp16 radius; uint8 qs[16]}, README.md:73-78); a row is whole heads of
 * head_dim (64 or 128) elements; a head is rotated by R (q_rot = R x), its
 * fp32 radius (the 128-slot tree, csrc/flash_turboquant.cu:141-148) stored
 * as fp16 saturated at 65504 in each of its blocks, and each direction
 * coordinate stored as the first nearest of 16 codebook entries; its value
 * is (r16 c[code]) R. */
#define PQKV_GGML_QK_PQ4 32
#define PQKV_GGML_PQ4_TYPE_SIZE 18

/* CPU type traits with an explicit head_dim, R ([head_dim][head_dim] fp32)
 * and codebook (16 fp32), host memory; k elements per call (whole heads).
 * The rotation is one fp32 FMA chain per coordinate over k ascending and the
 * rest the GPU encoder's rounding, so rows match pqkv_ggml_cpy_pq4 bytewise. */
int pqkv_pq4_quantize_rows_host(const float *x, void *y, int64_t k, int head_dim, const float *R,
                                const float *codebook);
int pqkv_pq4_dequantize_rows_host(const void *x, float *y, int64_t k, int head_dim, const float *R,
                                  const float *codebook);
/* The default type's rotation: Gram-Schmidt over rand() after srand(42), as
 * polarquant_init_c builds it (patch:549-579; it re-seeds the C library's
 * rand() the first time it runs for a head_dim). */
int pqkv_ggml_pq4_rotation(float *R, int head_dim);
/* ggml's type-trait signatures (from_float_ref, to_float) for the default
 * type: head_dim 128, the rotation above, the 4-bit table of patch:978-983
 * (the one polarquant_init_c uploads). k must be a multiple of 128. */
void pqkv_ggml_quantize_row_pq4_ref(const float *x, void *y, int64_t k);
void pqkv_ggml_dequantize_row_pq4(const void *x, float *y, int64_t k);

/* Backend op cpy: f32 / f16 src [ne0][ne1][ne2][ne3] (ne0 fastest, byte
 * strides nb, nb[0] the element size) into PQ4 rows dst (byte strides
 * nb_dst, nb_dst[0] = PQKV_GGML_PQ4_TYPE_SIZE) with the state's rotation and
 * 4-bit codebook (st from polarquant_init_c with n_bits 4). ne0 is whole
 * heads of st->head_dim. Stream-ordered; the rotation is the FMA chain of
 * pqkv_rotate, so the bytes equal pqkv_pq4_quantize_rows_host's. */
int pqkv_ggml_cpy_pq4(const polarquant_state *st, const void *src, int src_type, const int64_t ne[4],
                      const size_t nb[4], void *dst, const size_t nb_dst[4], void *stream);

/* Backend op flash_attn_ext over PQ4 keys and values, ggml's shapes:
 *   q    f32 [d][n_q][Hq][n_seq]        (byte strides nb_q, nb_q[0] = 4)
 *   k, v PQ4 [d][n_kv][Hkv][n_seq_kv]   (nb[1] bytes between tokens, nb[2]
 *                                        between heads, nb[3] between
 *                                        sequences; n_seq_kv 1 or n_seq)
 *   mask f16 [>= n_kv][>= n_q][1][1 or n_seq], additive, or NULL
 *   dst  f32 [d][Hq][n_q][n_seq], contiguous
 *   dst = softmax(scale q k^T + mask) v with k, v the rows' values; query
 *   head h reads kv head h / (Hq / Hkv); a row whose tokens are all masked
 *   (-inf) is 0. max_bias and logit_softcap must be 0 (PQKV_ERR_UNSUPPORTED
 *   otherwise: a backend's supports_op declines those). d = st->head_dim.
 * The workspace (pqkv_ggml_flash_attn_ext_pq4_workspace_bytes, 0 for an
 * invalid shape) needs no initialisation. Several query rows per sequence
 * (n_q > 1) each stream the whole key / value sequence. */
size_t pqkv_ggml_flash_attn_ext_pq4_workspace_bytes(const polarquant_state *st, const int64_t ne_q[4],
                                                    const int64_t ne_k[4]);
int pqkv_ggml_flash_attn_ext_pq4(const polarquant_state *st, const float *q, const int64_t ne_q[4],
                                 const size_t nb_q[4], const void *k, const int64_t ne_k[4], const size_t nb_k[4],
                                 const void *v, const int64_t ne_v[4], const size_t nb_v[4], const void *mask,
                                 const int64_t ne_m[4], const size_t nb_m[4], float scale, float max_bias,
                                 float logit_softcap, float *dst, void *workspace, size_t workspace_bytes,
                                 void *stream);

#ifdef __cplusplus
}
#endif

#endif /* PQKV_H */
