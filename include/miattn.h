/*
 * miattn.h — C ABI of the MI355X (gfx950) attention hot path.
 *
 * Every entry point takes raw device pointers, element strides (int64, in
 * elements, not bytes), a dtype code and the hipStream_t to launch on (as
 * void*).  Nothing here allocates, frees or synchronises: outputs and
 * workspaces are owned by the caller (the Python layer takes them from
 * torch's caching allocator, which keeps every call legal under hipGraph
 * capture).  Launch geometry depends only on shapes and capacities, never
 * on device-resident values, so captured graphs stay valid across replays.
 *
 * Return value: 0 on success; negative = invalid argument / unsupported
 * shape (nothing was launched); positive = hipError_t reported by the
 * runtime right after the launch.  mi_last_error() returns a description of
 * the most recent failure on the calling thread.
 *
 * Reference interfaces (Analysis196884/llm-infer-engine) each entry point
 * replaces are cited next to it as path:line.
 */
#ifndef MIATTN_H_
#define MIATTN_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes */
#define MI_DTYPE_BF16 0
#define MI_DTYPE_F16 1
#define MI_DTYPE_F32 2

/* status codes */
#define MI_OK 0
#define MI_ERR_INVALID -1     /* bad pointer / shape / stride / alignment */
#define MI_ERR_UNSUPPORTED -2 /* valid request this build has no kernel for */

/* Library version (major*10000 + minor*100 + patch). */
int32_t mi_version(void);

/* Description of the last failure on this thread ("" if none). */
const char* mi_last_error(void);

/*
 * Split-KV single-token decode, phase 1: per (batch, kv-head, split) partial
 * softmax state for ALL query heads of the GQA group (each KV byte is read
 * once per group, not once per query head).
 *
 * Replaces _flash_decode_split_kernel + its launch
 *   src/flash_decode.py:8-137, src/flash_decode.py:300-342.
 *
 * q        [batch, n_heads, 1, head_dim]      strides (q_sb, q_sh, q_sd)
 * k, v     [batch, n_kv_heads, kv_len, head_dim], innermost stride 1,
 *          element-aligned                     strides (*_sb, *_sh, *_sl)
 * head_dim 1 to 256 (src/flash_decode.py:274-277).  Rows that are 16-byte
 *          aligned are read with 128-bit loads (a head_dim that is not a
 *          multiple of 16 bytes, or unaligned rows, use element loads).
 * mask     optional bool bytes; key j of batch b participates iff
 *          mask[b*mask_sb + j*mask_sl] != 0 (mask_sb = 0 broadcasts)
 *          (src/flash_decode.py:87-95, :215-233)
 * seq_lens optional int64 [batch] on device: keys j >= seq_lens[b] are
 *          neither read nor counted (graph-safe variable lengths)
 * part_m, part_l  fp32 [batch, n_heads, num_splits]      (contiguous)
 * part_acc        fp32 [batch, n_heads, num_splits, head_dim] (contiguous)
 *          part_m holds the running max of the scaled scores in log2 units;
 *          part_l/part_acc the matching sum / unnormalised accumulator.
 *          An empty split stores l = 0 (src/flash_decode.py:97-99,131-137).
 * Keys are split into num_splits contiguous ranges of ceil(kv_len/num_splits).
 */
int32_t mi_decode_split(const void* q, const void* k, const void* v,
                        const uint8_t* mask, int64_t mask_sb, int64_t mask_sl,
                        const int64_t* seq_lens, float* part_m, float* part_l,
                        float* part_acc, int64_t batch, int64_t n_heads,
                        int64_t n_kv_heads, int64_t kv_len, int64_t head_dim,
                        int64_t num_splits, int64_t q_sb, int64_t q_sh,
                        int64_t q_sd, int64_t k_sb, int64_t k_sh, int64_t k_sl,
                        int64_t v_sb, int64_t v_sh, int64_t v_sl,
                        float sm_scale, int32_t dtype, void* stream);

/*
 * Split-KV decode, phase 2: log-sum-exp combine of the partials.
 * Replaces _flash_decode_reduce_kernel + its launch
 *   src/flash_decode.py:140-212, src/flash_decode.py:344-369.
 *
 * out [batch, n_heads, 1, head_dim] (strides o_sb, o_sh, o_sd), dtype of q.
 * lse optional fp32 [batch, n_heads] (natural log of the scaled scores).
 * Rows with no participating key produce 0 (src/flash_decode.py:204-205),
 * or NaN when empty_rows_nan != 0 (the 0/0 of src/decode_attn.py:70), and
 * lse = -inf.
 */
int32_t mi_decode_combine(const float* part_m, const float* part_l,
                          const float* part_acc, void* out, float* lse,
                          int64_t batch, int64_t n_heads, int64_t head_dim,
                          int64_t num_splits, int64_t o_sb, int64_t o_sh,
                          int64_t o_sd, int32_t empty_rows_nan, int32_t dtype,
                          void* stream);

/*
 * Both decode phases in one call (what flash_decode / decode_attention use).
 * With num_splits == 1 the partial buffers may be NULL: the split kernel then
 * normalises and writes out/lse itself (single launch).
 * arrive   optional uint64 [batch * n_heads] arrival counters (e.g. from
 *          mi_decode_arrive_counters; batch * n_heads <= MI_DECODE_ARRIVE_SLAB
 *          for one of its slabs): all zero before the first call, and every
 *          call leaves them zero.  Calls that share one counter array must not
 *          overlap in time (issue them on one stream).  With counters, a call
 *          whose split blocks are few and short (no mask, a power-of-two
 *          head_dim, 2..16 splits, at most one block per compute unit) runs the
 *          LSE combine inside the split launch: the splits of each (batch,
 *          kv-head) group are dealt to one XCD and the last of them to finish
 *          combines the group's partials from that XCD's L2 -- one launch
 *          instead of two, the same bits as the wave combine kernel.  Other
 *          calls, and NULL, run two launches.  A group whose splits did not all
 *          run on one XCD (never on a device that deals workgroups
 *          round-robin, as gfx950 does) yields NaN outputs and lse instead of
 *          a result.
 * Replaces flash_decode() src/flash_decode.py:236-370 and
 * decode_attention() src/decode_attn.py:137-166.
 */
int32_t mi_flash_decode(const void* q, const void* k, const void* v,
                        const uint8_t* mask, int64_t mask_sb, int64_t mask_sl,
                        const int64_t* seq_lens, float* part_m, float* part_l,
                        float* part_acc, uint64_t* arrive, void* out, float* lse,
                        int64_t batch,
                        int64_t n_heads, int64_t n_kv_heads, int64_t kv_len,
                        int64_t head_dim, int64_t num_splits, int64_t q_sb,
                        int64_t q_sh, int64_t q_sd, int64_t k_sb, int64_t k_sh,
                        int64_t k_sl, int64_t v_sb, int64_t v_sh, int64_t v_sl,
                        int64_t o_sb, int64_t o_sh, int64_t o_sd,
                        float sm_scale, int32_t empty_rows_nan, int32_t dtype,
                        void* stream);

/*
 * Arrival counters for mi_flash_decode's `arrive`, owned by the library:
 * *counters = a slab of MI_DECODE_ARRIVE_SLAB zeroed uint64 counters of the
 * current device reserved for `stream` (the same slab on every call with that
 * stream; calls on one stream never overlap, so they may share it).  The slabs
 * are part of the library's code object (no allocation); once
 * MI_DECODE_ARRIVE_SLABS streams of a device hold one, further streams get
 * MI_ERR_UNSUPPORTED (pass NULL: two launches).  A graph captured on a stream
 * keeps that stream's slab: replay it on that stream, or while no other call
 * runs on it.  No counterpart in the reference.
 */
#define MI_DECODE_ARRIVE_SLAB 8192
#define MI_DECODE_ARRIVE_SLABS 32
int32_t mi_decode_arrive_counters(void* stream, uint64_t** counters);

/*
 * mi_flash_decode without a caller workspace: the same kernels, with the split
 * partials kept in a library-owned device array of
 * MI_DECODE_NOALLOC_SCRATCH_BYTES per GPU (held until the process ends).  It
 * calls no hipMalloc/hipFree and allocates nothing, for callers that cannot
 * allocate (code under graph capture, serving loops that forbid allocation).
 * No counterpart in the reference.  The partials need
 * batch*n_heads*num_splits*(head_dim+2)*4 bytes (each array rounded up to 256
 * bytes) of the array's first 16 MiB - 64 KiB; larger calls return
 * MI_ERR_UNSUPPORTED before launching anything.  The last 64 KiB hold the
 * arrival counters of the in-launch combine (batch * n_heads <= 8192; larger
 * calls combine in a second launch).
 * Every call on one GPU shares that GPU's array: calls that overlap in time on
 * one device (different streams, or host threads) race and must not be issued.
 * num_splits == 1 uses no scratch.
 */
#define MI_DECODE_NOALLOC_SCRATCH_BYTES (16u << 20)
int32_t mi_flash_decode_noalloc(const void* q, const void* k, const void* v,
                                const uint8_t* mask, int64_t mask_sb, int64_t mask_sl,
                                const int64_t* seq_lens, void* out, float* lse,
                                int64_t batch, int64_t n_heads, int64_t n_kv_heads,
                                int64_t kv_len, int64_t head_dim, int64_t num_splits,
                                int64_t q_sb, int64_t q_sh, int64_t q_sd, int64_t k_sb,
                                int64_t k_sh, int64_t k_sl, int64_t v_sb, int64_t v_sh,
                                int64_t v_sl, int64_t o_sb, int64_t o_sh, int64_t o_sd,
                                float sm_scale, int32_t empty_rows_nan, int32_t dtype,
                                void* stream);

/*
 * Split count flash_decode runs for a requested num_splits on the current
 * device: unchanged once B * kv-head-groups * num_splits blocks cover the
 * compute units; below that, each requested split is subdivided into key
 * ranges of >= 1024 keys until they do (the output differs from the requested
 * split only in fp32 summation order).  The Python flash_decode and
 * mi_flash_decode_noalloc apply it; mi_flash_decode / mi_decode_split run
 * exactly the num_splits they are given.  No counterpart in the reference
 * (whose split size is fixed at 256 keys, src/flash_decode.py:271-272).
 */
int64_t mi_decode_effective_splits(int64_t batch, int64_t n_heads, int64_t n_kv_heads,
                                   int64_t kv_len, int64_t head_dim, int64_t num_splits);

/*
 * Split count the library would pick for a decode of this shape on the
 * current device (used when the caller passes no explicit num_splits).
 */
int64_t mi_decode_default_splits(int64_t batch, int64_t n_heads,
                                 int64_t n_kv_heads, int64_t kv_len,
                                 int64_t head_dim);

/*
 * Rotate-half RoPE of x [batch, n_heads, seq_len, head_dim] into out (any
 * strides).  Row s uses cos/sin row s of the [seq_len, head_dim/2] tables
 * (the caller slices the table at start_pos), or row positions[s] when
 * positions (device int64 [seq_len]) is not NULL.  table_rows is the number of
 * cos/sin rows (>= seq_len without positions; a position outside
 * [0, table_rows) uses the nearest row, as the fused prefill and decode RoPE
 * do).  cdtype is the table dtype.
 * Replaces rope_kernel + apply_rotary  src/rope.py:48-91, src/rope.py:94-119.
 */
int32_t mi_rope(const void* x, void* out, const void* cos, const void* sin,
                const int64_t* positions, int64_t table_rows, int64_t batch,
                int64_t n_heads, int64_t seq_len,
                int64_t head_dim, int64_t x_sb, int64_t x_sh, int64_t x_ss,
                int64_t x_sd, int64_t o_sb, int64_t o_sh, int64_t o_ss,
                int64_t o_sd, int64_t c_ss, int64_t c_sd, int64_t s_ss,
                int64_t s_sd, int32_t dtype, int32_t cdtype, void* stream);

/*
 * Fused K-RoPE + KV-cache append: cache_k[b, h, pos] = RoPE(xk[b, h, s]) and
 * cache_v[b, h, pos] = xv[b, h, s] (bitwise copy), with
 * pos = start_pos + s, or pos = positions[s] (device int64, one position per
 * token shared by the batch) when positions != NULL.  cache_k/cache_v point
 * at the layer view [batch, n_kv_heads, capacity, head_dim]; slots outside
 * [0, capacity) are never written.  cos/sin rows are indexed by s, or by pos
 * when cos_by_position != 0 (device-resident full table; a slot past its
 * table_rows rows uses the last row).  table_rows >= seq_len otherwise.  With
 * cos = sin = NULL, K is copied unrotated (plain cache write, KVCache.update)
 * and table_rows is ignored.
 * Replaces _rope_k_cache_write_seq_kernel / _scatter_kernel +
 * rope_and_cache_update  src/rope.py:122-252, src/rope.py:255-313.
 */
int32_t mi_rope_kv_append(const void* xk, const void* xv, const void* cos,
                          const void* sin, void* cache_k, void* cache_v,
                          int64_t start_pos, const int64_t* positions,
                          int64_t table_rows, int64_t batch,
                          int64_t n_kv_heads, int64_t seq_len,
                          int64_t head_dim, int64_t capacity, int64_t xk_sb,
                          int64_t xk_sh, int64_t xk_ss, int64_t xk_sd,
                          int64_t xv_sb, int64_t xv_sh, int64_t xv_ss,
                          int64_t xv_sd, int64_t ck_sb, int64_t ck_sh,
                          int64_t ck_st, int64_t ck_sd, int64_t cv_sb,
                          int64_t cv_sh, int64_t cv_st, int64_t cv_sd,
                          int64_t c_ss, int64_t c_sd, int64_t s_ss,
                          int64_t s_sd, int32_t cos_by_position, int32_t dtype,
                          int32_t cdtype, void* stream);

/*
 * Causal GQA prefill attention with optional fp32 LSE output.
 * q [batch, n_heads, seq_len, head_dim], k/v [batch, n_kv_heads, kv_len,
 * head_dim] (kv_len >= seq_len; only the first seq_len keys are used and
 * query row i attends keys 0..i), out like q, lse [batch, n_heads, seq_len]
 * fp32 (natural log of the scaled scores) or NULL.  Unit head-dim stride,
 * 16-byte aligned rows.  head_dim 16, 32, 64, 128 or 256 (any power of two
 * the reference kernel's tl.dot takes): bf16/fp16 at 32 to 256 run on MFMA,
 * head_dim 16 and fp32 on a VALU kernel in fp32 arithmetic.
 * Query head h reads kv head h / (n_heads / n_kv_heads).
 * Replaces flash_attention_kernel + flash_attention
 *   src/flash_attn.py:5-83, src/flash_attn.py:85-111.
 */
int32_t mi_attn_prefill(const void* q, const void* k, const void* v, void* out,
                        float* lse, int64_t batch, int64_t n_heads,
                        int64_t n_kv_heads, int64_t seq_len, int64_t kv_len,
                        int64_t head_dim, int64_t q_sb, int64_t q_sh,
                        int64_t q_ss, int64_t k_sb, int64_t k_sh, int64_t k_ss,
                        int64_t v_sb, int64_t v_sh, int64_t v_ss, int64_t o_sb,
                        int64_t o_sh, int64_t o_ss, float sm_scale,
                        int32_t dtype, void* stream);

/*
 * mi_attn_prefill with the rotate-half RoPE of q applied in the kernel's Q
 * prologue (q is read unrotated and never written): query row s of every
 * head uses row positions[s] of cos/sin (clamped into [0, table_rows)), or
 * row s when positions is NULL.  cos/sin [table_rows, >= head_dim/2] in q's
 * dtype, unit column stride, rows of table_row_stride elements (16-byte
 * aligned for bf16/fp16).  The result is bitwise that of mi_rope on q
 * followed by mi_attn_prefill.
 * Replaces apply_rotary(xq) + flash_attention of one prefill step
 *   src/rope.py:48-119 (rope_kernel, apply_rotary), src/flash_attn.py:5-111,
 *   as called by src/model.py:62-79.
 */
int32_t mi_attn_prefill_rope(const void* q, const void* k, const void* v, void* out,
                             float* lse, int64_t batch, int64_t n_heads, int64_t n_kv_heads,
                             int64_t seq_len, int64_t kv_len, int64_t head_dim, int64_t q_sb,
                             int64_t q_sh, int64_t q_ss, int64_t k_sb, int64_t k_sh,
                             int64_t k_ss, int64_t v_sb, int64_t v_sh, int64_t v_ss,
                             int64_t o_sb, int64_t o_sh, int64_t o_ss, float sm_scale,
                             const void* cos, const void* sin, int64_t table_rows,
                             int64_t table_row_stride, const int64_t* positions,
                             int32_t dtype, void* stream);

/*
 * RMSNorm over the last dim: y[r] = x[r] * rsqrt(mean(x[r]^2) + eps) * w,
 * fp32 internally, y in x's dtype (wdtype = weight dtype).  rows x n with row
 * strides x_rs / y_rs.
 * Replaces rms_norm_fwd_kernel + rmsnorm_triton  src/rms_norm.py:18-77.
 */
int32_t mi_rmsnorm(const void* x, const void* w, void* y, int64_t rows,
                   int64_t n, int64_t x_rs, int64_t y_rs, float eps,
                   int32_t dtype, int32_t wdtype, void* stream);

/*
 * Symmetric per-output-channel int8 quantisation of w [n_rows, k] (dtype):
 * scales[n] = dtype(max(max|w[n,:]|, 1e-12) / 127), q = clamp(rne(w / s),
 * -128, 127), every step IEEE-rounded (bit-exact with the reference recipe).
 * Replaces quantize_weight_symmetric_per_channel  src/quant_utils.py:7-36.
 */
int32_t mi_quantize_int8(const void* w, int8_t* q, void* scales,
                         int64_t n_rows, int64_t k, int64_t w_rs, int64_t q_rs,
                         int32_t dtype, void* stream);

/*
 * W8A16 GEMV, 1 <= m <= 16: y[m, n] = (sum_k x[m,k] * w[n,k]) * scales[n],
 * fp32 accumulate on MFMA, y in x's dtype (bf16/fp16).  w int8 [n, k] with
 * 16-byte aligned rows, k % 16 == 0.  sdtype = scales dtype.
 * Replaces w8a16_gemv_kernel + w8a16_gemv_launch
 *   src/quant_linear.py:7-63, src/quant_linear.py:66-120.
 */
int32_t mi_w8a16_gemv(const void* x, const int8_t* w, const void* scales,
                      void* y, int64_t m, int64_t n, int64_t k, int64_t x_sm,
                      int64_t x_sk, int64_t w_sn, int64_t s_sn, int64_t y_sm,
                      int64_t y_sn, int32_t dtype, int32_t sdtype,
                      void* stream);

/*
 * W8A16 GEMM for prefill-sized inputs (any m >= 1):
 * y[m, n] = (sum_k x[m,k] * w[n,k]) * scales[n], int8 widened exactly to x's
 * dtype, fp32 accumulate on MFMA, y in x's dtype (bf16/fp16).  x rows
 * (unit k stride, row stride x_sm elements) and w rows (w_sn bytes) 16-byte
 * aligned; k % 64 == 0; y has unit column stride and row stride y_sm.
 * Replaces w8a16_gemm_kernel + w8a16_gemm_launch
 *   src/quant_linear.py:123-188, src/quant_linear.py:191-247.
 */
int32_t mi_w8a16_gemm(const void* x, const int8_t* w, const void* scales,
                      void* y, int64_t m, int64_t n, int64_t k, int64_t x_sm,
                      int64_t w_sn, int64_t s_sn, int64_t y_sm, int32_t dtype,
                      int32_t sdtype, void* stream);

/*
 * Split count for mi_w8a16_gemm_splitk on the current device: 1 when the
 * 128 x 256 output tiles alone occupy every CU (use mi_w8a16_gemm), else the
 * number of K splits (each at least 128 deep, fp32 partials <= 64 MiB).
 * Same interface role as mi_w8a16_gemm (src/quant_linear.py:191-247).
 */
int64_t mi_w8a16_gemm_splits(int64_t m, int64_t n, int64_t k);

/*
 * mi_w8a16_gemm for grids too small to occupy the GPU: the K range is split
 * across `splits` workgroups per output tile, each writing unscaled fp32 sums
 * to part[split][m][n] (caller's workspace, >= splits * m * n elements), then
 * a second launch adds the splits in split order, applies scales[n] and
 * rounds to x's dtype.  2 <= splits <= min(k / 64, 64); other requirements as
 * mi_w8a16_gemm.  Replaces w8a16_gemm_kernel + w8a16_gemm_launch
 *   src/quant_linear.py:123-188, src/quant_linear.py:191-247 (small M).
 */
int32_t mi_w8a16_gemm_splitk(const void* x, const int8_t* w, const void* scales,
                             void* y, int64_t m, int64_t n, int64_t k,
                             int64_t x_sm, int64_t w_sn, int64_t s_sn,
                             int64_t y_sm, float* part, int64_t part_elems,
                             int64_t splits, int32_t dtype, int32_t sdtype,
                             void* stream);

/*
 * mi_w8a16_gemm (splits <= 1) or mi_w8a16_gemm_splitk (splits >= 2, with its
 * workspace) with the block's residual added in the epilogue:
 *   y[m, n] = dtype(res[m, n] + dtype((sum_k x[m,k] w[n,k]) * scales[n]))
 * (the roundings of the projection and of the add as separate ops); res
 * [m, n] in x's dtype, unit column stride, row stride res_sm (>= n).
 * Replaces h = x + self.wo(attn) and out = h + self.w2(...) of a prefill
 * block  src/model.py:113-127 with src/quant_linear.py:191-292.
 */
int32_t mi_w8a16_gemm_residual(const void* x, const int8_t* w, const void* scales,
                               const void* res, void* y, int64_t m, int64_t n,
                               int64_t k, int64_t x_sm, int64_t w_sn, int64_t s_sn,
                               int64_t res_sm, int64_t y_sm, float* part,
                               int64_t part_elems, int64_t splits, int32_t dtype,
                               int32_t sdtype, void* stream);

/*
 * The gated feed-forward input of a prefill block in one launch:
 *   y[m, n] = dtype(dtype(silu(y1)) * y3),  y1 = dtype((x w1^T)[m, n] * s1[n]),
 *                                           y3 = dtype((x w3^T)[m, n] * s3[n])
 * (the roundings of w1(x), w3(x), silu and the product as separate ops; silu
 * is evaluated with the hardware exp2 and reciprocal, so an element can be
 * one unit in the last place off the separate ops' result), with w1 and w3
 * [n, k] int8 and everything else as mi_w8a16_gemm; neither projection is
 * written out.  Replaces silu(self.w1(x)) * self.w3(x) of the
 * W8A16 feed-forward  src/model.py:23, src/quant_linear.py:191-292.
 */
int32_t mi_w8a16_gemm_swiglu(const void* x, const int8_t* w1, const void* scales1,
                             const int8_t* w3, const void* scales3, void* y,
                             int64_t m, int64_t n, int64_t k, int64_t x_sm,
                             int64_t w1_sn, int64_t s1_sn, int64_t w3_sn,
                             int64_t s3_sn, int64_t y_sm, int32_t dtype,
                             int32_t sdtype, void* stream);

/*
 * n_mats (1..4) GEMMs of the same activation x in one launch, e.g. a layer's
 * q, k and v projections: y_i = mi_w8a16_gemm(x, w_i, scales_i) for each i,
 * bit for bit, with the output tiles of all matrices in one grid (no tail
 * round per matrix).  w, scales and y are host arrays of n_mats device
 * pointers; n, w_sn, s_sn and y_sm host arrays of n_mats values; each matrix
 * meets mi_w8a16_gemm's requirements.  Replaces the three
 * W8A16Linear.forward -> w8a16_gemm_launch calls of a prefill attention block
 *   src/model.py:54 with src/quant_linear.py:191-247, 250-292.
 */
int32_t mi_w8a16_gemm_multi(const void* x, int64_t m, int64_t k, int64_t x_sm,
                            int32_t n_mats, const int8_t* const* w,
                            const void* const* scales, void* const* y,
                            const int64_t* n, const int64_t* w_sn,
                            const int64_t* s_sn, const int64_t* y_sm,
                            int32_t dtype, int32_t sdtype, void* stream);

/*
 * Fused decode-step projection (1 <= m <= 16 rows; k one of 512, 1024, 1536,
 * 2048, 3072, 4096, 6144, 8192):
 *   a   = rmsnorm(x, norm_w, eps) if norm_w != NULL else x   (rounded to dtype)
 *   y_a = dtype((sum_k a[m,k] * w_a[n,k]) * s_a[n])
 * then, by epilogue:
 *   0  y = y_a
 *   1  y = dtype(res + y_a)                                   (residual add)
 *   2  y = dtype(dtype(silu(y_a)) * y_b), y_b from w_b / s_b  (SwiGLU, k <= 4096)
 * Weights int8 [n, k] with 16-byte aligned rows (row strides w_sn_* bytes),
 * scales in the activation dtype (bf16/fp16), x/res/y rows in elements.  With
 * norm_w, m*k*2 <= 64 KB and k <= 2048 above 8 rows.  Each weight matrix and
 * x must span < 2 GB (32-bit buffer offsets).  Unsupported shapes
 * return MI_ERR_UNSUPPORTED.  Each step rounds where the reference's separate ops
 * round, so results equal the unfused chain up to fp32 summation order.
 * Replaces, fused into one launch: rmsnorm_triton  src/rms_norm.py:42-77;
 *   W8A16Linear / w8a16_gemv_launch  src/quant_linear.py:66-120, :250-292;
 *   the residual adds  src/model.py:113-127; silu(w1 x) * w3 x  src/model.py:23.
 */
int32_t mi_w8a16_linear_fused(const void* x, int64_t x_sm, const void* norm_w,
                              float eps, const int8_t* w_a, const void* s_a,
                              int64_t w_sn_a, const int8_t* w_b, const void* s_b,
                              int64_t w_sn_b, const void* res, int64_t res_sm,
                              void* y, int64_t y_sm, int64_t m, int64_t n,
                              int64_t k, int32_t epilogue, int32_t dtype,
                              void* stream);

/*
 * Fused decode-step attention input (1 <= m <= 16 rows): a = rmsnorm(x) (if
 * norm_w), q/k/v = W8A16 projections of a (rounded to dtype), then
 *   q_out[m, h, d]           = RoPE(q)   (q_out [m, n_heads, head_dim])
 *   cache_k[m, kvh, pos, d]  = RoPE(k),   cache_v[m, kvh, pos, d] = v
 * with pos = *pos (device int64, shared by all rows; slots outside
 * [0, capacity) are not written) and RoPE rows cos/sin[pos - rope_row0]
 * (rope_rows rows, row stride c_ss), rotate-half in fp32 with products and
 * sum rounded separately.  Cache views are the layer's [m, kvh, T, head_dim]
 * with element strides (c_sb, c_sh, c_st, 1).
 * Replaces, fused into one launch: rmsnorm_triton  src/rms_norm.py:42-77;
 *   wq / wk / wv  src/model_quantized.py:57-60; apply_rotary  src/rope.py:94-119;
 *   rope_and_cache_update (scatter path)  src/rope.py:188-252, :255-313.
 */
int32_t mi_w8a16_qkv_rope_append(
    const void* x, int64_t x_sm, const void* norm_w, float eps, const int8_t* wq,
    const void* sq, int64_t wq_sn, const int8_t* wk, const void* sk, int64_t wk_sn,
    const int8_t* wv, const void* sv, int64_t wv_sn, const void* cos, const void* sin,
    int64_t c_ss, int64_t rope_row0, int64_t rope_rows, const int64_t* pos, void* q_out,
    void* cache_k, void* cache_v, int64_t c_sb, int64_t c_sh, int64_t c_st,
    int64_t capacity, int64_t m, int64_t k, int64_t n_heads, int64_t n_kv_heads,
    int64_t head_dim, int32_t dtype, void* stream);

/*
 * Decode-step output projection (lm_head), 1 <= m <= 16 rows, k % 512 == 0,
 * k <= 4096, bf16/fp16:
 *   a        = rmsnorm(x, norm_w, eps) if norm_w != NULL else x  (rounded to dtype)
 *   y[m, n]  = dtype(sum_k a[m, k] * w[n, k])                    (fp32 accumulate)
 *   argmax_out[m] = first n with y[m, n] == max_n y[m, n]   (if argmax_out != NULL)
 * x [m, k] (row stride x_sm), w [n, k] in x's dtype (row stride w_sn), y [m, n]
 * (row stride y_sm); x/w/norm_w rows 16-byte aligned.  The
 * argmax needs fp32 part_v and int32 part_i workspaces of n_parts >=
 * mi_lm_head_partials(m, n) entries per row (row stride n_parts); NaN logits
 * are not ranked.  Two launches with argmax, one without.
 * Replaces, fused: the final norm + output Linear  src/model.py:137,183
 * (RMSNorm src/rms_norm.py:32-38) and greedy sampling's torch.argmax
 * src/sampler.py:30 (the per-token host sync of main.py:260 becomes a device
 * tensor).
 */
int32_t mi_lm_head(const void* x, int64_t x_sm, const void* norm_w, float eps,
                   const void* w, int64_t w_sn, void* y, int64_t y_sm,
                   int64_t* argmax_out, float* part_v, int32_t* part_i,
                   int64_t n_parts, int64_t m, int64_t n, int64_t k, int32_t dtype,
                   void* stream);

/* Partial-buffer entries per row that mi_lm_head's argmax needs (0 if m or n <= 0). */
int64_t mi_lm_head_partials(int64_t m, int64_t n);

#ifdef __cplusplus
}
#endif

#endif /* MIATTN_H_ */
