/*
 * dexter_gfx950.h -- C ABI of the MI355X (gfx950) blockwise-causal attention path.
 *
 * One shared library, libdexter_gfx950.so, exports these entry points. They
 * replace the device side of three pieces of dexter (raikonenfnu/dexter-labs),
 * cited below as path:line under python/dexter/:
 *
 *   dx_qk_norm_rope          ops/gfx1151/rope/qk_norm_rope.py:93-110
 *                            (semantics: ops/reference/rope.py:10-56,
 *                             dispatcher ops/__init__.py:66-86)
 *   dx_qk_norm_rope_append   the same, plus KVCache.append of the rotated k and
 *                            the raw v (models/dreamzero/model.py:53-58,166-175)
 *   dx_kv_append             KVCache.append, models/dreamzero/model.py:53-58
 *   dx_blockwise_causal_attention
 *                            ops/gfx1151/attention/blockwise_causal.py:146-173
 *                            (semantics: ops/reference/attention.py:22-77,
 *                             dispatcher ops/__init__.py:127-147)
 *   dx_blockwise_causal_attention_varlen
 *                            the same with one cache length per sequence; the
 *                            reference has a scalar cache_len only, and a
 *                            ragged batch there is one call per sequence.
 *   dx_qk_norm_rope_append_dev, dx_kv_append_dev, dx_blockwise_causal_attention_dev
 *                            the same three with the cache cursor (start row /
 *                            cached length) read from device memory, so one
 *                            captured graph serves every control step while
 *                            the cache grows; the reference captures only
 *                            cache-free steps (runtime/graph.py:50-74)
 *   dx_qkv_norm_rope         the q/k/v projections of SelfAttention.forward
 *                            (models/dreamzero/model.py:162-165, three
 *                            nn.Linear calls; on gfx1151 hipBLASLt through
 *                            ops/gfx1151/gemm) fused with dx_qk_norm_rope(_append)
 *                            (model.py:166-175)
 *   dx_adaln_modulate        ops/gfx1151/norm/adaln.py:108-128 (kernel :20-48;
 *                            semantics ops/reference/norm.py:16-20, dispatcher
 *                            ops/__init__.py:39-49)
 *   dx_gated_residual        ops/gfx1151/norm/adaln.py:131-148 (kernel :51-67;
 *                            semantics ops/reference/norm.py:23-25, dispatcher
 *                            ops/__init__.py:52-54)
 *
 * Conventions
 *  - Tensors are device pointers with explicit element strides; the last
 *    (head_dim) dimension must be contiguous. [B, L, H, D] tensors take
 *    strides (sb, sl, sh). A KV cache [2, B, S, H, D] takes (plane, sb, ss, sh):
 *    plane 0 holds K, plane 1 holds V.
 *  - dtype codes: DX_BF16, DX_F16, DX_F32.
 *  - stream is a hipStream_t (NULL = the legacy default stream). Every entry
 *    point only enqueues work: no allocation, no host synchronisation, so the
 *    calls are safe under HIP graph capture. Functions are re-entrant and may
 *    be called from any host thread.
 *  - Return 0 on success or a DX_E* code; dx_last_error() then describes the
 *    failure of the calling thread's last failed call.
 */
#ifndef DEXTER_GFX950_H
#define DEXTER_GFX950_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DX_OK 0
#define DX_EINVAL 1   /* bad shape, stride, dtype or argument */
#define DX_ELAUNCH 2  /* the HIP runtime refused a launch */
#define DX_EFULL 3    /* KV cache overflow: start + n > capacity */
#define DX_EWORKSPACE 4 /* workspace smaller than dx_attention_workspace_bytes() */

#define DX_BF16 0
#define DX_F16 1
#define DX_F32 2
#define DX_I32 3
#define DX_I64 4

/* Message for the calling thread's last failed call ("" if none). */
const char* dx_last_error(void);

/* ABI revision of this header; the Python loader checks it. */
int dx_abi_version(void);
#define DX_ABI_VERSION 10

/*
 * Launch-schedule overrides, for measurement and tests only: process-wide,
 * 0 (the default) leaves the choice to the library. Results stay within the
 * documented accuracy under every override; schedules differ in rounding.
 * Nothing in the library reads the environment.
 *   DX_TUNE_ATTN_SPLITS  key splits per attention work item (1..16)
 *   DX_TUNE_ATTN_KERNEL  attention kernel: 1 single-stream, 2 dual-stream
 *                        with a separate merge kernel, 3 paired prefill,
 *                        4 one-launch decode
 *   DX_TUNE_NORM_WAVES   waves per row of the adaLN / gated-residual kernels (1..16)
 *   DX_TUNE_QKV_SPLITS   K splits of the fused QKV GEMM (1..16)
 *   DX_TUNE_QKV_WAVES    fused QKV GEMM form: 0 the LDS-DMA form (waves of 64
 *                        features), 2 or 4 the register-ring form with that
 *                        many waves of 32 features
 *   DX_TUNE_ATTN_MERGE   one-launch decode merge: 1 through the L2 when the
 *                        splits share an XCD (the default), 2 at device
 *                        scope only (for tests)
 *   DX_TUNE_ATTN_PMERGE  key splits of the paired and dual-stream kernels:
 *                        1 merged by a separate merge kernel, 2 in the same
 *                        launch (the last split of each query tile to finish
 *                        merges all of its partials), 3 in the same launch
 *                        spread over the splits (dual-stream kernel: each
 *                        split merges a chunk of the rows once its group has
 *                        arrived; the paired kernel takes 2). Default: 2
 *                        for the paired kernel and for ragged batches on the
 *                        dual-stream kernel, else 1
 * Returns DX_EINVAL for an unknown key or an out-of-range value.
 * No reference counterpart (the reference's tuning is Triton's autotuner).
 */
#define DX_TUNE_ATTN_SPLITS 0
#define DX_TUNE_ATTN_KERNEL 1
#define DX_TUNE_NORM_WAVES 2
#define DX_TUNE_QKV_SPLITS 3
#define DX_TUNE_QKV_WAVES 4
#define DX_TUNE_ATTN_MERGE 5
#define DX_TUNE_ATTN_PMERGE 6
#define DX_TUNE_KEYS 7
int dx_set_tuning(int key, int value);

/*
 * QK-RMSNorm + rotary on q and k, one token's whole H*D plane at a time.
 *   out = rope(round_io(x * rsqrt(mean(x^2 over H*D) + eps) * w))
 * with the rotation in fp32 and a final round to the io dtype, the order of
 * ops/reference/rope.py:29-40 then :10-26. interleaved != 0 pairs (2j, 2j+1);
 * otherwise (j, j + D/2). cos/sin are [L, D/2] rows (row strides cos_sl,
 * sin_sl), shared by every batch and head. q_out/k_out are contiguous
 * [B, L, H, D]. io_dtype: DX_BF16 or DX_F16; weight_dtype and table_dtype:
 * DX_BF16, DX_F16 or DX_F32.
 * Replaces: ops/gfx1151/rope/qk_norm_rope.py:93-110.
 */
int dx_qk_norm_rope(const void* q, int64_t q_sb, int64_t q_sl, int64_t q_sh,
                    const void* k, int64_t k_sb, int64_t k_sl, int64_t k_sh,
                    int io_dtype,
                    const void* q_weight, const void* k_weight, int weight_dtype,
                    const void* cos, int64_t cos_sl, const void* sin, int64_t sin_sl,
                    int table_dtype,
                    void* q_out, void* k_out,
                    int64_t B, int64_t L, int64_t H, int64_t D,
                    float eps, int interleaved, void* stream);

/*
 * dx_qk_norm_rope, and in the same pass the rotated k and the unmodified v
 * [B, L, H, D] are written to rows [start, start + L) of the cache planes.
 * Returns DX_EFULL (nothing launched) when start + L > capacity.
 * Replaces: ops/gfx1151/rope/qk_norm_rope.py:93-110 followed by
 * models/dreamzero/model.py:53-58 (KVCache.append).
 */
int dx_qk_norm_rope_append(const void* q, int64_t q_sb, int64_t q_sl, int64_t q_sh,
                           const void* k, int64_t k_sb, int64_t k_sl, int64_t k_sh,
                           const void* v, int64_t v_sb, int64_t v_sl, int64_t v_sh,
                           int io_dtype,
                           const void* q_weight, const void* k_weight, int weight_dtype,
                           const void* cos, int64_t cos_sl, const void* sin, int64_t sin_sl,
                           int table_dtype,
                           void* q_out, void* k_out,
                           void* cache, int64_t c_plane, int64_t c_sb, int64_t c_ss,
                           int64_t c_sh, int64_t capacity, int64_t start,
                           int64_t B, int64_t L, int64_t H, int64_t D,
                           float eps, int interleaved, void* stream);

/*
 * Copy k and v [B, n, H, D] into rows [start, start + n) of planes 0 and 1 of
 * a [2, B, capacity, H, D] cache. Bit-exact copy. dtype: DX_BF16, DX_F16 or
 * DX_F32. Returns DX_EFULL (nothing launched) when start + n > capacity.
 * Replaces: models/dreamzero/model.py:53-58 (KVCache.append).
 */
int dx_kv_append(const void* k, int64_t k_sb, int64_t k_sl, int64_t k_sh,
                 const void* v, int64_t v_sb, int64_t v_sl, int64_t v_sh,
                 void* cache, int64_t c_plane, int64_t c_sb, int64_t c_ss, int64_t c_sh,
                 int dtype, int64_t B, int64_t n, int64_t H, int64_t D,
                 int64_t capacity, int64_t start, void* stream);

/*
 * Blockwise-causal flash attention forward.
 *   keys/values = [cache rows 0..cache_len) | k/v rows 0..Lk)]
 *   query i sees key j iff j < cache_len + end(i), where end(i) is
 *     causal != 0          : i + 1
 *     n_blocks == 0        : Lk (one block: every current key)
 *     otherwise            : the union over the pairs (lo, hi) of consecutive
 *                            entries of (starts..., Lq) whose row slice
 *                            [lo:hi] holds i (Python slicing over Lq rows),
 *                            of pair_end(hi): min(hi, Lq) for hi >= 0; for
 *                            hi < 0, max(cache_len + Lq + hi, 0) when
 *                            cache_len + hi < 0 (the reference's column stop
 *                            cache_len + hi then counts from the end of the
 *                            key axis), else 0; 0 if no pair holds i
 *   (ops/reference/attention.py:22-47). With causal or block starts Lk must
 *   equal Lq, as the reference's mask shape requires. Lk != Lq with
 *   n_blocks == 0 and causal == 0 is cross-attention: every key visible (the
 *   reference's mask cannot take it, attention.py:30; the model calls it so,
 *   models/dreamzero/model.py:234-241). A query with no visible key yields NaN,
 *   as the reference's softmax over an all -inf row does.
 * Grouped-query attention: q has H heads, k, v and the cache Hkv heads, H a
 *   multiple of Hkv; query head h reads K/V head h / (H / Hkv), the head that
 *   k.repeat_interleave(H / Hkv, dim=2) would put at h (vla/groot/backbone.py:109-114).
 * block_starts: device pointer to n_blocks int32 (starts_dtype DX_I32) or
 * int64 (DX_I64) block start indices, read on the device (no host sync), in
 * any order and of any sign, as the reference takes them; ascending
 * non-negative starts (the reference builds them with torch.arange) let the
 * kernels skip whole future tiles, any other list is masked key by key.
 * softmax_scale multiplies q.k before the softmax (the reference's default
 * is 1/sqrt(D); callers pass it explicitly). dtype: DX_BF16, DX_F16 or DX_F32
 * (q, k, v, the cache and out all of it); D: 16, 32, 64, 128 or 256. bf16/f16
 * at D 64 or 128 run on the 16-bit MFMA kernels; fp32 (any D) and bf16/f16 at
 * D 16, 32 or 256 on the general kernels (fp32 softmax and sums, products of
 * the inputs as they are: fp32, or 16-bit MFMA for bf16/f16 at D 32 and 256;
 * one rounding to dtype). Strides are multiples of 16 bytes.
 * out may be strided like q. cache may be NULL when cache_len == 0.
 * workspace must hold dx_attention_workspace_bytes(...) bytes for the same
 * shape (it may be NULL when that is 0). Its first 256 KiB hold the
 * arrival counters of the kernels that merge key splits in the same launch
 * (by default the prefill kernel and the decode kernel on ragged batches; the
 * one-launch decode kernel under DX_TUNE_ATTN_KERNEL 4): they must be zero
 * before a workspace is first used, and every completed call leaves them
 * zero. The rest needs no initialisation. Calls that share a workspace must
 * not overlap.
 * Replaces: ops/gfx1151/attention/blockwise_causal.py:146-173.
 */
int dx_blockwise_causal_attention(
    const void* q, int64_t q_sb, int64_t q_sl, int64_t q_sh,
    const void* k, int64_t k_sb, int64_t k_sl, int64_t k_sh,
    const void* v, int64_t v_sb, int64_t v_sl, int64_t v_sh,
    const void* cache, int64_t c_plane, int64_t c_sb, int64_t c_ss, int64_t c_sh,
    void* out, int64_t o_sb, int64_t o_sl, int64_t o_sh,
    int dtype, int64_t B, int64_t Lq, int64_t Lk, int64_t H, int64_t Hkv, int64_t D,
    int64_t cache_len, const void* block_starts, int starts_dtype, int64_t n_blocks,
    int causal, float softmax_scale,
    void* workspace, int64_t workspace_bytes, void* stream);

/*
 * As dx_blockwise_causal_attention, allocating nothing: the workspace is a
 * static per-device scratch of DX_ATTN_SCRATCH_BYTES (64 MiB) in the
 * library, held by each device the library runs on until the process ends.
 * A call whose dx_attention_workspace_bytes(...) exceeds it fails with
 * DX_EWORKSPACE before any launch. The call makes no hipMalloc/hipFree; the
 * first call on a device also launches a small kernel that clears the
 * scratch's counter region. Every call on a device shares that device's
 * scratch, so calls that overlap on one device (concurrent streams) race.
 * No counterpart in the reference: for callers that cannot allocate (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).
 */
#define DX_ATTN_SCRATCH_BYTES (64ll << 20)
int dx_blockwise_causal_attention_noalloc(
    const void* q, int64_t q_sb, int64_t q_sl, int64_t q_sh,
    const void* k, int64_t k_sb, int64_t k_sl, int64_t k_sh,
    const void* v, int64_t v_sb, int64_t v_sl, int64_t v_sh,
    const void* cache, int64_t c_plane, int64_t c_sb, int64_t c_ss, int64_t c_sh,
    void* out, int64_t o_sb, int64_t o_sl, int64_t o_sh,
    int dtype, int64_t B, int64_t Lq, int64_t Lk, int64_t H, int64_t Hkv, int64_t D,
    int64_t cache_len, const void* block_starts, int starts_dtype, int64_t n_blocks,
    int causal, float softmax_scale, void* stream);

/*
 * As dx_blockwise_causal_attention, with cache_lens[b] (a host array of B
 * values, copied into the launch arguments) as sequence b's cached length.
 * B <= 64.
 */
int dx_blockwise_causal_attention_varlen(
    const void* q, int64_t q_sb, int64_t q_sl, int64_t q_sh,
    const void* k, int64_t k_sb, int64_t k_sl, int64_t k_sh,
    const void* v, int64_t v_sb, int64_t v_sl, int64_t v_sh,
    const void* cache, int64_t c_plane, int64_t c_sb, int64_t c_ss, int64_t c_sh,
    void* out, int64_t o_sb, int64_t o_sl, int64_t o_sh,
    int dtype, int64_t B, int64_t Lq, int64_t Lk, int64_t H, int64_t Hkv, int64_t D,
    const int64_t* cache_lens, const void* block_starts, int starts_dtype,
    int64_t n_blocks, int causal, float softmax_scale,
    void* workspace, int64_t workspace_bytes, void* stream);

/*
 * SelfAttention's decode step in one call: the QK-RMSNorm + rotary prologue
 * of dx_qk_norm_rope (q_out, k_out written [B, L, H, D] contiguous, 16-byte
 * aligned), with append != 0 also the cache write of dx_qk_norm_rope_append
 * (rotated k and v into rows [cache_len, cache_len + L); DX_EFULL when
 * cache_len + L > capacity), then dx_blockwise_causal_attention of q_out over
 * the cache's first cache_len rows and k_out, v (Lq = Lk = L, H = Hkv).
 * Arguments as in those entry points; workspace: dx_attention_workspace_bytes
 * (B, L, L, H, D, cache_len, NULL) bytes, under the same zero-counter rule.
 * Two launches (the prologue kernel, then attention) behind one call: q_out,
 * k_out, the cache rows and out are the same bits as dx_qk_norm_rope(_append)
 * followed by dx_blockwise_causal_attention.
 * Replaces: models/dreamzero/model.py:166-182 (SelfAttention.forward's
 * ops.qk_norm_rope, kv_cache.append and ops.blockwise_causal_attention).
 */
int dx_qk_norm_rope_attention(
    const void* q, int64_t q_sb, int64_t q_sl, int64_t q_sh,
    const void* k, int64_t k_sb, int64_t k_sl, int64_t k_sh,
    const void* v, int64_t v_sb, int64_t v_sl, int64_t v_sh,
    int io_dtype, const void* q_weight, const void* k_weight, int weight_dtype,
    const void* cos, int64_t cos_sl, const void* sin, int64_t sin_sl, int table_dtype,
    float eps, int interleaved, void* q_out, void* k_out,
    void* cache, int64_t c_plane, int64_t c_sb, int64_t c_ss, int64_t c_sh,
    int64_t capacity, int64_t cache_len, int append,
    void* out, int64_t o_sb, int64_t o_sl, int64_t o_sh,
    int64_t B, int64_t L, int64_t H, int64_t D,
    const void* block_starts, int starts_dtype, int64_t n_blocks, int causal,
    float softmax_scale, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Device-cursor forms. The cache row count (attention) or start row (appends)
 * is an int32 in device memory, read by the kernels when they run: a HIP
 * graph captured once replays correctly after the cursor moves (a captured
 * torch add_ on the cursor moves it). The host cannot check the cursor, so:
 *  - attention clamps it to [0, cache_capacity] and is planned (split count,
 *    workspace) for cache_capacity rows: call dx_attention_workspace_bytes
 *    with cache_len = cache_capacity;
 *  - an append whose block would not fit in capacity rows writes no cache row
 *    and sets *status to 1 (status may be NULL); the prologue still writes
 *    q_out and k_out.
 * Otherwise identical to dx_blockwise_causal_attention, dx_kv_append and
 * dx_qk_norm_rope_append.
 * Replaces: the cache-free restriction of runtime/graph.py:50-74
 * (capture_denoise_step), with models/dreamzero/model.py:53-58,166-175.
 */
int dx_blockwise_causal_attention_dev(
    const void* q, int64_t q_sb, int64_t q_sl, int64_t q_sh,
    const void* k, int64_t k_sb, int64_t k_sl, int64_t k_sh,
    const void* v, int64_t v_sb, int64_t v_sl, int64_t v_sh,
    const void* cache, int64_t c_plane, int64_t c_sb, int64_t c_ss, int64_t c_sh,
    void* out, int64_t o_sb, int64_t o_sl, int64_t o_sh,
    int dtype, int64_t B, int64_t Lq, int64_t Lk, int64_t H, int64_t Hkv, int64_t D,
    const void* cache_len_dev, int64_t cache_capacity,
    const void* block_starts, int starts_dtype, int64_t n_blocks,
    int causal, float softmax_scale,
    void* workspace, int64_t workspace_bytes, void* stream);

int dx_kv_append_dev(const void* k, int64_t k_sb, int64_t k_sl, int64_t k_sh,
                     const void* v, int64_t v_sb, int64_t v_sl, int64_t v_sh,
                     void* cache, int64_t c_plane, int64_t c_sb, int64_t c_ss, int64_t c_sh,
                     int dtype, int64_t B, int64_t n, int64_t H, int64_t D,
                     int64_t capacity, const void* start_dev, void* status, void* stream);

int dx_qk_norm_rope_append_dev(const void* q, int64_t q_sb, int64_t q_sl, int64_t q_sh,
                               const void* k, int64_t k_sb, int64_t k_sl, int64_t k_sh,
                               const void* v, int64_t v_sb, int64_t v_sl, int64_t v_sh,
                               int io_dtype,
                               const void* q_weight, const void* k_weight, int weight_dtype,
                               const void* cos, int64_t cos_sl, const void* sin, int64_t sin_sl,
                               int table_dtype,
                               void* q_out, void* k_out,
                               void* cache, int64_t c_plane, int64_t c_sb, int64_t c_ss,
                               int64_t c_sh, int64_t capacity, const void* start_dev,
                               void* status,
                               int64_t B, int64_t L, int64_t H, int64_t D,
                               float eps, int interleaved, void* stream);

/*
 * Workspace bytes the attention entry points need for this shape on the
 * current device (split-KV partial results); 0 when the launch does not split.
 * Pass cache_len and cache_lens = NULL for dx_blockwise_causal_attention, or
 * the same cache_lens array (cache_len ignored) for the varlen entry point.
 * It takes no dtype: the bytes cover every dtype of the shape (at D 64 and
 * 128 an fp32 call splits its keys no further than fits the bf16/f16 plan's
 * bytes). The general kernel never writes the first 256 KiB (the counters).
 * Returns a negative DX_E* code on a bad shape.
 */
int64_t dx_attention_workspace_bytes(int64_t B, int64_t Lq, int64_t Lk, int64_t H,
                                     int64_t D, int64_t cache_len,
                                     const int64_t* cache_lens);

/*
 * QKV projection of a decode chunk fused with the QK-RMSNorm + rotary
 * prologue and the KV-cache write:
 *   q = x wq^T + bq, k = x wk^T + bk, v = x wv^T + bv   (nn.Linear, rounded
 *       once to io_dtype: the projections' outputs)
 *   (q_out, k_out) = dx_qk_norm_rope(q, k, ...), v_out = v
 *   and, when cache != NULL, the rotated k and v written to rows
 *   [start, start + L) of the cache (start from start_dev when that is not
 *   NULL, with the device-cursor rules of dx_kv_append_dev).
 * x is [B, L, C] (strides x_sb, x_sl; C contiguous); wq/wk/wv are [H*D, C]
 * (row stride w_row, the nn.Linear weight layout); bq/bk/bv are [H*D] or NULL.
 * q_out, k_out, v_out are contiguous [B, L, H, D]. Limits: B*L <= 128 tokens
 * (decode chunks), C a multiple of 512, H*D a multiple of 128 and at most
 * 8192, x spanning less than 2^31 bytes, w_row below 2^22 elements. workspace: dx_qkv_workspace_bytes(...) bytes, 16-byte aligned (fp32
 * split-K partial products; no initialisation needed).
 * Replaces: models/dreamzero/model.py:162-175 (three nn.Linear, then
 * ops.qk_norm_rope and KVCache.append).
 */
int dx_qkv_norm_rope(const void* x, int64_t x_sb, int64_t x_sl, int io_dtype,
                     const void* wq, const void* wk, const void* wv, int64_t w_row,
                     const void* bq, const void* bk, const void* bv,
                     const void* q_weight, const void* k_weight, int weight_dtype,
                     const void* cos, int64_t cos_sl, const void* sin, int64_t sin_sl,
                     int table_dtype,
                     void* q_out, void* k_out, void* v_out,
                     void* cache, int64_t c_plane, int64_t c_sb, int64_t c_ss, int64_t c_sh,
                     int64_t capacity, int64_t start, const void* start_dev, void* status,
                     int64_t B, int64_t L, int64_t C, int64_t H, int64_t D,
                     float eps, int interleaved,
                     void* workspace, int64_t workspace_bytes, void* stream);

/* Workspace bytes dx_qkv_norm_rope needs for this shape; negative DX_E* on a bad shape. */
int64_t dx_qkv_workspace_bytes(int64_t B, int64_t L, int64_t C, int64_t H, int64_t D);

/*
 * Adaptive LayerNorm modulation of a [B, L, C] activation:
 *   out = layer_norm(x over C, no affine, eps) * (1 + scale) + shift
 * (ops/reference/norm.py:16-20). Statistics and arithmetic in fp32 with one
 * final rounding (the math of ops/gfx1151/norm/adaln.py:36-48). scale and
 * shift are [B, L, C] through their strides: stride 0 broadcasts, so a
 * [B, 1, C] modulation takes sc_sl = 0 and a [C] one takes sc_sb = sc_sl = 0.
 * The last dim of every operand is contiguous. scale and shift share
 * mod_dtype; out_dtype must be the torch promotion of x_dtype and mod_dtype
 * (equal types stay, any other pair is DX_F32). Dtypes: DX_BF16, DX_F16, DX_F32.
 * C <= 65536 for 16-bit x, 32768 for f32 x.
 * Replaces: ops/gfx1151/norm/adaln.py:108-128.
 */
int dx_adaln_modulate(const void* x, int64_t x_sb, int64_t x_sl, int x_dtype,
                      const void* scale, int64_t sc_sb, int64_t sc_sl,
                      const void* shift, int64_t sh_sb, int64_t sh_sl, int mod_dtype,
                      void* out, int64_t o_sb, int64_t o_sl, int out_dtype,
                      int64_t B, int64_t L, int64_t C, float eps, void* stream);

/*
 * Gated residual of [B, L, C] activations: out = x + y * gate
 * (ops/reference/norm.py:23-25), as an fp32 product and an fp32 sum, each
 * rounded, then one rounding to out_dtype. x and y share x_dtype; gate is
 * [B, L, C] through its strides (0 broadcasts) with gate_dtype; out_dtype
 * must be the promotion of x_dtype and gate_dtype. Same limits as
 * dx_adaln_modulate.
 * Replaces: ops/gfx1151/norm/adaln.py:131-148.
 */
int dx_gated_residual(const void* x, int64_t x_sb, int64_t x_sl,
                      const void* y, int64_t y_sb, int64_t y_sl, int x_dtype,
                      const void* gate, int64_t g_sb, int64_t g_sl, int gate_dtype,
                      void* out, int64_t o_sb, int64_t o_sl, int out_dtype,
                      int64_t B, int64_t L, int64_t C, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DEXTER_GFX950_H */
