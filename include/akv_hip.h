/*
 * akv_hip.h -- C ABI of libakv_hip.so, the MI355X (gfx950) warm-tier hot path
 * of Adaptive KV Memory: bit-packing, block-affine quantize + pack, fused
 * dequant-attention over a hot fp16 + warm packed KV cache, and the
 * attention-sum importance update.
 *
 * Conventions (every entry point):
 *   - plain pointers to DEVICE memory and sizes; no framework types;
 *   - contiguous row-major tensors unless a field says otherwise;
 *   - work is enqueued asynchronously on `stream` (a hipStream_t, NULL = the
 *     default stream); nothing synchronises, nothing allocates device memory,
 *     no pointer is kept after return;
 *   - the return value is AKV_OK (0) or a negative AKV_E_* code, with a
 *     readable message in akv_last_error() (thread-local);
 *   - device pointers must be 16-byte aligned (AKV_E_ALIGN otherwise).
 *
 * Reference interfaces each entry point replaces are cited as file:line of
 * the reference repository (Arvind679715/adaptive-kv-memory).
 */
#ifndef AKV_HIP_H
#define AKV_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AKV_ABI_VERSION 5

/* status codes */
#define AKV_OK 0
#define AKV_E_INVALID (-1)     /* bad argument (null pointer, negative size, ...) */
#define AKV_E_BITS (-2)        /* unsupported bit width (reference raises ValueError) */
#define AKV_E_SHAPE (-3)       /* inconsistent or unsupported shape */
#define AKV_E_ALIGN (-4)       /* pointer not 16-byte aligned */
#define AKV_E_DTYPE (-5)       /* unsupported dtype */
#define AKV_E_WORKSPACE (-6)   /* workspace missing or too small */
#define AKV_E_UNSUPPORTED (-7) /* valid request this build does not implement */
#define AKV_E_HIP (-8)         /* HIP runtime error (launch failure) */
#define AKV_E_ABI (-9)         /* args struct built for another ABI version */

/* element types */
#define AKV_DT_F16 0
#define AKV_DT_BF16 1
#define AKV_DT_F32 2

/* warm-tier layouts */
#define AKV_WARM_NONE 0
/* Block-affine warm tier, one per (batch, kv-head) (akv/affine_quantizer.py:63-189
 * applied per T-token block for K and per G-channel group for V):
 *   k_codes [B][Hkv][Nw][D*bits_k/8] u8 (akv/bitpack.py layout along D)
 *   k_scale, k_zero [B][Hkv][ceil(Nw/T)][D] f16   (per channel, per block)
 *   v_codes [B][Hkv][Nw][D*bits_v/8] u8
 *   v_scale, v_zero [B][Hkv][Nw][D/G] f16          (per token, per group)
 *   optional outliers (n_out > 0): k_oidx, v_oidx [B][ceil(Nw/T)][n_out] i64
 *   (shared by the heads of a block, as one quantize_keys call shares them),
 *   k_odata, v_odata [B][Hkv][Nw][n_out] f16 (replace the dequantized value). */
#define AKV_WARM_AFFINE 1
/* Legacy per-token-group warm tier of the reference's public attention ops
 * (akv/triton_ops.py:657-713, akv/fused_attention.py:281-317):
 *   k_codes [Hw][Nw][row] u8 with row = pD*bits/8, pD = D rounded up to group_size
 *   k_scale, k_zero [Hw][Nw][pD/group_size] of meta_dtype
 *   Hw = 1 (one warm tier broadcast to every batch element and head) or
 *   Hw = Hkv (one per head, broadcast over the batch);
 *   dequant in fp32: u*s + z, or (u - maxv/2)*s when every zero-point is 0
 *   (legacy_sym = -1 detects this on the device, 0/1 force it); bits 2/4/8. */
#define AKV_WARM_LEGACY 2

typedef struct akv_warm_desc {
    int32_t kind;          /* AKV_WARM_* */
    int32_t bits_k, bits_v;
    int64_t n_warm;        /* warm tokens Nw */
    /* AKV_WARM_AFFINE */
    int32_t block_t;       /* K token block T (multiple of 16) */
    int32_t group_v;       /* V channel group G (multiple of 8, divides D) */
    int32_t n_out;         /* outlier channels per block, 0 = none */
    int32_t _pad0;
    const void *k_codes, *v_codes;
    const void *k_scale, *k_zero, *v_scale, *v_zero;
    const int64_t *k_oidx, *v_oidx;
    const void *k_odata, *v_odata;
    /* AKV_WARM_LEGACY */
    int32_t group_size;    /* group size along D */
    int32_t meta_dtype;    /* AKV_DT_* of scales / zeros */
    int32_t warm_heads;    /* Hw: 1 (shared), Hkv (per kv head) or, in decode, B * Hkv (per batch and kv head) */
    int32_t legacy_sym;    /* -1 detect, 0 asymmetric, 1 symmetric */
    /* token rows per warm head (LEGACY) or per (batch, kv-head) (AFFINE, dequant only) of
     * the codes, V meta and outlier values, >= n_warm; 0 = n_warm.  Lets a preallocated
     * store (PackedKVArena's [H][S][...] buffers, AKVLayer's growing tier) be read in
     * place while only its first n_warm rows are filled.  A LEGACY tier with a stride above
     * n_warm must force legacy_sym (0 or 1): the detection reads dense rows. */
    int64_t token_stride;
} akv_warm_desc;

/* ---------------------------------------------------------------- decode */

typedef struct akv_decode_args {
    int32_t abi_version;   /* AKV_ABI_VERSION */
    int32_t B, Hq, Hkv, M, D;  /* D in {64, 128}; Hq % Hkv == 0 */
    int32_t q_dtype;       /* AKV_DT_F16 */
    const void *q;         /* [B][Hq][M][D] */
    const void *k_hot, *v_hot; /* [B][Hkv][n_hot][D], q dtype (may be NULL when n_hot == 0) */
    int64_t n_hot;
    int32_t hot_first;     /* token order: 1 = [hot, warm] (reference ops), 0 = [warm, hot] */
    float sm_scale;        /* softmax scale (1/sqrt(D) in the reference); > 0 */
    akv_warm_desc warm;
    void *out;             /* [B][Hq][M][D], q dtype */
    float *attn_weights;   /* optional [B][Hq][M][N] fp32, N = n_hot + n_warm, 16-byte aligned */
    float *scores;         /* optional importance scores (n_scores,), updated in place */
    int64_t n_scores;
    float decay;
    int32_t num_splits;    /* 0 = choose */
    void *workspace;       /* device scratch of akv_decode_workspace_bytes() bytes.  Its first
                              akv_decode_counter_bytes() bytes are the split arrival counters: they must
                              read zero when a call starts, and every completed call leaves them zero; the
                              rest of the workspace needs no initial value.  Reusing a workspace for a
                              call with a larger counter region (more batch x kv-head x row-chunk pairs)
                              needs that region zeroed again, since the earlier call kept other data
                              there.  Calls that share a workspace must not overlap. */
    int64_t workspace_bytes;
    int64_t hot_stride;    /* token rows per (batch, kv-head) of k_hot / v_hot, >= n_hot; 0 = n_hot
                              (a preallocated hot buffer read in place) */
} akv_decode_args;

/* Bytes of device workspace akv_decode_attn needs for `args`. */
int64_t akv_decode_workspace_bytes(const akv_decode_args *args);

/* Bytes at the start of that workspace holding the split arrival counters
 * (256-byte multiple, B * Hkv * ceil(Hq/Hkv * M / 16) counters of 8 bytes); they must
 * be zero when a call starts.  No counterpart in the reference (its Triton launches
 * need no scratch): callers that keep one workspace per shape zero only this prefix. */
int64_t akv_decode_counter_bytes(const akv_decode_args *args);

/* Fused dequant-attention over hot fp16 + warm packed tiers (split-K, GQA),
 * optional normalised attention weights and importance EMA
 *   scores[n] = scores[n]*decay + sum_m mean_{b,h} attn[b,h,m,n].
 * Replaces: triton_kernels.fused_decode_attention (akv/triton_kernels.py:281-347),
 * triton_ops.fused_mixed_precision_attention (akv/triton_ops.py:466-515),
 * triton_ops.fused_quantized_attention (akv/triton_ops.py:330-377),
 * fused_attention.fused_int4_decode_attention (akv/fused_attention.py:213-278),
 * fused_attention.mixed_precision_decode_attention (akv/fused_attention.py:324-366),
 * and, with `scores`, triton_ops.fused_importance_update (akv/triton_ops.py:604-650). */
int akv_decode_attn(const akv_decode_args *args, void *stream);

/* Scratch limits of akv_decode_attn_noalloc: the bytes akv_decode_workspace_bytes()
 * reports, less the split counters, must not exceed AKV_NOALLOC_SCRATCH_BYTES, and
 * B * Hkv * ceil(Hq/Hkv * M / 16) must not exceed AKV_NOALLOC_COUNTER_BYTES / 8. */
#define AKV_NOALLOC_SCRATCH_BYTES (16ll << 20)
#define AKV_NOALLOC_COUNTER_BYTES (64ll << 10)

/* akv_decode_attn without the caller's workspace and without allocating: the same
 * kernels and results, with their scratch in a device array the library holds for the
 * rest of the process (one per GPU, AKV_NOALLOC_SCRATCH_BYTES plus the counters).
 * `workspace` and `workspace_bytes` are ignored; a call that needs more scratch than
 * the limits above returns AKV_E_WORKSPACE and launches nothing.  No hipMalloc, no
 * hipFree, no memset node: it may run inside a HIP graph capture.  All calls on one
 * GPU share that GPU's array, so calls that overlap on one GPU (different streams,
 * or graphs replayed concurrently) race and must be serialised by the caller.
 * No counterpart in the reference: it is for callers that cannot allocate device
 * memory (code under graph capture, tight serving loops, harnesses that forbid it). */
int akv_decode_attn_noalloc(const akv_decode_args *args, void *stream);

/* -------------------------------------------------------------- quantize */

/* quantize layouts */
/* K per channel over T-token blocks, V per token over G-channel groups, fp16
 * scale/zero, bit-packed codes: the AKV_WARM_AFFINE warm tier. */
#define AKV_QUANT_AFFINE 0
/* K and V per token over groups of group_v channels along D (D zero-padded to a
 * multiple of group_v), scale/zero in the input dtype, 2/4-bit codes packed,
 * 3/8-bit codes one per byte: triton_kernels.fused_quantize_evict
 * (akv/triton_kernels.py:464-500).  Outputs [B][H][n_sel][...] rows. */
#define AKV_QUANT_TOKEN_GROUPS 1
/* KVQuantizer.quantize (akv/quantizer.py:71-143): per-token groups of group_v
 * channels (D zero-padded), fp32 arithmetic whatever the input dtype, scale
 * clamp 1e-10, scales/zeros cast to the input dtype, 2/4-bit packed and 8-bit
 * raw; `symmetric` selects the symmetric branch (zero = 0, codes offset by
 * maxv//2).  bits 2, 4, 8. */
#define AKV_QUANT_KVQ 2
/* PackedKVArena.quantize_and_append (akv/packed_layout.py:106-161): the
 * TOKEN_GROUPS arithmetic (input dtype, per-token groups along D, zero-padded)
 * with the scale clamp at 1e-10 as the input dtype rounds it; bits 2, 4, 8.
 * Rows are the TOKEN_GROUPS rows: the arena keeps their first D * bits / 8 bytes. */
#define AKV_QUANT_ARENA 3

typedef struct akv_quant_args {
    int32_t abi_version;
    int32_t B, H, D;       /* D in {64, 128} */
    int32_t in_dtype;      /* AKV_DT_F16 / BF16 / F32: arithmetic is per-op rounded to it */
    int32_t layout;        /* AKV_QUANT_* */
    const void *k, *v;     /* [B][H][n_src][D] (either may be NULL to skip it) */
    int64_t n_src;
    const int64_t *sel;    /* optional [B][n_sel] token indices in [0, n_src) (NULL: tokens 0..n_sel-1) */
    int64_t n_sel;
    int32_t bits_k, bits_v;    /* AFFINE: 2, 3, 4, 8; TOKEN_GROUPS: 2, 3, 4, 8; KVQ, ARENA: 2, 4, 8 */
    int32_t block_t, group_v;  /* T (>= 1), G (32, 64 or 128; divides D for AFFINE) */
    int32_t n_out;             /* AFFINE outlier channels per block (0 = none) */
    int32_t symmetric;         /* KVQ only: symmetric branch */
    /* outputs; AFFINE: the AKV_WARM_AFFINE layout with Nw = n_sel */
    void *k_codes, *k_scale, *k_zero;
    void *v_codes, *v_scale, *v_zero;
    int64_t *k_oidx, *v_oidx;
    void *k_odata, *v_odata;
} akv_quant_args;

/* Gather -> quantize -> bit-pack (demotion).  AFFINE is bit-exact with
 * AffineQuantizer.quantize_keys / quantize_values + bitpack.pack
 * (akv/affine_quantizer.py:63-176, akv/bitpack.py:95-103) applied per block;
 * the gather replaces the index_select of AKVLayer demotion
 * (akv/drop_in.py:681-715).  TOKEN_GROUPS is bit-exact with the quantize
 * step of triton_kernels.fused_quantize_evict (akv/triton_kernels.py:464-507). */
int akv_quant_pack(const akv_quant_args *args, void *stream);

/* ------------------------------------------------------------- dequant */

typedef struct akv_dequant_args {
    int32_t abi_version;
    int32_t B, Hkv, D;     /* AFFINE: B, Hkv as stored; LEGACY: B ignored, Hkv = warm_heads */
    int32_t out_dtype;     /* AKV_DT_F16 (AFFINE); F16/BF16/F32 (LEGACY) */
    int32_t _pad0;
    akv_warm_desc warm;
    void *k_out, *v_out;   /* [B][Hkv][Nw][D] (AFFINE) or [Hw][Nw][D] (LEGACY); either may be NULL */
    void *workspace;       /* >= 256 bytes of device scratch when warm.legacy_sym == -1, else unused */
    /* AFFINE tiers built from blocks of any length (AKVLayer's demotion events, one
     * block per event): all optional, 0 / NULL = the fixed block_t layout above. */
    const int32_t *block_of_token; /* [Nw] K-meta / outlier block row of each warm token */
    int64_t n_blocks;              /* K-meta rows per (batch, kv-head) and outlier-index rows per
                                      batch element when block_of_token is given */
    const int64_t *out_slot;       /* [Nw] output token row of each warm token: the outputs are then
                                      [B][Hkv][out_tokens][D] and other rows are not written */
    int64_t out_tokens;
} akv_dequant_args;

/* Unpack + dequantize a warm tier to dense values, bit-exact with
 * AffineQuantizer.dequantize_keys / dequantize_values
 * (akv/affine_quantizer.py:112-124, :178-189), triton_ops._dequantize_packed
 * (akv/triton_ops.py:657-713) and fused_attention._dequant_int4_tile
 * (akv/fused_attention.py:281-317).  With block_of_token / out_slot it also
 * serves AKVLayer's chronological view: the dequantized working copy of every
 * demotion event (akv/drop_in.py:694-715) scattered to its tokens' positions
 * (akv/drop_in.py:762-787).  AFFINE outputs are float16, or float32 holding the
 * float16 values (the reference's cat with float32 / bfloat16 hot tokens). */
int akv_dequant_unpack(const akv_dequant_args *args, void *stream);

/* -------------------------------------------------------------- bitpack */

/* codes [rows][dim] u8 -> packed [rows][packed_dim] u8 (akv/bitpack.py:13-103);
 * bits 2/3/4 (any other width copies). */
int akv_bitpack(const void *codes, void *packed, int64_t rows, int32_t dim, int32_t bits, void *stream);
/* packed [rows][packed_dim] -> codes [rows][orig_dim] (akv/bitpack.py:22-114). */
int akv_bitunpack(const void *packed, void *codes, int64_t rows, int32_t packed_dim, int32_t orig_dim,
                  int32_t bits, void *stream);

/* ----------------------------------------------------------- importance */

typedef struct akv_importance_args {
    int32_t abi_version;
    int32_t attn_dtype;    /* AKV_DT_F16 / BF16 / F32 */
    const void *attn;      /* [B][H][M][N] */
    int64_t B, H, M, N;
    float *scores;         /* (n_scores,) fp32, updated in place */
    int64_t n_scores;
    float decay;
    int32_t q_window;      /* > 0: only the last q_window query rows count (0 = all M rows) */
    int32_t pool_kernel;   /* > 1 (and < N): average-pool the per-key importance over pool_kernel keys
                              (stride 1, zero padding pool_kernel / 2, divided by pool_kernel), at most 64 */
    int32_t _pad0;
} akv_importance_args;

/* scores = scores*decay + sum_m mean_{b,h} attn (truncated / zero-padded to
 * n_scores): triton_ops.fused_importance_update (akv/triton_ops.py:604-650) and
 * ImportanceScorer.update's accumulate rule (akv/importance.py:88-92, :127-128);
 * with q_window / pool_kernel, the OBSERVATION_WINDOW rule (akv/importance.py:96-115):
 * the last q_window queries summed, then avg_pool1d(kernel, stride 1, padding kernel // 2). */
int akv_importance_update(const akv_importance_args *args, void *stream);

/* --------------------------------------------------------------- prefill */

typedef struct akv_prefill_args {
    int32_t abi_version;   /* AKV_ABI_VERSION */
    int32_t B, Hq, Hkv, M, D;  /* D = 128; Hq % Hkv == 0; M query positions per head */
    int32_t q_dtype;       /* AKV_DT_F16 or AKV_DT_BF16 (bf16 is converted to fp16: exact in fp16's range) */
    const void *q;         /* [B][Hq][M][D] */
    const void *k_hot, *v_hot; /* [B][Hkv][n_hot][D] f16 (may be NULL when n_hot == 0) */
    int64_t n_hot;
    float sm_scale;        /* softmax scale (1/sqrt(D) in the reference); > 0 */
    int32_t num_splits;    /* token splits, 0 = choose */
    akv_warm_desc warm;    /* AKV_WARM_NONE, or AKV_WARM_AFFINE with block_t % 32 == 0,
                              group_v in {32, 64, 128} and n_out == 0 */
    void *out;             /* [B][Hq][M][D], q dtype */
    void *workspace;       /* akv_prefill_workspace_bytes() bytes (0 with a single split) */
    int64_t workspace_bytes;
    const void *k_chunk, *v_chunk; /* optional [B][Hkv][M][D] in q's dtype: the chunk's own keys and
                              values, attended after the cache with a causal mask (query position m
                              sees chunk tokens 0..m); both NULL = the cache only */
} akv_prefill_args;

/* Bytes of device workspace akv_prefill_attn needs for `args` (split partials). */
int64_t akv_prefill_workspace_bytes(const akv_prefill_args *args);

/* Chunked prefill: M query positions per head (a prompt chunk after every
 * cached token, so no mask over the cache) attend to the hot fp16 + warm
 * block-affine cache and, when k_chunk / v_chunk are given, causally to the
 * chunk's own tokens; no attention weights.  QK^T and PV run on MFMA over
 * dequantized LDS tiles shared by the GQA group's heads.  The causal part has
 * no counterpart in the reference (its attention over a chunk is the model's).
 * Replaces, for M > 1 without weights: triton_ops.fused_quantized_attention
 * (akv/triton_ops.py:330-377) and triton_ops.fused_mixed_precision_attention
 * (akv/triton_ops.py:466-515), which dequantize the whole warm tier first. */
int akv_prefill_attn(const akv_prefill_args *args, void *stream);

/* ------------------------------------------------------- demote selection */

/* AKVLayer._select_demote_indices (akv/drop_in.py:392-413) on the device: for each of `rows`
 * rows of `len` fp32 importance scores, the indices of the n_demote smallest after positions
 * [0, protect_first) and [max(0, len - protect_last), len) are set to +inf; written ascending to
 * out [rows][n_demote] i64.  Equal scores take the lower index first (NaN sorts above +inf). */
int akv_select_demote(const float *scores, int64_t rows, int64_t len, int64_t n_demote,
                      int32_t protect_first, int32_t protect_last, int64_t *out, void *stream);

/* --------------------------------------------------------------- misc */

int akv_abi_version(void);
const char *akv_last_error(void);
/* sizeof of the args structs, for bindings that mirror them (ctypes, cgo):
 * 0 akv_warm_desc, 1 akv_decode_args, 2 akv_quant_args, 3 akv_dequant_args,
 * 4 akv_importance_args, 5 akv_prefill_args; -1 for an unknown id. */
int64_t akv_struct_size(int32_t which);
/* A measurement helper with no counterpart in the reference: reads `bytes` (a multiple of
 * 16, 16-byte aligned) once with 16-byte non-temporal loads, as fast as a read-once kernel
 * goes on this GPU; `sink` (4 bytes of device memory) is written only if the XOR of the data
 * equals a sentinel.  Its time beside a kernel's, over the same byte count, is the streaming
 * roofline the benchmark reports. */
int akv_stream_read(const void *data, int64_t bytes, uint32_t *sink, void *stream);
/* Measurement helpers with no counterpart in the reference: the per-wave timeline of the
 * fast decode kernel, recorded only by the timeline build of the library (`make timeline`,
 * compiled with -DAKV_TIMELINE; 16 words per wave, s_memrealtime ticks at 100 MHz, the
 * word meanings are listed in csrc/decode_fast.hip).  akv_timeline_words returns the
 * number of words the build records (0 in the normal build, where fetch and clear return
 * AKV_E_UNSUPPORTED).  fetch copies the first `words` words to host memory (synchronous);
 * clear zeroes them on `stream`. */
int64_t akv_timeline_words(void);
int akv_timeline_fetch(uint64_t *host, int64_t words);
int akv_timeline_clear(void *stream);

#ifdef __cplusplus
}
#endif

#endif /* AKV_HIP_H */
