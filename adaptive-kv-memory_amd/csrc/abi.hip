// extern "C" entry points of libakv_hip.so: argument validation, split
// planning, workspace carving and dispatch to the kernels.
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>

#include "akv_common.h"
#include "decode.h"
#include "prefill.h"
#include "misc.h"
#include "quant.h"

namespace {

thread_local std::string g_err;

int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}
int ok() {
    g_err.clear();
    return AKV_OK;
}
int hip_fail(hipError_t e, const char *what) {
    return fail(AKV_E_HIP, "%s: %s", what, hipGetErrorString(e));
}
bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }
bool pow2(int x) { return x > 0 && (x & (x - 1)) == 0; }
int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }
int64_t align256(int64_t x) { return round_up(x, 256); }

struct Plan {
    int nchunk, prows, n_wsplit, n_hsplit, nsplit;
    int64_t wsplit_len, hsplit_len, N;
    int64_t ctr_bytes, part_bytes, rowstat_bytes, flag_bytes, stash_bytes, total;
    bool fused;  // the fast split kernel merges its own splits (arrival counters at offset 0)
};

constexpr int kWaves = 4;

// Deterministic split schedule.  Splits are sized by bytes so a hot split (fp16
// K/V, 4*D bytes per token) and a warm split (packed codes + meta) stream
// about the same amount; each is a multiple of its token unit and holds at
// least one unit per wave.  Without an explicit count the schedule aims at a
// few workgroups per compute unit of the 256-CU MI355X.
constexpr int kCUs = 256;
// Largest split count the fast kernel merges itself (its last workgroup reads
// every partial of a row chunk); larger counts use decode_reduce_kernel.
constexpr int kFusedMaxSplits = 32;

bool fast_path(const akv_decode_args *a) {
    const akv_warm_desc &w = a->warm;
    if (w.kind == AKV_WARM_LEGACY)  // per-token group meta, read like the affine V meta
        return w.bits_k == w.bits_v && akv::decode_fast_legacy_shape(a->D, w.bits_k, w.group_size, w.meta_dtype) &&
               akv::decode_fast_meta_aligned(w.token_stride > 0 ? w.token_stride : w.n_warm, w.group_size,
                                             w.warm_heads) &&
               akv::decode_fast_lds_bytes(akv::decode_fast_slot_bytes(w.bits_k, w.bits_v, w.group_size, 0, true), 0) <=
                   160 * 1024;
    if (!(w.kind == AKV_WARM_AFFINE && a->D == 128 && w.block_t % 32 == 0 &&
          (w.group_v == 32 || w.group_v == 64 || w.group_v == 128) &&
          akv::decode_fast_meta_aligned(w.n_warm, w.group_v, (int64_t)a->B * a->Hkv)))
        return false;
    // outlier channels: up to 4 per block with 32-channel V groups; the ring must fit the LDS
    if (w.n_out != 0 && !(w.n_out <= 4 && w.group_v == 32 && w.k_odata && w.v_odata && w.k_oidx && w.v_oidx))
        return false;
    return akv::decode_fast_lds_bytes(akv::decode_fast_slot_bytes(w.bits_k, w.bits_v, w.group_v, w.n_out, false),
                                      w.n_out) <= 160 * 1024;
}

void make_plan(const akv_decode_args *a, Plan *pl) {
    const akv_warm_desc &w = a->warm;
    const int64_t nw = w.kind == AKV_WARM_NONE ? 0 : w.n_warm;
    const int64_t nh = a->n_hot;
    const int g = a->Hq / a->Hkv;
    const int R = g * a->M;
    const bool fast = fast_path(a);
    pl->nchunk = (R + 15) / 16;
    pl->prows = R < 16 ? R : 16;
    pl->N = nw + nh;
    const int64_t pairs = (int64_t)a->B * a->Hkv * pl->nchunk;
    // bytes streamed per token
    double bw = 0.0;
    if (w.kind == AKV_WARM_AFFINE)
        bw = a->D * (w.bits_k + w.bits_v) / 8.0 + 4.0 * a->D / w.block_t + 4.0 * a->D / w.group_v;
    else if (w.kind == AKV_WARM_LEGACY)
        bw = 2.0 * a->D * w.bits_k / 8.0 + 4.0 * a->D / (w.group_size > 0 ? w.group_size : 32);
    const double bhot = 4.0 * a->D;
    if (fast) {
        // One workgroup of many waves per CU and (batch, kv-head, row chunk);
        // its waves share the range's hot tiles and warm units dynamically.
        const int64_t units = (nw + 31) / 32, tiles = (nh + 15) / 16;
        int64_t cp = a->num_splits > 0 ? a->num_splits : kCUs / pairs;
        // Short contexts: about 3 items per 4 waves.  The launch then costs its fixed latency
        // chain (first loads, one item, the merges) rather than several items per wave; more
        // splits only lengthen the final merge (4k Qwen layer: 13.0 us at 2 items per wave,
        // 10.3 us here, 11.3-12.2 us at 24-64 splits).
        const int64_t by_items =
            (units + tiles) * 4 / (3 * akv::decode_fast_waves(w.kind == AKV_WARM_AFFINE ? w.n_out : 0));
        if (a->num_splits <= 0 && cp > by_items) cp = by_items;
        if (cp < 1) cp = 1;
        pl->wsplit_len = (units + cp - 1) / cp * 32;
        pl->hsplit_len = (tiles + cp - 1) / cp * 16;
        if (pl->wsplit_len < 32) pl->wsplit_len = 32;
        if (pl->hsplit_len < 16) pl->hsplit_len = 16;
        pl->n_wsplit = (int)cp;
        pl->n_hsplit = 0;
        pl->nsplit = (int)cp;
    } else {
    int64_t target;
    if (a->num_splits > 0) {
        target = a->num_splits;
    } else {
        target = (kCUs * 4 + pairs - 1) / pairs;
    }
    if (target < 1) target = 1;
    // Hot splits first (each about one split's worth of bytes), then the warm
    // tier takes the rest of the target, so the grid never exceeds it: a grid
    // one workgroup over the resident capacity runs a second, nearly idle round.
    const double pair_bytes = nw * bw + nh * bhot;
    const double split_bytes = pair_bytes / (double)target;
    const int64_t wunit = (w.kind == AKV_WARM_AFFINE) ? w.block_t : 16;
    int64_t n_h = nh > 0 ? (int64_t)std::ceil(nh * bhot / split_bytes - 1e-9) : 0;
    if (nh > 0 && n_h < 1) n_h = 1;
    if (nw > 0 && n_h > target - 1) n_h = target > 1 ? target - 1 : 1;
    const int64_t n_w = nw > 0 ? (target - n_h > 1 ? target - n_h : 1) : 0;
    const int64_t hlen = n_h > 0 ? (nh + n_h - 1) / n_h : 0;
    const int64_t wlen = n_w > 0 ? (nw + n_w - 1) / n_w : 0;
    pl->wsplit_len = round_up(wlen > kWaves * wunit ? wlen : kWaves * wunit, wunit);
    pl->hsplit_len = round_up(hlen > kWaves * 16 ? hlen : kWaves * 16, 16);
    pl->n_wsplit = nw > 0 ? (int)((nw + pl->wsplit_len - 1) / pl->wsplit_len) : 0;
    pl->n_hsplit = nh > 0 ? (int)((nh + pl->hsplit_len - 1) / pl->hsplit_len) : 0;
    pl->nsplit = pl->n_wsplit + pl->n_hsplit;
    }
    pl->fused = fast && pl->nsplit <= kFusedMaxSplits;
    pl->ctr_bytes = align256(pairs * 8);
    pl->part_bytes = align256(pairs * pl->nsplit * (int64_t)pl->prows * (a->D + 4) * 4);
    pl->rowstat_bytes = align256((int64_t)a->B * a->Hq * a->M * 2 * 4);
    pl->flag_bytes = 256;
    const bool need_stash = a->attn_weights == nullptr && a->scores != nullptr;
    pl->stash_bytes = need_stash ? align256((int64_t)a->B * a->Hq * a->M * pl->N * 4) : 0;
    pl->total = pl->ctr_bytes + pl->part_bytes + pl->rowstat_bytes + pl->flag_bytes + pl->stash_bytes;
}

int check_decode(const akv_decode_args *a) {
    if (!a) return fail(AKV_E_INVALID, "args is NULL");
    if (a->abi_version != AKV_ABI_VERSION)
        return fail(AKV_E_ABI, "args built for ABI %d, library is ABI %d", a->abi_version, AKV_ABI_VERSION);
    if (a->q_dtype != AKV_DT_F16) return fail(AKV_E_DTYPE, "decode attention takes float16 queries");
    if (a->D != 64 && a->D != 128) return fail(AKV_E_SHAPE, "head_dim %d unsupported (64 or 128)", a->D);
    if (a->B < 1 || a->Hq < 1 || a->Hkv < 1 || a->M < 1)
        return fail(AKV_E_SHAPE, "B, Hq, Hkv, M must be >= 1");
    if (a->Hq % a->Hkv) return fail(AKV_E_SHAPE, "Hq (%d) must be a multiple of Hkv (%d)", a->Hq, a->Hkv);
    // the online softmax takes the largest raw score as the largest scaled one
    if (!(a->sm_scale > 0.0f) || !(a->sm_scale < INFINITY))
        return fail(AKV_E_INVALID, "sm_scale must be positive and finite (got %g)", (double)a->sm_scale);
    if (a->n_hot < 0) return fail(AKV_E_SHAPE, "n_hot < 0");
    const akv_warm_desc &w = a->warm;
    const int64_t nw = w.kind == AKV_WARM_NONE ? 0 : w.n_warm;
    if (nw < 0) return fail(AKV_E_SHAPE, "n_warm < 0");
    if (a->n_hot + nw < 1) return fail(AKV_E_SHAPE, "no tokens to attend to");
    if (!a->q || !a->out) return fail(AKV_E_INVALID, "q and out are required");
    if (!aligned16(a->q) || !aligned16(a->out)) return fail(AKV_E_ALIGN, "q/out must be 16-byte aligned");
    // the weights are written and read back with 16-byte accesses
    if (a->attn_weights && !aligned16(a->attn_weights))
        return fail(AKV_E_ALIGN, "attn_weights must be 16-byte aligned");
    if (a->n_hot > 0) {
        if (!a->k_hot || !a->v_hot) return fail(AKV_E_INVALID, "k_hot/v_hot required when n_hot > 0");
        if (!aligned16(a->k_hot) || !aligned16(a->v_hot)) return fail(AKV_E_ALIGN, "hot tier must be 16-byte aligned");
        if (a->n_hot * a->D * 2 >= (int64_t)1 << 32) return fail(AKV_E_SHAPE, "hot tier per head exceeds 4 GiB");
    }
    if (a->hot_stride != 0 && a->hot_stride < a->n_hot) return fail(AKV_E_SHAPE, "hot_stride < n_hot");
    if (w.kind == AKV_WARM_AFFINE && w.token_stride != 0 && w.token_stride != w.n_warm)
        return fail(AKV_E_UNSUPPORTED, "decode reads an affine warm tier with token_stride == n_warm only");
    if (w.kind == AKV_WARM_LEGACY && w.token_stride != 0 && w.token_stride < w.n_warm)
        return fail(AKV_E_SHAPE, "token_stride < n_warm");
    if (w.kind == AKV_WARM_AFFINE) {
        for (int bits : {w.bits_k, w.bits_v})
            if (bits < 2 || bits > 4) return fail(AKV_E_BITS, "Unsupported bits: %d", bits);
        if (w.block_t < 16 || w.block_t % 16) return fail(AKV_E_SHAPE, "block_t must be a positive multiple of 16");
        if (w.group_v < 8 || w.group_v % 8 || a->D % w.group_v)
            return fail(AKV_E_SHAPE, "group_v must be a multiple of 8 dividing D");
        if (!w.k_codes || !w.v_codes || !w.k_scale || !w.k_zero || !w.v_scale || !w.v_zero)
            return fail(AKV_E_INVALID, "warm tier pointers missing");
        if (w.n_out < 0 || w.n_out > a->D) return fail(AKV_E_SHAPE, "n_out out of range");
        if (w.n_out > 0 && (!w.k_oidx || !w.v_oidx || !w.k_odata || !w.v_odata))
            return fail(AKV_E_INVALID, "outlier pointers missing");
        if (nw * (int64_t)a->D >= (int64_t)1 << 32) return fail(AKV_E_SHAPE, "warm tier per head exceeds 4 GiB");
    } else if (w.kind == AKV_WARM_LEGACY) {
        if (w.bits_k != w.bits_v) return fail(AKV_E_BITS, "legacy warm tier uses one width for K and V");
        if (w.bits_k != 2 && w.bits_k != 4 && w.bits_k != 8) return fail(AKV_E_BITS, "Unsupported bits: %d", w.bits_k);
        if (!pow2(w.group_size) || w.group_size < 8) return fail(AKV_E_UNSUPPORTED, "group_size must be a power of two >= 8");
        if (w.meta_dtype < 0 || w.meta_dtype > 2) return fail(AKV_E_DTYPE, "bad meta dtype");
        if (w.warm_heads != 1 && w.warm_heads != a->Hkv && w.warm_heads != a->B * a->Hkv)
            return fail(AKV_E_SHAPE, "warm_heads must be 1, Hkv or B * Hkv");
        if (w.legacy_sym < 0 && w.token_stride > w.n_warm)
            return fail(AKV_E_UNSUPPORTED, "symmetric-branch detection reads dense rows: force legacy_sym with a token stride");
        if (!w.k_codes || !w.v_codes || !w.k_scale || !w.k_zero || !w.v_scale || !w.v_zero)
            return fail(AKV_E_INVALID, "warm tier pointers missing");
        if (nw * (int64_t)a->D * 2 >= (int64_t)1 << 32) return fail(AKV_E_SHAPE, "warm tier per head exceeds 4 GiB");
    } else if (w.kind != AKV_WARM_NONE) {
        return fail(AKV_E_INVALID, "unknown warm kind %d", w.kind);
    }
    if (w.kind != AKV_WARM_NONE && nw > 0) {
        if (!aligned16(w.k_codes) || !aligned16(w.v_codes) || !aligned16(w.k_scale) || !aligned16(w.v_scale) ||
            !aligned16(w.k_zero) || !aligned16(w.v_zero))
            return fail(AKV_E_ALIGN, "warm tier must be 16-byte aligned");
    }
    if (a->scores && a->n_scores < 0) return fail(AKV_E_SHAPE, "n_scores < 0");
    return AKV_OK;
}

struct PrefillPlan {
    int R, n_row_tiles, nsplit, nchunk, prows;
    int64_t tiles_per_split, part_bytes;
};

int check_prefill(const akv_prefill_args *a) {
    if (!a) return fail(AKV_E_INVALID, "args is NULL");
    if (a->abi_version != AKV_ABI_VERSION)
        return fail(AKV_E_ABI, "args built for ABI %d, library is ABI %d", a->abi_version, AKV_ABI_VERSION);
    if (a->q_dtype != AKV_DT_F16 && a->q_dtype != AKV_DT_BF16)
        return fail(AKV_E_DTYPE, "prefill takes float16 or bfloat16 queries");
    if (a->D != 128) return fail(AKV_E_SHAPE, "prefill supports head_dim 128 (got %d)", a->D);
    if (a->B < 1 || a->Hq < 1 || a->Hkv < 1 || a->M < 1) return fail(AKV_E_SHAPE, "B, Hq, Hkv, M must be >= 1");
    if (a->Hq % a->Hkv) return fail(AKV_E_SHAPE, "Hq (%d) must be a multiple of Hkv (%d)", a->Hq, a->Hkv);
    // the online softmax takes the largest raw score as the largest scaled one
    if (!(a->sm_scale > 0.0f) || !(a->sm_scale < INFINITY))
        return fail(AKV_E_INVALID, "sm_scale must be positive and finite (got %g)", (double)a->sm_scale);
    if (a->n_hot < 0) return fail(AKV_E_SHAPE, "n_hot < 0");
    const akv_warm_desc &w = a->warm;
    const int64_t nw = w.kind == AKV_WARM_NONE ? 0 : w.n_warm;
    if (nw < 0) return fail(AKV_E_SHAPE, "n_warm < 0");
    if (!a->k_chunk != !a->v_chunk) return fail(AKV_E_INVALID, "k_chunk and v_chunk go together");
    if (a->k_chunk && (!aligned16(a->k_chunk) || !aligned16(a->v_chunk)))
        return fail(AKV_E_ALIGN, "k_chunk/v_chunk must be 16-byte aligned");
    if (a->n_hot + nw < 1 && !a->k_chunk) return fail(AKV_E_SHAPE, "no tokens to attend to");
    if (!a->q || !a->out) return fail(AKV_E_INVALID, "q and out are required");
    if (!aligned16(a->q) || !aligned16(a->out)) return fail(AKV_E_ALIGN, "q/out must be 16-byte aligned");
    if (a->n_hot > 0) {
        if (!a->k_hot || !a->v_hot) return fail(AKV_E_INVALID, "k_hot/v_hot required when n_hot > 0");
        if (!aligned16(a->k_hot) || !aligned16(a->v_hot)) return fail(AKV_E_ALIGN, "hot tier must be 16-byte aligned");
        if (a->n_hot * a->D * 2 >= (int64_t)1 << 32) return fail(AKV_E_SHAPE, "hot tier per head exceeds 4 GiB");
    }
    if (w.token_stride != 0 && w.token_stride != nw)
        return fail(AKV_E_UNSUPPORTED, "prefill reads a warm tier with token_stride == n_warm only");
    if (w.kind == AKV_WARM_AFFINE) {
        for (int bits : {w.bits_k, w.bits_v})
            if (bits < 2 || bits > 4) return fail(AKV_E_BITS, "Unsupported bits: %d", bits);
        if (w.block_t < 32 || w.block_t % 32) return fail(AKV_E_UNSUPPORTED, "prefill needs block_t a multiple of 32");
        if (w.group_v != 32 && w.group_v != 64 && w.group_v != 128)
            return fail(AKV_E_UNSUPPORTED, "prefill needs group_v 32, 64 or 128");
        if (w.n_out != 0) return fail(AKV_E_UNSUPPORTED, "prefill does not take outlier channels");
        if (nw > 0) {
            if (!w.k_codes || !w.v_codes || !w.k_scale || !w.k_zero || !w.v_scale || !w.v_zero)
                return fail(AKV_E_INVALID, "warm tier pointers missing");
            if (!aligned16(w.k_codes) || !aligned16(w.v_codes) || !aligned16(w.k_scale) || !aligned16(w.v_scale) ||
                !aligned16(w.k_zero) || !aligned16(w.v_zero))
                return fail(AKV_E_ALIGN, "warm tier must be 16-byte aligned");
        }
        if (nw * (int64_t)a->D >= (int64_t)1 << 32) return fail(AKV_E_SHAPE, "warm tier per head exceeds 4 GiB");
    } else if (w.kind != AKV_WARM_NONE) {
        return fail(AKV_E_UNSUPPORTED, "prefill takes the block-affine warm tier only");
    }
    return AKV_OK;
}

// Row tiles of 256 query rows per (batch, kv-head); token splits until there
// is one workgroup (8 waves, two per SIMD) per compute unit, each split at
// least 8 tiles.
void make_prefill_plan(const akv_prefill_args *a, PrefillPlan *pl) {
    const int g = a->Hq / a->Hkv;
    pl->R = g * a->M;
    pl->n_row_tiles = (pl->R + akv::kPrefillRows - 1) / akv::kPrefillRows;
    const int64_t nw = a->warm.kind == AKV_WARM_NONE ? 0 : a->warm.n_warm;
    const int64_t nt = (a->n_hot + 31) / 32 + (nw + 31) / 32 + (a->k_chunk ? (a->M + 31) / 32 : 0);
    const int64_t wgs = (int64_t)a->B * a->Hkv * pl->n_row_tiles;
    int64_t ns = a->num_splits > 0 ? a->num_splits : (kCUs + wgs - 1) / wgs;
    if (a->num_splits <= 0 && ns > nt / 8) ns = nt / 8;
    if (ns > nt) ns = nt;
    if (ns < 1) ns = 1;
    pl->tiles_per_split = (nt + ns - 1) / ns;
    pl->nsplit = (int)((nt + pl->tiles_per_split - 1) / pl->tiles_per_split);
    pl->nchunk = (pl->R + 15) / 16;
    pl->prows = pl->R < 16 ? pl->R : 16;
    pl->part_bytes = pl->nsplit > 1
        ? align256((int64_t)a->B * a->Hkv * pl->nchunk * pl->nsplit * pl->prows * (a->D + 4) * 4) : 0;
}

}  // namespace

extern "C" {

int akv_abi_version(void) { return AKV_ABI_VERSION; }
const char *akv_last_error(void) { return g_err.c_str(); }

int64_t akv_struct_size(int32_t which) {
    switch (which) {
        case 0: return (int64_t)sizeof(akv_warm_desc);
        case 1: return (int64_t)sizeof(akv_decode_args);
        case 2: return (int64_t)sizeof(akv_quant_args);
        case 3: return (int64_t)sizeof(akv_dequant_args);
        case 4: return (int64_t)sizeof(akv_importance_args);
        case 5: return (int64_t)sizeof(akv_prefill_args);
        default: return -1;
    }
}

int64_t akv_decode_workspace_bytes(const akv_decode_args *a) {
    if (check_decode(a) != AKV_OK) return -1;
    Plan pl;
    make_plan(a, &pl);
    return pl.total;
}

int64_t akv_decode_counter_bytes(const akv_decode_args *a) {
    if (check_decode(a) != AKV_OK) return -1;
    Plan pl;
    make_plan(a, &pl);
    return pl.ctr_bytes;
}

}  // extern "C"

namespace {

// One decode call with its scratch carved as: the split arrival counters at `ctr`
// (pl.ctr_bytes, zero on entry; a completed call leaves them zero again) and the
// partials, row statistics, flags and logit stash from `ws` on.
int decode_run(const akv_decode_args *a, const Plan &pl, char *ctr, char *ws, void *stream) {
    const akv_warm_desc &w = a->warm;
    akv::DecodeParams p{};
    p.B = a->B; p.Hq = a->Hq; p.Hkv = a->Hkv; p.M = a->M; p.D = a->D;
    p.g = a->Hq / a->Hkv; p.R = p.g * a->M; p.nchunk = pl.nchunk; p.prows = pl.prows;
    p.q = (const _Float16 *)a->q;
    p.khot = (const _Float16 *)a->k_hot; p.vhot = (const _Float16 *)a->v_hot;
    p.n_hot = a->n_hot;
    p.h_stride = a->hot_stride > 0 ? a->hot_stride : a->n_hot;
    const int wk = w.kind == AKV_WARM_NONE ? AKV_WARM_AFFINE : w.kind;
    p.n_warm = w.kind == AKV_WARM_NONE ? 0 : w.n_warm;
    p.w_stride = w.token_stride > 0 ? w.token_stride : p.n_warm;
    int kb = 4, vb = 4;
    int sym_src[2] = {0, 0};
    const int *sym_ptr = nullptr;
    if (pl.fused) p.split_ctr = (uint64_t *)ctr;
    p.part = (float *)ws;
    p.rowstats = (float *)(ws + pl.part_bytes);
    int *flags = (int *)(ws + pl.part_bytes + pl.rowstat_bytes);
    float *stash_ws = (float *)(ws + pl.part_bytes + pl.rowstat_bytes + pl.flag_bytes);
    if (w.kind == AKV_WARM_AFFINE) {
        kb = w.bits_k; vb = w.bits_v;
        p.kc = w.k_codes; p.vc = w.v_codes;
        p.ks = w.k_scale; p.kz = w.k_zero; p.vs = w.v_scale; p.vz = w.v_zero;
        p.kc_row = a->D * kb / 8; p.vc_row = a->D * vb / 8;
        p.T = w.block_t; p.Gv = w.group_v;
        p.tshift = -1;
        if (w.block_t % 32 == 0 && pow2(w.block_t / 32)) {
            p.tshift = 0;
            while ((32 << p.tshift) < w.block_t) ++p.tshift;
        }
        p.nblk = (p.n_warm + w.block_t - 1) / w.block_t;
        p.n_out = w.n_out;
        p.k_oidx = w.k_oidx; p.v_oidx = w.v_oidx;
        p.k_odata = (const _Float16 *)w.k_odata; p.v_odata = (const _Float16 *)w.v_odata;
        p.warm_heads = a->Hkv;
    } else if (w.kind == AKV_WARM_LEGACY) {
        kb = vb = w.bits_k;
        const int pD = (int)round_up(a->D, w.group_size);
        p.kc = w.k_codes; p.vc = w.v_codes;
        p.ks = w.k_scale; p.kz = w.k_zero; p.vs = w.v_scale; p.vz = w.v_zero;
        p.kc_row = p.vc_row = pD * kb / 8;
        p.gs = w.group_size; p.lg = pD / w.group_size; p.meta_dt = w.meta_dtype;
        p.warm_heads = w.warm_heads;
        p.half_max_k = p.half_max_v = (float)(((1 << kb) - 1) / 2);
        p.T = 16;
        if (w.legacy_sym < 0) {
            p.sym_flags = flags;
            sym_src[0] = w.meta_dtype;
            sym_src[1] = (int)((int64_t)w.warm_heads * p.n_warm * p.lg);
            sym_ptr = sym_src;
        } else {
            p.legacy_sym = w.legacy_sym ? 1 : 0;
        }
    } else {
        p.T = 16; p.Gv = 32;
    }
    p.scale_log2 = a->sm_scale * 1.4426950408889634f;
    p.hot_first = a->hot_first ? 1 : 0;
    p.N = pl.N;
    p.n_wsplit = pl.n_wsplit; p.n_hsplit = pl.n_hsplit; p.nsplit = pl.nsplit;
    p.wsplit_len = pl.wsplit_len; p.hsplit_len = pl.hsplit_len;
    p.fd_nsplit = akv::make_fast_div((uint32_t)pl.nsplit);
    p.fd_hkv = akv::make_fast_div((uint32_t)a->Hkv);
    p.fd_nchunk = akv::make_fast_div((uint32_t)pl.nchunk);
    p.fd_m = akv::make_fast_div((uint32_t)a->M);
    p.out = (_Float16 *)a->out;
    p.attn_out = a->attn_weights;
    p.stash = a->attn_weights ? a->attn_weights : (a->scores ? stash_ws : nullptr);
    p.scores = a->scores;
    p.n_scores = a->scores ? a->n_scores : 0;
    p.decay = a->decay;
    if (w.kind == AKV_WARM_AFFINE) p.slot_bytes = (int)akv::decode_fast_slot_bytes(kb, vb, w.group_v, w.n_out, false);
    if (w.kind == AKV_WARM_LEGACY && fast_path(a)) {
        p.Gv = w.group_size;
        p.slot_bytes = (int)akv::decode_fast_slot_bytes(kb, vb, w.group_size, 0, true);
    }
    hipError_t e = akv::decode_launch(p, kb, vb, wk, sym_ptr, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "decode launch");
    return ok();
}

// ---------------------------------------------------------------- scratch
// Device scratch of the no-allocation decode entry point: one copy per GPU,
// held until the process ends.  The first kScratchCtrBytes hold the split
// arrival counters (8 bytes per (batch, kv-head, row chunk)) and nothing else
// writes there; every completed call leaves them zero.  The rest takes the
// partials, row statistics, flags and logit stash of one call.
constexpr int64_t kScratchBytes = AKV_NOALLOC_SCRATCH_BYTES + AKV_NOALLOC_COUNTER_BYTES;
constexpr int64_t kScratchCtrBytes = AKV_NOALLOC_COUNTER_BYTES;
constexpr int kMaxDevices = 64;

}  // namespace

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

std::mutex g_scratch_mu;
char *g_scratch_ptr[kMaxDevices] = {};

// The address of this device's `scratch`, found once per device (with that device
// current) by hipGetSymbolAddress.  The counter region starts zero: the array is
// zero-initialised when the code object is loaded, and every completed call leaves its
// counters zero.  On the first call on a device the region is also cleared by a kernel
// on `stream` -- unless that stream is being captured, where the clear would only become
// a graph node that runs at replay (after eager calls made before it); such a first call
// relies on the load-time zero initialisation alone.
int scratch_base(void *stream, char **out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (stream) {
        int sdev = -1;
        e = hipStreamGetDevice((hipStream_t)stream, &sdev);
        if (e != hipSuccess) return hip_fail(e, "hipStreamGetDevice");
        if (sdev != dev) return fail(AKV_E_INVALID, "stream belongs to device %d, but device %d is current", sdev, dev);
    }
    if (dev < 0 || dev >= kMaxDevices) return fail(AKV_E_INVALID, "device index %d out of range", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
        if (!ptr) return fail(AKV_E_HIP, "hipGetSymbolAddress(scratch) returned NULL");
        hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
        e = hipStreamIsCapturing((hipStream_t)stream, &cap);
        if (e != hipSuccess) return hip_fail(e, "hipStreamIsCapturing");
        if (cap == hipStreamCaptureStatusNone) {
            e = akv::zero_fill_launch(ptr, kScratchCtrBytes, (hipStream_t)stream);
            if (e != hipSuccess) return hip_fail(e, "scratch counter clear");
        }
        g_scratch_ptr[dev] = (char *)ptr;
    }
    *out = g_scratch_ptr[dev];
    return AKV_OK;
}

}  // namespace

extern "C" {

int akv_decode_attn(const akv_decode_args *a, void *stream) {
    int rc = check_decode(a);
    if (rc != AKV_OK) return rc;
    Plan pl;
    make_plan(a, &pl);
    if (!a->workspace || a->workspace_bytes < pl.total)
        return fail(AKV_E_WORKSPACE, "workspace of %lld bytes needed", (long long)pl.total);
    if (!aligned16(a->workspace)) return fail(AKV_E_ALIGN, "workspace must be 16-byte aligned");
    char *ws = (char *)a->workspace;
    return decode_run(a, pl, ws, ws + pl.ctr_bytes, stream);
}

int akv_decode_attn_noalloc(const akv_decode_args *a, void *stream) {
    int rc = check_decode(a);
    if (rc != AKV_OK) return rc;
    Plan pl;
    make_plan(a, &pl);
    if (pl.ctr_bytes > kScratchCtrBytes)
        return fail(AKV_E_WORKSPACE, "%lld split counters exceed the %lld the no-allocation entry point holds",
                    (long long)(pl.ctr_bytes / 8), (long long)(kScratchCtrBytes / 8));
    if (pl.total - pl.ctr_bytes > kScratchBytes - kScratchCtrBytes)
        return fail(AKV_E_WORKSPACE, "this call needs %lld bytes of scratch; the no-allocation entry point holds %lld",
                    (long long)(pl.total - pl.ctr_bytes), (long long)(kScratchBytes - kScratchCtrBytes));
    char *base = nullptr;
    if ((rc = scratch_base(stream, &base)) != AKV_OK) return rc;
    return decode_run(a, pl, base, base + kScratchCtrBytes, stream);
}

int akv_quant_pack(const akv_quant_args *a, void *stream) {
    if (!a) return fail(AKV_E_INVALID, "args is NULL");
    if (a->abi_version != AKV_ABI_VERSION) return fail(AKV_E_ABI, "ABI mismatch");
    if (a->D != 64 && a->D != 128) return fail(AKV_E_SHAPE, "head_dim %d unsupported (64 or 128)", a->D);
    if (a->B < 1 || a->H < 1 || a->n_src < 0 || a->n_sel < 0) return fail(AKV_E_SHAPE, "bad sizes");
    if (a->in_dtype < 0 || a->in_dtype > 2) return fail(AKV_E_DTYPE, "bad input dtype");
    if (a->n_sel == 0) return ok();
    if (!a->sel && a->n_sel > a->n_src) return fail(AKV_E_SHAPE, "n_sel > n_src without indices");
    const bool affine = a->layout == AKV_QUANT_AFFINE;
    const bool kvq = a->layout == AKV_QUANT_KVQ;
    const bool arena = a->layout == AKV_QUANT_ARENA;
    if (!affine && !kvq && !arena && a->layout != AKV_QUANT_TOKEN_GROUPS)
        return fail(AKV_E_INVALID, "unknown layout");
    for (int bits : {a->bits_k, a->bits_v}) {
        // 8 bits: raw codes, one per byte (akv/bitpack.py:95-103 passes them through)
        const bool okb = (kvq || arena) ? (bits == 2 || bits == 4 || bits == 8) : (bits >= 2 && bits <= 4) || bits == 8;
        if (!okb) return fail(AKV_E_BITS, "Unsupported bits: %d", bits);
    }
    if (a->group_v != 32 && a->group_v != 64 && a->group_v != 128) return fail(AKV_E_UNSUPPORTED, "group_v must be 32, 64 or 128");
    if (affine && a->D % a->group_v) return fail(AKV_E_SHAPE, "group_v must divide D");
    if (a->block_t < 1) return fail(AKV_E_SHAPE, "block_t must be >= 1");
    if (a->n_out < 0 || a->n_out > a->D || (a->n_out > 0 && !affine)) return fail(AKV_E_SHAPE, "bad n_out");
    if (a->k && (!a->k_codes || !a->k_scale || !a->k_zero)) return fail(AKV_E_INVALID, "K outputs missing");
    if (a->v && (!a->v_codes || !a->v_scale || !a->v_zero)) return fail(AKV_E_INVALID, "V outputs missing");
    if (a->n_out > 0 && ((a->k && (!a->k_oidx || !a->k_odata)) || (a->v && (!a->v_oidx || !a->v_odata))))
        return fail(AKV_E_INVALID, "outlier outputs missing");
    for (const void *ptr : {(const void *)a->k_codes, (const void *)a->v_codes})
        if (ptr && !aligned16(ptr)) return fail(AKV_E_ALIGN, "code outputs must be 16-byte aligned");
    akv::QuantParams p{};
    p.B = a->B; p.H = a->H; p.D = a->D;
    p.in_dt = a->in_dtype;
    // arithmetic dtype and the scale clamp as that dtype rounds it
    p.ar_dt = kvq ? AKV_DT_F32 : a->in_dtype;
    if (kvq) p.lo = 1e-10f;
    else if (p.ar_dt == AKV_DT_F16) p.lo = 0.0f;  // 1e-8 and 1e-10 underflow in fp16
    else if (p.ar_dt == AKV_DT_BF16)
        p.lo = __builtin_bit_cast(float, arena ? 0x2edc0000u : 0x322c0000u);  // bfloat16(1e-10), bfloat16(1e-8)
    else p.lo = arena ? 1e-10f : 1e-8f;
    p.symmetric = kvq && a->symmetric;
    p.k = a->k; p.v = a->v;
    p.n_src = a->n_src; p.n_sel = a->n_sel; p.sel = a->sel;
    p.bits_k = a->bits_k; p.bits_v = a->bits_v;
    p.G_v = a->group_v;
    p.n_out = a->n_out;
    p.k_codes = a->k_codes; p.k_scale = a->k_scale; p.k_zero = a->k_zero;
    p.v_codes = a->v_codes; p.v_scale = a->v_scale; p.v_zero = a->v_zero;
    p.k_oidx = a->k_oidx; p.v_oidx = a->v_oidx; p.k_odata = a->k_odata; p.v_odata = a->v_odata;
    if (affine) {
        p.pD = a->D;
        p.k_mode = 0;
        p.T = a->block_t;
        p.G_k = a->group_v;
        p.sbits_k = a->bits_k; p.sbits_v = a->bits_v;
        p.meta_dt = AKV_DT_F16;
    } else {
        p.pD = (int)round_up(a->D, a->group_v);
        p.k_mode = 1;
        p.T = 32;
        p.G_k = a->group_v;
        p.sbits_k = (a->bits_k == 2 || a->bits_k == 4) ? a->bits_k : 8;
        p.sbits_v = (a->bits_v == 2 || a->bits_v == 4) ? a->bits_v : 8;
        p.meta_dt = a->in_dtype;
    }
    p.k_row = p.pD * p.sbits_k / 8;
    p.v_row = p.pD * p.sbits_v / 8;
    p.nblk = (a->n_sel + p.T - 1) / p.T;
    hipError_t e = akv::quant_launch(p, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "quant launch");
    return ok();
}

int akv_dequant_unpack(const akv_dequant_args *a, void *stream) {
    if (!a) return fail(AKV_E_INVALID, "args is NULL");
    if (a->abi_version != AKV_ABI_VERSION) return fail(AKV_E_ABI, "ABI mismatch");
    const akv_warm_desc &w = a->warm;
    if (a->D % 8 || a->D < 8) return fail(AKV_E_SHAPE, "D must be a positive multiple of 8");
    if (w.n_warm < 0) return fail(AKV_E_SHAPE, "n_warm < 0");
    akv::DequantParams p{};
    p.kind = w.kind;
    p.D = a->D;
    p.n_warm = w.n_warm;
    p.bits_k = w.bits_k; p.bits_v = w.bits_v;
    p.kc = w.k_codes; p.vc = w.v_codes;
    p.ks = w.k_scale; p.kz = w.k_zero; p.vs = w.v_scale; p.vz = w.v_zero;
    p.out_dt = a->out_dtype;
    p.k_out = a->k_out; p.v_out = a->v_out;
    const bool events = a->block_of_token != nullptr;
    if (w.token_stride != 0 && w.token_stride < w.n_warm) return fail(AKV_E_SHAPE, "token_stride < n_warm");
    if (a->out_slot && a->out_tokens < 1) return fail(AKV_E_SHAPE, "out_slot needs out_tokens >= 1");
    p.tok_stride = w.token_stride > 0 ? w.token_stride : w.n_warm;
    p.out_slot = a->out_slot;
    p.out_tokens = a->out_tokens;
    if (w.kind == AKV_WARM_AFFINE) {
        for (int bits : {w.bits_k, w.bits_v})
            if ((bits < 2 || bits > 4) && bits != 8) return fail(AKV_E_BITS, "Unsupported bits: %d", bits);
        if (w.block_t < 1 || w.group_v < 1 || a->D % w.group_v) return fail(AKV_E_SHAPE, "bad block_t / group_v");
        if (a->out_dtype != AKV_DT_F16 && a->out_dtype != AKV_DT_F32)
            return fail(AKV_E_DTYPE, "affine dequant produces float16 (or float32 holding float16 values)");
        if (events && a->n_blocks < 1) return fail(AKV_E_SHAPE, "block_of_token needs n_blocks >= 1");
        p.nbh = a->B * a->Hkv; p.Hkv = a->Hkv;
        p.kc_row = a->D * w.bits_k / 8; p.vc_row = a->D * w.bits_v / 8;
        p.T = w.block_t; p.Gv = w.group_v;
        p.nblk = events ? a->n_blocks : (w.n_warm + w.block_t - 1) / w.block_t;
        p.blk_of = a->block_of_token;
        p.n_out = w.n_out;
        p.k_oidx = w.k_oidx; p.v_oidx = w.v_oidx; p.k_odata = w.k_odata; p.v_odata = w.v_odata;
    } else if (w.kind == AKV_WARM_LEGACY) {
        if (events || a->out_slot) return fail(AKV_E_INVALID, "event blocks and output slots apply to the affine tier");
        if (w.token_stride != 0 && w.token_stride < w.n_warm) return fail(AKV_E_SHAPE, "token_stride < n_warm");
        if (w.legacy_sym < 0 && w.token_stride > w.n_warm)
            return fail(AKV_E_UNSUPPORTED, "symmetric-branch detection reads dense rows: force legacy_sym with a token stride");
        if (w.bits_k != w.bits_v) return fail(AKV_E_BITS, "legacy warm tier uses one width for K and V");
        if (w.bits_k != 2 && w.bits_k != 4 && w.bits_k != 8) return fail(AKV_E_BITS, "Unsupported bits: %d", w.bits_k);
        if (w.group_size < 1) return fail(AKV_E_SHAPE, "bad group_size");
        if (a->out_dtype < 0 || a->out_dtype > 2) return fail(AKV_E_DTYPE, "bad out dtype");
        const int pD = (int)round_up(a->D, w.group_size);
        p.nbh = w.warm_heads; p.Hkv = w.warm_heads;
        p.kc_row = p.vc_row = pD * w.bits_k / 8;
        p.gs = w.group_size; p.lg = pD / w.group_size; p.meta_dt = w.meta_dtype;
        p.legacy_sym = w.legacy_sym;
        if (w.legacy_sym < 0) {
            if (!a->workspace || !aligned16(a->workspace))
                return fail(AKV_E_WORKSPACE, "symmetric-branch detection needs a 256-byte workspace");
            p.sym_flags = (const int *)a->workspace;
            hipError_t e = akv::legacy_sym_launch(w.k_zero, w.v_zero, (int64_t)w.warm_heads * w.n_warm * p.lg,
                                                  w.meta_dtype, (int *)a->workspace, (hipStream_t)stream);
            if (e != hipSuccess) return hip_fail(e, "legacy symmetric detection");
        }
    } else {
        return fail(AKV_E_INVALID, "unknown warm kind %d", w.kind);
    }
    hipError_t e = akv::dequant_launch(p, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "dequant launch");
    return ok();
}

int akv_bitpack(const void *codes, void *packed, int64_t rows, int32_t dim, int32_t bits, void *stream) {
    if (bits != 2 && bits != 3 && bits != 4) return fail(AKV_E_BITS, "bitpack handles 2/3/4 bits, got %d", bits);
    if (rows < 0 || dim < 0) return fail(AKV_E_SHAPE, "bad sizes");
    if ((rows > 0 && dim > 0) && (!codes || !packed)) return fail(AKV_E_INVALID, "null pointer");
    const int prow = bits == 4 ? (dim + 1) / 2 : bits == 2 ? (dim + 3) / 4 : 3 * ((dim + 7) / 8);
    hipError_t e = akv::bitpack_launch(codes, packed, rows, dim, bits, prow, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "bitpack launch");
    return ok();
}

int akv_bitunpack(const void *packed, void *codes, int64_t rows, int32_t packed_dim, int32_t orig_dim, int32_t bits,
                  void *stream) {
    if (bits != 2 && bits != 3 && bits != 4) return fail(AKV_E_BITS, "bitunpack handles 2/3/4 bits, got %d", bits);
    if (rows < 0 || packed_dim < 0 || orig_dim < 0) return fail(AKV_E_SHAPE, "bad sizes");
    const int cap = bits == 4 ? 2 * packed_dim : bits == 2 ? 4 * packed_dim : 8 * (packed_dim / 3);
    if (bits == 2 && orig_dim != 4 * packed_dim) return fail(AKV_E_SHAPE, "2-bit unpack needs orig_dim == 4 * packed_dim");
    if (orig_dim > cap) return fail(AKV_E_SHAPE, "orig_dim %d exceeds the %d packed codes", orig_dim, cap);
    if ((rows > 0 && orig_dim > 0) && (!codes || !packed)) return fail(AKV_E_INVALID, "null pointer");
    hipError_t e = akv::bitunpack_launch(packed, codes, rows, packed_dim, orig_dim, bits, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "bitunpack launch");
    return ok();
}

int64_t akv_prefill_workspace_bytes(const akv_prefill_args *a) {
    if (check_prefill(a) != AKV_OK) return -1;
    PrefillPlan pl;
    make_prefill_plan(a, &pl);
    return pl.part_bytes;
}

int akv_prefill_attn(const akv_prefill_args *a, void *stream) {
    int rc = check_prefill(a);
    if (rc != AKV_OK) return rc;
    PrefillPlan pl;
    make_prefill_plan(a, &pl);
    if (pl.part_bytes > 0) {
        if (!a->workspace || a->workspace_bytes < pl.part_bytes)
            return fail(AKV_E_WORKSPACE, "workspace of %lld bytes needed", (long long)pl.part_bytes);
        if (!aligned16(a->workspace)) return fail(AKV_E_ALIGN, "workspace must be 16-byte aligned");
    }
    const akv_warm_desc &w = a->warm;
    akv::PrefillParams p{};
    p.B = a->B; p.Hq = a->Hq; p.Hkv = a->Hkv; p.M = a->M; p.g = a->Hq / a->Hkv; p.R = pl.R;
    p.q_bf16 = a->q_dtype == AKV_DT_BF16;
    p.q = a->q; p.out = a->out;
    p.khot = (const _Float16 *)a->k_hot; p.vhot = (const _Float16 *)a->v_hot; p.n_hot = a->n_hot;
    if (w.kind == AKV_WARM_AFFINE) {
        p.kc = w.k_codes; p.vc = w.v_codes;
        p.ks = (const _Float16 *)w.k_scale; p.kz = (const _Float16 *)w.k_zero;
        p.vs = (const _Float16 *)w.v_scale; p.vz = (const _Float16 *)w.v_zero;
        p.n_warm = w.n_warm; p.T = w.block_t; p.Gv = w.group_v;
        p.nblk = (w.n_warm + w.block_t - 1) / w.block_t;
        p.bits_k = w.bits_k; p.bits_v = w.bits_v;
    } else {
        p.n_warm = 0; p.T = 32; p.Gv = 32; p.nblk = 0; p.bits_k = p.bits_v = 4;
    }
    p.scale_log2 = a->sm_scale * 1.4426950408889634f;
    p.n_row_tiles = pl.n_row_tiles;
    p.nsplit = pl.nsplit;
    p.tiles_per_split = pl.tiles_per_split;
    p.part = (float *)a->workspace;
    p.nchunk = pl.nchunk; p.prows = pl.prows;
    p.kcur = a->k_chunk; p.vcur = a->v_chunk;
    p.n_cur = a->k_chunk ? a->M : 0;
    hipError_t e = akv::prefill_launch(p, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "prefill launch");
    return ok();
}

int64_t akv_timeline_words(void) { return akv::decode_fast_timeline_words(); }

int akv_timeline_fetch(uint64_t *host, int64_t words) {
    if (akv::decode_fast_timeline_words() == 0)
        return fail(AKV_E_UNSUPPORTED, "this build records no timeline (build it with make timeline)");
    if (!host || words < 0) return fail(AKV_E_INVALID, "bad timeline buffer");
    hipError_t e = akv::decode_fast_timeline_fetch((unsigned long long *)host, words);
    if (e != hipSuccess) return hip_fail(e, "timeline fetch");
    return ok();
}

int akv_timeline_clear(void *stream) {
    if (akv::decode_fast_timeline_words() == 0)
        return fail(AKV_E_UNSUPPORTED, "this build records no timeline (build it with make timeline)");
    hipError_t e = akv::decode_fast_timeline_clear((hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "timeline clear");
    return ok();
}

int akv_stream_read(const void *data, int64_t bytes, uint32_t *sink, void *stream) {
    if (bytes < 0 || bytes % 16) return fail(AKV_E_SHAPE, "bytes must be a non-negative multiple of 16");
    if (bytes > 0 && (!data || !sink)) return fail(AKV_E_INVALID, "null pointer");
    if (bytes > 0 && !aligned16(data)) return fail(AKV_E_ALIGN, "data must be 16-byte aligned");
    hipError_t e = akv::stream_read_launch(data, bytes, sink, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "stream read launch");
    return ok();
}

int akv_select_demote(const float *scores, int64_t rows, int64_t len, int64_t n_demote, int32_t protect_first,
                      int32_t protect_last, int64_t *out, void *stream) {
    if (rows < 0 || len < 0 || n_demote < 0) return fail(AKV_E_SHAPE, "negative size");
    if (n_demote > len) return fail(AKV_E_SHAPE, "n_demote (%lld) > len (%lld)", (long long)n_demote, (long long)len);
    if (protect_first < 0 || protect_last < 0) return fail(AKV_E_SHAPE, "negative protection");
    if (rows == 0 || n_demote == 0) return ok();
    if (!scores || !out) return fail(AKV_E_INVALID, "scores and out are required");
    if (!aligned16(scores) || !aligned16(out)) return fail(AKV_E_ALIGN, "scores/out must be 16-byte aligned");
    if (len >= ((int64_t)1 << 31)) return fail(AKV_E_SHAPE, "len too large");
    hipError_t e = akv::select_launch(scores, rows, len, n_demote, protect_first, protect_last, out, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "select launch");
    return ok();
}

int akv_importance_update(const akv_importance_args *a, void *stream) {
    if (!a) return fail(AKV_E_INVALID, "args is NULL");
    if (a->abi_version != AKV_ABI_VERSION) return fail(AKV_E_ABI, "ABI mismatch");
    if (a->attn_dtype < 0 || a->attn_dtype > 2) return fail(AKV_E_DTYPE, "bad attention dtype");
    if (a->B < 1 || a->H < 1 || a->M < 1 || a->N < 0 || a->n_scores < 0) return fail(AKV_E_SHAPE, "bad sizes");
    if ((a->n_scores > 0 && !a->scores) || (a->N > 0 && !a->attn)) return fail(AKV_E_INVALID, "null pointer");
    akv::ImportanceParams p{};
    p.attn = a->attn; p.attn_dt = a->attn_dtype;
    p.B = a->B; p.H = a->H; p.M = a->M; p.N = a->N;
    p.scores = a->scores; p.n_scores = a->n_scores; p.decay = a->decay;
    if (a->q_window < 0 || a->pool_kernel < 0 || a->pool_kernel > 64)
        return fail(AKV_E_SHAPE, "q_window must be >= 0 and pool_kernel in [0, 64]");
    p.m0 = (a->q_window > 0 && a->q_window < a->M) ? a->M - a->q_window : 0;
    // the reference pools only when kv_len > kernel (akv/importance.py:111)
    p.pool = (a->pool_kernel > 1 && a->N > a->pool_kernel) ? a->pool_kernel : 1;
    hipError_t e = akv::importance_launch(p, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "importance launch");
    return ok();
}

}  // extern "C"
