// Device helpers shared by the LDS-tiled attention kernels over the
// block-affine warm tier (decode_fast.hip, prefill.hip): buffer loads into
// LDS, exact fp16 dequant of packed code pairs and the code windows of each
// bit width, the hot-K channel permutation, and the online softmax of one
// 16-token MFMA tile.
#pragma once

#include "akv_common.h"

namespace akv {
namespace {

constexpr float kThreshF = 8.0f;
constexpr float kPLog2F = 7.0f;

template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt out of range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14)); }

// Buffer resource as four scalars (raw buffer, no stride, range-checked to `bytes`).
__device__ __forceinline__ u4 rsrc4(const void *base, uint32_t bytes) {
    const uint64_t b = (uint64_t)base;
    return (u4){(uint32_t)b, (uint32_t)(b >> 32) & 0xFFFFu, bytes, (uint32_t)kRsrcWord3};
}

// One LDS-DMA instruction: for each lane i set in `mask`, 16 bytes at buffer
// offset soff + voff_i are written to LDS [lds + 16 i]; bytes past the
// resource range arrive as zeros.  Written as one asm block so the compiler
// can neither merge two of them under divergent control flow nor change how
// many are issued (the vmcnt waits count them); M0 is restored afterwards.
// M0 is written several instructions before the load that reads it.  The
// loads are non-temporal (each byte is read once; measured 0.5 us per layer
// faster at the 32k decode workload than the default policy).
// Inline asm is opaque to the compiler's hazard checks, so each block brings the
// wait states its first load needs: a VMEM instruction may read an SGPR only 5
// wait states after a VALU wrote it, and the compiler keeps some buffer
// descriptors spilled in VGPR lanes and reloads them with v_readlane_b32 (a VALU
// write) right before a block.  Here the four SALU instructions and the s_nop 0
// make 5; the block of dma_lean opens with two and an s_nop 2.
__device__ __forceinline__ void dma16(u4 rsrc, uint32_t lds, uint32_t voff, uint32_t soff, uint64_t mask) {
    uint64_t saved;
    uint32_t saved_m0;
    asm volatile(
        "s_mov_b32 %[sm0], m0\n\t"
        "s_mov_b32 m0, %[lds]\n\t"
        "s_mov_b64 %[sv], exec\n\t"
        "s_and_b64 exec, exec, %[mask]\n\t"
        "s_nop 0\n\t"
        "buffer_load_dwordx4 %[voff], %[rsrc], %[soff] offen nt lds\n\t"
        "s_mov_b64 exec, %[sv]\n\t"
        "s_mov_b32 m0, %[sm0]"
        : [sv] "=&s"(saved), [sm0] "=&s"(saved_m0)
        : [lds] "s"(lds), [mask] "s"(mask), [voff] "v"(voff), [rsrc] "s"(rsrc), [soff] "s"(soff)
        : "memory");
}
// One contiguous range of BYTES bytes (buffer offset soff) into LDS [lds, lds + BYTES)
// with every lane active: 1 KiB pieces as 16-byte loads, 256-byte pieces as 4-byte
// loads.  The instruction's immediate offset advances the buffer and the LDS address
// alike, so one M0 value (set once, restored at the end of the block) serves the whole
// range.  v16 = lane * 16, v4 = lane * 4.  dma_count<BYTES>() is the number of loads
// issued (the vmcnt accounting of the callers counts them).
template <int BYTES>
__host__ __device__ constexpr bool dma_lean_ok() {
    return BYTES == 256 || BYTES == 512 || BYTES == 1024 || BYTES == 1536 || BYTES == 2048 || BYTES == 3072 ||
           BYTES == 4096;
}
template <int BYTES>
__host__ __device__ constexpr int dma_count() {
    return BYTES / 1024 + (BYTES % 1024) / 256;
}
#define AKV_DMA_HEAD "s_mov_b32 %[sm0], m0\n\ts_mov_b32 m0, %[lds]\n\ts_nop 2\n\t"
#define AKV_DMA_X4(off) "buffer_load_dwordx4 %[v16], %[rsrc], %[soff] offen offset:" #off " nt lds\n\t"
#define AKV_DMA_X1(off) "buffer_load_dword %[v4], %[rsrc], %[soff] offen offset:" #off " nt lds\n\t"
#define AKV_DMA_TAIL "s_mov_b32 m0, %[sm0]"
#define AKV_DMA_ARGS                                                                           \
    : [sm0] "=&s"(saved_m0)                                                                    \
    : [lds] "s"(lds), [v16] "v"(v16), [v4] "v"(v4), [rsrc] "s"(rsrc), [soff] "s"(soff) : "memory"
template <int BYTES>
__device__ __forceinline__ void dma_lean(u4 rsrc, uint32_t lds, uint32_t soff, uint32_t v16, uint32_t v4) {
    static_assert(dma_lean_ok<BYTES>(), "range size without a full-lane load pattern");
    uint32_t saved_m0;
    if constexpr (BYTES == 256) {
        asm volatile(AKV_DMA_HEAD AKV_DMA_X1(0) AKV_DMA_TAIL AKV_DMA_ARGS);
    } else if constexpr (BYTES == 512) {
        asm volatile(AKV_DMA_HEAD AKV_DMA_X1(0) AKV_DMA_X1(256) AKV_DMA_TAIL AKV_DMA_ARGS);
    } else if constexpr (BYTES == 1024) {
        asm volatile(AKV_DMA_HEAD AKV_DMA_X4(0) AKV_DMA_TAIL AKV_DMA_ARGS);
    } else if constexpr (BYTES == 1536) {
        asm volatile(AKV_DMA_HEAD AKV_DMA_X4(0) AKV_DMA_X1(1024) AKV_DMA_X1(1280) AKV_DMA_TAIL AKV_DMA_ARGS);
    } else if constexpr (BYTES == 2048) {
        asm volatile(AKV_DMA_HEAD AKV_DMA_X4(0) AKV_DMA_X4(1024) AKV_DMA_TAIL AKV_DMA_ARGS);
    } else if constexpr (BYTES == 3072) {
        asm volatile(AKV_DMA_HEAD AKV_DMA_X4(0) AKV_DMA_X4(1024) AKV_DMA_X4(2048) AKV_DMA_TAIL AKV_DMA_ARGS);
    } else {
        asm volatile(AKV_DMA_HEAD AKV_DMA_X4(0) AKV_DMA_X4(1024) AKV_DMA_X4(2048) AKV_DMA_X4(3072) AKV_DMA_TAIL
                         AKV_DMA_ARGS);
    }
}
#undef AKV_DMA_HEAD
#undef AKV_DMA_X4
#undef AKV_DMA_X1
#undef AKV_DMA_TAIL
#undef AKV_DMA_ARGS

__device__ __forceinline__ uint64_t lane_mask(int bytes) {  // lanes covering `bytes` (>= 16)
    return bytes >= 1024 ? ~0ull : ((1ull << (bytes >> 4)) - 1ull);
}
__device__ __forceinline__ uint32_t lds_addr(const unsigned char *p) { return (uint32_t)(uintptr_t)p; }

// A value the compiler must keep in a VGPR (not rematerialize as a literal),
// so (x & m) | c selects one v_and_or_b32 with m in a VGPR and c in an SGPR.
__device__ __forceinline__ uint32_t in_vgpr(uint32_t x) {
    asm volatile("" : "+v"(x));
    return x;
}

// An LDS pointer made from a 32-bit LDS byte address (for example one kept opaque by
// in_vgpr, so that the constant parts of later addresses become instruction offsets).
typedef const __attribute__((address_space(3))) uint32_t lds_cu32;
template <typename T>
__device__ __forceinline__ const __attribute__((address_space(3))) T *lds_ptr(uint32_t a) {
    return (const __attribute__((address_space(3))) T *)(size_t)a;
}

__device__ __forceinline__ h2 pk_fma(h2 a, h2 b, h2 c) { return __builtin_elementwise_fma(a, b, c); }

__device__ __forceinline__ float wmax16(float x) {
    x = fmaxf(x, __shfl_xor(x, 16));
    x = fmaxf(x, __shfl_xor(x, 32));
    return x;
}
__device__ __forceinline__ float wsum16(float x) {
    x += __shfl_xor(x, 16);
    x += __shfl_xor(x, 32);
    return x;
}

// fp16 bits of 2^(10-o): a code at bit offset o of that number's mantissa reads as 2^(10-o) + c.
__host__ __device__ constexpr uint32_t magic_of(int o) { return (uint32_t)(25 - o) << 10; }
__host__ __device__ constexpr uint32_t magic2(int o) { return magic_of(o) * 0x00010001u; }
__host__ __device__ constexpr float magic_val(int o) { return (float)(1 << (10 - o)); }

// --------------------------------------------------------------- K windows
// Pair pi (0..15) of a lane's 32 channels: window dword and bit offset; the
// channels (relative to the lane's group) of its halves are kpair_chan().
template <int BK>
__host__ __device__ constexpr int koff(int pi) {
    return BK == 3 ? ((pi % 8) == 0 ? 0 : (pi % 8) == 1 ? 3 : (pi % 8) == 2 ? 6 : (pi % 8) == 3 ? 1
                      : (pi % 8) == 4 ? 4 : (pi % 8) == 5 ? 7 : (pi % 8) == 6 ? 2 : 5)
         : BK == 4 ? (pi % 2) * 4
                   : 2 * (pi % 4);
}
template <int BK>
struct KWin {
    uint32_t w[BK == 3 ? 6 : (BK == 4 ? 8 : 4)];
};
// r: the lane's raw code bytes (BK*4 bytes) as little-endian dwords
template <int BK>
__device__ __forceinline__ void k_windows(const uint32_t *r, KWin<BK> &W) {
    if constexpr (BK == 3) {
        W.w[0] = perm(r[1], r[0], 0x04050102u);
        W.w[1] = perm(r[1], r[0], 0x03040001u);
        W.w[2] = perm(r[1], r[0], 0x0C030C00u);
        W.w[3] = perm(r[2], r[1], 0x06070304u);
        W.w[4] = perm(r[2], r[1], 0x05060203u);
        W.w[5] = perm(r[2], r[1], 0x0C050C02u);
    } else if constexpr (BK == 4) {
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            W.w[2 * d] = r[d];
            W.w[2 * d + 1] = perm(0u, r[d], 0x0C030C01u);
        }
    } else {
#pragma unroll
        for (int d = 0; d < 2; ++d) {
            W.w[2 * d] = r[d];
            W.w[2 * d + 1] = perm(0u, r[d], 0x0C030C01u);
        }
    }
}
template <int BK>
__device__ __forceinline__ uint32_t k_window_of(const KWin<BK> &W, int pi) {
    if (BK == 3) {
        const int k = pi % 8, base = 3 * (pi / 8);
        return W.w[base + (k < 3 ? 0 : (k < 6 ? 1 : 2))];
    } else if (BK == 4) {
        return W.w[2 * (pi / 4) + ((pi % 4) >= 2 ? 1 : 0)];
    } else {
        return W.w[2 * (pi / 8) + ((pi % 8) >= 4 ? 1 : 0)];
    }
}

// --------------------------------------------------------------- V windows
// One token pair (a, b) of an 8-channel chunk.  da / db: the chunk's bytes
// of each token at byte 0 of a dword (memory order).  Code k (channel k of
// the chunk) sits in window vwin(k) at bit offset voff(k), in both halves.
template <int BV>
struct VSlot {
    static constexpr int NW = BV == 3 ? 3 : (BV == 4 ? 4 : 2);
};
template <int BV>
__host__ __device__ constexpr int vwin(int k) {
    // 3-bit: codes 7,6,5 in window 0; 4,3,2 in 1; 1,0 in 2
    // 4-bit: ch1,ch0 in 0; ch3,ch2 in 1; ch5,ch4 in 2; ch7,ch6 in 3
    // 2-bit: codes 3..0 in 0; 7..4 in 1
    return BV == 3 ? (k >= 5 ? 0 : (k >= 2 ? 1 : 2)) : BV == 4 ? (k / 2) : (k / 4);
}
template <int BV>
__host__ __device__ constexpr int voff(int k) {
    return BV == 3 ? (k >= 5 ? 3 * (7 - k) : (k >= 2 ? 3 * (4 - k) : 3 * (1 - k)))
         : BV == 4 ? ((k & 1) ? 0 : 4)
                   : 2 * (3 - (k & 3));
}
template <int BV>
__device__ __forceinline__ void v_windows(uint32_t da, uint32_t db, uint32_t *win) {
    if (BV == 3) {
        win[0] = perm(db, da, 0x05060102u);            // [a.x2 a.x1 | b.x2 b.x1]: W bits 0-15
        const uint32_t w1 = perm(db, da, 0x04050001u); // [a.x1 a.x0 | b.x1 b.x0]: W bits 8-23
        win[1] = w1 >> 1;
        win[2] = w1 >> 10;
    } else if (BV == 4) {
        const uint32_t lo = perm(db, da, 0x05040100u); // bytes 0,1 of a | of b
        const uint32_t hi = perm(db, da, 0x07060302u); // bytes 2,3
        win[0] = lo;
        win[1] = lo >> 8;
        win[2] = hi;
        win[3] = hi >> 8;
    } else {
        const uint32_t w = perm(db, da, 0x05040100u);  // bytes 0,1 of a | of b
        win[0] = w;
        win[1] = w >> 8;
    }
}
template <int BV>
__host__ __device__ constexpr int v_ostep() { return BV == 3 ? 3 : (BV == 4 ? 4 : 2); }
template <int BV>
__host__ __device__ constexpr int v_noffs() { return BV == 3 ? 3 : (BV == 4 ? 2 : 4); }

// Masks of a code at bit offset o (both halves), one VGPR per offset the bit
// width uses (3 bits: any of 0..7; 4 bits: 0, 4; 2 bits: 0, 2, 4, 6).
template <int B>
struct Masks {
    uint32_t m[8];
    __device__ __forceinline__ void init() {
#pragma unroll
        for (int o = 0; o < 8; ++o)
            if (B == 3 || (B == 4 && o % 4 == 0) || (B == 2 && o % 2 == 0))
                m[o] = in_vgpr((((1u << B) - 1u) << o) * 0x00010001u);
    }
};

// --------------------------------------------------------------- layouts
struct Soft {
    float m2, l;
    f4 acc[8];  // O^T: channel 8*chunk + j of chunk 4*grp + i, row col
    f4 accz;    // sum_t P * (V zero-point of the chunk's group): added to every channel of the chunk at the end
};

// Online softmax over one 16-token tile.  s: raw q.k of tokens 4*grp+i for
// row col.  The running max of a row only moves when some score exceeds it by
// more than 2^8 (log2 units); the test needs no cross-lane traffic, since a
// row's tile max passes the bound iff one of its four lanes' maxima does.  On
// the rare update the four lanes of a row agree on the new max through two
// shuffles.  Returns the fp16 P^T operand (x 2^7).
// Maximum of a tile's scores straight from the MFMAs, as IEEE maximum (nested, so
// one or two v_maximum3_f32).  fmaxf over values the compiler cannot prove
// canonical (MFMA results) costs an extra v_max per operand to quiet signalling
// NaNs; maximum needs none, and the scores never hold a NaN, so both give the same
// max.  It must be an operation the compiler sees: a VALU may read the result of
// v_mfma_f32_16x16x32_f16 only 8 wait states after it issues, and the compiler
// inserts those only before instructions it knows.  An inline-asm v_max3_f32 here
// read stale registers once nothing else separated it from the last MFMA.
__device__ __forceinline__ float mfma_max4(f4 s) {
    return __builtin_elementwise_maximum(
        __builtin_elementwise_maximum(__builtin_elementwise_maximum(s[0], s[1]), s[2]), s[3]);
}
__device__ __forceinline__ float mfma_max8(f4 a, f4 b) {
    const float m0 = __builtin_elementwise_maximum(__builtin_elementwise_maximum(a[0], a[1]), a[2]);
    const float m1 = __builtin_elementwise_maximum(__builtin_elementwise_maximum(a[3], b[0]), b[1]);
    const float m2 = __builtin_elementwise_maximum(__builtin_elementwise_maximum(b[2], b[3]), b[3]);
    return __builtin_elementwise_maximum(__builtin_elementwise_maximum(m0, m1), m2);
}

__device__ __forceinline__ h4 softmax16(Soft &st, f4 s, float sl2) {
    const float t = mfma_max4(s) * sl2;
    if (__builtin_amdgcn_ballot_w64(t > st.m2 + kThreshF)) {
        const float tm2 = wmax16(t);
        const float mn = fmaxf(st.m2, tm2);
        const float alpha = __builtin_amdgcn_exp2f(st.m2 - mn);
        st.l *= alpha;
#pragma unroll
        for (int j = 0; j < 8; ++j) st.acc[j] *= alpha;
        st.accz *= alpha;
        st.m2 = mn;
    }
    const float bias = kPLog2F - st.m2;
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[i], sl2, bias));
    st.l += (p[0] + p[1]) + (p[2] + p[3]);
    return (h4){(_Float16)p[0], (_Float16)p[1], (_Float16)p[2], (_Float16)p[3]};
}

// The same over a 32-token tile given as two 16-token halves: returns the
// fp16 P^T operand of a 16x16x32 MFMA whose K index 8*grp + j is token
// 4*grp + j of half 0 (j < 4) or of half 1 (j >= 4).
__device__ __forceinline__ h8 softmax32(Soft &st, f4 s0, f4 s1, float sl2) {
    const float t = mfma_max8(s0, s1) * sl2;
    if (__builtin_amdgcn_ballot_w64(t > st.m2 + kThreshF)) {
        const float tm2 = wmax16(t);
        const float mn = fmaxf(st.m2, tm2);
        const float alpha = __builtin_amdgcn_exp2f(st.m2 - mn);
        st.l *= alpha;
#pragma unroll
        for (int j = 0; j < 8; ++j) st.acc[j] *= alpha;
        st.accz *= alpha;
        st.m2 = mn;
    }
    const float bias = kPLog2F - st.m2;
    float p[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        p[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s0[i], sl2, bias));
        p[4 + i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s1[i], sl2, bias));
    }
    st.l += ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
    return (h8){(_Float16)p[0], (_Float16)p[1], (_Float16)p[2], (_Float16)p[3],
                (_Float16)p[4], (_Float16)p[5], (_Float16)p[6], (_Float16)p[7]};
}

__device__ __forceinline__ uint32_t lds_u16(const unsigned char *p) { return *(const uint16_t *)p; }
__device__ __forceinline__ h2 lds_h2(const unsigned char *a, const unsigned char *b) {
    return (h2){*(const _Float16 *)a, *(const _Float16 *)b};
}
__device__ __forceinline__ bool finite2(uint32_t x) {
    return ((x & 0x7C00u) != 0x7C00u) && ((x & 0x7C000000u) != 0x7C000000u);
}

}  // namespace

// Natural-order hot K (16 dwords of channel pairs 2d, 2d+1 of the lane's 32
// channels) -> the warm pair order: pair pi holds channels kpair_chan(pi, 0/1),
// which always have the same parity, so one byte permute builds each pair.
template <int BK>
__device__ __forceinline__ void hot_k_pairs(const uint32_t *nat, uint32_t *pairs) {
#pragma unroll
    for (int pi = 0; pi < 16; ++pi) {
        const int c0 = kpair_chan<BK>(pi, 0), c1 = kpair_chan<BK>(pi, 1);
        const uint32_t sel = (c0 & 1) ? 0x07060302u : 0x05040100u;
        pairs[pi] = perm(nat[c1 >> 1], nat[c0 >> 1], sel);
    }
}

}  // namespace akv
