// Device-side helpers shared by the warm-tier kernels (gfx950 / CDNA4).
//
// Every kernel here is written for 64-lane wavefronts.  Code bytes are read
// through buffer resources (bounds-checked: an offset past `num_records`
// returns 0), code pairs are turned into fp16 with the 0x6400 exponent trick,
// and the reference's fp16 dequant (two roundings, no FMA) is done with packed
// half arithmetic -- the library is compiled with -ffp-contract=off.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "akv_hip.h"

namespace akv {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));
typedef uint32_t u3 __attribute__((ext_vector_type(3)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

// Third descriptor word of a raw (untyped) buffer resource on gfx9-family parts.
constexpr int kRsrcWord3 = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, kRsrcWord3);
}
__device__ __forceinline__ uint32_t bld32(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
__device__ __forceinline__ u2 bld64(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
}
__device__ __forceinline__ u3 bld96(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b96(r, off, 0, 0);
}
__device__ __forceinline__ u4 bld128(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}
__device__ __forceinline__ uint16_t bld16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}

__device__ __forceinline__ h2 as_h2(uint32_t x) { return __builtin_bit_cast(h2, x); }
__device__ __forceinline__ uint32_t as_u32(h2 x) { return __builtin_bit_cast(uint32_t, x); }

// v_perm_b32: result byte i = byte sel[i] of the 8-byte value {hi, lo} (0-3 from lo).
__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}

// Two small unsigned codes held in the low bits of each 16-bit half -> exact fp16 values.
__device__ __forceinline__ h2 codes_to_h2(uint32_t pair) {
    const h2 magic = {(_Float16)1024.0f, (_Float16)1024.0f};
    return as_h2(pair | 0x64006400u) - magic;
}

// Reference fp16 dequant of a code pair: codes.half() * scale (rounded) + zero (rounded).
__device__ __forceinline__ h2 deq_affine(uint32_t pair, h2 s, h2 z) {
    h2 c = codes_to_h2(pair);
    h2 t = c * s;
    return t + z;
}

__device__ __forceinline__ f4 mfma_k32(h8 a, h8 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f4 mfma_k16(h4 a, h4 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);  // quiet NaN
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// Value of a meta / activation element of dtype `dt` as float.
__device__ __forceinline__ float load_as_f32(const void *p, int64_t i, int dt) {
    if (dt == AKV_DT_F16) return (float)((const _Float16 *)p)[i];
    if (dt == AKV_DT_BF16) return bf16_to_f32(((const uint16_t *)p)[i]);
    return ((const float *)p)[i];
}

// ---------------------------------------------------------------------------
// Code-pair extraction.  A "pair" is two codes placed in the low bits of the
// two 16-bit halves of a dword, ready for codes_to_h2.  Which two channels a
// pair carries depends on the packing; the *_chan functions give it so the
// other operand of the dot product can be permuted to match.
// ---------------------------------------------------------------------------

// K side: one token, LCH = D/4 consecutive channels held by a lane as raw
// little-endian dwords r[] (the bitpack bytes in memory order).
// Channel (relative to the lane's first channel) of half `hf` of pair `pi`.
template <int BITS>
__host__ __device__ constexpr int kpair_chan(int pi, int hf) {
    if (BITS == 3) {  // word pairs (2wp, 2wp+1); codes 7..3 from the low window, 2..0 from the high
        return 8 * (2 * (pi / 8) + hf) + (7 - pi % 8);
    } else if (BITS == 4) {  // dword d: (b0.lo,b2.lo),(b0.hi,b2.hi),(b1.lo,b3.lo),(b1.hi,b3.hi)
        return 8 * (pi / 4) + (pi % 4 == 0 ? 1 : pi % 4 == 1 ? 0 : pi % 4 == 2 ? 3 : 2) + 4 * hf;
    } else if (BITS == 2) {  // dword d: crumb r of bytes (0,2) for r<4, of (1,3) for r>=4
        return 16 * (pi / 8) + (pi % 8 < 4 ? 3 - pi % 8 : 11 - pi % 8) + 8 * hf;
    } else if (BITS == 8) {  // dword d: (b0,b2),(b1,b3)
        return 4 * (pi / 2) + pi % 2 + 2 * hf;
    } else {  // 16: fp16 values in natural order
        return 2 * pi + hf;
    }
}

template <int BITS>
__device__ __forceinline__ uint32_t kpair_extract(const uint32_t *r, int pi) {
    if (BITS == 3) {
        const int wp = pi / 8, k = pi % 8;
        // bytes of word pair wp: 6wp..6wp+5
        uint32_t zlo, zhi;
        if (wp == 0) {
            zlo = perm(r[1], r[0], 0x04050102u);  // [b2 b1 b5 b4]
            zhi = perm(r[1], r[0], 0x03040001u);  // [b1 b0 b4 b3]
        } else {
            zlo = perm(r[2], r[1], 0x06070304u);  // [b8 b7 b11 b10]
            zhi = perm(r[2], r[1], 0x05060203u);  // [b7 b6 b10 b9]
        }
        return k < 5 ? (zlo >> (3 * k)) & 0x00070007u : (zhi >> (7 + 3 * (k - 5))) & 0x00070007u;
    } else if (BITS == 4) {
        return (r[pi / 4] >> (4 * (pi % 4))) & 0x000F000Fu;
    } else if (BITS == 2) {
        return (r[pi / 8] >> (2 * (pi % 8))) & 0x00030003u;
    } else {  // 8
        return (r[pi / 2] >> (8 * (pi % 2))) & 0x00FF00FFu;
    }
}

// V side: one 8-channel chunk of two tokens a, b.  `wa`, `wb` hold the
// chunk's bytes in memory order starting at byte 0 of the dword (8-bit codes
// need two dwords each: wa[0..1], wb[0..1]).  Pair j carries channel vchan(j)
// of token a (low half) and of token b (high half).
template <int BITS>
__host__ __device__ constexpr int vpair_chan(int j) {
    if (BITS == 3) return 7 - j;
    if (BITS == 4) return j ^ 1;
    if (BITS == 2) return (j < 4) ? 3 - j : 11 - j;
    return j;  // 8-bit and fp16: natural
}

template <int BITS>
__device__ __forceinline__ uint32_t vpair_extract(const uint32_t *wa, const uint32_t *wb, int j) {
    if (BITS == 3) {
        if (j < 5) {
            uint32_t z = perm(wb[0], wa[0], 0x05060102u);  // [a.b2 a.b1 b.b2 b.b1]
            return (z >> (3 * j)) & 0x00070007u;
        }
        uint32_t z = perm(wb[0], wa[0], 0x04050001u);  // [a.b1 a.b0 b.b1 b.b0]
        return (z >> (7 + 3 * (j - 5))) & 0x00070007u;
    } else if (BITS == 4) {
        uint32_t z = j < 4 ? perm(wb[0], wa[0], 0x05040100u) : perm(wb[0], wa[0], 0x07060302u);
        return (z >> (4 * (j & 3))) & 0x000F000Fu;
    } else if (BITS == 2) {
        uint32_t z = (wa[0] & 0xFFFFu) | (wb[0] << 16);
        return (z >> (2 * j)) & 0x00030003u;
    } else {  // 8
        const int d = j / 4, k = j % 4;
        // bytes k of wa[d] and wb[d] into the low byte of each half
        return perm(wb[d], wa[d], (uint32_t)(k | (0x0C << 8) | ((4 + k) << 16) | (0x0C << 24)));
    }
}

// Code of channel c from one packed row in the bitpack layout (akv/bitpack.py).
__device__ __forceinline__ uint32_t extract_code(const unsigned char *row, int c, int bits) {
    if (bits == 4) {
        const uint32_t by = row[c >> 1];
        return (c & 1) ? (by & 15u) : (by >> 4);
    }
    if (bits == 2) return ((uint32_t)row[c >> 2] >> (6 - 2 * (c & 3))) & 3u;
    if (bits == 3) {
        const int w = c >> 3, i = c & 7;
        const uint32_t W = ((uint32_t)row[3 * w] << 16) | ((uint32_t)row[3 * w + 1] << 8) | row[3 * w + 2];
        return (W >> (21 - 3 * i)) & 7u;
    }
    return row[c];
}

}  // namespace akv
