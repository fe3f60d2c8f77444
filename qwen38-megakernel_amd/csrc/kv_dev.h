// Device-side building blocks of the quantized KV path for gfx950 (CDNA4, wave64).
//
// Row formats (one row = 256 values of one (layer, kv head, position, K or V)); both are the reference's
// (qwen38_mk.cu:2003-2097) so that stored bytes are bit-identical:
//   q8 : 256 int8 codes in natural order, one fp16 scale per 32 values (am / 127).
//   b-bit, b = 4..7 : bytes 0..127 = low nibbles (word w = values 8w..8w+7: values 0..3 in the low nibbles of bytes
//        0..3, values 4..7 in the high nibbles); bytes 128 + w (b-4) .. = the high bits, value k at bit (b-4) k of
//        that little-endian field; code n = q + 2^(b-1); one fp16 scale d = (signed max) / -2^(b-1) per 32 values.
// Scales live in a separate [row][8] fp16 array.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "kv_layout.h"

namespace qkv {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

// The value of lane l ^ M, by VALU lane exchanges instead of ds_bpermute (an LDS round trip per exchange): DPP
// quad_perm for M = 1, 2; quad_perm + row_half_mirror (l ^ 3 ^ 7) for 4; row_mirror + row_half_mirror (l ^ 15 ^ 7)
// for 8; v_permlane16_swap / v_permlane32_swap for 16 / 32, which leave the partner row's value in one of the two
// registers depending on the lane's row (inline assembly: the builtin folds the two results when both inputs are the
// same value; s_nop covers the VALU-write -> permlane-read hazard).
template <int M>
__device__ __forceinline__ unsigned xor_lane_u(unsigned v) {
    if constexpr (M == 1) return __builtin_amdgcn_update_dpp(0u, v, 0xB1, 0xf, 0xf, false); // quad_perm 1,0,3,2
    else if constexpr (M == 2) return __builtin_amdgcn_update_dpp(0u, v, 0x4E, 0xf, 0xf, false); // quad_perm 2,3,0,1
    else if constexpr (M == 4) {
        const unsigned x = __builtin_amdgcn_update_dpp(0u, v, 0x1B, 0xf, 0xf, false); // quad_perm 3,2,1,0
        return __builtin_amdgcn_update_dpp(0u, x, 0x141, 0xf, 0xf, false);              // row_half_mirror
    } else if constexpr (M == 8) {
        const unsigned x = __builtin_amdgcn_update_dpp(0u, v, 0x140, 0xf, 0xf, false); // row_mirror
        return __builtin_amdgcn_update_dpp(0u, x, 0x141, 0xf, 0xf, false);             // row_half_mirror
    } else if constexpr (M == 16) {
        unsigned a = v, b = v;
        asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
        return (threadIdx.x & 16) ? a : b;
    } else {
        static_assert(M == 32, "lane exchange masks 1..32");
        unsigned a = v, b = v;
        asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
        return (threadIdx.x & 32) ? a : b;
    }
}
__device__ __forceinline__ unsigned shfl_xor_u(unsigned v, int m) {
    switch (m) { // m is a constant after unrolling
    case 1: return xor_lane_u<1>(v);
    case 2: return xor_lane_u<2>(v);
    case 4: return xor_lane_u<4>(v);
    case 8: return xor_lane_u<8>(v);
    case 16: return xor_lane_u<16>(v);
    default: return xor_lane_u<32>(v);
    }
}
__device__ __forceinline__ float shfl_xor(float v, int m) { return __builtin_bit_cast(float, shfl_xor_u(__builtin_bit_cast(unsigned, v), m)); }

// max / sum over the four lanes l, l ^ 16, l ^ 32, l ^ 48 with v_permlane16_swap / v_permlane32_swap (VALU exchanges
// between 16-lane rows, no LDS round trip).  Two copies of the value go in; afterwards one register holds rows
// (0, 0, 2, 2) and the other rows (1, 1, 3, 3) (then halves (lo, lo) / (hi, hi)), so every lane gets
// op(op(x_r0, x_r1), op(x_r2, x_r3)), each op's operands in either order (exact: max and add are commutative).
// Inline assembly: the compiler's builtin folds the two results into one when both inputs are the same value.  The
// s_nops cover the VALU-write -> permlane-read hazard.
__device__ __forceinline__ float quad_max(float v) {
    float a = v, b = v;
    asm("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\tv_max_f32 %0, %0, %1\n\tv_mov_b32 %1, %0\n\t"
        "s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\tv_max_f32 %0, %0, %1"
        : "+v"(a), "+v"(b));
    return a;
}
__device__ __forceinline__ float quad_sum(float v) {
    float a = v, b = v;
    asm("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\tv_add_f32 %0, %0, %1\n\tv_mov_b32 %1, %0\n\t"
        "s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\tv_add_f32 %0, %0, %1"
        : "+v"(a), "+v"(b));
    return a;
}

// ------------------------------------------------------------------------------------------------ quantizers
// One row per wave: lane l holds values 4l .. 4l+3 (a 32-value block = 8 lanes).

// 256-point FWHT, stage order over index bits 0..7 ascending, butterfly (a+b, a-b), then * 1/16 (qwen38_mk.cu:2048-2068).
// Index i = 4 lane + k: bits 0..1 in-lane, bits 2..7 = lane bits 0..5.
__device__ __forceinline__ void fwht256_w64(float (&v)[4]) {
#pragma unroll
    for (int m = 1; m < 4; m <<= 1)
#pragma unroll
        for (int k = 0; k < 4; k++)
            if (!(k & m)) {
                const float a = v[k], b = v[k | m];
                v[k] = a + b;
                v[k | m] = a - b;
            }
    const int lane = lane_id();
    // lane-bit stages: v' = o + s v with s = -1 in the upper lane of each pair (o - v) and +1 in the lower (v + o), one
    // FMA each: a product with +-1 is exact, so the FMA rounds o +- v once, the same bits as the add or subtract
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
        const float sg = (lane & m) ? -1.f : 1.f;
#pragma unroll
        for (int k = 0; k < 4; k++) v[k] = __builtin_fmaf(sg, v[k], shfl_xor(v[k], m));
    }
#pragma unroll
    for (int k = 0; k < 4; k++) v[k] *= 0.0625f;
}

// Q/K prep of one row per wave (lane l holds values 4l .. 4l+3): RMSNorm over the 256 values with weight w and
// eps 1e-6, then NeoX RoPE on values 0..63, pair (i, i + 32) rotated by the table row rc[i] = (cos, sin) of the
// row's position (qwen38_mk.cu:2623-2636, 2903-2910, mk_shared.cuh:239).  The arithmetic order is fixed so that a
// scalar restatement reproduces it bit for bit: per-lane sum of squares as an FMA chain, xor-butterfly over the
// wave, 1 / sqrt (both correctly rounded), products and FMAs named explicitly.  All 64 lanes must call it.
__device__ __forceinline__ void qk_prep(float (&v)[4], const float * w, const float2 * rc) {
    const int lane = lane_id();
    float s = __builtin_fmaf(v[3], v[3], __builtin_fmaf(v[2], v[2], __builtin_fmaf(v[1], v[1], v[0] * v[0])));
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) s = s + shfl_xor(s, m);
    const float rs = 1.0f / __builtin_sqrtf(s / 256.0f + 1e-6f);
    const float4 wv = *reinterpret_cast<const float4 *>(w + 4 * lane);
    v[0] = v[0] * (rs * wv.x);
    v[1] = v[1] * (rs * wv.y);
    v[2] = v[2] * (rs * wv.z);
    v[3] = v[3] * (rs * wv.w);
    float o[4];
#pragma unroll
    for (int k = 0; k < 4; k++) o[k] = shfl_xor(v[k], 8);
    if (lane < 16) {
        const float4 * tab = reinterpret_cast<const float4 *>(rc + 4 * (lane & 7));
        const float4 c01 = tab[0], c23 = tab[1];
        const float c[4] = {c01.x, c01.z, c23.x, c23.z}, sn[4] = {c01.y, c01.w, c23.y, c23.w};
#pragma unroll
        for (int k = 0; k < 4; k++)
            v[k] = lane < 8 ? __builtin_fmaf(v[k], c[k], -(o[k] * sn[k])) : __builtin_fmaf(o[k], sn[k], v[k] * c[k]);
    }
}

// float -> int32 by the hardware conversion: truncates, saturates, NaN -> 0 (the reference's cvt.rzi; a C cast leaves
// out-of-range and NaN undefined, so the instruction is named explicitly)
__device__ __forceinline__ int f2i_rz(float x) {
    int r;
    asm("v_cvt_i32_f32 %0, %1" : "=v"(r) : "v"(x));
    return r;
}
// round half to even, then convert (__float2int_rn)
__device__ __forceinline__ int f2i_rn(float x) { return f2i_rz(__builtin_rintf(x)); }

__device__ __forceinline__ uint16_t f2h_bits(float x) {
    const _Float16 h = (_Float16) x;
    return __builtin_bit_cast(uint16_t, h);
}
__device__ __forceinline__ float h2f_bits(uint16_t b) { return (float) __builtin_bit_cast(_Float16, b); }

// q8_0 codes of this lane's 4 values as one word and the scale of its block, given the block's max |v| am
__device__ __forceinline__ unsigned quant_q8_am(const float (&v)[4], float am, uint16_t & sc) {
    const float id = am > 0.f ? 127.0f / am : 0.f;
    unsigned w = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) w |= ((unsigned) f2i_rn(v[k] * id) & 0xffu) << (8 * k);
    sc = f2h_bits(am / 127.0f);
    return w;
}
// max |v| over the lane's 32-value block (8 lanes)
__device__ __forceinline__ float block_absmax(const float (&v)[4]) {
    float am = 0.f;
#pragma unroll
    for (int k = 0; k < 4; k++) am = fmaxf(am, fabsf(v[k]));
    am = fmaxf(am, shfl_xor(am, 1));
    am = fmaxf(am, shfl_xor(am, 2));
    return fmaxf(am, shfl_xor(am, 4));
}
// q8_0 store of one row (kv_store_q8, qwen38_mk.cu:2005-2022): codes of this lane's 4 values as one word, scale of its block
__device__ __forceinline__ unsigned quant_q8(const float (&v)[4], uint16_t & sc) { return quant_q8_am(v, block_absmax(v), sc); }

// b-bit store (kv_store_q4 :2029-2046 / kv_store_qn :2075-2097): signed max (ties -> larger value), d = sv / -h,
// id = 1/d, n = min(2h-1, (int) fma(v, id, h + 0.5)).  Returns the 4 codes n (one per byte).
__device__ __forceinline__ unsigned quant_qn(const float (&v)[4], int bits, uint16_t & sc, float & amax) {
    const int h = 1 << (bits - 1);
    float am = 0.f, sv = 0.f;
    // (selects, not branches: the row is one dependent chain per wave)
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const float a = fabsf(v[k]);
        const bool take = a > am || (a == am && v[k] > sv);
        am = take ? a : am;
        sv = take ? v[k] : sv;
    }
#pragma unroll
    for (int m = 1; m <= 4; m <<= 1) {
        const float oa = shfl_xor(am, m), os = shfl_xor(sv, m);
        const bool take = oa > am || (oa == am && os > sv);
        am = take ? oa : am;
        sv = take ? os : sv;
    }
    amax = am; // the block's max |v| (the q8 ring copy's)
    const float d = sv / (float) -h, id = d != 0.f ? 1.0f / d : 0.f;
    unsigned codes = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int n = min(2 * h - 1, f2i_rz(__builtin_fmaf(v[k], id, (float) h + 0.5f)));
        codes |= ((unsigned) n & 0xffu) << (8 * k);
    }
    sc = f2h_bits(d);
    return codes;
}

// ------------------------------------------------------------------------------------------------ kv_store of one row
// One row per wave: lane l holds values 4l .. 4l+3 (kv_store, qwen38_mk.cu:2099-2116).  Used by the append kernel and
// by the attention kernel's fused append (mk_kv_append_attend), so both store the same bytes.

// the store geometry a row's addresses need (the part of StoreLayout a called function takes as plain values)
struct RowGeo {
    const int * ptab;
    int pt_stride, page, n_pages, kvrc;
};
__device__ __forceinline__ RowGeo geo_of(const StoreLayout & S) { return RowGeo{S.ptab, S.pt_stride, S.page, S.n_pages, S.kvrc}; }

__device__ __forceinline__ size_t main_row(const RowGeo & S, int seq, int g, int p) {
    const int lp = p / S.page;
    const int phys = S.ptab[seq * S.pt_stride + lp];
    return (size_t) (g * S.n_pages + phys) * S.page + (p - lp * S.page);
}
__device__ __forceinline__ size_t main_row(const StoreLayout & S, int seq, int g, int p) { return main_row(geo_of(S), seq, g, p); }
__device__ __forceinline__ size_t ring_row(const RowGeo & S, int seq, int g, int p) {
    return (size_t) (seq * NKV + g) * S.kvrc + p % S.kvrc;
}
__device__ __forceinline__ size_t ring_row(const StoreLayout & S, int seq, int g, int p) { return ring_row(geo_of(S), seq, g, p); }

// the lane's 4 values of input row `row` (elements row .. row + 255) of fp16 (f16) or fp32 data
__device__ __forceinline__ void load_row4(const void * in, size_t row, int f16, float (&v)[4]) {
    const size_t src = row + 4 * lane_id();
    if (f16) {
        const uint2 raw = *reinterpret_cast<const uint2 *>(static_cast<const _Float16 *>(in) + src);
        const half2v a = __builtin_bit_cast(half2v, raw.x), b = __builtin_bit_cast(half2v, raw.y);
        v[0] = (float) a[0];
        v[1] = (float) a[1];
        v[2] = (float) b[0];
        v[3] = (float) b[1];
    } else {
        const float4 raw = *reinterpret_cast<const float4 *>(static_cast<const float *>(in) + src);
        v[0] = raw.x;
        v[1] = raw.y;
        v[2] = raw.z;
        v[3] = raw.w;
    }
}

// the row of position p (kv head g of sequence seq) on side sd: optional FWHT, the main row in the side's format and,
// when ring and the side has a window, the q8 ring copy of the same rotated values.  All 64 lanes call it.
// row: the main-store row of (seq, g, p); rr: its ring row (used when ring)
// the row's stores carry the non-temporal hint: the rows are read back by other workgroups, from beyond the writing
// XCD's L2 (config 2: 3.05 against 3.30 µs per step, the same bits)
template <typename X>
__device__ __forceinline__ void st_row(X * p, X v) {
    __builtin_nontemporal_store(v, p);
}
__device__ __forceinline__ void store_row_at(const SideLayout & sd, size_t row, size_t rr, bool ring, float (&v)[4]) {
    const int lane = lane_id();
    if (sd.rot) fwht256_w64(v);
    uint16_t sc;
    float am; // the block's max |v|, shared by the main row's quantizer and the ring copy
    if (sd.bits == 8) {
        am = block_absmax(v);
        const unsigned word = quant_q8_am(v, am, sc);
        st_row(reinterpret_cast<unsigned *>(sd.vals + row * HD + 4 * lane), word);
    } else {
        const int bits = sd.bits, hb = bits - 4, odd = lane & 1;
        const unsigned codes = quant_qn(v, bits, sc, am);
        // word lane/2 of the row: the even lane's values are its low nibbles, the odd lane's the high nibbles
        unsigned nib = codes & 0x0f0f0f0fu;
        if (odd) nib <<= 4;
        unsigned hi = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) hi |= ((codes >> (8 * k + 4)) & 0xfu) << (hb * (k + 4 * odd));
        nib |= shfl_xor_u(nib, 1);
        hi |= shfl_xor_u(hi, 1);
        uint8_t * rp = sd.vals + row * row_bytes(bits);
        if (!odd) {
            st_row(reinterpret_cast<unsigned *>(rp + 4 * (lane >> 1)), nib);
            uint8_t * hp = rp + 128 + (lane >> 1) * hb;
            for (int k = 0; k < hb; k++) st_row(hp + k, (uint8_t) (hi >> (8 * k)));
        }
    }
    if ((lane & 7) == 0) st_row(sd.scs + row * 8 + (lane >> 3), sc);
    if (ring && sd.ring) {
        uint16_t rs;
        const unsigned word = quant_q8_am(v, am, rs);
        st_row(reinterpret_cast<unsigned *>(sd.ring + rr * HD + 4 * lane), word);
        if ((lane & 7) == 0) st_row(sd.rsc + rr * 8 + (lane >> 3), rs);
    }
}
__device__ __forceinline__ void store_row(const RowGeo & S, const SideLayout & sd, int seq, int g, int p, bool ring, float (&v)[4]) {
    store_row_at(sd, main_row(S, seq, g, p), S.kvrc > 0 ? ring_row(S, seq, g, p) : 0, ring, v);
}

__device__ __forceinline__ void store_row(const StoreLayout & S, const SideLayout & sd, int seq, int g, int p, bool ring, float (&v)[4]) {
    store_row(geo_of(S), sd, seq, g, p, ring, v);
}

// ------------------------------------------------------------------------------------------------ dequantization
// fp16 operands are built with the 0x6400 magic: the half with bits 0x6400 | n is 1024 + n exactly (n < 1024), so
// (0x6400 | n) - (1024 + bias) is the integer code exactly and one fp16 multiply by the scale rounds d * q once,
// the same value as the reference's half_rn(d * (float) q) (q8_to_f16 :2336, qn_to_f16 :2458).

__device__ __forceinline__ unsigned perm_b32(unsigned hi_src, unsigned lo_src, unsigned sel) {
    return __builtin_amdgcn_perm(hi_src, lo_src, sel);
}

__device__ __forceinline__ half2v as_h2(unsigned x) { return __builtin_bit_cast(half2v, x); }
__device__ __forceinline__ unsigned as_u(half2v x) { return __builtin_bit_cast(unsigned, x); }

// the hb-bit fields 0..3 of x (field k at bit hb k) moved to bits 4 .. 4+hb-1 of byte k
template <int HB>
__device__ __forceinline__ unsigned spread4(unsigned x) {
    // 24-bit multiplies (full rate): the compiler cannot always prove the operands fit and would otherwise emit the
    // quarter-rate 32-bit multiply
    if constexpr (HB == 1) return __umul24((x << 4) & 0xf0u, 0x00204081u) & 0x10101010u; // bit k -> bit 8k + 4
    if constexpr (HB == 2) {
        x = __umul24(x & 0xffu, 0x10010u) & 0x00f000f0u; // fields 0,1 at bits 4..7, fields 2,3 at 20..23
        return __umul24(x, 0x41u) & 0x30303030u;       // field 1 -> 12..13, field 3 -> 28..29
    }
    if constexpr (HB == 3) {
        x &= 0xfffu;
        x = (x | (x << 10)) & 0x003f003fu;
        x = (x | (x << 5)) & 0x07070707u;
        return x << 4;
    }
    return 0u;
}

// the biased codes n of the 8 values of one nibble word W (+ its high-bit field H): bytes of lo = values 0..3,
// bytes of hi = values 4..7
template <int B>
__device__ __forceinline__ void word_codes(unsigned W, unsigned H, unsigned & lo, unsigned & hi) {
    constexpr int HB = B - 4;
    lo = W & 0x0f0f0f0fu;
    hi = (W >> 4) & 0x0f0f0f0fu;
    if constexpr (HB > 0) {
        lo |= spread4<HB>(H);
        hi |= spread4<HB>(H >> (4 * HB));
    }
}

} // namespace qkv
