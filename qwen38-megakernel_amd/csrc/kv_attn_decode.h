// Split-K decode attention over the mixed q8-ring / packed KV store (gfx950, wave64, MFMA f16): k_attn computes the
// query preparation and every segment's partial (m, l, O); k_combine merges a head's segments into the output.
//
// Work: one workgroup of 4 waves per (sequence, layer, kv head, canonical segment).  The segment length depends only on
// L's 640-position bucket (seg_len), so the partition -- and with it every rounding -- is independent of the grid,
// the split count and the number of query tokens sharing the bucket.  Wave w takes the 32-position tiles w, w+4, ..
// of the segment with its own online-softmax state; the 4 states are merged in wave order into the segment's partial.
// k_combine merges the segments of a head in segment order (fixed orders: no bit depends on scheduling).
//
// Per tile and wave: the tile's packed rows are copied HBM -> LDS by global_load_lds_dwordx4 into the wave's stage,
// read into registers in MFMA operand layout, and the stage is refilled with the wave's next tile before the math
// starts (one tile in flight per wave while it computes, 8 per CU at two workgroups per CU):
//   S^T = K Q^T   v_mfma_f32_16x16x32_f16, A = 16 positions x 32 dims of K (lane: position l%16, 8 consecutive dims of
//                 its quarter l/16 of the row), B = Q^T with column n = query row n/2 of an 8-row group (the tile
//                 section below).  Two 16-position subtiles.
//   softmax       lane (n, quarter q) owns the scores of its row at positions 4q..4q+3 and 16+4q..16+4q+3: 8 values,
//                 max / sum across the 4 quarters by v_permlane16/32_swap; exp2 in log2 units.
//   O += P V      the MFMA's K as 16 positions x 2 adjacent dims: A = two adjacent dims of one position of V,
//                 B = P in the (row, dim parity) column pairs.
// Dequantization happens in registers with the 0x6400 magic (kv_dev.h): fp16 values half_rn(d q), the reference's
// operands (q8_to_f16 qwen38_mk.cu:2336, qn_to_f16 :2458).  The arithmetic of a row follows attn_core_t
// (qwen38_mk.cu:2757-3080): S in fp32 from fp16 operands, masked positions -> -inf, P rounded to fp16, O in fp32.
//
// This header holds the decode kernel template (k_attn) and its device helpers: kv_attn.hip instantiates the plain
// kernels, kv_attn_fused.hip the ones with the fused append (mk_kv_append_attend), in two translation units.
#pragma once
#include <type_traits>
#include "kv_dev.h"
#include "kv_launch.h"

namespace qkv {

constexpr float LOG2E = 1.4426950408889634f;
constexpr unsigned C64 = 0x64646464u;

// The page table is read through the constant address space (no kernel writes it during a launch): a scalar load,
// which waits on lgkmcnt only, never on the tile copies in flight.  Its latency under a full HBM stream is of the order
// of a tile's, so the tile loops look a tile's page up one step ahead (page_of), before they wait for the current tile.
typedef const __attribute__((address_space(4))) int * const_int_p;

// physical page of the logical page holding position p (wave-uniform) of sequence seq; Geo: StoreLayout or RowGeo (the
// same member names)
template <class Geo>
__device__ __forceinline__ int page_of(const Geo & S, int seq, int p) {
    const int lp = __builtin_amdgcn_readfirstlane(p / S.page);
    return ((const_int_p) S.ptab)[seq * S.pt_stride + lp];
}

// main-store row of (g, p) in physical page phys (the page of p)
template <class Geo>
__device__ __forceinline__ size_t attn_main_row(const Geo & S, int g, int p, int phys) {
    const int lp = __builtin_amdgcn_readfirstlane(p / S.page);
    return (size_t) (g * S.n_pages + phys) * S.page + (p - lp * S.page);
}

__device__ __forceinline__ half2v splat_h(unsigned s, int upper) {
    const unsigned x = upper ? (s >> 16) : (s & 0xffffu);
    return as_h2(x | (x << 16));
}

// ------------------------------------------------------------------------------------------------ K operand
// One lane's share of a 16-position K subtile: the row of position (l % 16), bytes of its quarter q = l / 16.
template <int B>
struct KSub {
    static constexpr int HB = B - 4;
    unsigned d[B == 8 ? 16 : 8]; // q8: 64 bytes (dims 64q..64q+63); packed: 32 bytes of nibbles (words 8q..8q+7)
    unsigned h[B == 8 ? 1 : 2 * (B - 4) + (B == 4)]; // packed: the 8 words' high-bit fields (8 HB bytes)
    unsigned s;                   // scales of blocks 2q, 2q+1
};

template <int B>
__device__ __forceinline__ void load_ksub(KSub<B> & k, const uint8_t * row, const uint16_t * sc, int q) {
    if constexpr (B == 8) {
        const uint4 * p = reinterpret_cast<const uint4 *>(row + 64 * q);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint4 x = p[i];
            k.d[4 * i] = x.x;
            k.d[4 * i + 1] = x.y;
            k.d[4 * i + 2] = x.z;
            k.d[4 * i + 3] = x.w;
        }
    } else {
        const uint4 * p = reinterpret_cast<const uint4 *>(row + 32 * q);
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const uint4 x = p[i];
            k.d[4 * i] = x.x;
            k.d[4 * i + 1] = x.y;
            k.d[4 * i + 2] = x.z;
            k.d[4 * i + 3] = x.w;
        }
        constexpr int HB = B - 4;
        const uint8_t * hp = row + 128 + 8 * q * HB;
        if constexpr (HB == 1) {
            const uint2 x = *reinterpret_cast<const uint2 *>(hp);
            k.h[0] = x.x;
            k.h[1] = x.y;
        } else if constexpr (HB == 2) {
            const uint4 x = *reinterpret_cast<const uint4 *>(hp);
            k.h[0] = x.x;
            k.h[1] = x.y;
            k.h[2] = x.z;
            k.h[3] = x.w;
        } else if constexpr (HB == 3) {
#pragma unroll
            for (int i = 0; i < 3; i++) {
                const uint2 x = reinterpret_cast<const uint2 *>(hp)[i];
                k.h[2 * i] = x.x;
                k.h[2 * i + 1] = x.y;
            }
        }
    }
    k.s = *reinterpret_cast<const unsigned *>(sc + 2 * q);
}

// the high-bit field of word ks (HB * 8 bits)
template <int HB>
__device__ __forceinline__ unsigned hi_field(const unsigned * h, int ks) {
    if constexpr (HB == 1) return (h[ks >> 2] >> (8 * (ks & 3))) & 0xffu;
    if constexpr (HB == 2) return (h[ks >> 1] >> (16 * (ks & 1))) & 0xffffu;
    if constexpr (HB == 3) {
        const int bit = 24 * ks, dw = bit >> 5, sh = bit & 31;
        unsigned x = h[dw] >> sh;
        if (sh > 8) x |= h[dw + 1] << (32 - sh);
        return x & 0xffffffu;
    }
    return 0u;
}

// fp16 A fragment of K step ks: values 8 ks .. 8 ks + 7 of the lane's row quarter, natural order
template <int B>
__device__ __forceinline__ half8 kfrag(const KSub<B> & k, int ks) {
    unsigned lo, hi;
    float bias;
    if constexpr (B == 8) {
        lo = k.d[2 * ks] ^ 0x80808080u; // signed q -> q + 128
        hi = k.d[2 * ks + 1] ^ 0x80808080u;
        bias = 1152.f;
    } else {
        word_codes<B>(k.d[ks], hi_field<B - 4>(k.h, ks), lo, hi);
        bias = (float) (1024 + (1 << (B - 1)));
    }
    const half2v b2 = {(_Float16) -bias, (_Float16) -bias};
    const half2v d2 = splat_h(k.s, ks >= 4);
    const half2v p0 = (as_h2(perm_b32(lo, C64, 0x00050004u)) + b2) * d2;
    const half2v p1 = (as_h2(perm_b32(lo, C64, 0x00070006u)) + b2) * d2;
    const half2v p2 = (as_h2(perm_b32(hi, C64, 0x00050004u)) + b2) * d2;
    const half2v p3 = (as_h2(perm_b32(hi, C64, 0x00070006u)) + b2) * d2;
    half8 r;
    r[0] = p0[0];
    r[1] = p0[1];
    r[2] = p1[0];
    r[3] = p1[1];
    r[4] = p2[0];
    r[5] = p2[1];
    r[6] = p3[0];
    r[7] = p3[1];
    return r;
}

// ------------------------------------------------------------------------------------------------ V operand
// One lane's share of a V tile: dims 16 m .. 16 m + 15 (m = l % 16) of the 8 positions of its quarter q = l / 16:
// j = 0..3 -> 4q + j, j = 4..7 -> 16 + 4q + j - 4 (the positions of the lane's P values).
template <int B>
struct VRaw {
    unsigned d[8][B == 8 ? 4 : 2]; // q8: 16 code bytes; packed: nibble words 2m, 2m+1
    unsigned h[8][B == 7 ? 2 : 1]; // packed: high-bit fields of the two words (2 HB bytes)
    unsigned s[8];                 // the scale of block m / 2
};

template <int B>
__device__ __forceinline__ void load_vpos(VRaw<B> & v, int j, const uint8_t * row, const uint16_t * sc, int m) {
    if constexpr (B == 8) {
        const uint4 x = *reinterpret_cast<const uint4 *>(row + 16 * m);
        v.d[j][0] = x.x;
        v.d[j][1] = x.y;
        v.d[j][2] = x.z;
        v.d[j][3] = x.w;
    } else {
        const uint2 x = *reinterpret_cast<const uint2 *>(row + 8 * m);
        v.d[j][0] = x.x;
        v.d[j][1] = x.y;
        constexpr int HB = B - 4;
        const uint8_t * hp = row + 128 + 2 * m * HB;
        if constexpr (HB == 1) v.h[j][0] = *reinterpret_cast<const uint16_t *>(hp);
        else if constexpr (HB == 2) v.h[j][0] = *reinterpret_cast<const unsigned *>(hp);
        else if constexpr (HB == 3) {
            const uint16_t * h16 = reinterpret_cast<const uint16_t *>(hp);
            v.h[j][0] = (unsigned) h16[0] | ((unsigned) h16[1] << 16);
            v.h[j][1] = h16[2];
        }
    }
    v.s[j] = sc[m >> 1];
}

// code bytes of the lane's 16 dims for position j: c[a] byte b = biased code of dim 16 m + 4 a + b
template <int B>
__device__ __forceinline__ void vcodes(const VRaw<B> & v, int j, unsigned (&c)[4]) {
    if constexpr (B == 8) {
#pragma unroll
        for (int a = 0; a < 4; a++) c[a] = v.d[j][a];
    } else {
        constexpr int HB = B - 4;
        unsigned h0 = 0, h1 = 0;
        if constexpr (HB == 1) {
            h0 = v.h[j][0] & 0xffu;
            h1 = (v.h[j][0] >> 8) & 0xffu;
        } else if constexpr (HB == 2) {
            h0 = v.h[j][0] & 0xffffu;
            h1 = v.h[j][0] >> 16;
        } else if constexpr (HB == 3) {
            h0 = v.h[j][0] & 0xffffffu;
            h1 = (v.h[j][0] >> 24) | (v.h[j][1] << 8);
        }
        word_codes<B>(v.d[j][0], h0, c[0], c[1]);
        word_codes<B>(v.d[j][1], h1, c[2], c[3]);
    }
}

// the code bytes of nibble word w (0, 1) of the lane's 16 dims for position j: c[0] byte b = dim 16 m + 8 w + b,
// c[1] byte b = dim 16 m + 8 w + 4 + b (biased codes; q8: the signed bytes)
template <int B>
__device__ __forceinline__ void vcodes_word(const VRaw<B> & v, int j, int w, unsigned (&c)[2]) {
    if constexpr (B == 8) {
        c[0] = v.d[j][2 * w];
        c[1] = v.d[j][2 * w + 1];
    } else {
        constexpr int HB = B - 4;
        unsigned hw = 0;
        if constexpr (HB == 1) hw = (v.h[j][0] >> (8 * w)) & 0xffu;
        else if constexpr (HB == 2) hw = w ? v.h[j][0] >> 16 : v.h[j][0] & 0xffffu;
        else if constexpr (HB == 3) hw = w ? (v.h[j][0] >> 24) | (v.h[j][1] << 8) : v.h[j][0] & 0xffffffu;
        word_codes<B>(v.d[j][w], hw, c[0], c[1]);
    }
}

// ------------------------------------------------------------------------------------------------ tile staging
// Tiles move HBM -> LDS with global_load_lds_dwordx4 (16 bytes per lane, 1 KiB per wave instruction, written at
// M0 + 16 lane), issued from inline assembly so that the waits are explicit: the compiler would otherwise wait for
// every outstanding copy before the first LDS read.  Nothing else in the tile loop issues vector-memory loads, so
// `s_waitcnt vmcnt(n)` with n = the copies of the younger tile in flight is exact.  M0 is not allocatable; only
// these copies set it in this kernel.
// Stage layout (STAGE_BYTES, one per wave and stage): K rows [32][32 KB], V rows [32][32 VB], K scales [32][8],
// V scales [32][8] (fp16).  Rows past the end of the context are copies of the last row (finite, masked later).
// The copies carry the non-temporal hint (nt): each tile is read once, so it is streamed through the L2 without
// displacing what is read again (code, kernel arguments, page tables, the partials the combine reads).  Measured on
// configs 3 and 5: 1-2% shorter steps, the same bits.
#ifndef QKV_DMA_CPOL
#define QKV_DMA_CPOL " nt"
#endif
// NT = false: without the hint, for tiles that other work items read again (prefill row blocks of one key segment,
// the row batches of one decode segment)
template <bool NT = true>
__device__ __forceinline__ void dma16(const void * g, unsigned lds) {
    if constexpr (NT) asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" QKV_DMA_CPOL ::"s"(lds), "v"(g) : "memory");
    else asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds), "v"(g) : "memory");
}
__device__ __forceinline__ void dma16_keep(const void * g, unsigned lds) { dma16<false>(g, lds); }
// the same with a scalar base address and a 32-bit per-lane byte offset (no 64-bit vector address per copy)
template <bool NT = true>
__device__ __forceinline__ void dma16s(const void * base, unsigned voff, unsigned lds) {
    if constexpr (NT)
        asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" QKV_DMA_CPOL ::"s"(lds), "v"(voff), "s"(base) : "memory");
    else asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds), "v"(voff), "s"(base) : "memory");
}
// N (1..4) consecutive 1 KiB pieces from one scalar base: M0 set once, the instruction offset (0, 1024, 2048, 3072)
// added to both the global and the LDS address of each copy
#define QKV_DMA_AT(O, C) "global_load_lds_dwordx4 %1, %2 offset:" #O C "\n\t"
template <int N, bool NT = true>
__device__ __forceinline__ void dma16s_run(const void * base, unsigned voff, unsigned lds) {
    static_assert(N >= 1 && N <= 4, "one to four pieces");
    if constexpr (NT) {
        if constexpr (N == 1) asm volatile("s_mov_b32 m0, %0\n\t" QKV_DMA_AT(0, QKV_DMA_CPOL) ::"s"(lds), "v"(voff), "s"(base) : "memory");
        if constexpr (N == 2)
            asm volatile("s_mov_b32 m0, %0\n\t" QKV_DMA_AT(0, QKV_DMA_CPOL) QKV_DMA_AT(1024, QKV_DMA_CPOL) ::"s"(lds), "v"(voff), "s"(base) : "memory");
        if constexpr (N == 3)
            asm volatile("s_mov_b32 m0, %0\n\t" QKV_DMA_AT(0, QKV_DMA_CPOL) QKV_DMA_AT(1024, QKV_DMA_CPOL) QKV_DMA_AT(2048, QKV_DMA_CPOL)
                         ::"s"(lds), "v"(voff), "s"(base) : "memory");
        if constexpr (N == 4)
            asm volatile("s_mov_b32 m0, %0\n\t" QKV_DMA_AT(0, QKV_DMA_CPOL) QKV_DMA_AT(1024, QKV_DMA_CPOL) QKV_DMA_AT(2048, QKV_DMA_CPOL)
                             QKV_DMA_AT(3072, QKV_DMA_CPOL) ::"s"(lds), "v"(voff), "s"(base) : "memory");
    } else {
        if constexpr (N == 1) asm volatile("s_mov_b32 m0, %0\n\t" QKV_DMA_AT(0, "") ::"s"(lds), "v"(voff), "s"(base) : "memory");
        if constexpr (N == 2) asm volatile("s_mov_b32 m0, %0\n\t" QKV_DMA_AT(0, "") QKV_DMA_AT(1024, "") ::"s"(lds), "v"(voff), "s"(base) : "memory");
        if constexpr (N == 3)
            asm volatile("s_mov_b32 m0, %0\n\t" QKV_DMA_AT(0, "") QKV_DMA_AT(1024, "") QKV_DMA_AT(2048, "") ::"s"(lds), "v"(voff), "s"(base) : "memory");
        if constexpr (N == 4)
            asm volatile("s_mov_b32 m0, %0\n\t" QKV_DMA_AT(0, "") QKV_DMA_AT(1024, "") QKV_DMA_AT(2048, "") QKV_DMA_AT(3072, "")
                         ::"s"(lds), "v"(voff), "s"(base) : "memory");
    }
}
// n pieces (compile time) from base into LDS at lds: runs of four
template <int N, bool NT = true>
__device__ __forceinline__ void dma16s_pieces(const uint8_t * base, unsigned voff, unsigned lds) {
    if constexpr (N >= 4) {
        dma16s_run<4, NT>(base, voff, lds);
        if constexpr (N > 4) dma16s_pieces<N - 4, NT>(base + 4096, voff, lds + 4096);
    } else if constexpr (N > 0) {
        dma16s_run<N, NT>(base, voff, lds);
    }
}
// a segment partial's four values, stored with the non-temporal hint: the combine reads them from beyond the L2 of the
// XCD that wrote them (configs 3 fused, 4, 5: 1-2% shorter launches, the same bits)
__device__ __forceinline__ void store_part(float * p, const float4 & y) {
    typedef float f4v __attribute__((ext_vector_type(4)));
    __builtin_nontemporal_store(f4v{y.x, y.y, y.z, y.w}, reinterpret_cast<f4v *>(p));
}
__device__ __forceinline__ void lds_drain() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
// a workgroup barrier for LDS data only: __syncthreads() also waits for every vector-memory operation of the wave,
// which would expose the latency of the tile copies in flight at the barrier
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
template <int N>
__device__ __forceinline__ void vm_wait() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// a 16-byte load the compiler does not track: the caller waits for it with vm_wait and then pins the value (pin_after)
// -- a tracked load would make the compiler's own wait before the first use also drain the tile copies issued after it
__device__ __forceinline__ f32x4 gload16(const void * g) {
    f32x4 r;
    asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(r) : "v"(g) : "memory");
    return r;
}
__device__ __forceinline__ void pin_after(f32x4 & x) { asm volatile("" : "+v"(x)); }
struct TileSrc {
    const uint8_t * k;
    const uint16_t * ks;
    const uint8_t * v;
    const uint16_t * vs;
};

// the source rows of the 32 positions from p0 (wave-uniform) of (seq, kv head g): window tiles (ring) are q8 rows
// from the ring of sides that have one, else from the main store (q8 sides); other tiles are main-store rows of
// KB / VB bits.  ring0 = the first ring row of (seq, g); mr = the main-store row of p0 (read only for a side without a
// ring or a packed tile)
template <int KB, int VB>
__device__ __forceinline__ TileSrc tile_src_row(int kvrc, const SideLayout & SK, const SideLayout & SV, size_t mr, int p0, size_t ring0,
                                               bool ring) {
    TileSrc t;
    size_t rr = 0;
    if (ring) {
        int rows = max(kvrc, 1);
        asm volatile("" : "+s"(rows)); // the division's set-up stays on this path (not hoisted out of a caller's loop)
        rr = ring0 + __builtin_amdgcn_readfirstlane(p0 % rows);
    }
    if (ring && SK.ring) {
        t.k = reinterpret_cast<const uint8_t *>(SK.ring) + rr * HD;
        t.ks = SK.rsc + rr * 8;
    } else {
        t.k = SK.vals + mr * (ring ? HD : 32 * KB);
        t.ks = SK.scs + mr * 8;
    }
    if (ring && SV.ring) {
        t.v = reinterpret_cast<const uint8_t *>(SV.ring) + rr * HD;
        t.vs = SV.rsc + rr * 8;
    } else {
        t.v = SV.vals + mr * (ring ? HD : 32 * VB);
        t.vs = SV.scs + mr * 8;
    }
    return t;
}
// the same with the main-store row from phys, the physical page of p0 (page_of), looked up by the caller
template <int KB, int VB, class Geo>
__device__ __forceinline__ TileSrc tile_src(const Geo & S, const SideLayout & SK, const SideLayout & SV, int g, int p0, int phys,
                                           size_t ring0, bool ring) {
    const size_t mr = !ring || !SK.ring || !SV.ring ? attn_main_row(S, g, p0, phys) : 0;
    return tile_src_row<KB, VB>(S.kvrc, SK, SV, mr, p0, ring0, ring);
}

// copies of one tile into the stage at LDS address `lds` (KB + VB + 1 copy instructions per lane).
// Full tiles copy contiguous bytes (one address add per instruction); the last, partial tile of a context clamps each
// 16-byte chunk to the last valid row.
// PART: 0 = the whole tile, 1 = the K rows and scales, 2 = the V rows and scales (two waves sharing one stage, each
// copying what it stores in a fused append)
template <int KB, int VB, int PART = 0, bool NT = true>
__device__ __forceinline__ void issue_tile(const TileSrc & t, int nv, unsigned lds, int lane) {
    constexpr int KR = 2 * KB, VR = 2 * VB; // 16-byte chunks per row
    constexpr bool DK = PART != 2, DV = PART != 1;
    if (nv == ATP) {
        const unsigned off = 16 * lane;
        if constexpr (DK) dma16s_pieces<KB, NT>(t.k, off, lds);
        if constexpr (DV) dma16s_pieces<VB, NT>(t.v, off, lds + 1024 * KB);
    } else {
        if constexpr (DK)
#pragma unroll
            for (int j = 0; j < KB; j++) {
                int c = j * 64 + lane;
                const int r = c / KR;
                if (r >= nv) c = (nv - 1) * KR + (c - r * KR);
                dma16<NT>(t.k + 16 * c, lds + 1024 * j);
            }
        if constexpr (DV)
#pragma unroll
            for (int j = 0; j < VB; j++) {
                int c = j * 64 + lane;
                const int r = c / VR;
                if (r >= nv) c = (nv - 1) * VR + (c - r * VR);
                dma16<NT>(t.v + 16 * c, lds + 1024 * (KB + j));
            }
    }
    const int r = min(lane & 31, nv - 1);
    if constexpr (PART == 0) {
        dma16<NT>(lane < 32 ? static_cast<const void *>(t.ks + 8 * r) : static_cast<const void *>(t.vs + 8 * r), lds + 1024 * (KB + VB));
    } else if ((lane < 32) == (PART == 1)) { // half the lanes: the same LDS slots (lane-indexed) as the whole copy
        dma16<NT>(PART == 1 ? static_cast<const void *>(t.ks + 8 * r) : static_cast<const void *>(t.vs + 8 * r), lds + 1024 * (KB + VB));
    }
}

// a q8 tile through a stage smaller than one (three workgroups per CU): part 0 = the K rows at 0 and every scale at
// 8 KiB, part 1 = the V rows at 0 once the K operands are in registers; partial tiles clamp as issue_tile does
template <int PART, bool NT = true>
__device__ __forceinline__ void issue_q8_part(const TileSrc & t, int nv, unsigned lds, int lane) {
    const uint8_t * const src = PART == 0 ? t.k : t.v;
    if (nv == ATP) {
        const unsigned off = 16 * lane;
        dma16s_pieces<8, NT>(src, off, lds);
    } else {
#pragma unroll
        for (int j = 0; j < 8; j++) {
            int c = j * 64 + lane;
            const int r = c / 16;
            if (r >= nv) c = (nv - 1) * 16 + (c - r * 16);
            dma16<NT>(src + 16 * c, lds + 1024 * j);
        }
    }
    if constexpr (PART == 0) {
        const int r = min(lane & 31, nv - 1);
        dma16<NT>(lane < 32 ? static_cast<const void *>(t.ks + 8 * r) : static_cast<const void *>(t.vs + 8 * r), lds + 8192);
    }
}

template <int KB, int VB>
struct RawTile {
    KSub<KB> k0, k1; // subtile rows n, 16 + n
    VRaw<VB> v;      // the lane's 8 positions
};

// the lane's operands of a staged tile into registers (row n = l % 16, quarter q = l / 16): the K subtiles, then,
// separately, the V positions (read after the scores, so the K and V registers are never live together)
template <int KB, int VB>
__device__ __forceinline__ void read_k(RawTile<KB, VB> & r, const uint8_t * kr, const uint16_t * ksc, int n, int q) {
    load_ksub<KB>(r.k0, kr + n * 32 * KB, ksc + n * 8, q);
    load_ksub<KB>(r.k1, kr + (16 + n) * 32 * KB, ksc + (16 + n) * 8, q);
}
template <int KB, int VB>
__device__ __forceinline__ void read_k(RawTile<KB, VB> & r, const uint8_t * st, int n, int q) {
    read_k<KB, VB>(r, st, reinterpret_cast<const uint16_t *>(st + 1024 * (KB + VB)), n, q);
}
template <int KB, int VB>
__device__ __forceinline__ void read_v(RawTile<KB, VB> & r, const uint8_t * vr, const uint16_t * vsc, int n, int q) {
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int row = j < 4 ? 4 * q + j : 16 + 4 * q + j - 4;
        load_vpos<VB>(r.v, j, vr + row * 32 * VB, vsc + row * 8, n);
    }
}
template <int KB, int VB>
__device__ __forceinline__ void read_v(RawTile<KB, VB> & r, const uint8_t * st, int n, int q) {
    read_v<KB, VB>(r, st + 1024 * KB, reinterpret_cast<const uint16_t *>(st + 1024 * (KB + VB)) + 8 * ATP, n, q);
}

// ------------------------------------------------------------------------------------------------ the tile
// Query rows go in NP groups of 8 (compute_tile: one group; 16 and 24 rows take compute_tile_v below, which shares
// the O += P V form).  Both MFMA products use the 16 columns as (row, e) pairs, row = 8 h + n / 2 of group h and
// e = n % 2:
//   S^T = K Q^T   column n of Q^T is query row 8 h + n / 2 (each score is computed in lanes n and n ^ 1), so lane
//                 (n, q) owns its row's scores at positions 4 q + e and 16 + 4 q + e (e = 0..3);
//   O += P V      the MFMA's K = 32 is 16 positions x (e = 0, 1):
//                 O[row][16 m + 2 b + e'] = sum_{p, e} A[m][(p, e)] B[(p, e)][(row, e')],
//                 A = V[p][16 m + 2 b + e],  B = P[p][row] if e = e' else 0,
//                 so an A register holds two adjacent dims of one position: a byte pair of the position's code word
//                 and one scale per register, shared by every row group.
// A row's arithmetic does not depend on its group or on T, so the partials are bitwise T-invariant.
template <int NP>
struct WaveState {
    f32x4 acc[NP][8]; // group h, block b, element i -> dim 16 (4 q + i) + 2 b + (n & 1) of row 8 h + n / 2
    float m[NP], l[NP];
    int lim[NP];      // last visible position of the lane's row (-1: padding row)
    int lim_min;      // last position visible to every real row (L - T), wave-uniform
    // one 8-row group: the lane's Q^T operands of the 8 K steps stay in registers for the whole item (32 VGPRs);
    // more groups read them from LDS per tile
    half8 qf[NP == 1 ? 8 : 1];
};

// query rows in LDS: fp16 [RP][256] with 16-byte chunk c of row r stored at chunk c ^ (r % 16)
__device__ __forceinline__ int qchunk(int r, int c) { return r * (HD / 8) + (c ^ (r & 15)); }

template <int K, int V>
struct Fmt {
    static constexpr int kb = K, vb = V;
};

struct NoHook {
    template <typename... A>
    __device__ void operator()(A &&...) const {}
};

// LATE_V: raw.v is unset on entry; load_v(raw, n, q) reads the V operands from the stage after the scores, and after_v()
// (which refills the stage) runs once they are in registers -- K and V are never live together next to the state
template <int NP, int KB, int VB, bool LATE_V = false, typename FV = NoHook, typename FA = NoHook>
__device__ __forceinline__ void compute_tile(WaveState<NP> & st, const half8 * sQ, int p0, RawTile<KB, VB> & raw, FV load_v = FV(),
                                             FA after_v = FA()) {
    int lane = lane_id(); // opaque: lane-derived LDS addresses are recomputed per tile, not held across the loop
    asm volatile("" : "+v"(lane));
    const int q = lane >> 4, n = lane & 15;
    // ---- S^T = K Q^T, two 16-position subtiles
    f32x4 s[NP][2];
#pragma unroll
    for (int h = 0; h < NP; h++) s[h][0] = s[h][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 8; ks++) {
        const half8 a0 = kfrag<KB>(raw.k0, ks);
        const half8 a1 = kfrag<KB>(raw.k1, ks);
#pragma unroll
        for (int h = 0; h < NP; h++) {
            const half8 b = NP == 1 ? st.qf[ks] : sQ[qchunk(8 * h + (n >> 1), 8 * q + ks)];
            s[h][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, b, s[h][0], 0, 0, 0);
            s[h][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, b, s[h][1], 0, 0, 0);
        }
    }
    // ---- online softmax (log2 units).  The running max moves only when a tile's max exceeds it by more than
    // RESCALE_LOG2 (and on the first visible tile): until then P = exp2(s - m) <= 2^RESCALE_LOG2 (in fp16 range) and
    // O, l keep their scale, so most tiles need no rescale of O.  A function of the data order within the fixed
    // partition only: deterministic.
    constexpr float RESCALE_LOG2 = 8.f;
    // every position of the tile visible to every row (uniform: a scalar branch, no per-value mask on full tiles)
    const bool full = __builtin_amdgcn_readfirstlane(p0 + ATP - 1 <= st.lim_min);
    // B operands of the two 16-position groups G: (P, 0) in even columns, (0, P) in odd ones; built per row group
    // right after its softmax so that only the packed fp16 P stays live
    const unsigned odd = n & 1;
    const unsigned sel_lo = odd ? 0x05040c0cu : 0x0c0c0504u, sel_hi = odd ? 0x07060c0cu : 0x0c0c0706u;
    half8 pb[NP][2];
    float alpha[NP];
    bool rescale = false;
#pragma unroll
    for (int h = 0; h < NP; h++) {
        float t[8];
        float mx = -INFINITY;
        if (full) {
#pragma unroll
            for (int e = 0; e < 8; e++) {
                t[e] = (e < 4 ? s[h][0][e] : s[h][1][e - 4]) * LOG2E;
                mx = fmaxf(mx, t[e]);
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int pos = p0 + (e < 4 ? 4 * q + e : 16 + 4 * q + e - 4);
                const float sv = (e < 4 ? s[h][0][e] : s[h][1][e - 4]) * LOG2E;
                t[e] = pos <= st.lim[h] ? sv : -INFINITY;
                mx = fmaxf(mx, t[e]);
            }
        }
        mx = quad_max(mx);
        const float mold = st.m[h];
        const float mnew = mx > mold + RESCALE_LOG2 ? mx : mold; // (mold = -inf: any finite mx)
        float al = 1.f, ps = 0.f;
        float p[8];
        if (mnew != -INFINITY) {
            al = mold == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mold - mnew);
#pragma unroll
            for (int e = 0; e < 8; e++) {
                p[e] = __builtin_amdgcn_exp2f(t[e] - mnew);
                ps += p[e];
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++) p[e] = 0.f;
        }
        ps = quad_sum(ps);
        st.l[h] = __builtin_fmaf(st.l[h], al, ps);
        st.m[h] = mnew;
        alpha[h] = al;
        rescale |= al != 1.f && mold != -INFINITY; // (O is still zero before the first visible tile)
#pragma unroll
        for (int G = 0; G < 2; G++)
#pragma unroll
            for (int k = 0; k < 2; k++) {
                half2v x2;
                x2[0] = (_Float16) p[4 * G + 2 * k];
                x2[1] = (_Float16) p[4 * G + 2 * k + 1];
                const unsigned x = as_u(x2);
                const half2v y0 = as_h2(perm_b32(x, 0u, sel_lo)), y1 = as_h2(perm_b32(x, 0u, sel_hi));
                pb[h][G][4 * k] = y0[0];
                pb[h][G][4 * k + 1] = y0[1];
                pb[h][G][4 * k + 2] = y1[0];
                pb[h][G][4 * k + 3] = y1[1];
            }
    }
    if (__any(rescale)) { // alpha == 1 exactly leaves O unchanged: the skip is exact
#pragma unroll
        for (int h = 0; h < NP; h++)
#pragma unroll
            for (int b = 0; b < 8; b++) st.acc[h][b] *= alpha[h];
    }
    if constexpr (LATE_V) {
        load_v(raw, n, q); // (the tile's lane indices: recomputed per tile)
        lds_drain();
        after_v();
    }
    // ---- O += P V: block b = dims 16 m + 2 b, + 1 of the lane's V row m (nibble word b / 4, values 2 (b % 4), + 1)
    half2v dv[8];
#pragma unroll
    for (int j = 0; j < 8; j++) dv[j] = as_h2((raw.v.s[j] & 0xffffu) * 0x10001u);
    constexpr unsigned QX = VB == 8 ? 0x80808080u : 0u; // q8: signed byte -> byte + 128
    constexpr float VBIAS = VB == 8 ? 1152.f : (float) (1024 + (1 << (VB - 1)));
    const half2v vb2 = {(_Float16) -VBIAS, (_Float16) -VBIAS};
#pragma unroll
    for (int w = 0; w < 2; w++) {
        unsigned c[8][2];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            vcodes_word<VB>(raw.v, j, w, c[j]);
            c[j][0] ^= QX;
            c[j][1] ^= QX;
        }
#pragma unroll
        for (int bb = 0; bb < 4; bb++) {
            const int b = 4 * w + bb;
            const unsigned sel = (bb & 1) ? 0x00070006u : 0x00050004u;
#pragma unroll
            for (int G = 0; G < 2; G++) {
                half8 va;
#pragma unroll
                for (int jj = 0; jj < 4; jj++) {
                    const int j = 4 * G + jj;
                    const half2v x = (as_h2(perm_b32(c[j][bb >> 1], C64, sel)) + vb2) * dv[j];
                    va[2 * jj] = x[0];
                    va[2 * jj + 1] = x[1];
                }
#pragma unroll
                for (int h = 0; h < NP; h++) st.acc[h][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb[h][G], st.acc[h][b], 0, 0, 0);
            }
        }
    }
}

// ------------------------------------------------------------------------------------------------ 24-row tile
// compute_tile for 16 or 24 rows (NP = 2, 3) with each score computed once: the S^T MFMAs take 16 distinct query rows
// per column block (block 0: rows 0..15, block 1: rows 16..23 and, in lanes 8..15, copies of them), so the online
// softmax runs over NB = 1 or 2 blocks instead of NP 8-row groups held twice.  The P V operands keep
// compute_tile's (row, dim parity) column pairs: group h's lane n takes row 8 h + n / 2's fp16 P from the lane that
// owns that row (ds_bpermute within the lane's 16-lane row).  A row's scores, softmax, P and P V are the same
// operations on the same values as in compute_tile (an MFMA output element does not depend on its column): bitwise
// the same partials as k_attn's 24-row kernel.
template <int NP>
struct RowState {
    static constexpr int NB = (NP + 1) / 2;
    f32x4 acc[NP][8]; // as WaveState::acc: group h, lane (n, q) -> row 8 h + n / 2
    float m[NB], l[NB];
    int lim[NB];      // last visible position of the lane's block row 16 H + n (-1: padding)
    int lim_min;
};

// load_v(raw, n, q) reads the V operands after the scores; after_v() runs once they are in registers
template <int NP, int KB, int VB, typename FV, typename FA = NoHook>
__device__ __forceinline__ void compute_tile_v(RowState<NP> & st, const half8 * sQ, int p0, RawTile<KB, VB> & raw, FV load_v,
                                               FA after_v = FA()) {
    static_assert(NP == 2 || NP == 3, "16 or 24 rows");
    constexpr int NB = RowState<NP>::NB;
    // (the lane index stays visible here: its LDS addresses are held across the tile loop, which fits these kernels'
    // registers and saves ~60 VALU instructions per tile)
    const int lane = lane_id();
    const int q = lane >> 4, n = lane & 15;
    f32x4 s[NB][2];
#pragma unroll
    for (int H = 0; H < NB; H++) s[H][0] = s[H][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 8; ks++) {
        const half8 a0 = kfrag<KB>(raw.k0, ks);
        const half8 a1 = kfrag<KB>(raw.k1, ks);
#pragma unroll
        for (int H = 0; H < NB; H++) {
            const half8 b = sQ[qchunk(H ? 16 + (n & 7) : n, 8 * q + ks)];
            s[H][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, b, s[H][0], 0, 0, 0);
            s[H][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, b, s[H][1], 0, 0, 0);
        }
    }
    constexpr float RESCALE_LOG2 = 8.f;
    const bool full = __builtin_amdgcn_readfirstlane(p0 + ATP - 1 <= st.lim_min);
    unsigned w[NB][2][2]; // block H, group G, pair k: the lane's fp16 P of positions 16 G + 4 q + 2 k, + 1
    float alpha[NB];
    bool rescale = false;
#pragma unroll
    for (int H = 0; H < NB; H++) {
        float t[8];
        float mx = -INFINITY;
        if (full) {
#pragma unroll
            for (int e = 0; e < 8; e++) {
                t[e] = (e < 4 ? s[H][0][e] : s[H][1][e - 4]) * LOG2E;
                mx = fmaxf(mx, t[e]);
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int pos = p0 + (e < 4 ? 4 * q + e : 16 + 4 * q + e - 4);
                const float sv = (e < 4 ? s[H][0][e] : s[H][1][e - 4]) * LOG2E;
                t[e] = pos <= st.lim[H] ? sv : -INFINITY;
                mx = fmaxf(mx, t[e]);
            }
        }
        mx = quad_max(mx);
        const float mold = st.m[H];
        const float mnew = mx > mold + RESCALE_LOG2 ? mx : mold;
        float al = 1.f, ps = 0.f;
        float p[8];
        if (mnew != -INFINITY) {
            al = mold == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mold - mnew);
#pragma unroll
            for (int e = 0; e < 8; e++) {
                p[e] = __builtin_amdgcn_exp2f(t[e] - mnew);
                ps += p[e];
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++) p[e] = 0.f;
        }
        ps = quad_sum(ps);
        st.l[H] = __builtin_fmaf(st.l[H], al, ps);
        st.m[H] = mnew;
        alpha[H] = al;
        rescale |= al != 1.f && mold != -INFINITY && (H == 0 || n < 8);
#pragma unroll
        for (int G = 0; G < 2; G++)
#pragma unroll
            for (int k = 0; k < 2; k++) {
                half2v x2;
                x2[0] = (_Float16) p[4 * G + 2 * k];
                x2[1] = (_Float16) p[4 * G + 2 * k + 1];
                w[H][G][k] = as_u(x2);
            }
    }
    // group h's lane n takes row 8 h + n / 2: block h / 2, lane (8 h + n / 2) % 16 of the same 16-lane row
    const int src[3] = {4 * (16 * q + (n >> 1)), 4 * (16 * q + 8 + (n >> 1)), 4 * (16 * q + (n >> 1))};
    if (__any(rescale)) { // alpha == 1 exactly leaves O unchanged: the skip is exact
#pragma unroll
        for (int h = 0; h < NP; h++) {
            const float a = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src[h], __builtin_bit_cast(int, alpha[h >> 1])));
#pragma unroll
            for (int b = 0; b < 8; b++) st.acc[h][b] *= a;
        }
    }
    const unsigned odd = n & 1;
    const unsigned sel_lo = odd ? 0x05040c0cu : 0x0c0c0504u, sel_hi = odd ? 0x07060c0cu : 0x0c0c0706u;
    half8 pb[NP][2];
#pragma unroll
    for (int h = 0; h < NP; h++)
#pragma unroll
        for (int G = 0; G < 2; G++)
#pragma unroll
            for (int k = 0; k < 2; k++) {
                const unsigned x = (unsigned) __builtin_amdgcn_ds_bpermute(src[h], (int) w[h >> 1][G][k]);
                const half2v y0 = as_h2(perm_b32(x, 0u, sel_lo)), y1 = as_h2(perm_b32(x, 0u, sel_hi));
                pb[h][G][4 * k] = y0[0];
                pb[h][G][4 * k + 1] = y0[1];
                pb[h][G][4 * k + 2] = y1[0];
                pb[h][G][4 * k + 3] = y1[1];
            }
    load_v(raw, n, q);
    lds_drain();
    after_v();
    // ---- O += P V as compute_tile
    half2v dv[8];
#pragma unroll
    for (int j = 0; j < 8; j++) dv[j] = as_h2((raw.v.s[j] & 0xffffu) * 0x10001u);
    constexpr unsigned QX = VB == 8 ? 0x80808080u : 0u;
    constexpr float VBIAS = VB == 8 ? 1152.f : (float) (1024 + (1 << (VB - 1)));
    const half2v vb2 = {(_Float16) -VBIAS, (_Float16) -VBIAS};
#pragma unroll
    for (int wd = 0; wd < 2; wd++) {
        unsigned c[8][2];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            vcodes_word<VB>(raw.v, j, wd, c[j]);
            c[j][0] ^= QX;
            c[j][1] ^= QX;
        }
#pragma unroll
        for (int bb = 0; bb < 4; bb++) {
            const int b = 4 * wd + bb;
            const unsigned sel = (bb & 1) ? 0x00070006u : 0x00050004u;
#pragma unroll
            for (int G = 0; G < 2; G++) {
                half8 va;
#pragma unroll
                for (int jj = 0; jj < 4; jj++) {
                    const int j = 4 * G + jj;
                    const half2v x = (as_h2(perm_b32(c[j][bb >> 1], C64, sel)) + vb2) * dv[j];
                    va[2 * jj] = x[0];
                    va[2 * jj + 1] = x[1];
                }
#pragma unroll
                for (int h = 0; h < NP; h++) st.acc[h][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb[h][G], st.acc[h][b], 0, 0, 0);
            }
        }
    }
}

// The fused append's rows of one wave (mk_kv_append_attend): positions L - T .. L - 1 of segment [c0, c1) whose tile
// falls in slice sl, sides w0 .. w1 (0 = K, 1 = V), each stored by store_row exactly as k_append stores it.  Plain
// values (a called function: inlined, its code made the fused kernels' tile loop slower); called only from the
// fused-append kernels (APPEND), so the plain kernels carry neither the store code nor a call.
static __device__ __noinline__ void append_rows(const void * kin, const void * vin, int f16, int kin_nl, const int * ptab, int pt_stride, int page,
                                         int n_pages, int kvrc, uint8_t * kvals, uint16_t * kscs, int8_t * kring, uint16_t * krsc,
                                         int kbits, int krot, uint8_t * vvals, uint16_t * vscs, int8_t * vring, uint16_t * vrsc,
                                         int vbits, int vrot, int seq, int g, int l, int si, int L, int T, int c0, int c1, int sl, int w0,
                                         int w1) {
    const RowGeo G{ptab, pt_stride, page, n_pages, kvrc};
    const SideLayout K{kvals, kscs, kring, krsc, kbits, krot}, V{vvals, vscs, vring, vrsc, vbits, vrot};
    const int pa = max(L - T, c0), pb = min(L, c1);
    for (int p = pa; p < pb; p++) {
        if (((p - c0) >> 5) % AWAVES != sl) continue;
        const size_t row = ((((size_t) si * T + (p - (L - T))) * kin_nl + l) * NKV + g) * HD;
        for (int w = w0; w <= w1; w++) {
            float v[4];
            load_row4(w ? vin : kin, row, f16, v);
            store_row(G, w ? V : K, seq, g, p, true, v);
        }
    }
}

// wave issue priority 0..3 from the tiles a wave has left: the instruction arbiter otherwise favours the older
// workgroup on a CU, which then finishes early and leaves the younger one's waves to run the launch's tail alone.
// A uniform value; s_setprio takes an immediate.
__device__ __forceinline__ void set_prio(int left) {
    if (left >= 6) __builtin_amdgcn_s_setprio(3);
    else if (left >= 5) __builtin_amdgcn_s_setprio(2);
    else if (left >= 4) __builtin_amdgcn_s_setprio(1);
    else __builtin_amdgcn_s_setprio(0);
}

// ------------------------------------------------------------------------------------------------ launch head
// AttnHead (the first 192 bytes of the kernel arguments) in scalar registers: three 16-dword loads and one wait.  The
// values come out of the asm, so the compiler keeps them in registers (or VGPR lanes) and never re-reads a field from
// the argument segment in the middle of the prologue.
typedef unsigned u32x16 __attribute__((ext_vector_type(16)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
struct HeadRegs {
    u32x16 a, b, c;
    u32x4 d;
};
__device__ __forceinline__ HeadRegs load_head() {
    HeadRegs r;
    asm volatile("s_load_dwordx16 %0, %4, 0x0\n\ts_load_dwordx16 %1, %4, 0x40\n\ts_load_dwordx16 %2, %4, 0x80\n\t"
                 "s_load_dwordx4 %3, %4, 0xc0\n\ts_waitcnt lgkmcnt(0)"
                 : "=&s"(r.a), "=&s"(r.b), "=&s"(r.c), "=&s"(r.d)
                 : "s"(__builtin_amdgcn_kernarg_segment_ptr()));
    return r;
}
template <int I>
__device__ __forceinline__ unsigned head_dw(const HeadRegs & r) {
    if constexpr (I < 16) return r.a[I];
    else if constexpr (I < 32) return r.b[I - 16];
    else if constexpr (I < 48) return r.c[I - 32];
    else return r.d[I - 48];
}
template <typename T, int OFF>
__device__ __forceinline__ T head_get(const HeadRegs & r) {
    static_assert(OFF % 4 == 0 && OFF + sizeof(T) <= sizeof(AttnHead), "a dword-aligned head field");
    constexpr int I = OFF / 4;
    if constexpr (sizeof(T) == 8) return __builtin_bit_cast(T, ((unsigned long long) head_dw<I + 1>(r) << 32) | head_dw<I>(r));
    else return __builtin_bit_cast(T, head_dw<I>(r));
}
// floor(n / d) from M = magic31(d) (kv_launch.h): exact for n d < 2^31, one multiply instead of a division sequence
__device__ __forceinline__ int div_m(int n, unsigned M) { return (int) __umulhi(2u * (unsigned) n, M); }
#define QKV_HEAD(r, f) head_get<std::remove_cv_t<decltype(AttnHead::f)>, offsetof(AttnHead, f)>(r)

// ------------------------------------------------------------------------------------------------ the kernel
// More than 16 query rows (T >= 3) are held as 24 rows per wave (three groups; 48 rows of accumulators in one wave
// spill).  T = 3, 4: one 24-row pass.  T = 5..8: k_verify below (one pass, 8 waves), or (knob) batches of 24 rows
// here: work item = (sequence, layer, kv head, segment, row batch), batch-minor, each batch streaming the segment's
// tiles again.  Every row sees the same slices, tile arithmetic and merge whatever T and whichever kernel.
// SMALL (one 8-row group, KB + VB <= 11): three workgroups per CU for launches with many work items.  The stages hold
// one packed tile (32 (KB + VB) + 1 KiB); a q8 window tile goes through in two halves (issue_q8_part); the V operands
// are read after the scores (168 registers).  Same slices and arithmetic: bitwise the same partials.
template <int NP, int KB, int VB, bool SMALL = false, bool APPEND = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(SMALL ? 3 : 2, SMALL ? 3 : 2))) void k_attn(AttnArgs a) {
    static_assert(!SMALL || (NP == 1 && KB + VB <= 11), "small stages: one row group, packed tiles of at most 11 KiB");
    constexpr int RP = 8 * NP; // query rows held (the padding rows are zero)
    constexpr int SB = SMALL ? 1024 * (KB + VB) + 1024 : STAGE_BYTES, SLDS = AWAVES * SB; // stage bytes, all stages
    // NP = 3: the V operands are read from the stage after the scores (the stage is refilled only then), so a wave
    // never holds a whole raw tile in registers next to 24 rows of accumulators, and two workgroups fit a CU
    constexpr bool LATE_V = NP >= 3 || SMALL;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    // the wave index as a scalar: tile positions, page lookups and source selection stay scalar (SMEM loads, uniform
    // branches); vector loads there would need vmcnt waits that also drain the tile copies in flight
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // the lane index is made opaque at each item's start and again before its merge: lane-derived values of the start
    // and the merge are not held (and spilled) across the tile loop, as a spill reload waits for every copy in flight
    int lane = threadIdx.x & 63;
    const int sl = wv; // the wave's slice of tiles: w, w + 4, ..
    const StoreLayout & S = a.S; // (the layouts of layers after layer0, the fused append's geometry)
    const unsigned lds0 = (unsigned) (size_t) (__attribute__((address_space(3))) uint8_t *) smem;
    const unsigned st_lds0 = (unsigned) __builtin_amdgcn_readfirstlane(lds0 + wv * SB);
    half8 * const sQ = reinterpret_cast<half8 *>(smem + SLDS); // [RP][256] fp16, chunk-swizzled (qchunk)
    // The first tile copy of an item waits on every scalar load before it, and each round trip to the kernel arguments
    // costs a few hundred ns at launch: the common case (one sequence, one layer) takes everything from the launch head
    // (AttnHead, one round of loads); only other sequences / layers read more.
    const HeadRegs hr = load_head();
    const int n_items = QKV_HEAD(hr, n_items), n_base = QKV_HEAD(hr, n_base), nseq0 = QKV_HEAD(hr, nseq), kvrc = QKV_HEAD(hr, kvrc),
              spage = QKV_HEAD(hr, page);
    const int T = QKV_HEAD(hr, T), R = QKV_HEAD(hr, R), layer0 = QKV_HEAD(hr, layer0), qs = QKV_HEAD(hr, qs);
    const unsigned krot = QKV_HEAD(hr, krot);
    const int * const ptab = QKV_HEAD(hr, ptab);
    const int pt_stride = QKV_HEAD(hr, pt_stride), n_pages = QKV_HEAD(hr, n_pages);
    const SeqDesc sd0{QKV_HEAD(hr, seq),  QKV_HEAD(hr, L),     QKV_HEAD(hr, ws),   QKV_HEAD(hr, cs),
                      QKV_HEAD(hr, nseg), QKV_HEAD(hr, item0), QKV_HEAD(hr, pbase), QKV_HEAD(hr, nseg_m)};
    const unsigned T_m = QKV_HEAD(hr, T_m);
    const SideLayout K0{QKV_HEAD(hr, kvals), QKV_HEAD(hr, kscs), QKV_HEAD(hr, kring), QKV_HEAD(hr, krsc), APPEND ? a.side0[0].bits : KB,
                        APPEND ? a.side0[0].rot : 0};
    const SideLayout V0{QKV_HEAD(hr, vvals), QKV_HEAD(hr, vscs), QKV_HEAD(hr, vring), QKV_HEAD(hr, vrsc), APPEND ? a.side0[1].bits : VB,
                        APPEND ? a.side0[1].rot : 0};
    const float * const qp = QKV_HEAD(hr, q);
    const float * const qnw = QKV_HEAD(hr, qnw);
    const float2 * const rope = QKV_HEAD(hr, rope);
    float * const part = QKV_HEAD(hr, part);
    float2 * const ml = QKV_HEAD(hr, ml);
    for (int bitem = blockIdx.x; bitem < n_items; bitem += gridDim.x) {
        asm volatile("" : "+v"(lane));
        // the stage address and the sequence count are made opaque per item as well: values derived from them (the 16
        // copy destinations of a stage, the sequence tests) are computed where they are used instead of once before
        // the loop and kept in VGPR lanes, which costs more instructions before an item's first copy than it saves
        unsigned st_lds = st_lds0;
        int nseq = nseq0;
        asm volatile("" : "+s"(st_lds), "+s"(nseq));
        int n = lane & 15, q = lane >> 4;
        // one row batch per item, or two (n_items = 2 n_base: T = 5..8 in 24-row batches)
        int item = bitem, batch = 0;
        if (n_items != n_base) {
            // two row batches of one item run on workgroup indices 8 apart: the same XCD (workgroups are dealt to the
            // 8 XCDs round robin by index) and dispatched together there, so the second batch's tile copies find the
            // first's in that XCD's L2 instead of streaming the segment from HBM again.  The items past the last
            // whole group of 8 keep the batch-minor order.
            const int full = (n_base >> 3) << 3;
            if (bitem < 2 * full) {
                const int k = bitem >> 3;
                item = ((k >> 1) << 3) + (bitem & 7);
                batch = k & 1;
            } else {
                item = full + ((bitem - 2 * full) >> 1);
                batch = (bitem - 2 * full) & 1;
            }
        }
        const int row0 = RP * batch;
        int si = 0;
        SeqDesc sd = sd0;
        if (nseq > 1) {
            int it0[MAX_SEQ];
#pragma unroll
            for (int i = 0; i < MAX_SEQ; i++) it0[i] = a.sd[i].item0; // independent loads, one round
#pragma unroll
            for (int i = 1; i < MAX_SEQ; i++)
                if (i < nseq && item >= it0[i]) si = i;
            sd = a.sd[si];
        }
        const int local = item - sd.item0;
        const int lg = div_m(local, sd.nseg_m), seg = local - lg * sd.nseg;
        const int g = lg % NKV, l = lg / NKV;
        const int L = sd.L, ws = sd.ws, seq = sd.seq;
        const int c0 = seg * sd.cs, c1 = min(L, c0 + sd.cs);
        const int ntiles = (c1 - c0 + ATP - 1) / ATP;
        const int my = ntiles > sl ? (ntiles - sl + AWAVES - 1) / AWAVES : 0; // tiles sl, sl+4, ..
        SideLayout SK = K0, SV = V0;
        if (l > 0) {
            SK = S.side[layer0 + l][0];
            SV = S.side[layer0 + l][1];
        }
        const RowGeo geo{ptab, pt_stride, spage, n_pages, kvrc};
        const size_t ring0 = (size_t) (seq * NKV + g) * kvrc;
        const size_t gbase = (size_t) (g * n_pages + sd.pbase) * spage;
        // (the page-table path divides by the page size, made opaque there, so that the division's set-up is
        // not hoisted out of the item loop onto the common path)
        auto paged_geo = [&]() {
            RowGeo G = geo;
            asm volatile("" : "+s"(G.page));
            return G;
        };
        auto main_row_of = [&](int p, int phys) { return sd.pbase >= 0 ? gbase + p : attn_main_row(paged_geo(), g, p, phys); };

        // tile i of the wave starts at position c0 + 32 (sl + 4 i); phys: its physical page; into the stage at lds_to
        auto issue = [&](int i, int phys, unsigned lds_to) {
            const int p0 = c0 + ATP * (sl + AWAVES * i), nv = min(ATP, L - p0);
            const bool ring = kvrc > 0 && p0 >= ws; // the window: q8 rows (ring, or the main store of q8 sides)
            const TileSrc t = tile_src_row<KB, VB>(kvrc, SK, SV, main_row_of(p0, phys), p0, ring0, ring);
            int ln = lane; // opaque: the per-lane chunk addresses are not hoisted out of the tile loop into registers
            asm volatile("" : "+v"(ln));
            // 24-row kernels (NP = 3) run T = 5..8 as two row batches that stream the same tiles: no non-temporal hint
            constexpr bool NT = NP < 3;
            if (ring) {
                if constexpr (SMALL) issue_q8_part<0, NT>(t, nv, lds_to, ln);
                else issue_tile<8, 8, 0, NT>(t, nv, lds_to, ln);
            } else {
                issue_tile<KB, VB, 0, NT>(t, nv, lds_to, ln);
            }
        };

        // physical page of tile i: the table is read only for sequences whose pages are not contiguous (0 otherwise:
        // the main-store row of position p is then gbase + p)
        auto tile_page = [&](int i) { return sd.pbase >= 0 ? 0 : page_of(paged_geo(), seq, c0 + ATP * (sl + AWAVES * i)); };
        int phys_cur = my > 0 ? tile_page(0) : 0; // page of the tile in the stage (tile i while step i runs)
        // fused append (APPEND kernels only): a wave whose tiles hold new positions (L - T .. L - 1) stores those rows
        // before its first copy (a called function waits for every load at entry, so it runs before any copy is issued)
        bool has_new = false;
        if (APPEND && a.kin) {
            const int pa = max(L - T, c0), pb = min(L, c1);
            for (int p = pa; p < pb; p++) has_new |= ((p - c0) >> 5) % AWAVES == sl;
        }
        // ---- queries: FWHT when K is stored rotated, * 1/16, fp16 (qwen38_mk.cu:2873-2880), rows r = hh T + t.  The
        // wave's rows are loaded before its first tile copy and waited for alone (loads return in order: vmcnt at most
        // the copy count), so they are converted while tile 0 streams.  Only the copy issue runs between the loads and
        // the wait (the loaded registers must not be read or moved before it).
        if constexpr (APPEND)
            if (has_new) {
                append_rows(a.kin, a.vin, a.kin_f16, a.kin_nl, geo.ptab, geo.pt_stride, geo.page, geo.n_pages, geo.kvrc, SK.vals, SK.scs, SK.ring,
                            SK.rsc, SK.bits, SK.rot, SV.vals, SV.scs, SV.ring, SV.rsc, SV.bits, SV.rot, seq, g, l, si, L, T, c0, c1, sl, 0, 1);
                vm_wait<0>(); // the stored rows are in L2 before this wave's copies read them
            }
        constexpr int QPW = RP / AWAVES; // rows per wave
        f32x4 qx[QPW];
#pragma unroll
        for (int j = 0; j < QPW; j++) {
            const int r = row0 + wv + AWAVES * j;
            if (r < R) {
                const int hh = div_m(r, T_m), t = r - hh * T;
                qx[j] = gload16(qp + (((size_t) (l * nseq + si) * T + t) * NH + GQA * g + hh) * qs + 4 * lane);
            } else {
                qx[j] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
        }
        if (my > 0) {
            issue(0, phys_cur, st_lds);
            // copy instructions of tile 0 (issue_tile / issue_q8_part): every load before them has returned
            const bool ring = kvrc > 0 && c0 + ATP * sl >= ws;
            if (ring) {
                vm_wait<SMALL ? 8 + 1 : 8 + 8 + 1>();
            } else {
                vm_wait<KB + VB + 1>();
            }
        } else {
            vm_wait<0>();
        }
#pragma unroll
        for (int j = 0; j < QPW; j++) {
            pin_after(qx[j]);
            const int r = wv + AWAVES * j, gr = row0 + r;
            half2v o0 = {(_Float16) 0.f, (_Float16) 0.f}, o1 = o0;
            if (gr < R) {
                const int t = gr - div_m(gr, T_m) * T;
                float v[4] = {qx[j][0], qx[j][1], qx[j][2], qx[j][3]};
                if (qnw) qk_prep(v, qnw + (size_t) l * HD, rope + (size_t) (L - T + t) * 32);
                if ((krot >> (layer0 + l)) & 1u) fwht256_w64(v);
                o0[0] = (_Float16) (v[0] * 0.0625f);
                o0[1] = (_Float16) (v[1] * 0.0625f);
                o1[0] = (_Float16) (v[2] * 0.0625f);
                o1[1] = (_Float16) (v[3] * 0.0625f);
            }
            reinterpret_cast<uint2 *>(sQ + qchunk(r, lane >> 1))[lane & 1] = make_uint2(as_u(o0), as_u(o1));
        }
        // one 8-row group: compute_tile (each row in two columns); 16 or 24 rows: compute_tile_v (distinct rows)
        constexpr bool DISTINCT = NP >= 2;
        std::conditional_t<DISTINCT, RowState<(DISTINCT ? NP : 2)>, WaveState<NP>> st;
        if constexpr (DISTINCT) {
#pragma unroll
            for (int H = 0; H < RowState<NP>::NB; H++) {
                st.m[H] = -INFINITY;
                st.l[H] = 0.f;
                const int row = row0 + 16 * H + n; // (block 1, lanes 8..15: padding)
                st.lim[H] = (H == 0 || n < 8) && row < R ? L - T + (row - div_m(row, T_m) * T) : -1;
            }
        } else {
#pragma unroll
            for (int h = 0; h < NP; h++) {
                st.m[h] = -INFINITY;
                st.l[h] = 0.f;
                const int row = row0 + 8 * h + (n >> 1);
                st.lim[h] = row < R ? L - T + (row - div_m(row, T_m) * T) : -1;
            }
        }
#pragma unroll
        for (int h = 0; h < NP; h++)
#pragma unroll
            for (int b = 0; b < 8; b++) st.acc[h][b] = f32x4{0.f, 0.f, 0.f, 0.f};
        st.lim_min = L - T;
        __syncthreads(); // the query rows are complete
        if constexpr (NP == 1) {
#pragma unroll
            for (int ks = 0; ks < 8; ks++) st.qf[ks] = sQ[qchunk(n >> 1, 8 * q + ks)];
        }
        const uint8_t * const stp = smem + wv * SB; // (derived from smem: LDS reads)
        // one tile: operands into registers, then the stage is free and the next tile streams in during the math
        auto step = [&](auto fmt, int i) {
            constexpr int K2 = decltype(fmt)::kb, V2 = decltype(fmt)::vb;
            set_prio(my - i);
            const int phys_next = i + 1 < my ? tile_page(i + 1) : 0; // the scalar load overlaps the wait below
            vm_wait<0>(); // tile i has landed (the wave's only copies in flight)
            RawTile<K2, V2> raw;
            const int p0 = c0 + ATP * (sl + AWAVES * i);
            if constexpr (SMALL && K2 == 8 && V2 == 8) { // a q8 window tile in two halves
                const uint16_t * const sc = reinterpret_cast<const uint16_t *>(stp + 8192);
                read_k<8, 8>(raw, stp, sc, n, q);
                lds_drain(); // the K rows are in registers: the V half may overwrite them
                {
                    const TileSrc t = tile_src_row<KB, VB>(kvrc, SK, SV, main_row_of(p0, phys_cur), p0, ring0, true);
                    int ln = lane;
                    asm volatile("" : "+v"(ln));
                    issue_q8_part<1>(t, min(ATP, L - p0), st_lds, ln);
                }
                compute_tile<NP, 8, 8, true>(
                    st, sQ, p0, raw,
                    [&](RawTile<8, 8> & r, int tn, int tq) {
                        vm_wait<0>(); // the V half has landed
                        read_v<8, 8>(r, stp, sc + 8 * ATP, tn, tq);
                    },
                    [&]() {
                        if (i + 1 < my) issue(i + 1, phys_next, st_lds);
                    });
            } else if constexpr (LATE_V && DISTINCT) {
                read_k<K2, V2>(raw, stp, n, q);
                compute_tile_v<(DISTINCT ? NP : 2), K2, V2>(
                    st, sQ, p0, raw, [&](RawTile<K2, V2> & r, int tn, int tq) { read_v<K2, V2>(r, stp, tn, tq); },
                    [&]() {
                        if (i + 1 < my) issue(i + 1, phys_next, st_lds);
                    });
            } else if constexpr (LATE_V) {
                read_k<K2, V2>(raw, stp, n, q);
                compute_tile<NP, K2, V2, true>(
                    st, sQ, p0, raw, [&](RawTile<K2, V2> & r, int tn, int tq) { read_v<K2, V2>(r, stp, tn, tq); },
                    [&]() {
                        if (i + 1 < my) issue(i + 1, phys_next, st_lds);
                    });
            } else if constexpr (DISTINCT) {
                read_k<K2, V2>(raw, stp, n, q);
                read_v<K2, V2>(raw, stp, n, q);
                lds_drain();
                if (i + 1 < my) issue(i + 1, phys_next, st_lds);
                compute_tile_v<(DISTINCT ? NP : 2), K2, V2>(st, sQ, p0, raw, NoHook());
            } else {
                read_k<K2, V2>(raw, stp, n, q);
                read_v<K2, V2>(raw, stp, n, q);
                lds_drain();
                if (i + 1 < my) issue(i + 1, phys_next, st_lds);
                compute_tile<NP, K2, V2>(st, sQ, p0, raw);
            }
            phys_cur = phys_next;
        };
        // the wave's window (ring) tiles are its last ones: i >= i_ring, p0 >= ws.  Two loops, one tile format each,
        // keep a single tile body live per loop (one body holding both formats costs registers)
        int i_ring = my;
        if (kvrc > 0) {
            const int d = ws - c0 - ATP * sl;
            i_ring = d <= 0 ? 0 : min(my, (d + AWAVES * ATP - 1) / (AWAVES * ATP));
        }
        int i = 0;
        for (; i < i_ring; i++) step(Fmt<KB, VB>(), i);
        for (; i < my; i++) step(Fmt<8, 8>(), i);
        asm volatile("" : "+v"(lane));
        n = lane & 15;
        q = lane >> 4;
        // ---- merge the 4 waves in order: M = max m_w, O = sum e_w O_w, l = sum e_w l_w.  Per pass of 16 rows (two
        // groups) every wave writes its scaled O rows to its own LDS buffer (the stages are free), then each thread
        // adds the 4 buffers in wave order.
        constexpr int OLD = HD + 4;                                                   // row stride (floats) of a buffer
        constexpr int MR = NP == 1 ? 8 : 16;                                          // rows per wave buffer
        float * const s_m = reinterpret_cast<float *>(smem + AWAVES * MR * OLD * 4); // [AWAVES][RP]
        float * const s_l = s_m + AWAVES * RP;                                        // [AWAVES][RP]
        static_assert(AWAVES * MR * OLD * 4 + 2 * AWAVES * RP * 4 <= SLDS, "merge buffers inside the stages");
        __syncthreads(); // every wave is done with its stage
        if constexpr (DISTINCT) {
            if (q == 0) { // rows 16 H + n of the blocks
                s_m[wv * RP + n] = st.m[0];
                s_l[wv * RP + n] = st.l[0];
                if constexpr (NP == 3)
                    if (n < 8) {
                        s_m[wv * RP + 16 + n] = st.m[RowState<NP>::NB - 1];
                        s_l[wv * RP + 16 + n] = st.l[RowState<NP>::NB - 1];
                    }
            }
        } else if (q == 0 && !(n & 1)) {
#pragma unroll
            for (int h = 0; h < NP; h++) {
                s_m[wv * RP + 8 * h + (n >> 1)] = st.m[h];
                s_l[wv * RP + 8 * h + (n >> 1)] = st.l[h];
            }
        }
        __syncthreads();
        const int RB = min(RP, R - row0); // rows of this batch
        constexpr int NPASS = (NP + 1) / 2;
#pragma unroll
        for (int ps = 0; ps < NPASS; ps++) {
#pragma unroll
            for (int hh = 0; hh < 2; hh++) {
                const int h = 2 * ps + hh;
                if (h < NP) {
                    const int row = 8 * h + (n >> 1);
                    const float M = fmaxf(fmaxf(s_m[row], s_m[RP + row]), fmaxf(s_m[2 * RP + row], s_m[3 * RP + row]));
                    const float mr = DISTINCT ? s_m[wv * RP + row] : st.m[(DISTINCT ? 0 : h)]; // the wave's own m of the row
                    const float e = mr == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mr - M);
                    float * o = reinterpret_cast<float *>(smem) + (wv * MR + 8 * hh + (n >> 1)) * OLD + 64 * q + (n & 1);
#pragma unroll
                    for (int b = 0; b < 8; b++)
#pragma unroll
                        for (int i = 0; i < 4; i++) o[16 * i + 2 * b] = e * st.acc[h][b][i];
                }
            }
            __syncthreads();
            const int nrow = min(16, RB - 16 * ps);
            for (int idx = threadIdx.x; idx < nrow * (HD / 4); idx += 256) {
                const int r16 = idx / (HD / 4), c4 = idx % (HD / 4);
                const float * src = reinterpret_cast<const float *>(smem) + r16 * OLD + 4 * c4;
                float4 y = *reinterpret_cast<const float4 *>(src);
#pragma unroll
                for (int w = 1; w < AWAVES; w++) {
                    const float4 z = *reinterpret_cast<const float4 *>(src + w * MR * OLD);
                    y.x += z.x;
                    y.y += z.y;
                    y.z += z.z;
                    y.w += z.w;
                }
                store_part(part + ((size_t) item * R + row0 + 16 * ps + r16) * HD + 4 * c4, y);
            }
            if (ps + 1 < NPASS) __syncthreads();
        }
        if (threadIdx.x < RB) {
            const int row = threadIdx.x;
            const float M = fmaxf(fmaxf(s_m[row], s_m[RP + row]), fmaxf(s_m[2 * RP + row], s_m[3 * RP + row]));
            float lsum = 0.f;
#pragma unroll
            for (int w = 0; w < AWAVES; w++) {
                const float ew = s_m[w * RP + row] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(s_m[w * RP + row] - M);
                lsum += ew * s_l[w * RP + row];
            }
            ml[(size_t) item * R + row0 + row] = make_float2(M, lsum);
        }
        __syncthreads(); // the LDS is reused by the next item
    }
}

// ------------------------------------------------------------------------------------------------ verify kernel
// 25..48 query rows per kv head (T = 5..8) in one pass over each segment, persistent: one workgroup of 8 waves per CU
// walks the work items blockIdx.x, + gridDim.x, ...  Waves w and w + 4 take tile slice w (tiles w, w + 4, ..) for rows
// 0..23 and 24..47 and share the slice's two LDS stages; at step i (after a workgroup barrier) tile i + 1 is copied
// into the other stage -- the K rows and K scales by the first wave of the pair, the V rows and V scales by the
// second -- while both compute tile i.  After an item's last step the copies of the next item's first tiles go into the
// free stages during the merge, so an item starts with them on their way.  A row's
// slices, tile arithmetic and merge order are those of k_attn: bitwise the same partials.
// APPEND (mk_kv_append_attend): the new rows are stored before an item's first copy, so nothing is started early.
template <typename P>
__device__ __forceinline__ P * uniform_ptr(P * p) {
    const unsigned long long x = (unsigned long long) p;
    const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned) x), hi = __builtin_amdgcn_readfirstlane((unsigned) (x >> 32));
    return reinterpret_cast<P *>(((unsigned long long) hi << 32) | lo);
}
struct ItemGeo {
    int si, seq, L, ws, c0, c1, ntiles, g, l, pbase;
    SideLayout SK, SV;
    size_t ring0;
};
__device__ __forceinline__ ItemGeo item_geo(const AttnArgs & a, int item) {
    ItemGeo G;
    int si = 0;
#pragma unroll
    for (int i = 1; i < MAX_SEQ; i++)
        if (i < a.nseq && item >= a.sd[i].item0) si = i;
    const SeqDesc sd = a.sd[si];
    const int local = item - sd.item0, lg = div_m(local, sd.nseg_m), seg = local - lg * sd.nseg;
    G.si = si;
    G.seq = sd.seq;
    G.L = sd.L;
    G.ws = sd.ws;
    G.g = lg % NKV;
    G.l = lg / NKV;
    G.pbase = sd.pbase;
    G.c0 = seg * sd.cs;
    G.c1 = min(sd.L, G.c0 + sd.cs);
    G.ntiles = (G.c1 - G.c0 + ATP - 1) / ATP;
    G.SK = a.S.side[a.layer0 + G.l][0];
    G.SV = a.S.side[a.layer0 + G.l][1];
    G.ring0 = (size_t) (sd.seq * NKV + G.g) * a.S.kvrc;
    return G;
}

template <int KB, int VB, bool APPEND = false>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_verify(AttnArgs a) {
    constexpr int NP = 3, RP = 24, NW = 2 * AWAVES, QPW = 2 * RP / NW, SB = STAGE_BYTES;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // the lane index is made opaque at each item's start and again before its merge, so that lane-derived values of the
    // item's start and merge are not held (and spilled) across the tile loop: a spill reload waits for every copy in
    // flight, the next item's first tiles included
    int lane = threadIdx.x & 63;
    const int sl = wv & (AWAVES - 1), hf = wv / AWAVES, row0 = RP * hf;
    const StoreLayout & S = a.S;
    const unsigned lds0 = (unsigned) (size_t) (__attribute__((address_space(3))) uint8_t *) smem;
    auto stage = [&](int b) { return 2 * sl + (b & 1); }; // stage b of the wave's slice
    half8 * const sQ = reinterpret_cast<half8 *>(smem + NW * SB); // [48][256] fp16, chunk-swizzled per half of 24 rows
    const half8 * const sQh = sQ + hf * RP * (HD / 8);
    const int T = a.T, R = a.R;
    const unsigned T_m = a.h.T_m;

    // physical page of position p of item G: the table is read only for sequences whose pages are not contiguous (0
    // otherwise: the main-store row of p is then (g n_pages + pbase) page + p)
    auto tile_phys = [&](const ItemGeo & G, int p) { return G.pbase >= 0 ? 0 : page_of(S, G.seq, p); };
    // the wave's half of tile i of an item (its first position c0, length L, window start ws, kv head g, sides SK / SV,
    // first ring row ring0) into stage b
    auto issue = [&](SideLayout SK, SideLayout SV, int c0, int L, int ws, int g, int pbase, size_t ring0, int i, int phys, int b) {
        const int p0 = c0 + ATP * (sl + AWAVES * i), nv = min(ATP, L - p0);
        const bool ring = S.kvrc > 0 && p0 >= ws;
        const size_t mr = pbase >= 0 ? (size_t) (g * S.n_pages + pbase) * S.page + p0 : attn_main_row(S, g, p0, phys);
        TileSrc t = tile_src_row<KB, VB>(S.kvrc, SK, SV, mr, p0, ring0, ring);
        t.k = uniform_ptr(t.k); // (wave-uniform by construction; stated, so that the copies take the scalar base)
        t.v = uniform_ptr(t.v);
        const unsigned to = (unsigned) __builtin_amdgcn_readfirstlane(lds0 + stage(b) * SB);
        int ln = lane;
        asm volatile("" : "+v"(ln));
        if (ring) {
            if (hf == 0) issue_tile<8, 8, 1>(t, nv, to, ln);
            else issue_tile<8, 8, 2>(t, nv, to, ln);
        } else {
            if (hf == 0) issue_tile<KB, VB, 1>(t, nv, to, ln);
            else issue_tile<KB, VB, 2>(t, nv, to, ln);
        }
    };
    // the wave's query rows r = wv + 8 j of item G (rows hh T + t of the kv head)
    auto q_addr = [&](const ItemGeo & G, int j) {
        const int r = wv + NW * j, hh = div_m(r, T_m), t = r - hh * T;
        return a.q + (((size_t) (G.l * a.nseq + G.si) * T + t) * NH + GQA * G.g + hh) * a.qs + 4 * lane;
    };

    int par = 0;      // stage parity of the item's tile 0
    bool pre = false; // the item's first tiles were started by the previous item
    for (int item = blockIdx.x; item < a.n_items; item += gridDim.x) {
        asm volatile("" : "+v"(lane));
        int n = lane & 15, q = lane >> 4;
        const ItemGeo G = item_geo(a, item);
        const SideLayout SK = G.SK, SV = G.SV;
        const int my = G.ntiles > sl ? (G.ntiles - sl + AWAVES - 1) / AWAVES : 0;
        const int my0 = (G.ntiles + AWAVES - 1) / AWAVES;
        const int nxt = item + gridDim.x;
        const bool chain = !(APPEND && a.kin) && nxt < a.n_items;
        f32x4 qx[QPW];
        if (pre) { // (tile 0 was copied during the previous merge: waiting for the rows finds it landed too)
#pragma unroll
            for (int j = 0; j < QPW; j++)
                qx[j] = wv + NW * j < R ? *reinterpret_cast<const f32x4 *>(q_addr(G, j)) : f32x4{0.f, 0.f, 0.f, 0.f};
        } else {
            if constexpr (APPEND) {
                bool has_new = false;
                if (a.kin)
                    for (int p = max(G.L - T, G.c0); p < min(G.L, G.c1); p++) has_new |= ((p - G.c0) >> 5) % AWAVES == sl;
                if (has_new) {
                    append_rows(a.kin, a.vin, a.kin_f16, a.kin_nl, S.ptab, S.pt_stride, S.page, S.n_pages, S.kvrc, G.SK.vals, G.SK.scs,
                                G.SK.ring, G.SK.rsc, G.SK.bits, G.SK.rot, G.SV.vals, G.SV.scs, G.SV.ring, G.SV.rsc, G.SV.bits, G.SV.rot,
                                G.seq, G.g, G.l, G.si, G.L, T, G.c0, G.c1, sl, hf, hf);
                    vm_wait<0>(); // the stored rows are in L2 before this wave's copies read them
                }
            }
            // loaded before the first copy and waited for alone (loads return in order), as in k_attn
#pragma unroll
            for (int j = 0; j < QPW; j++) qx[j] = wv + NW * j < R ? gload16(q_addr(G, j)) : f32x4{0.f, 0.f, 0.f, 0.f};
            if (my > 0) {
                issue(SK, SV, G.c0, G.L, G.ws, G.g, G.pbase, G.ring0, 0, tile_phys(G, G.c0 + ATP * sl), par);
                const bool ring = S.kvrc > 0 && G.c0 + ATP * sl >= G.ws;
                if (ring) vm_wait<8 + 1>();
                else if (hf == 0) vm_wait<KB + 1>();
                else vm_wait<VB + 1>();
            } else {
                vm_wait<0>();
            }
#pragma unroll
            for (int j = 0; j < QPW; j++) pin_after(qx[j]);
        }
        // ---- queries: FWHT when K is stored rotated, * 1/16, fp16 (qwen38_mk.cu:2873-2880)
#pragma unroll
        for (int j = 0; j < QPW; j++) {
            const int r = wv + NW * j;
            half2v o0 = {(_Float16) 0.f, (_Float16) 0.f}, o1 = o0;
            if (r < R) {
                const int t = r - div_m(r, T_m) * T;
                float v[4] = {qx[j][0], qx[j][1], qx[j][2], qx[j][3]};
                if (a.qnw) qk_prep(v, a.qnw + (size_t) G.l * HD, a.rope + (size_t) (G.L - T + t) * 32);
                if ((a.krot >> (a.layer0 + G.l)) & 1u) fwht256_w64(v);
                o0[0] = (_Float16) (v[0] * 0.0625f);
                o0[1] = (_Float16) (v[1] * 0.0625f);
                o1[0] = (_Float16) (v[2] * 0.0625f);
                o1[1] = (_Float16) (v[3] * 0.0625f);
            }
            reinterpret_cast<uint2 *>(sQ + (r / RP) * RP * (HD / 8) + qchunk(r % RP, lane >> 1))[lane & 1] = make_uint2(as_u(o0), as_u(o1));
        }
        RowState<NP> st;
#pragma unroll
        for (int H = 0; H < 2; H++) {
            st.m[H] = -INFINITY;
            st.l[H] = 0.f;
            const int row = row0 + 16 * H + n; // (block 1, lanes 8..15: padding)
            st.lim[H] = (H == 0 || n < 8) && row < R ? G.L - T + (row - div_m(row, T_m) * T) : -1;
        }
#pragma unroll
        for (int h = 0; h < NP; h++)
#pragma unroll
            for (int b = 0; b < 8; b++) st.acc[h][b] = f32x4{0.f, 0.f, 0.f, 0.f};
        st.lim_min = G.L - T;
        // ---- the tiles: one workgroup barrier per step (the first also completes the query rows)
        int i_ring = my;
        if (S.kvrc > 0) {
            const int d = G.ws - G.c0 - ATP * sl;
            i_ring = d <= 0 ? 0 : min(my, (d + AWAVES * ATP - 1) / (AWAVES * ATP));
        }
        auto vstep = [&](auto fmt, int i) {
            constexpr int K2 = decltype(fmt)::kb, V2 = decltype(fmt)::vb;
            set_prio(my - i);
            const int phys_next = i + 1 < my ? tile_phys(G, G.c0 + ATP * (sl + AWAVES * (i + 1))) : 0;
            vm_wait<0>();    // this wave's half of tile i has landed
            __syncthreads(); // both halves of every slice's tile i are staged; every wave is done with tile i - 1
            if (i + 1 < my) issue(SK, SV, G.c0, G.L, G.ws, G.g, G.pbase, G.ring0, i + 1, phys_next, par + i + 1);
            if (i < my) {
                const uint8_t * const sp = smem + stage(par + i) * SB;
                RawTile<K2, V2> raw;
                read_k<K2, V2>(raw, sp, n, q);
                compute_tile_v<NP, K2, V2>(st, sQh, G.c0 + ATP * (sl + AWAVES * i), raw,
                                               [&](RawTile<K2, V2> & r, int tn, int tq) { read_v<K2, V2>(r, sp, tn, tq); });
            }
        };
        int i = 0;
        for (; i < i_ring; i++) vstep(Fmt<KB, VB>(), i);
        for (; i < my0; i++) vstep(Fmt<8, 8>(), i);
        // the next item's first tile of this slice, on its way during the merge (into the stage parity the last step left
        // free: its tile my0 - 2 was read before that step's barrier)
        if (chain) {
            const ItemGeo N = item_geo(a, nxt);
            if (N.ntiles > sl) issue(N.SK, N.SV, N.c0, N.L, N.ws, N.g, N.pbase, N.ring0, 0, tile_phys(N, N.c0 + ATP * sl), par + my0);
        }
        asm volatile("" : "+v"(lane));
        n = lane & 15;
        q = lane >> 4;
        // ---- merge the 4 slices of each row in order (as k_attn), one 8-row group per pass.  Wave w's buffer is half of
        // stage 2 (w / 2) + the parity of the last tile (read by now); the next item's first tiles sit in the other parity.
        constexpr int OLD = HD + 4, MB = 8 * OLD * 4; // row stride (floats), one wave's buffer (bytes)
        static_assert(2 * MB <= SB, "two wave buffers per stage");
        const int bl = (par + my0 - 1) & 1;
        auto wbuf = [&](int w) { return reinterpret_cast<float *>(smem + (2 * (w >> 1) + bl) * SB + (w & 1) * MB); };
        float * const s_m = reinterpret_cast<float *>(sQ); // [8][24] (the query rows are read by now)
        float * const s_l = s_m + NW * RP;
        lds_barrier(); // every wave is done with its tiles and the query rows
        if (q == 0) { // rows 16 H + n of the blocks
            s_m[wv * RP + n] = st.m[0];
            s_l[wv * RP + n] = st.l[0];
            if (n < 8) {
                s_m[wv * RP + 16 + n] = st.m[1];
                s_l[wv * RP + 16 + n] = st.l[1];
            }
        }
        const int th = threadIdx.x / 256, tl = threadIdx.x - 256 * th, wb = AWAVES * th;
        const int trow0 = RP * th, RB = min(RP, R - trow0);
        const float * const s_mh = s_m + wb * RP, * const s_mw = s_m + hf * AWAVES * RP;
        lds_barrier();
#pragma unroll
        for (int h = 0; h < NP; h++) {
            {
                const int row = 8 * h + (n >> 1);
                const float M = fmaxf(fmaxf(s_mw[row], s_mw[RP + row]), fmaxf(s_mw[2 * RP + row], s_mw[3 * RP + row]));
                const float mr = s_mw[wv % AWAVES * RP + row]; // the wave's own m of the row
                const float e = mr == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mr - M);
                float * o = wbuf(wv) + (n >> 1) * OLD + 64 * q + (n & 1);
#pragma unroll
                for (int b = 0; b < 8; b++)
#pragma unroll
                    for (int k = 0; k < 4; k++) o[16 * k + 2 * b] = e * st.acc[h][b][k];
            }
            lds_barrier();
            const int nrow = min(8, RB - 8 * h);
            for (int idx = tl; idx < nrow * (HD / 4); idx += 256) {
                const int r8 = idx / (HD / 4), c4 = idx % (HD / 4);
                float4 y = *reinterpret_cast<const float4 *>(wbuf(wb) + r8 * OLD + 4 * c4);
#pragma unroll
                for (int w = 1; w < AWAVES; w++) {
                    const float4 z = *reinterpret_cast<const float4 *>(wbuf(wb + w) + r8 * OLD + 4 * c4);
                    y.x += z.x;
                    y.y += z.y;
                    y.z += z.z;
                    y.w += z.w;
                }
                store_part(a.part + ((size_t) item * R + trow0 + 8 * h + r8) * HD + 4 * c4, y);
            }
            if (h + 1 < NP) lds_barrier();
        }
        if (tl < RB) {
            const int row = tl;
            const float M = fmaxf(fmaxf(s_mh[row], s_mh[RP + row]), fmaxf(s_mh[2 * RP + row], s_mh[3 * RP + row]));
            float lsum = 0.f;
#pragma unroll
            for (int w = 0; w < AWAVES; w++) {
                const float ew = s_mh[w * RP + row] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(s_mh[w * RP + row] - M);
                lsum += ew * s_l[(wb + w) * RP + row];
            }
            a.ml[(size_t) item * R + trow0 + row] = make_float2(M, lsum);
        }
        lds_barrier(); // the buffers and the query rows are reused by the next item
        par = (par + my0) & 1;
        pre = chain;
    }
}

typedef void (*AttnKernel)(AttnArgs);
template <bool APPEND>
static AttnKernel verify_of(int kb, int vb) {
#define QKV_VB(K)                                                                                                      \
    switch (vb) {                                                                                                      \
    case 4: return k_verify<K, 4, APPEND>;                                                                             \
    case 5: return k_verify<K, 5, APPEND>;                                                                             \
    case 6: return k_verify<K, 6, APPEND>;                                                                             \
    case 7: return k_verify<K, 7, APPEND>;                                                                             \
    case 8: return k_verify<K, 8, APPEND>;                                                                             \
    default: return nullptr;                                                                                           \
    }
    switch (kb) {
    case 4: QKV_VB(4)
    case 5: QKV_VB(5)
    case 6: QKV_VB(6)
    case 7: QKV_VB(7)
    case 8: QKV_VB(8)
    default: return nullptr;
    }
#undef QKV_VB
}
// the fused-append kernels (kv_attn_fused.hip): np row groups, wide (np = 3, 48 rows), K / V bits
AttnKernel pick_fused(int np, bool wide, int kb, int vb);

} // namespace qkv
