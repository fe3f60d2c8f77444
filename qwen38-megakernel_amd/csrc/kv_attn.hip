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
#include "kv_dev.h"
#include "kv_launch.h"

namespace qkv {

constexpr float LOG2E = 1.4426950408889634f;
constexpr unsigned C64 = 0x64646464u;

// The page table is read through the constant address space (no kernel writes it during a launch): a scalar load,
// which waits on lgkmcnt only, never on the tile copies in flight.  Its latency under a full HBM stream is of the order
// of a tile's, so the tile loops look a tile's page up one step ahead (page_of), before they wait for the current tile.
typedef const __attribute__((address_space(4))) int * const_int_p;

// physical page of the logical page holding position p (wave-uniform) of sequence seq
__device__ __forceinline__ int page_of(const StoreLayout & S, int seq, int p) {
    const int lp = __builtin_amdgcn_readfirstlane(p / S.page);
    return ((const_int_p) S.ptab)[seq * S.pt_stride + lp];
}

// main-store row of (g, p) in physical page phys (the page of p)
__device__ __forceinline__ size_t attn_main_row(const StoreLayout & S, int g, int p, int phys) {
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
__device__ __forceinline__ void dma16(const void * g, unsigned lds) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds), "v"(g) : "memory");
}
// the same with a scalar base address and a 32-bit per-lane byte offset (no 64-bit vector address per copy)
__device__ __forceinline__ void dma16s(const void * base, unsigned voff, unsigned lds) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds), "v"(voff), "s"(base) : "memory");
}
__device__ __forceinline__ void lds_drain() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
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
// KB / VB bits.  ring0 = the first ring row of (seq, g).
// phys: the physical page of p0 (page_of), looked up by the caller
template <int KB, int VB>
__device__ __forceinline__ TileSrc tile_src(const StoreLayout & S, const SideLayout & SK, const SideLayout & SV, int g, int p0, int phys,
                                           size_t ring0, bool ring) {
    TileSrc t;
    size_t mr = 0;
    if (!ring || !SK.ring || !SV.ring) mr = attn_main_row(S, g, p0, phys);
    const size_t rr = ring ? ring0 + __builtin_amdgcn_readfirstlane(p0 % max(S.kvrc, 1)) : 0;
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

// copies of one tile into the stage at LDS address `lds` (KB + VB + 1 copy instructions per lane).
// Full tiles copy contiguous bytes (one address add per instruction); the last, partial tile of a context clamps each
// 16-byte chunk to the last valid row.
// PART: 0 = the whole tile, 1 = the K rows and scales, 2 = the V rows and scales (two waves sharing one stage, each
// copying what it stores in a fused append)
template <int KB, int VB, int PART = 0>
__device__ __forceinline__ void issue_tile(const TileSrc & t, int nv, unsigned lds, int lane) {
    constexpr int KR = 2 * KB, VR = 2 * VB; // 16-byte chunks per row
    constexpr bool DK = PART != 2, DV = PART != 1;
    if (nv == ATP) {
        const unsigned off = 16 * lane;
        if constexpr (DK)
#pragma unroll
            for (int j = 0; j < KB; j++) dma16s(t.k + 1024 * j, off, lds + 1024 * j);
        if constexpr (DV)
#pragma unroll
            for (int j = 0; j < VB; j++) dma16s(t.v + 1024 * j, off, lds + 1024 * (KB + j));
    } else {
        if constexpr (DK)
#pragma unroll
            for (int j = 0; j < KB; j++) {
                int c = j * 64 + lane;
                const int r = c / KR;
                if (r >= nv) c = (nv - 1) * KR + (c - r * KR);
                dma16(t.k + 16 * c, lds + 1024 * j);
            }
        if constexpr (DV)
#pragma unroll
            for (int j = 0; j < VB; j++) {
                int c = j * 64 + lane;
                const int r = c / VR;
                if (r >= nv) c = (nv - 1) * VR + (c - r * VR);
                dma16(t.v + 16 * c, lds + 1024 * (KB + j));
            }
    }
    const int r = min(lane & 31, nv - 1);
    if constexpr (PART == 0) {
        dma16(lane < 32 ? static_cast<const void *>(t.ks + 8 * r) : static_cast<const void *>(t.vs + 8 * r), lds + 1024 * (KB + VB));
    } else if ((lane < 32) == (PART == 1)) { // half the lanes: the same LDS slots (lane-indexed) as the whole copy
        dma16(PART == 1 ? static_cast<const void *>(t.ks + 8 * r) : static_cast<const void *>(t.vs + 8 * r), lds + 1024 * (KB + VB));
    }
}

// a q8 tile through a stage smaller than one (three workgroups per CU): part 0 = the K rows at 0 and every scale at
// 8 KiB, part 1 = the V rows at 0 once the K operands are in registers; partial tiles clamp as issue_tile does
template <int PART>
__device__ __forceinline__ void issue_q8_part(const TileSrc & t, int nv, unsigned lds, int lane) {
    const uint8_t * const src = PART == 0 ? t.k : t.v;
    if (nv == ATP) {
        const unsigned off = 16 * lane;
#pragma unroll
        for (int j = 0; j < 8; j++) dma16s(src + 1024 * j, off, lds + 1024 * j);
    } else {
#pragma unroll
        for (int j = 0; j < 8; j++) {
            int c = j * 64 + lane;
            const int r = c / 16;
            if (r >= nv) c = (nv - 1) * 16 + (c - r * 16);
            dma16(src + 16 * c, lds + 1024 * j);
        }
    }
    if constexpr (PART == 0) {
        const int r = min(lane & 31, nv - 1);
        dma16(lane < 32 ? static_cast<const void *>(t.ks + 8 * r) : static_cast<const void *>(t.vs + 8 * r), lds + 8192);
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
// Query rows go in NP groups of 8 (NP = 1, 2 or 3: 8, 16 or 24 rows per pass).  Both MFMA products use the 16
// columns as (row, e) pairs, row = 8 h + n / 2 of group h and e = n % 2:
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

// wave issue priority 0..3 from the tiles a wave has left: the instruction arbiter otherwise favours the older
// workgroup on a CU, which then finishes early and leaves the younger one's waves to run the launch's tail alone.
// A uniform value; s_setprio takes an immediate.
__device__ __forceinline__ void set_prio(int left) {
    if (left >= 6) __builtin_amdgcn_s_setprio(3);
    else if (left >= 5) __builtin_amdgcn_s_setprio(2);
    else if (left >= 4) __builtin_amdgcn_s_setprio(1);
    else __builtin_amdgcn_s_setprio(0);
}

// ------------------------------------------------------------------------------------------------ the kernel
// More than 16 query rows (T >= 3) are held as 24 rows per wave (three groups; 48 rows of accumulators in one wave
// spill).  T = 3, 4: one 24-row pass.  T = 5..8: the WIDE kernel below, or (knob) batches of 24 rows: work item =
// (sequence, layer, kv head, segment, row batch), batch-minor, each batch streaming the segment's tiles again.  Every
// row sees the same slices, tile arithmetic and merge whatever T and whichever kernel.
// WIDE (25..48 rows, T = 5..8): one pass instead of two batches.  8 waves: waves w and w + 4 take the same slice of
// tiles (w, w + 4, ..) for rows 0..23 and 24..47, and share two stages per slice: at step i (after a workgroup barrier)
// tile i + 1 is copied into the other stage -- the K rows by the first wave of the pair, the V rows by the second --
// while both compute tile i.  A row's slices, tile arithmetic and merge order are those of the batched kernel.
// SMALL (one 8-row group, KB + VB <= 11): three workgroups per CU for launches with many work items.  The stages hold
// one packed tile (32 (KB + VB) + 1 KiB); a q8 window tile goes through in two halves (issue_q8_part); the V operands
// are read after the scores (168 registers).  Same slices and arithmetic: bitwise the same partials.
template <int NP, int KB, int VB, bool SMALL = false, bool WIDE = false>
__global__ __launch_bounds__(WIDE ? 512 : 256) __attribute__((amdgpu_waves_per_eu(SMALL ? 3 : 2, SMALL ? 3 : 2))) void k_attn(AttnArgs a) {
    static_assert(!SMALL || (NP == 1 && KB + VB <= 11), "small stages: one row group, packed tiles of at most 11 KiB");
    static_assert(!WIDE || NP == 3, "wide: two halves of 24 rows");
    constexpr int RP = 8 * NP;                // query rows held by a wave (the padding rows are zero)
    constexpr int NW = WIDE ? 2 * AWAVES : AWAVES, NQ = WIDE ? 2 * RP : RP; // waves, query rows of the workgroup
    constexpr int SB = SMALL ? 1024 * (KB + VB) + 1024 : STAGE_BYTES, SLDS = NW * SB; // stage bytes, all stages
    // NP = 3: the V operands are read from the stage after the scores (the stage is refilled only then), so a wave
    // never holds a whole raw tile in registers next to 24 rows of accumulators, and two workgroups fit a CU
    constexpr bool LATE_V = NP >= 3 || SMALL;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    // the wave index as a scalar: tile positions, page lookups and source selection stay scalar (SMEM loads, uniform
    // branches); vector loads there would need vmcnt waits that also drain the tile copies in flight
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63, n = lane & 15, q = lane >> 4;
    const int sl = WIDE ? wv & (AWAVES - 1) : wv, hf = WIDE ? wv / AWAVES : 0; // the wave's slice of tiles, row half
    const StoreLayout & S = a.S;
    const unsigned lds0 = (unsigned) (size_t) (__attribute__((address_space(3))) uint8_t *) smem;
    // stage b (0, 1) of the wave's slice: one per wave, or two per slice (WIDE)
    auto stage_of = [&](int b) { return WIDE ? 2 * sl + b : wv; };
    const unsigned st_lds = (unsigned) __builtin_amdgcn_readfirstlane(lds0 + wv * SB);
    half8 * const sQ = reinterpret_cast<half8 *>(smem + SLDS); // [NQ][256] fp16, chunk-swizzled (qchunk) per half
    const half8 * const sQh = sQ + hf * RP * (HD / 8);          // the wave's rows
    // The first tile copy of an item waits on every scalar load before it, and each round trip to the kernel arguments
    // costs a few hundred ns at launch: the common case (one sequence, one layer) needs one round -- the header, sd[0]
    // and side0 at fixed offsets, made live together by the empty asm so that the loads issue back to back and are
    // waited for once -- and only other sequences / layers add a second.
    const int n_items = a.n_items, n_base = a.n_base, nseq = a.nseq, kvrc = S.kvrc, spage = S.page;
    const SeqDesc sd0 = a.sd[0];
    const SideLayout K0 = a.side0[0], V0 = a.side0[1];
    asm volatile("" ::"s"(n_items), "s"(n_base), "s"(nseq), "s"(kvrc), "s"(spage), "s"(sd0.L), "s"(sd0.ws), "s"(sd0.cs), "s"(sd0.nseg),
                 "s"(sd0.item0), "s"(sd0.pbase), "s"(sd0.seq), "s"(K0.vals), "s"(K0.scs), "s"(K0.ring), "s"(K0.rsc), "s"(V0.vals),
                 "s"(V0.scs), "s"(V0.ring), "s"(V0.rsc), "s"(a.T), "s"(a.R), "s"(a.layer0), "s"(a.krot), "s"(a.qs), "s"(a.q),
                 "s"(a.qnw), "s"(a.rope), "s"(S.ptab), "s"(S.pt_stride));
    for (int bitem = blockIdx.x; bitem < n_items; bitem += gridDim.x) {
        const int nb = n_items / n_base, item = bitem / nb, batch = bitem - item * nb, row0 = RP * (WIDE ? hf : batch);
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
        const int seg = local % sd.nseg, lg = local / sd.nseg;
        const int g = lg % NKV, l = lg / NKV;
        const int L = sd.L, ws = sd.ws, seq = sd.seq, T = a.T;
        const int c0 = seg * sd.cs, c1 = min(L, c0 + sd.cs);
        const int ntiles = (c1 - c0 + ATP - 1) / ATP;
        const int my = ntiles > sl ? (ntiles - sl + AWAVES - 1) / AWAVES : 0; // tiles sl, sl+4, ..
        const int my0 = (ntiles + AWAVES - 1) / AWAVES;                       // steps of the workgroup (slice 0)
        SideLayout SK = K0, SV = V0;
        if (l > 0) {
            SK = S.side[a.layer0 + l][0];
            SV = S.side[a.layer0 + l][1];
        }
        const size_t ring0 = (size_t) (seq * NKV + g) * kvrc;

        // tile i of the wave starts at position c0 + 32 (sl + 4 i); phys: its physical page; into the stage at lds_to
        auto issue = [&](int i, int phys, unsigned lds_to) {
            const int p0 = c0 + ATP * (sl + AWAVES * i), nv = min(ATP, L - p0);
            const bool ring = S.kvrc > 0 && p0 >= ws; // the window: q8 rows (ring, or the main store of q8 sides)
            const TileSrc t = tile_src<KB, VB>(S, SK, SV, g, p0, phys, ring0, ring);
            int ln = lane; // opaque: the per-lane chunk addresses are not hoisted out of the tile loop into registers
            asm volatile("" : "+v"(ln));
            if constexpr (WIDE) {
                if (ring) {
                    if (hf == 0) issue_tile<8, 8, 1>(t, nv, lds_to, ln);
                    else issue_tile<8, 8, 2>(t, nv, lds_to, ln);
                } else {
                    if (hf == 0) issue_tile<KB, VB, 1>(t, nv, lds_to, ln);
                    else issue_tile<KB, VB, 2>(t, nv, lds_to, ln);
                }
            } else if (ring) {
                if constexpr (SMALL) issue_q8_part<0>(t, nv, lds_to, ln);
                else issue_tile<8, 8>(t, nv, lds_to, ln);
            } else {
                issue_tile<KB, VB>(t, nv, lds_to, ln);
            }
        };

        // physical page of tile i: the table is read only for sequences whose pages are not contiguous
        auto tile_page = [&](int i) {
            const int p = c0 + ATP * (sl + AWAVES * i);
            return sd.pbase >= 0 ? sd.pbase + __builtin_amdgcn_readfirstlane(p / spage) : page_of(S, seq, p);
        };
        int phys_cur = my > 0 ? tile_page(0) : 0; // page of the tile in the stage (tile i while step i runs)
        // fused append: this wave's tiles that hold new positions (L - T .. L - 1) are copied only after the wave has
        // stored those rows (the vmcnt wait before the copy covers the stores); a new row in tile 0 is stored first
        int new_tile0 = my; // the wave's first tile holding a new position
        if (a.kin) {
            const int pa = max(L - T, c0), pb = min(L, c1);
            for (int p = pa; p < pb; p++)
                if (((p - c0) >> 5) % AWAVES == sl) new_tile0 = min(new_tile0, ((p - c0) >> 5) / AWAVES);
        }
        auto append_rows = [&]() {
            const int pa = max(L - T, c0), pb = min(L, c1);
            for (int p = pa; p < pb; p++) {
                if (((p - c0) >> 5) % AWAVES != sl) continue;
                const size_t row = ((((size_t) si * T + (p - (L - T))) * a.kin_nl + l) * NKV + g) * HD;
#pragma unroll
                for (int w = 0; w < 2; w++) {
                    if (WIDE && w != hf) continue; // (the pair's first wave stores K, the second V)
                    float v[4];
                    load_row4(w ? a.vin : a.kin, row, a.kin_f16, v);
                    store_row(S, w ? SV : SK, seq, g, p, true, v);
                }
            }
        };
        // ---- queries: FWHT when K is stored rotated, * 1/16, fp16 (qwen38_mk.cu:2873-2880), rows r = hh T + t.  The
        // wave's rows are loaded before its first tile copy and waited for alone (loads return in order: vmcnt at most
        // the copy count), so they are converted while tile 0 streams.  Only the copy issue runs between the loads and
        // the wait (the loaded registers must not be read or moved before it).
        if (new_tile0 == 0) {
            append_rows();
            vm_wait<0>(); // the stored rows are in L2 before this wave's copies read them
        }
        const int qrow0 = WIDE ? 0 : row0; // the workgroup's first row
        constexpr int QPW = NQ / NW;       // rows per wave
        f32x4 qx[QPW];
#pragma unroll
        for (int j = 0; j < QPW; j++) {
            const int r = qrow0 + wv + NW * j;
            if (r < a.R) {
                const int hh = r / T, t = r % T;
                qx[j] = gload16(a.q + (((size_t) (l * a.nseq + si) * T + t) * NH + GQA * g + hh) * a.qs + 4 * lane);
            } else {
                qx[j] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
        }
        if (my > 0) {
            issue(0, phys_cur, lds0 + stage_of(0) * SB);
            // copy instructions of tile 0 (issue_tile / issue_q8_part): every load before them has returned
            const bool ring = S.kvrc > 0 && c0 + ATP * sl >= ws;
            if constexpr (WIDE) {
                if (hf == 0) {
                    if (ring) vm_wait<8 + 1>();
                    else vm_wait<KB + 1>();
                } else {
                    if (ring) vm_wait<8 + 1>();
                    else vm_wait<VB + 1>();
                }
            } else if (ring) {
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
            const int r = wv + NW * j, gr = qrow0 + r;
            half2v o0 = {(_Float16) 0.f, (_Float16) 0.f}, o1 = o0;
            if (gr < a.R) {
                const int t = gr % T;
                float v[4] = {qx[j][0], qx[j][1], qx[j][2], qx[j][3]};
                if (a.qnw) qk_prep(v, a.qnw + (size_t) l * HD, a.rope + (size_t) (L - T + t) * 32);
                if ((a.krot >> (a.layer0 + l)) & 1u) fwht256_w64(v);
                o0[0] = (_Float16) (v[0] * 0.0625f);
                o0[1] = (_Float16) (v[1] * 0.0625f);
                o1[0] = (_Float16) (v[2] * 0.0625f);
                o1[1] = (_Float16) (v[3] * 0.0625f);
            }
            reinterpret_cast<uint2 *>(sQ + (r / RP) * RP * (HD / 8) + qchunk(r % RP, lane >> 1))[lane & 1] = make_uint2(as_u(o0), as_u(o1));
        }
        if (new_tile0 > 0 && new_tile0 < my) append_rows(); // stored while the first tiles stream
        WaveState<NP> st;
#pragma unroll
        for (int h = 0; h < NP; h++) {
            st.m[h] = -INFINITY;
            st.l[h] = 0.f;
            const int row = row0 + 8 * h + (n >> 1);
            st.lim[h] = row < a.R ? L - T + row % T : -1;
#pragma unroll
            for (int b = 0; b < 8; b++) st.acc[h][b] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
        st.lim_min = L - T;
        __syncthreads(); // the query rows are complete
        if constexpr (NP == 1) {
#pragma unroll
            for (int ks = 0; ks < 8; ks++) st.qf[ks] = sQh[qchunk(n >> 1, 8 * q + ks)];
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
                    const TileSrc t = tile_src<KB, VB>(S, SK, SV, g, p0, phys_cur, ring0, true);
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
            } else if constexpr (LATE_V) {
                read_k<K2, V2>(raw, stp, n, q);
                compute_tile<NP, K2, V2, true>(
                    st, sQ, p0, raw, [&](RawTile<K2, V2> & r, int tn, int tq) { read_v<K2, V2>(r, stp, tn, tq); },
                    [&]() {
                        if (i + 1 < my) issue(i + 1, phys_next, st_lds);
                    });
            } else {
                read_k<K2, V2>(raw, stp, n, q);
                read_v<K2, V2>(raw, stp, n, q);
                lds_drain();
                if (i + 1 < my) issue(i + 1, phys_next, st_lds);
                compute_tile<NP, K2, V2>(st, sQ, p0, raw);
            }
            phys_cur = phys_next;
        };
        // WIDE: one workgroup barrier per step; tile i + 1 streams into the slice's other stage during tile i's math
        auto wstep = [&](auto fmt, int i) {
            constexpr int K2 = decltype(fmt)::kb, V2 = decltype(fmt)::vb;
            set_prio(my - i);
            const int phys_next = i + 1 < my ? tile_page(i + 1) : 0;
            vm_wait<0>();    // this wave's half of tile i has landed
            __syncthreads(); // both halves of every slice's tile i are staged; every wave is done with tile i - 1
            if (i + 1 < my) issue(i + 1, phys_next, lds0 + stage_of((i + 1) & 1) * SB);
            if (i < my) {
                const uint8_t * const sp = smem + stage_of(i & 1) * SB;
                RawTile<K2, V2> raw;
                read_k<K2, V2>(raw, sp, n, q);
                compute_tile<NP, K2, V2, true>(st, sQh, c0 + ATP * (sl + AWAVES * i), raw,
                                               [&](RawTile<K2, V2> & r, int tn, int tq) { read_v<K2, V2>(r, sp, tn, tq); });
            }
            phys_cur = phys_next;
        };
        // the wave's window (ring) tiles are its last ones: i >= i_ring, p0 >= ws.  Two loops, one tile format each,
        // keep a single tile body live per loop (one body holding both formats costs registers)
        int i_ring = my;
        if (S.kvrc > 0) {
            const int d = ws - c0 - ATP * sl;
            i_ring = d <= 0 ? 0 : min(my, (d + AWAVES * ATP - 1) / (AWAVES * ATP));
        }
        int i = 0;
        if constexpr (WIDE) { // every wave takes part in the my0 barriers
            for (; i < i_ring; i++) wstep(Fmt<KB, VB>(), i);
            for (; i < my0; i++) wstep(Fmt<8, 8>(), i);
        } else {
            for (; i < i_ring; i++) step(Fmt<KB, VB>(), i);
            for (; i < my; i++) step(Fmt<8, 8>(), i);
        }
        // ---- merge the 4 waves (slices) of each row in order: M = max m_w, O = sum e_w O_w, l = sum e_w l_w.  Per pass
        // of 16 rows (two groups) every wave writes its scaled O rows to its own LDS buffer (the stages are free), then
        // each thread adds the 4 buffers of its rows' waves in slice order.
        constexpr int OLD = HD + 4;                                           // row stride (floats) of a buffer
        constexpr int MR = NP == 1 ? 8 : 16;                                  // rows per wave buffer
        float * const s_m = reinterpret_cast<float *>(smem + NW * MR * OLD * 4); // [NW][RP]
        float * const s_l = s_m + NW * RP;                                    // [NW][RP]
        static_assert(NW * MR * OLD * 4 + 2 * NW * RP * 4 <= SLDS, "merge buffers inside the stages");
        __syncthreads(); // every wave is done with its stage
        if (q == 0 && !(n & 1)) {
#pragma unroll
            for (int h = 0; h < NP; h++) {
                s_m[wv * RP + 8 * h + (n >> 1)] = st.m[h];
                s_l[wv * RP + 8 * h + (n >> 1)] = st.l[h];
            }
        }
        __syncthreads();
        const int R = a.R;
        // the merging thread's half (WIDE: threads 256 h .. 256 h + 255 add the buffers of waves 4 h .. 4 h + 3)
        const int th = WIDE ? threadIdx.x / 256 : 0, tl = threadIdx.x - 256 * th, wb = AWAVES * th;
        const int trow0 = WIDE ? RP * th : row0, RB = min(RP, R - trow0); // its rows
        const float * const s_mh = s_m + wb * RP, * const s_mw = s_m + hf * AWAVES * RP; // the thread's / the wave's half
        constexpr int NPASS = (NP + 1) / 2;
#pragma unroll
        for (int ps = 0; ps < NPASS; ps++) {
#pragma unroll
            for (int hh = 0; hh < 2; hh++) {
                const int h = 2 * ps + hh;
                if (h < NP) {
                    const int row = 8 * h + (n >> 1);
                    const float M = fmaxf(fmaxf(s_mw[row], s_mw[RP + row]), fmaxf(s_mw[2 * RP + row], s_mw[3 * RP + row]));
                    const float e = st.m[h] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(st.m[h] - M);
                    float * o = reinterpret_cast<float *>(smem) + (wv * MR + 8 * hh + (n >> 1)) * OLD + 64 * q + (n & 1);
#pragma unroll
                    for (int b = 0; b < 8; b++)
#pragma unroll
                        for (int i = 0; i < 4; i++) o[16 * i + 2 * b] = e * st.acc[h][b][i];
                }
            }
            __syncthreads();
            const int nrow = min(16, RB - 16 * ps);
            for (int idx = tl; idx < nrow * (HD / 4); idx += 256) {
                const int r16 = idx / (HD / 4), c4 = idx % (HD / 4);
                const float * src = reinterpret_cast<const float *>(smem) + (wb * MR + r16) * OLD + 4 * c4;
                float4 y = *reinterpret_cast<const float4 *>(src);
#pragma unroll
                for (int w = 1; w < AWAVES; w++) {
                    const float4 z = *reinterpret_cast<const float4 *>(src + w * MR * OLD);
                    y.x += z.x;
                    y.y += z.y;
                    y.z += z.z;
                    y.w += z.w;
                }
                *reinterpret_cast<float4 *>(a.part + ((size_t) item * R + trow0 + 16 * ps + r16) * HD + 4 * c4) = y;
            }
            if (ps + 1 < NPASS) __syncthreads();
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
        __syncthreads(); // the LDS is reused by the next item
    }
}

// ------------------------------------------------------------------------------------------------ prefetch
// The first `tiles` tiles of every wave slice of an attention launch's work items copied into LDS and dropped: the
// bytes pass through the L2 of the XCD that workgroup x runs on, and the attention launch with the same arguments puts
// work item x on workgroup x -- the same XCD (workgroups go round-robin over the XCDs by index) -- so its first tile
// copies hit that L2 (or the last-level cache) instead of HBM.  No results: issued ahead of the attention, on another
// stream beside independent work (the reference's pf_l2 in attn_proj, qwen38_mk.cu:2600-2621).
template <int KB, int VB>
__global__ __launch_bounds__(256) void k_prefetch(AttnArgs a, int tiles) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const StoreLayout & S = a.S;
    const unsigned st_lds = (unsigned) __builtin_amdgcn_readfirstlane((unsigned) (size_t) (__attribute__((address_space(3))) uint8_t *) smem + wv * STAGE_BYTES);
    for (int item = blockIdx.x; item < a.n_items; item += gridDim.x) {
        int si = 0;
        for (int i = 1; i < a.nseq; i++)
            if (item >= a.sd[i].item0) si = i;
        const SeqDesc sd = a.sd[si];
        const int local = item - sd.item0, seg = local % sd.nseg, lg = local / sd.nseg, g = lg % NKV, l = lg / NKV;
        const int c0 = seg * sd.cs, c1 = min(sd.L, c0 + sd.cs), ntiles = (c1 - c0 + ATP - 1) / ATP;
        const SideLayout SK = S.side[a.layer0 + l][0], SV = S.side[a.layer0 + l][1];
        const size_t ring0 = (size_t) (sd.seq * NKV + g) * S.kvrc;
        for (int i = 0; i < tiles; i++) {
            const int tix = wv + AWAVES * i;
            if (tix >= ntiles) break;
            const int p0 = c0 + ATP * tix, nv = min(ATP, sd.L - p0);
            const int phys = sd.pbase >= 0 ? sd.pbase + p0 / S.page : page_of(S, sd.seq, p0);
            const bool ring = S.kvrc > 0 && p0 >= sd.ws;
            const TileSrc t = tile_src<KB, VB>(S, SK, SV, g, p0, phys, ring0, ring);
            if (ring) issue_tile<8, 8>(t, nv, st_lds, lane);
            else issue_tile<KB, VB>(t, nv, st_lds, lane);
            vm_wait<0>(); // (the stage is reused by the next copy)
        }
    }
}

// ------------------------------------------------------------------------------------------------ output epilogue
// One output row y (head h of token row trow, lane l holding dims 4l .. 4l+3) after the merge: the V un-rotation when
// V is stored rotated, the sigmoid output gate (qwen38_mk.cu:4686) when grow is given, the fp32 store, and when q32a
// is given the o_proj activation units of q32_store (qwen38_mk.cu:283-307): block k = lane / 8 of the head's 8 blocks of
// 32 (j = 8 h + k), amax / 127, round half away from zero; unit gi = 8 h + 2 (k / 2) + half, bytes of the even blocks
// in a, odd ones in b.  All 64 lanes of the wave call it.
__device__ __forceinline__ void finish_row(float (&v)[4], bool vrot, const float * grow, float * orow, int8_t * q32a, int8_t * q32b,
                                           uint16_t * q32m, size_t trow, int h) {
    const int lane = lane_id();
    if (vrot) fwht256_w64(v);
    if (grow) {
        const float4 gt = *reinterpret_cast<const float4 *>(grow + 4 * lane);
        v[0] = v[0] / (1.0f + expf(-gt.x));
        v[1] = v[1] / (1.0f + expf(-gt.y));
        v[2] = v[2] / (1.0f + expf(-gt.z));
        v[3] = v[3] / (1.0f + expf(-gt.w));
    }
    *reinterpret_cast<float4 *>(orow + 4 * lane) = make_float4(v[0], v[1], v[2], v[3]);
    if (q32a) {
        float am = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
        am = fmaxf(am, shfl_xor(am, 1));
        am = fmaxf(am, shfl_xor(am, 2));
        am = fmaxf(am, shfl_xor(am, 4));
        const float d = am / 127.0f;
        int qv[4];
#pragma unroll
        for (int k = 0; k < 4; k++) qv[k] = am == 0.0f ? 0 : (int) roundf(v[k] / d);
        const int k8 = lane >> 3, part = k8 & 1, hh = (lane >> 2) & 1;
        const size_t gi = trow * 192 + 8 * h + 2 * (k8 >> 1) + hh;
        const unsigned packed = (qv[0] & 0xff) | (qv[1] & 0xff) << 8 | (qv[2] & 0xff) << 16 | (unsigned) (qv[3] & 0xff) << 24;
        *reinterpret_cast<unsigned *>((part ? q32b : q32a) + gi * 16 + 4 * (lane & 3)) = packed;
        int sum = qv[0] + qv[1] + qv[2] + qv[3];
        sum += __shfl_xor(sum, 1, 64);
        sum += __shfl_xor(sum, 2, 64);
        if ((lane & 3) == 0) {
            q32m[gi * 4 + part] = f2h_bits(d);
            q32m[gi * 4 + 2 + part] = (uint16_t) (int16_t) sum;
        }
    }
}

// ------------------------------------------------------------------------------------------------ combine
// The merge of a head's segment partials (attn_combine, qwen38_mk.cu:4617-4700: y = sum_c e_c O_c / sum_c e_c l_c with
// e_c = exp(m_c - M)), in two forms with fixed orders (no bit depends on scheduling):
//   row form   (combine_row)  one workgroup per output row (layer, sequence, kv head, row r).  Wave w loads the
//              segments c = w, w+4, .. at once, weights them by exp2(m_c - M_w) against its own maximum M_w and sums
//              them in segment order; the four wave sums are rescaled to M = max M_w and added in wave order; y = O / l,
//              then the V un-rotation, gate and o_proj units (finish_row).
//   split form (combine_split) one workgroup per (output row, 64-dim quarter), for launches without rotated V, gate or
//              units.  Lane group s = 4 w + l / 16 takes the segments c = s, s + 16, .. and sums them the same way;
//              the 4 groups of a wave are merged by permlane swaps, the 4 waves in wave order.
// Both run as a kernel of their own after the attention launch (an in-launch merge by extra workgroups that wait for
// a head's segments measured slower: partials then have to be written through to the coherence point shared by the
// XCDs before the waiting workgroup may read them).  scratch: LDS of 4 KiB + 32 B.
// the output row of combine workgroup b of a launch: (layer, sequence, kv head, row r) with r fastest
struct CombineRow {
    int l, si, g, r;
};
__device__ __forceinline__ CombineRow combine_row_of(const AttnArgs & a, int b) {
    CombineRow c;
    c.r = b % a.R;
    b /= a.R;
    c.g = b % NKV;
    b /= NKV;
    c.si = b % a.nseq;
    c.l = b / a.nseq;
    return c;
}

__device__ __forceinline__ void combine_row(const AttnArgs & a, const CombineRow & cr, uint8_t * scratch) {
    float4 (*s_num)[64] = reinterpret_cast<float4 (*)[64]>(scratch);         // [AWAVES][64]
    float2 * s_md = reinterpret_cast<float2 *>(scratch + AWAVES * 64 * 16); // [AWAVES] (max, denominator)
    const int R = a.R, T = a.T, r = cr.r, g = cr.g, si = cr.si, l = cr.l;
    const SeqDesc & sd = a.sd[si];
    const int nseg = sd.nseg;
    const size_t head0 = (size_t) sd.item0 + (size_t) (l * NKV + g) * nseg;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    // one round of loads: wave w's segments c = w, w + 4, .. (all issued before any is used)
    constexpr int PER = MAX_SEG / AWAVES;
    float2 ml[PER];
    float4 o[PER];
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const int c = wv + AWAVES * k;
        if (c < nseg) {
            ml[k] = a.ml[(head0 + c) * R + r];
            o[k] = *reinterpret_cast<const float4 *>(a.part + ((head0 + c) * R + r) * HD + 4 * lane);
        }
    }
    float Mw = -INFINITY;
#pragma unroll
    for (int k = 0; k < PER; k++)
        if (wv + AWAVES * k < nseg) Mw = fmaxf(Mw, ml[k].x);
    float4 num = make_float4(0.f, 0.f, 0.f, 0.f);
    float den = 0.f;
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const int c = wv + AWAVES * k;
        if (c < nseg) {
            const float e = ml[k].x == -INFINITY ? 0.f : exp2f(ml[k].x - Mw);
            num.x = __builtin_fmaf(e, o[k].x, num.x);
            num.y = __builtin_fmaf(e, o[k].y, num.y);
            num.z = __builtin_fmaf(e, o[k].z, num.z);
            num.w = __builtin_fmaf(e, o[k].w, num.w);
            den = __builtin_fmaf(e, ml[k].y, den);
        }
    }
    s_num[wv][lane] = num;
    if (lane == 0) s_md[wv] = make_float2(Mw, den);
    __syncthreads();
    if (wv == 0) {
        // the 4 wave sums in wave order, each rescaled to the overall max
        float M = s_md[0].x;
#pragma unroll
        for (int k = 1; k < AWAVES; k++) M = fmaxf(M, s_md[k].x);
        float4 y = make_float4(0.f, 0.f, 0.f, 0.f);
        float dd = 0.f;
#pragma unroll
        for (int k = 0; k < AWAVES; k++) {
            const float2 md = s_md[k];
            const float e = md.x == -INFINITY ? 0.f : exp2f(md.x - M);
            const float4 z = s_num[k][lane];
            y.x = __builtin_fmaf(e, z.x, y.x);
            y.y = __builtin_fmaf(e, z.y, y.y);
            y.z = __builtin_fmaf(e, z.z, y.z);
            y.w = __builtin_fmaf(e, z.w, y.w);
            dd = __builtin_fmaf(e, md.y, dd);
        }
        float v[4] = {y.x / dd, y.y / dd, y.z / dd, y.w / dd};
        const int h = GQA * g + r / T, t = r % T;
        const size_t trow = (size_t) (l * a.nseq + si) * T + t; // the token's row of 24 x 256 outputs
        finish_row(v, (a.vrot >> (a.layer0 + l)) & 1u, a.gate ? a.gate + (trow * NH + h) * a.gs : nullptr, a.out + (trow * NH + h) * HD,
                   a.q32a, a.q32b, a.q32m, trow, h);
    }
}

__device__ __forceinline__ void combine_split(const AttnArgs & a, const CombineRow & cr, int dq, uint8_t * scratch) {
    float4 (*s_num)[16] = reinterpret_cast<float4 (*)[16]>(scratch);        // [AWAVES][16]
    float2 * s_md = reinterpret_cast<float2 *>(scratch + AWAVES * 16 * 16); // [AWAVES]
    const int R = a.R, T = a.T, r = cr.r, g = cr.g, si = cr.si, l = cr.l;
    const SeqDesc & sd = a.sd[si];
    const int nseg = sd.nseg;
    const size_t head0 = (size_t) sd.item0 + (size_t) (l * NKV + g) * nseg;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, sub = lane >> 4, dl = lane & 15;
    const int slot = 4 * wv + sub, dim = 64 * dq + 4 * dl;
    constexpr int PER = MAX_SEG / 16;
    float2 ml[PER];
    float4 o[PER];
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const int c = slot + 16 * k;
        if (c < nseg) {
            ml[k] = a.ml[(head0 + c) * R + r];
            o[k] = *reinterpret_cast<const float4 *>(a.part + ((head0 + c) * R + r) * HD + dim);
        }
    }
    float Ms = -INFINITY;
#pragma unroll
    for (int k = 0; k < PER; k++)
        if (slot + 16 * k < nseg) Ms = fmaxf(Ms, ml[k].x);
    float4 num = make_float4(0.f, 0.f, 0.f, 0.f);
    float den = 0.f;
#pragma unroll
    for (int k = 0; k < PER; k++) {
        if (slot + 16 * k < nseg) {
            const float e = ml[k].x == -INFINITY ? 0.f : exp2f(ml[k].x - Ms);
            num.x = __builtin_fmaf(e, o[k].x, num.x);
            num.y = __builtin_fmaf(e, o[k].y, num.y);
            num.z = __builtin_fmaf(e, o[k].z, num.z);
            num.w = __builtin_fmaf(e, o[k].w, num.w);
            den = __builtin_fmaf(e, ml[k].y, den);
        }
    }
    // the wave's 4 lane groups (same dims, slots 4 w .. 4 w + 3)
    const float Mw = quad_max(Ms);
    const float ew = Ms == -INFINITY ? 0.f : exp2f(Ms - Mw);
    num.x = quad_sum(ew * num.x);
    num.y = quad_sum(ew * num.y);
    num.z = quad_sum(ew * num.z);
    num.w = quad_sum(ew * num.w);
    den = quad_sum(ew * den);
    if (sub == 0) s_num[wv][dl] = num;
    if (lane == 0) s_md[wv] = make_float2(Mw, den);
    __syncthreads();
    if (wv == 0 && sub == 0) {
        float M = s_md[0].x;
#pragma unroll
        for (int k = 1; k < AWAVES; k++) M = fmaxf(M, s_md[k].x);
        float4 y = make_float4(0.f, 0.f, 0.f, 0.f);
        float dd = 0.f;
#pragma unroll
        for (int k = 0; k < AWAVES; k++) {
            const float2 md = s_md[k];
            const float e = md.x == -INFINITY ? 0.f : exp2f(md.x - M);
            const float4 z = s_num[k][dl];
            y.x = __builtin_fmaf(e, z.x, y.x);
            y.y = __builtin_fmaf(e, z.y, y.y);
            y.z = __builtin_fmaf(e, z.z, y.z);
            y.w = __builtin_fmaf(e, z.w, y.w);
            dd = __builtin_fmaf(e, md.y, dd);
        }
        const int h = GQA * g + r / T, t = r % T;
        *reinterpret_cast<float4 *>(a.out + (((size_t) (l * a.nseq + si) * T + t) * NH + h) * HD + dim) =
            make_float4(y.x / dd, y.y / dd, y.z / dd, y.w / dd);
    }
}

__global__ __launch_bounds__(256) void k_combine(AttnArgs a) {
    __shared__ __attribute__((aligned(16))) uint8_t scratch[AWAVES * 64 * 16 + AWAVES * 8];
    combine_row(a, combine_row_of(a, blockIdx.x), scratch);
}

__global__ __launch_bounds__(256) void k_combine_split(AttnArgs a) {
    __shared__ __attribute__((aligned(16))) uint8_t scratch[AWAVES * 16 * 16 + AWAVES * 8];
    combine_split(a, combine_row_of(a, blockIdx.x >> 2), blockIdx.x & 3, scratch);
}

// launches whose rows need the whole row in one workgroup (V stored rotated, gate, o_proj units) use the row form
static bool host_combine_needs_rows(const AttnArgs & a) {
    const unsigned vrot = (a.vrot >> a.layer0) & ((a.nl >= 32 ? 0u : 1u << a.nl) - 1u);
    return vrot || a.gate || a.q32a;
}

hipError_t launch_combine(const AttnArgs & a, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1) {
    const unsigned rows = (unsigned) (a.nl * a.nseq * NKV * a.R);
    if (host_combine_needs_rows(a)) hipExtLaunchKernelGGL(k_combine, dim3(rows), dim3(256), 0, st, ev0, ev1, 0, a);
    else hipExtLaunchKernelGGL(k_combine_split, dim3(4 * rows), dim3(256), 0, st, ev0, ev1, 0, a);
    return hipGetLastError();
}

// ------------------------------------------------------------------------------------------------ prefill
// Causal attention of one prefill piece (pk_attn8's exact form, prefill_attn.cuh:698-702; pieces and window
// prefill_host.cu:606-615).  Keys are cut into absolute segments of a.seg positions (a function of the row's bucket); a
// row's partial for segment k is one online softmax over the segment's tiles in order, and the combine folds the row's
// segments 0 .. pos / a.seg in order: each output is a function of its position and the store only, whatever the
// chunking of the prefill.

// 32 values of scale block b (dims 32 b .. 32 b + 31) of one staged row of B bits -> 16 fp16 pairs fp16_rn(d q), the
// same values as the decode operands (kfrag)
template <int B>
__device__ __forceinline__ void dequant_block(const uint8_t * row, uint16_t sc, int b, half2v (&o)[16]) {
    const half2v d2 = as_h2((unsigned) sc * 0x10001u);
    constexpr float bias = B == 8 ? 1152.f : (float) (1024 + (1 << (B - 1)));
    const half2v b2 = {(_Float16) -bias, (_Float16) -bias};
#pragma unroll
    for (int w = 0; w < 4; w++) {
        unsigned lo, hi;
        if constexpr (B == 8) {
            const uint2 x = *reinterpret_cast<const uint2 *>(row + 32 * b + 8 * w);
            lo = x.x ^ 0x80808080u;
            hi = x.y ^ 0x80808080u;
        } else {
            constexpr int HB = B - 4;
            const int word = 4 * b + w;
            const unsigned W = *reinterpret_cast<const unsigned *>(row + 4 * word);
            unsigned H = 0;
#pragma unroll
            for (int k = 0; k < HB; k++) H |= (unsigned) row[128 + word * HB + k] << (8 * k);
            word_codes<B>(W, H, lo, hi);
        }
        o[4 * w] = (as_h2(perm_b32(lo, C64, 0x00050004u)) + b2) * d2;
        o[4 * w + 1] = (as_h2(perm_b32(lo, C64, 0x00070006u)) + b2) * d2;
        o[4 * w + 2] = (as_h2(perm_b32(hi, C64, 0x00050004u)) + b2) * d2;
        o[4 * w + 3] = (as_h2(perm_b32(hi, C64, 0x00070006u)) + b2) * d2;
    }
}

// fp16 tile layouts in LDS: K [32][SK_LD] (row = position), V transposed [256][SVT_LD] (row = dim) with the positions in
// the order of the P V operands (position bits 2 and 3 swapped)
constexpr int SK_LD = HD + 8;
constexpr int SVT_LD = ATP + 8;
typedef float f32x16 __attribute__((ext_vector_type(16)));

// Prefill attention on 32x32x16 MFMAs: workgroup = (128 query rows, kv head, key segment), row block fastest so the
// workgroups of one segment run side by side; 8 waves.  Waves 0-3 (consumers) hold 32 query
// rows each and run the MFMAs and the softmax on the fp16 tile of buffer i % 2; waves 4-7 (producers) each copy an
// 8-position quarter of the tiles (two tiles in flight) and dequantize exactly what they copied into the other
// buffer.  One barrier per tile hands a buffer over; on each SIMD a producer's VALU work overlaps a consumer's MFMAs.
constexpr int PQ_REGION = 5120;                           // per producer and stage: K rows 2 KB, V rows 2 KB, scales 1 KB
constexpr int PQ_STAGES = 2 * 4 * PQ_REGION;              // two stages of the 4 producers
constexpr int PQ_BUF = (ATP * SK_LD + HD * SVT_LD + 64) * 2; // one fp16 tile: K [32][SK_LD], V^T [256][SVT_LD] + skew
// V^T row r starts at r SVT_LD + 8 (r / 32): the 8 rows a producer wave writes at once (32 apart) fall in different banks
constexpr int PQ_LDS = PQ_STAGES + 2 * PQ_BUF;
static_assert(PQ_LDS >= PF2_ROWS * SK_LD * 2, "query staging inside the tile buffers");

// the 8 positions of quarter pw of tile i: one producer wave's copies (5 instructions, always) into its region
template <int KB, int VB>
__device__ __forceinline__ void pq_issue(const TileSrc & t, int nq, unsigned lds, int lane) {
    constexpr int KRB = 32 * KB, VRB = 32 * VB; // row bytes
#pragma unroll
    for (int j = 0; j < 2; j++) {
        int o = 1024 * j + 16 * lane;
        if (o >= nq * KRB) o = nq * KRB - 16;
        dma16(t.k + o, lds + 1024 * j);
    }
#pragma unroll
    for (int j = 0; j < 2; j++) {
        int o = 1024 * j + 16 * lane;
        if (o >= nq * VRB) o = nq * VRB - 16;
        dma16(t.v + o, lds + 2048 + 1024 * j);
    }
    const int r = min(lane & 7, nq - 1);
    dma16(lane < 8 ? static_cast<const void *>(t.ks + 8 * r) : static_cast<const void *>(t.vs + 8 * r), lds + 4096);
}

// one producer lane: position lane % 8 of its quarter, scale block lane / 8, K and V into the fp16 buffer
template <int KB, int VB>
__device__ __forceinline__ void pq_dequant(const uint8_t * reg, int pw, int lane, _Float16 * sK, _Float16 * sVt) {
    const int pl = lane & 7, b = lane >> 3, p = 8 * pw + pl;
    const uint16_t * ksc = reinterpret_cast<const uint16_t *>(reg + 4096);
    half2v o[16];
    dequant_block<KB>(reg + pl * 32 * KB, ksc[pl * 8 + b], b, o);
    uint4 * kd = reinterpret_cast<uint4 *>(sK + p * SK_LD + 32 * b);
#pragma unroll
    for (int k = 0; k < 4; k++) kd[k] = make_uint4(as_u(o[4 * k]), as_u(o[4 * k + 1]), as_u(o[4 * k + 2]), as_u(o[4 * k + 3]));
    dequant_block<VB>(reg + 2048 + pl * 32 * VB, ksc[64 + pl * 8 + b], b, o);
    const int x = (p & ~12) | ((p >> 1) & 4) | ((p << 1) & 8);
    _Float16 * vd = sVt + (32 * b) * SVT_LD + 8 * b + x;
#pragma unroll
    for (int k = 0; k < 16; k++) {
        vd[(2 * k) * SVT_LD] = o[k][0];
        vd[(2 * k + 1) * SVT_LD] = o[k][1];
    }
}

template <int KB, int VB>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_prefill3(PrefillArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63, c = lane & 31, hf = lane >> 5;
    const bool producer = wv >= 4;
    const int pw = wv - 4;
    const StoreLayout & S = a.S;
    int bi = blockIdx.x;
    const int rb = bi % a.nrb;
    bi /= a.nrb;
    const int g = bi % NKV, k = bi / NKV;
    const int r0 = PF2_ROWS * rb, rlast = min(a.R, r0 + PF2_ROWS) - 1;
    const int pmax = a.n0 + rlast / GQA;
    const int c0 = k * a.seg;
    if (c0 > pmax) return;
    const int c1 = min(c0 + a.seg, pmax + 1);
    const int ntiles = (c1 - c0 + ATP - 1) / ATP;
    const unsigned lds0 = (unsigned) (size_t) (__attribute__((address_space(3))) uint8_t *) smem;
    _Float16 * const buf0 = reinterpret_cast<_Float16 *>(smem + PQ_STAGES);
    const SideLayout & SK = S.side[a.layer][0];
    const SideLayout & SV = S.side[a.layer][1];
    const size_t ring0 = (size_t) (a.seq * NKV + g) * S.kvrc;
    const int L = a.L, ws = a.ws;
    auto is_ring = [&](int i) { return S.kvrc > 0 && c0 + ATP * i >= ws; };
    // producer: the copies of quarter pw of tile i into stage i % 2
    auto issue = [&](int i) {
        const int p0t = c0 + ATP * i, nv = min(ATP, L - p0t);
        const int q0 = min(8 * pw, nv - 1), nq = min(8, nv - q0), p0 = p0t + q0;
        const unsigned lds = (unsigned) __builtin_amdgcn_readfirstlane(lds0 + ((i & 1) * 4 + pw) * PQ_REGION);
        const bool ring = is_ring(i);
        const TileSrc t = tile_src<KB, VB>(S, SK, SV, g, p0, page_of(S, a.seq, p0), ring0, ring);
        if (ring) pq_issue<8, 8>(t, nq, lds, lane);
        else pq_issue<KB, VB>(t, nq, lds, lane);
    };
    auto dequant = [&](int i) {
        const uint8_t * reg = smem + ((i & 1) * 4 + pw) * PQ_REGION;
        _Float16 * sK = buf0 + (i & 1) * (PQ_BUF / 2);
        _Float16 * sVt = sK + ATP * SK_LD;
        if (is_ring(i)) pq_dequant<8, 8>(reg, pw, lane, sK, sVt);
        else pq_dequant<KB, VB>(reg, pw, lane, sK, sVt);
    };
    // ---- query rows: all 8 waves stage 16 rows each (prep, FWHT for rotated K, * 1/16, fp16), consumers take fragments
    _Float16 * const qs = reinterpret_cast<_Float16 *>(smem);
    for (int j = 0; j < 16; j++) {
        const int rl = 16 * wv + j, r = r0 + rl;
        half2v o0 = {(_Float16) 0.f, (_Float16) 0.f}, o1 = o0;
        if (r < a.R) {
            const int t = r / GQA, hh = r - GQA * t;
            const float4 x = *reinterpret_cast<const float4 *>(a.q + ((size_t) t * NH + GQA * g + hh) * a.qs + 4 * lane);
            float v[4] = {x.x, x.y, x.z, x.w};
            if (a.qnw) qk_prep(v, a.qnw, a.rope + (size_t) (a.n0 + t) * 32);
            if (a.krot) fwht256_w64(v);
            o0[0] = (_Float16) (v[0] * 0.0625f);
            o0[1] = (_Float16) (v[1] * 0.0625f);
            o1[0] = (_Float16) (v[2] * 0.0625f);
            o1[1] = (_Float16) (v[3] * 0.0625f);
        }
        *reinterpret_cast<uint2 *>(qs + rl * SK_LD + 4 * lane) = make_uint2(as_u(o0), as_u(o1));
    }
    __syncthreads();
    // Both roles pass the same barriers: two after the staging, then one per tile.
    if (producer) {
        __syncthreads(); // the consumers hold their query fragments: the staging area is free
        issue(0);
        if (ntiles > 1) issue(1);
        if (ntiles > 1) vm_wait<5>();
        else vm_wait<0>();
        dequant(0);
        lds_drain();
        if (ntiles > 2) issue(2);
        __syncthreads(); // buffer 0 complete
        for (int i = 0; i < ntiles; i++) {
            if (i + 1 < ntiles) {
                if (i + 2 < ntiles) vm_wait<5>(); // tile i + 1 landed (tile i + 2 may be in flight)
                else vm_wait<0>();
                dequant(i + 1);
                lds_drain();
                if (i + 3 < ntiles) issue(i + 3);
            }
            __syncthreads(); // buffer (i + 1) % 2 complete, buffer i % 2 free
        }
        return;
    }
    half8 qf[16];
#pragma unroll
    for (int ks = 0; ks < 16; ks++) qf[ks] = *reinterpret_cast<const half8 *>(qs + (32 * wv + c) * SK_LD + 16 * ks + 8 * hf);
    __syncthreads();
    __syncthreads();
    const int row = r0 + 32 * wv + c;
    const int lim = row < a.R ? a.n0 + row / GQA : -1;
    const int lim_min = a.n0 + (r0 + 32 * wv) / GQA;
    float m = -INFINITY, l = 0.f;
    f32x16 O[8];
#pragma unroll
    for (int db = 0; db < 8; db++)
#pragma unroll
        for (int e = 0; e < 16; e++) O[db][e] = 0.f;
    constexpr float RESCALE_LOG2 = 8.f;
    for (int i = 0; i < ntiles; i++) {
        const _Float16 * const sK = buf0 + (i & 1) * (PQ_BUF / 2);
        const _Float16 * const sVt = sK + ATP * SK_LD;
        const int p0 = c0 + ATP * i;
        f32x16 sacc;
#pragma unroll
        for (int e = 0; e < 16; e++) sacc[e] = 0.f;
#pragma unroll
        for (int ks = 0; ks < 16; ks++) {
            const half8 ak = *reinterpret_cast<const half8 *>(sK + c * SK_LD + 16 * ks + 8 * hf);
            sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ak, qf[ks], sacc, 0, 0, 0);
        }
        const bool full = p0 + ATP - 1 <= lim_min;
        float mx = -INFINITY;
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const int pos = p0 + 8 * (e >> 2) + 4 * hf + (e & 3);
            sacc[e] = full || pos <= lim ? sacc[e] * LOG2E : -INFINITY;
            mx = fmaxf(mx, sacc[e]);
        }
        mx = fmaxf(mx, shfl_xor(mx, 32));
        const float mnew = mx > m + RESCALE_LOG2 ? mx : m;
        float al = 1.f, ps = 0.f;
        if (mnew != -INFINITY) {
            al = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - mnew);
#pragma unroll
            for (int e = 0; e < 16; e++) {
                sacc[e] = __builtin_amdgcn_exp2f(sacc[e] - mnew);
                ps += sacc[e];
            }
        } else {
#pragma unroll
            for (int e = 0; e < 16; e++) sacc[e] = 0.f;
        }
        ps += shfl_xor(ps, 32);
        const bool rescale = al != 1.f && m != -INFINITY;
        l = __builtin_fmaf(l, al, ps);
        m = mnew;
        if (__any(rescale)) {
#pragma unroll
            for (int db = 0; db < 8; db++) O[db] *= al;
        }
        half8 pb[2];
#pragma unroll
        for (int s2 = 0; s2 < 2; s2++)
#pragma unroll
            for (int e = 0; e < 8; e++) pb[s2][e] = (_Float16) sacc[8 * s2 + e];
#pragma unroll
        for (int db = 0; db < 8; db++)
#pragma unroll
            for (int s2 = 0; s2 < 2; s2++) {
                const half8 av = *reinterpret_cast<const half8 *>(sVt + (32 * db + c) * SVT_LD + 8 * db + 16 * s2 + 8 * hf);
                O[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, pb[s2], O[db], 0, 0, 0);
            }
        __syncthreads(); // buffer i % 2 free for the producers
    }
    if (row < a.R) {
        const size_t u = (size_t) (g * a.nseg + k) * a.R + row;
        if (hf == 0) a.ml[u] = make_float2(m, l);
        float * const dst = a.part + u * HD;
#pragma unroll
        for (int db = 0; db < 8; db++)
#pragma unroll
            for (int j = 0; j < 4; j++)
                *reinterpret_cast<float4 *>(dst + 32 * db + 8 * j + 4 * hf) =
                    make_float4(O[db][4 * j], O[db][4 * j + 1], O[db][4 * j + 2], O[db][4 * j + 3]);
    }
}

// One wave per (row, kv head) of a prefill piece: the row's segments 0 .. pos / a.seg folded in segment order
// (M' = max(M, m_k), O' = O e^(M - M') + O_k e^(m_k - M'), l likewise), y = O / l, then the output epilogue.
__global__ __launch_bounds__(256) void k_prefill_combine(PrefillArgs a) {
    const int wid = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (wid >= a.R * NKV) return;
    const int r = wid % a.R, g = wid / a.R;
    const int t = r / GQA, hh = r - GQA * t, pos = a.n0 + t;
    const int nk = pos / a.seg + 1;
    float M = -INFINITY, den = 0.f;
    float4 num = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int k = 0; k < nk; k++) {
        const size_t u = (size_t) (g * a.nseg + k) * a.R + r;
        const float2 ml = a.ml[u];
        const float4 o = *reinterpret_cast<const float4 *>(a.part + u * HD + 4 * lane);
        const float Mn = fmaxf(M, ml.x);
        const float e0 = M == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(M - Mn);
        const float e1 = ml.x == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ml.x - Mn);
        num.x = __builtin_fmaf(num.x, e0, e1 * o.x);
        num.y = __builtin_fmaf(num.y, e0, e1 * o.y);
        num.z = __builtin_fmaf(num.z, e0, e1 * o.z);
        num.w = __builtin_fmaf(num.w, e0, e1 * o.w);
        den = __builtin_fmaf(den, e0, e1 * ml.y);
        M = Mn;
    }
    float v[4] = {num.x / den, num.y / den, num.z / den, num.w / den};
    const int h = GQA * g + hh;
    finish_row(v, a.vrot, a.gate ? a.gate + ((size_t) t * NH + h) * a.gs : nullptr, a.out + ((size_t) t * NH + h) * HD, a.q32a,
               a.q32b, a.q32m, (size_t) t, h);
}

// ------------------------------------------------------------------------------------------------ dispatch
typedef void (*AttnKernel)(AttnArgs);

template <int NP, bool WIDE = false>
static AttnKernel pick(int kb, int vb) {
#define QKV_VB(K)                                                                                                      \
    switch (vb) {                                                                                                      \
    case 4: return k_attn<NP, K, 4, false, WIDE>;                                                                      \
    case 5: return k_attn<NP, K, 5, false, WIDE>;                                                                      \
    case 6: return k_attn<NP, K, 6, false, WIDE>;                                                                      \
    case 7: return k_attn<NP, K, 7, false, WIDE>;                                                                      \
    case 8: return k_attn<NP, K, 8, false, WIDE>;                                                                      \
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

template <int KB, int VB>
static AttnKernel small_or_null() {
    if constexpr (KB + VB <= 11) return k_attn<1, KB, VB, true>;
    else return nullptr;
}

static AttnKernel pick_small(int kb, int vb) {
#define QKV_VB(K)                                                                                                      \
    switch (vb) {                                                                                                      \
    case 4: return small_or_null<K, 4>();                                                                              \
    case 5: return small_or_null<K, 5>();                                                                              \
    case 6: return small_or_null<K, 6>();                                                                              \
    case 7: return small_or_null<K, 7>();                                                                              \
    default: return nullptr;                                                                                           \
    }
    switch (kb) {
    case 4: QKV_VB(4)
    case 5: QKV_VB(5)
    case 6: QKV_VB(6)
    case 7: QKV_VB(7)
    default: return nullptr;
    }
#undef QKV_VB
}

// CUs of the current device (cached per thread and device)
static int device_cus() {
    static thread_local int dev_cached = -1, cus = 0;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    if (dev != dev_cached) {
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
        dev_cached = dev;
    }
    return cus;
}

hipError_t launch_attn(const AttnArgs & a, int kb, int vb, int max_blocks, int occ, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1) {
    AttnKernel k = nullptr;
    const int np = a.RP / 8;
    // three workgroups per CU (small stages) when one 8-row group of a packed format of at most 11 KiB per tile has
    // more work items than two per CU hold (occ 0), or always (occ 3); occ 2 keeps two
    const bool small = np == 1 && kb + vb <= 11 && (occ == 3 || (occ == 0 && a.n_items > 2 * device_cus()));
    if (small) k = pick_small(kb, vb);
    else if (np == 1) k = pick<1>(kb, vb);
    else if (np == 2) k = pick<2>(kb, vb);
    else if (np == 3) k = a.wide ? pick<3, true>(kb, vb) : pick<3>(kb, vb);
    if (!k) return hipErrorInvalidValue;
    static thread_local const void * configured[128];
    static thread_local int n_configured = 0;
    bool done = false;
    for (int i = 0; i < n_configured; i++) done |= configured[i] == (const void *) k;
    const int lds = a.wide ? 2 * (ATTN_LDS + a.RP * HD * 2) : (small ? AWAVES * (1024 * (kb + vb) + 1024) : ATTN_LDS) + a.RP * HD * 2;
    if (!done) {
        const hipError_t e = hipFuncSetAttribute((const void *) k, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
        if (e != hipSuccess) return e;
        if (n_configured < 128) configured[n_configured++] = (const void *) k;
    }
    int blocks = a.n_items;
    if (max_blocks > 0 && blocks > max_blocks) blocks = max_blocks;
    hipExtLaunchKernelGGL(k, dim3(blocks), dim3(a.wide ? 512 : 256), lds, st, ev0, ev1, 0, a);
    return hipGetLastError();
}

typedef void (*PrefillKernel)(PrefillArgs);

static PrefillKernel pick_prefill(int kb, int vb) {
#define QKV_VB(K)                                                                                                      \
    switch (vb) {                                                                                                      \
    case 4: return k_prefill3<K, 4>;                                                                                    \
    case 5: return k_prefill3<K, 5>;                                                                                    \
    case 6: return k_prefill3<K, 6>;                                                                                    \
    case 7: return k_prefill3<K, 7>;                                                                                    \
    case 8: return k_prefill3<K, 8>;                                                                                    \
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

hipError_t launch_prefill(const PrefillArgs & a, int kb, int vb, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1) {
    PrefillKernel k = pick_prefill(kb, vb);
    if (!k) return hipErrorInvalidValue;
    constexpr int lds = PQ_LDS;
    static thread_local const void * configured[32];
    static thread_local int n_configured = 0;
    bool done = false;
    for (int i = 0; i < n_configured; i++) done |= configured[i] == (const void *) k;
    if (!done) {
        const hipError_t e = hipFuncSetAttribute((const void *) k, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
        if (e != hipSuccess) return e;
        if (n_configured < 32) configured[n_configured++] = (const void *) k;
    }
    hipExtLaunchKernelGGL(k, dim3(a.nrb * NKV * a.nseg), dim3(512), lds, st, ev0, nullptr, 0, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipExtLaunchKernelGGL(k_prefill_combine, dim3((a.R * NKV + 3) / 4), dim3(256), 0, st, nullptr, ev1, 0, a);
    return hipGetLastError();
}


template <int KB, int VB>
static hipError_t prefetch_kb_vb(const AttnArgs & a, int tiles, hipStream_t st) {
    constexpr int lds = ATTN_LDS;
    static thread_local bool configured = false; // (per instantiation, as launch_attn does)
    if (!configured) {
        const hipError_t e = hipFuncSetAttribute((const void *) k_prefetch<KB, VB>, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
        if (e != hipSuccess) return e;
        configured = true;
    }
    hipLaunchKernelGGL((k_prefetch<KB, VB>), dim3(a.n_items), dim3(256), lds, st, a, tiles);
    return hipGetLastError();
}

hipError_t launch_prefetch(const AttnArgs & a, int kb, int vb, int tiles, hipStream_t st) {
#define QKV_VB(K)                                                                                                      \
    switch (vb) {                                                                                                      \
    case 4: return prefetch_kb_vb<K, 4>(a, tiles, st);                                                                 \
    case 5: return prefetch_kb_vb<K, 5>(a, tiles, st);                                                                 \
    case 6: return prefetch_kb_vb<K, 6>(a, tiles, st);                                                                 \
    case 7: return prefetch_kb_vb<K, 7>(a, tiles, st);                                                                 \
    case 8: return prefetch_kb_vb<K, 8>(a, tiles, st);                                                                 \
    default: return hipErrorInvalidValue;                                                                              \
    }
    switch (kb) {
    case 4: QKV_VB(4)
    case 5: QKV_VB(5)
    case 6: QKV_VB(6)
    case 7: QKV_VB(7)
    case 8: QKV_VB(8)
    default: return hipErrorInvalidValue;
    }
#undef QKV_VB
}

} // namespace qkv
