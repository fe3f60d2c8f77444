// Split-K decode attention over the mixed q8-ring / packed KV store (gfx950, wave64, MFMA f16).
//
// Work: one workgroup of 4 waves per (sequence, layer, kv head, canonical segment of SEG positions).  Wave w takes the
// 32-position tiles w, w+4, .. of the segment and keeps its own online-softmax state; at the end of the segment the 4
// states are merged in wave order and written as the segment's partial (m, l, O).  The partition is fixed by the
// positions alone, so the result never depends on the grid, the split count or the number of query tokens.
//
// Per tile and wave, everything stays in registers (no LDS, no barriers):
//   S^T = K Q^T   v_mfma_f32_16x16x32_f16, A = 16 positions x 32 dims of K (lane: position l%16, 8 consecutive dims of
//                 its quarter l/16 of the row), B = Q^T (lane: query row l%16, the same dims).  Two 16-position subtiles.
//   softmax       lane (row l%16, quarter q) owns S of positions 4q..4q+3 and 16+4q..16+4q+3 of its row: 8 values,
//                 max / sum across the 4 quarters by two xor shuffles; exp2 in log2 units.
//   O^T += V^T P^T  A = V^T (lane: dims 16 (l%16) + i for instruction i, its 8 positions), B = P^T (the lane's own 8 P
//                 values as fp16), C = O^T (lane: its row, dims 64q .. 64q+63).
// Dequantization happens in registers with the 0x6400 magic (kv_dev.h): fp16 values half_rn(d q), the reference's
// operands (q8_to_f16 qwen38_mk.cu:2336, qn_to_f16 :2458).  The arithmetic of a row follows attn_core_t
// (qwen38_mk.cu:2757-3080): S in fp32 from fp16 operands, masked positions -> -inf, P rounded to fp16, O in fp32.
#include "kv_dev.h"
#include "kv_launch.h"

namespace qkv {

constexpr float LOG2E = 1.4426950408889634f;
constexpr unsigned C64 = 0x64646464u;

__device__ __forceinline__ size_t attn_main_row(const StoreLayout & S, int seq, int g, int p) {
    const int lp = p / S.page;
    const int phys = S.ptab[seq * S.pt_stride + lp];
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

// ------------------------------------------------------------------------------------------------ the tile
template <int NR>
struct WaveState {
    f32x4 acc[NR][16]; // O^T: instruction i, element e -> dim 64 q + 16 e + i of the lane's row
    float m[NR], l[NR];
    int lim[NR];       // last visible position of the lane's row (-1: padding row)
};

template <int NR, int KB, int VB>
__device__ __forceinline__ void attend_tile(WaveState<NR> & st, const half8 (&qf)[NR][8], int p0, int nv, const uint8_t * kbase,
                                            const uint16_t * ksc, const uint8_t * vbase, const uint16_t * vsc) {
    const int lane = lane_id(), n = lane & 15, q = lane >> 4;
    constexpr int KRB = 32 * KB, VRB = 32 * VB;
    // ---- loads: K subtiles (position n and 16 + n) and V (the lane's 8 positions); rows past the end alias the last row
    KSub<KB> k0, k1;
    {
        const int r0 = min(n, nv - 1), r1 = min(16 + n, nv - 1);
        load_ksub<KB>(k0, kbase + (size_t) r0 * KRB, ksc + r0 * 8, q);
        load_ksub<KB>(k1, kbase + (size_t) r1 * KRB, ksc + r1 * 8, q);
    }
    VRaw<VB> vr;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int rr = min((j < 4 ? 4 * q + j : 16 + 4 * q + j - 4), nv - 1);
        load_vpos<VB>(vr, j, vbase + (size_t) rr * VRB, vsc + rr * 8, n);
    }
    // ---- S^T = K Q^T
    f32x4 s[2][NR];
#pragma unroll
    for (int rg = 0; rg < NR; rg++) s[0][rg] = s[1][rg] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 8; ks++) {
        const half8 a0 = kfrag<KB>(k0, ks);
        const half8 a1 = kfrag<KB>(k1, ks);
#pragma unroll
        for (int rg = 0; rg < NR; rg++) {
            s[0][rg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, qf[rg][ks], s[0][rg], 0, 0, 0);
            s[1][rg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, qf[rg][ks], s[1][rg], 0, 0, 0);
        }
    }
    // ---- online softmax (log2 units); lane: row n of group rg, positions p0 + 4q + e and p0 + 16 + 4q + e
    half8 pf[NR];
    bool rescale = false;
    float alpha[NR];
#pragma unroll
    for (int rg = 0; rg < NR; rg++) {
        float t[8];
        float mx = -INFINITY;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int pos = p0 + (e < 4 ? 4 * q + e : 16 + 4 * q + e - 4);
            const float sv = (e < 4 ? s[0][rg][e] : s[1][rg][e - 4]) * LOG2E;
            t[e] = pos <= st.lim[rg] ? sv : -INFINITY;
            mx = fmaxf(mx, t[e]);
        }
        mx = fmaxf(mx, shfl_xor(mx, 16));
        mx = fmaxf(mx, shfl_xor(mx, 32));
        const float mnew = fmaxf(st.m[rg], mx);
        float al = 1.f, ps = 0.f;
        float p[8];
        if (mnew != -INFINITY) {
            al = exp2f(st.m[rg] - mnew);
#pragma unroll
            for (int e = 0; e < 8; e++) {
                p[e] = exp2f(t[e] - mnew);
                ps += p[e];
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++) p[e] = 0.f;
        }
        ps += shfl_xor(ps, 16);
        ps += shfl_xor(ps, 32);
        st.l[rg] = __builtin_fmaf(st.l[rg], al, ps);
        st.m[rg] = mnew;
        alpha[rg] = al;
        rescale |= al != 1.f;
#pragma unroll
        for (int e = 0; e < 8; e++) pf[rg][e] = (_Float16) p[e];
    }
    if (__any(rescale)) {
#pragma unroll
        for (int rg = 0; rg < NR; rg++)
#pragma unroll
            for (int i = 0; i < 16; i++) st.acc[rg][i] *= alpha[rg];
    }
    // ---- O^T += V^T P^T, one instruction per dim 16 m + i of the lane
    half2v dv[4];
#pragma unroll
    for (int jp = 0; jp < 4; jp++) dv[jp] = as_h2((vr.s[2 * jp] & 0xffffu) | (vr.s[2 * jp + 1] << 16));
    unsigned c[8][4];
#pragma unroll
    for (int j = 0; j < 8; j++) vcodes<VB>(vr, j, c[j]);
    constexpr unsigned XMAG = VB == 8 ? 0x64806480u : 0x64006400u;
    constexpr float VBIAS = VB == 8 ? 1152.f : (float) (1024 + (1 << (VB - 1)));
    const half2v vb2 = {(_Float16) -VBIAS, (_Float16) -VBIAS};
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int a = i >> 2, b = i & 3;
        const unsigned sel = (unsigned) b | 0x0c00u | ((unsigned) (4 + b) << 16) | 0x0c000000u;
        half8 va;
#pragma unroll
        for (int jp = 0; jp < 4; jp++) {
            const half2v x = (as_h2(perm_b32(c[2 * jp + 1][a], c[2 * jp][a], sel) ^ XMAG) + vb2) * dv[jp];
            va[2 * jp] = x[0];
            va[2 * jp + 1] = x[1];
        }
#pragma unroll
        for (int rg = 0; rg < NR; rg++) st.acc[rg][i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pf[rg], st.acc[rg][i], 0, 0, 0);
    }
}

// ------------------------------------------------------------------------------------------------ the kernel
template <int NR, int KB, int VB>
__global__ __launch_bounds__(256) void k_attn(AttnArgs a) {
    constexpr int RP = 16 * NR;
    __shared__ float s_o[RP][HD + 4];
    __shared__ float s_m[AWAVES][RP], s_l[AWAVES][RP];
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63, n = lane & 15, q = lane >> 4;
    const StoreLayout & S = a.S;
    for (int item = blockIdx.x; item < a.n_items; item += gridDim.x) {
        int si = 0;
#pragma unroll
        for (int i = 1; i < 8; i++)
            if (i < a.nseq && item >= a.sd[i].item0) si = i;
        const SeqDesc & sd = a.sd[si];
        const int local = item - sd.item0;
        const int seg = local % sd.nseg, lg = local / sd.nseg;
        const int g = lg % NKV, l = lg / NKV;
        const int L = sd.L, ws = sd.ws, seq = sd.seq;
        const int c0 = seg * SEG, c1 = min(L, c0 + SEG);
        const int ntiles = (c1 - c0 + ATP - 1) / ATP;
        const SideLayout & SK = S.side[a.layer0 + l][0];
        const SideLayout & SV = S.side[a.layer0 + l][1];

        half8 qf[NR][8];
        {
            const _Float16 * qb = a.qh + ((size_t) ((l * a.nseq + si) * NKV + g) * RP) * HD;
#pragma unroll
            for (int rg = 0; rg < NR; rg++)
#pragma unroll
                for (int ks = 0; ks < 8; ks++)
                    qf[rg][ks] = *reinterpret_cast<const half8 *>(qb + (size_t) (16 * rg + n) * HD + 64 * q + 8 * ks);
        }
        WaveState<NR> st;
#pragma unroll
        for (int rg = 0; rg < NR; rg++) {
            st.m[rg] = -INFINITY;
            st.l[rg] = 0.f;
            const int row = 16 * rg + n;
            st.lim[rg] = row < a.R ? L - a.T + row % a.T : -1;
#pragma unroll
            for (int i = 0; i < 16; i++) st.acc[rg][i] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
        for (int tt = wv; tt < ntiles; tt += AWAVES) {
            const int p0 = c0 + ATP * tt, nv = min(ATP, L - p0);
            if (S.kvrc > 0 && p0 >= ws) { // the window: q8 rows from the rings (sides without one are q8 in the main store)
                const int rr = p0 % S.kvrc;
                const uint8_t *kb, *vb;
                const uint16_t *ks, *vs;
                if (SK.ring) {
                    const size_t r = (size_t) (seq * NKV + g) * S.kvrc + rr;
                    kb = reinterpret_cast<const uint8_t *>(SK.ring) + r * HD;
                    ks = SK.rsc + r * 8;
                } else {
                    const size_t r = attn_main_row(S, seq, g, p0);
                    kb = SK.vals + r * HD;
                    ks = SK.scs + r * 8;
                }
                if (SV.ring) {
                    const size_t r = (size_t) (seq * NKV + g) * S.kvrc + rr;
                    vb = reinterpret_cast<const uint8_t *>(SV.ring) + r * HD;
                    vs = SV.rsc + r * 8;
                } else {
                    const size_t r = attn_main_row(S, seq, g, p0);
                    vb = SV.vals + r * HD;
                    vs = SV.scs + r * 8;
                }
                attend_tile<NR, 8, 8>(st, qf, p0, nv, kb, ks, vb, vs);
            } else {
                const size_t r = attn_main_row(S, seq, g, p0);
                attend_tile<NR, KB, VB>(st, qf, p0, nv, SK.vals + r * (32 * KB), SK.scs + r * 8, SV.vals + r * (32 * VB), SV.scs + r * 8);
            }
        }
        // ---- merge the 4 waves in order: M = max m_w, O = sum e_w O_w, l = sum e_w l_w
        if (q == 0) {
#pragma unroll
            for (int rg = 0; rg < NR; rg++) {
                s_m[wv][16 * rg + n] = st.m[rg];
                s_l[wv][16 * rg + n] = st.l[rg];
            }
        }
        __syncthreads();
        float e[NR];
#pragma unroll
        for (int rg = 0; rg < NR; rg++) {
            const int row = 16 * rg + n;
            const float M = fmaxf(fmaxf(s_m[0][row], s_m[1][row]), fmaxf(s_m[2][row], s_m[3][row]));
            e[rg] = st.m[rg] == -INFINITY ? 0.f : exp2f(st.m[rg] - M);
        }
        for (int w = 0; w < AWAVES; w++) {
            if (wv == w) {
#pragma unroll
                for (int rg = 0; rg < NR; rg++) {
                    float * o = &s_o[16 * rg + n][64 * q];
#pragma unroll
                    for (int i = 0; i < 16; i++)
#pragma unroll
                        for (int ee = 0; ee < 4; ee++) {
                            const float x = st.acc[rg][i][ee];
                            o[16 * ee + i] = w == 0 ? e[rg] * x : __builtin_fmaf(e[rg], x, o[16 * ee + i]);
                        }
                }
            }
            __syncthreads();
        }
        float * part = a.part + (size_t) item * a.R * HD;
        for (int idx = threadIdx.x; idx < a.R * (HD / 4); idx += 256) {
            const int row = idx / (HD / 4), c4 = idx % (HD / 4);
            *reinterpret_cast<float4 *>(part + (size_t) row * HD + 4 * c4) = *reinterpret_cast<const float4 *>(&s_o[row][4 * c4]);
        }
        if (threadIdx.x < a.R) {
            const int row = threadIdx.x;
            const float M = fmaxf(fmaxf(s_m[0][row], s_m[1][row]), fmaxf(s_m[2][row], s_m[3][row]));
            float lsum = 0.f;
#pragma unroll
            for (int w = 0; w < AWAVES; w++) {
                const float ew = s_m[w][row] == -INFINITY ? 0.f : exp2f(s_m[w][row] - M);
                lsum = __builtin_fmaf(ew, s_l[w][row], lsum);
            }
            a.ml[(size_t) item * a.R + row] = make_float2(M, lsum);
        }
        __syncthreads(); // s_o / s_m are reused by the next item
    }
}

// ------------------------------------------------------------------------------------------------ dispatch
typedef void (*AttnKernel)(AttnArgs);

template <int NR>
static AttnKernel pick(int kb, int vb) {
#define QKV_VB(K)                                                                                                      \
    switch (vb) {                                                                                                      \
    case 4: return k_attn<NR, K, 4>;                                                                                   \
    case 5: return k_attn<NR, K, 5>;                                                                                   \
    case 6: return k_attn<NR, K, 6>;                                                                                   \
    case 7: return k_attn<NR, K, 7>;                                                                                   \
    case 8: return k_attn<NR, K, 8>;                                                                                   \
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

hipError_t launch_attn(const AttnArgs & a, int kb, int vb, int max_blocks, hipStream_t st) {
    AttnKernel k = nullptr;
    const int nr = a.RP / 16;
    if (nr == 1) k = pick<1>(kb, vb);
    else if (nr == 2) k = pick<2>(kb, vb);
    else if (nr == 3) k = pick<3>(kb, vb);
    if (!k) return hipErrorInvalidValue;
    int blocks = a.n_items;
    if (max_blocks > 0 && blocks > max_blocks) blocks = max_blocks;
    hipLaunchKernelGGL(k, dim3(blocks), dim3(256), 0, st, a);
    return hipGetLastError();
}

} // namespace qkv
