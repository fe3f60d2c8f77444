/*
 * kv_oracle.c -- CPU restatement of the reference's quantized KV-cache arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP path and the host-core
 * baseline that bench.py times beside it.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product library never links or calls it.
 *
 * Written from the reference's source semantics (CUDA, sm_86, nvcc defaults: IEEE division and
 * reciprocal, FMA contraction of a*b+c, RNE float->half, saturating float->int with NaN -> 0).
 * Build with -ffp-contract=off: every fused multiply-add below is an explicit fmaf().
 *
 * Pinning (what checks each function; see tests/test_oracle_*.py):
 *   kvo_fwht256        closed forms: basis vectors -> +-1/16 Sylvester signs, H.H = I, linearity, brute-force
 *                      matrix product in fp64 (ulp bound) and exact bits for power-of-two-friendly inputs.
 *   kvo_store_q8       crafted blocks (zero block, single +-x, ties at .5 to even), numpy property check
 *                      |q - v*127/am| <= 0.5 with ties-to-even, scale == float16(am/127).
 *   kvo_store_qn       crafted blocks (all zero -> n = h / scale -0, single value -> n = 0 or 2h-1, |x| ties
 *                      -> larger x), b = 4 bytes == the q4 layout, numpy floor(v*id + h + .5) clamp property,
 *                      pack/unpack round trip and hand-placed byte positions.
 *   kvo_ws / kvo_kvrc  the reference's documented spot values (W 2048 -> 2,561..3,200 positions, kvrc 3,232,
 *                      L 101,600 -> ws 98,560).
 *   kvo_attn_exact     brute-force fp64 softmax attention; pinned by closed forms (uniform keys -> mean of V,
 *                      one dominant key -> that V row, L = 1 -> V row) in the tests.
 *   kvo_attn_chunked   the reference's split-K arithmetic (attn_dims chunks, 32-position tiles, fp16 operands,
 *                      fp32 online softmax, attn_combine); pinned against kvo_attn_exact within 2e-3.
 *   kvo_dg_hash        FNV-style row hash; its byte loop is FNV-1a 64, pinned by the published FNV-1a test vectors;
 *                      its 8-byte word step by hand-computed words.
 *   kvo_gate           y / (1 + expf(-g)) (qwen38_mk.cu:4686); pinned by closed forms (g = 0 -> y / 2, large g -> y).
 *   kvo_q32_row        q32_store (qwen38_mk.cu:283-307) over one token's 24 x 256 output row: known answers (zero
 *                      block, single value -> +-127, half-away-from-zero ties) and the unit layout by hand-placed
 *                      blocks in the tests.
 *   kvo_rope_rows      the RoPE text table (loader.cu:1252-1258); pinned by numpy fp64 cos/sin of the same angles
 *                      (<= 1 float ulp) and row 0 = (1, 0).
 *   kvo_qk_prep        RMSNorm + NeoX RoPE on values 0..63 (qwen38_mk.cu:2623-2636, 2903-2910) in the HIP kernels'
 *                      fixed arithmetic order; pinned by an fp64 numpy RMSNorm / rotate-half within 2e-6 relative,
 *                      position 0 = RMSNorm alone, constant rows, and norm preservation of each rotated pair.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <pthread.h>
#include <time.h>

#define HD 256
#define ATP 32
#define ATT_NCH 20
#define ATT_BUCKET (ATT_NCH * ATP)

/* ---------------------------------------------------------------- fp16 / int conversions (CUDA semantics) */

/* float -> binary16, round to nearest even, overflow -> inf (__float2half_rn) */
uint16_t kvo_f2h(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t) (sign | (ax > 0x7f800000u ? 0x7fffu : 0x7c00u)); /* NaN / inf */
    if (ax >= 0x477ff000u) return (uint16_t) (sign | 0x7c00u); /* >= 65520: rounds to inf */
    if (ax < 0x33000000u) return (uint16_t) sign; /* < 2^-25: rounds to zero (2^-25 itself ties to even 0) */
    const int e = (int) (ax >> 23) - 127;
    uint32_t m = (ax & 0x7fffffu) | 0x800000u;
    if (e < -14) { /* subnormal half: value = m * 2^(e-23); half ulp 2^-24 */
        const int sh = -e - 14 + 13; /* bits to drop */
        const uint32_t q = m >> sh, r = m & ((1u << sh) - 1u), hf = 1u << (sh - 1);
        uint32_t h = q;
        if (r > hf || (r == hf && (q & 1u))) h++;
        return (uint16_t) (sign | h);
    }
    const uint32_t q = m >> 13, r = m & 0x1fffu;
    uint32_t h = ((uint32_t) (e + 15) << 10) | (q & 0x3ffu);
    if (r > 0x1000u || (r == 0x1000u && (q & 1u))) h++; /* carry into the exponent is the right result */
    return (uint16_t) (sign | h);
}

float kvo_h2f(uint16_t h) {
    const uint32_t sign = (uint32_t) (h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) x = sign;
        else { /* subnormal */
            float f = (float) m * 5.9604644775390625e-8f; /* 2^-24, exact */
            memcpy(&x, &f, 4);
            x |= sign;
        }
    } else if (e == 31) x = sign | 0x7f800000u | (m << 13);
    else x = sign | ((e + 112) << 23) | (m << 13);
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* (int) x: truncation, saturating, NaN -> 0 (cvt.rzi.s32.f32) */
static int cvt_rzi(float x) {
    if (x != x) return 0;
    if (x >= 2147483648.0f) return 2147483647;
    if (x <= -2147483648.0f) return (-2147483647 - 1);
    return (int) x;
}
/* __float2int_rn: round half to even, saturating, NaN -> 0 */
static int cvt_rni(float x) {
    if (x != x) return 0;
    const float r = nearbyintf(x); /* default rounding mode: nearest even */
    if (r >= 2147483648.0f) return 2147483647;
    if (r <= -2147483648.0f) return (-2147483647 - 1);
    return (int) r;
}

/* ---------------------------------------------------------------- quantizers (qwen38_mk.cu:2003-2097) */

/* q8_0 row (qwen38_mk.cu:2005-2022): per 32 values am = max |v|; id = 127/am (0 if am = 0);
 * q = rint_even(v * id); scale = half(am / 127). */
void kvo_store_q8(const float * v, int8_t * q, uint16_t * sc) {
    for (int b = 0; b < HD / 32; b++) {
        float am = 0.f;
        for (int k = 0; k < 32; k++) am = fmaxf(am, fabsf(v[32 * b + k]));
        const float id = am > 0.f ? 127.0f / am : 0.f;
        for (int k = 0; k < 32; k++) q[32 * b + k] = (int8_t) (cvt_rni(v[32 * b + k] * id) & 0xff);
        sc[b] = kvo_f2h(am / 127.0f);
    }
}

/* signed-max selection of kv_store_q4 / kv_store_qn (qwen38_mk.cu:2033-2041, 2079-2086): the value of
 * largest magnitude, ties to the larger value, starting from (0, +0); NaN never wins. */
static float signed_max(const float * v) {
    float am = 0.f, sv = 0.f;
    for (int k = 0; k < 32; k++) {
        const float a = fabsf(v[k]);
        if (a > am || (a == am && v[k] > sv)) { am = a; sv = v[k]; }
    }
    return sv;
}

/* 4..7-bit row (kv_store_q4 qwen38_mk.cu:2029-2046, kv_store_qn :2075-2097): d = sv / -h, id = 1/d (0 if d == 0),
 * n = min(2h-1, (int) fma(v, id, h + 0.5)); bytes 0..127 hold the low nibbles (word w = values 8w..8w+7: values 0..3 in
 * the low nibbles of bytes 0..3, values 4..7 in the high nibbles), bytes 128 + w (b-4) .. the high bits, value k at bit
 * (b-4) k of that little-endian field. */
void kvo_store_qn(const float * v, uint8_t * q, uint16_t * sc, int bits) {
    const int h = 1 << (bits - 1), hb = bits - 4;
    for (int b = 0; b < HD / 32; b++) {
        const float sv = signed_max(v + 32 * b);
        const float d = sv / (float) -h, id = d != 0.f ? 1.0f / d : 0.f;
        sc[b] = kvo_f2h(d);
        for (int wl = 0; wl < 4; wl++) {
            const int w = 4 * b + wl;
            uint32_t lo = 0, hi = 0;
            for (int k = 0; k < 8; k++) {
                int n = cvt_rzi(fmaf(v[8 * w + k], id, (float) h + 0.5f));
                if (n > 2 * h - 1) n = 2 * h - 1;
                const uint32_t un = (uint32_t) n;
                lo |= (un & 15u) << (k < 4 ? 8 * k : 8 * (k - 4) + 4);
                hi |= (un >> 4) << (hb * k);
            }
            memcpy(q + 4 * w, &lo, 4);
            for (int k = 0; k < hb; k++) q[128 + w * hb + k] = (uint8_t) ((hi >> (8 * k)) & 0xffu);
        }
    }
}

/* bytes of one stored row */
int kvo_row_bytes(int bits) { return HD * bits / 8; }

/* ---------------------------------------------------------------- Walsh-Hadamard (qwen38_mk.cu:2048-2068) */

/* Sylvester-ordered 256-point FWHT: stages over index bits 0..7 in ascending order, butterfly (a+b, a-b) with a the
 * lower index, then * 1/16 (exact). Stage order and butterfly form fix the bits. */
void kvo_fwht256(float * v) {
    for (int m = 1; m < HD; m <<= 1)
        for (int i = 0; i < HD; i++)
            if (!(i & m)) {
                const float a = v[i], b = v[i | m];
                v[i] = a + b;
                v[i | m] = a - b;
            }
    for (int i = 0; i < HD; i++) v[i] *= 0.0625f;
}

/* ---------------------------------------------------------------- dequantization */

/* integer codes of a stored row: q in [-h, h-1] (q8: int8) */
void kvo_codes(const uint8_t * q, int bits, int * out) {
    if (bits == 8) {
        for (int i = 0; i < HD; i++) out[i] = (int8_t) q[i];
        return;
    }
    const int h = 1 << (bits - 1), hb = bits - 4;
    for (int w = 0; w < 32; w++) {
        uint32_t lo;
        memcpy(&lo, q + 4 * w, 4);
        uint32_t hi = 0;
        for (int k = 0; k < hb; k++) hi |= (uint32_t) q[128 + w * hb + k] << (8 * k);
        for (int k = 0; k < 8; k++) {
            const uint32_t nib = (lo >> (k < 4 ? 8 * k : 8 * (k - 4) + 4)) & 15u;
            const uint32_t hv = hb ? (hi >> (hb * k)) & ((1u << hb) - 1u) : 0u;
            out[8 * w + k] = (int) (nib | (hv << 4)) - h;
        }
    }
}

/* fp32 dequantization d * q (k_ring_refill, qwen38_mk.cu:2497-2512) */
void kvo_dequant_f32(const uint8_t * q, const uint16_t * sc, int bits, float * out) {
    int c[HD];
    kvo_codes(q, bits, c);
    for (int i = 0; i < HD; i++) out[i] = kvo_h2f(sc[i / 32]) * (float) c[i];
}

/* the fp16 operand the attention kernels see: half_rn(d * q) (q8_to_f16 :2336, q4_to_f16 :2346, qn_to_f16 :2458) */
void kvo_dequant_f16(const uint8_t * q, const uint16_t * sc, int bits, float * out) {
    int c[HD];
    kvo_codes(q, bits, c);
    for (int i = 0; i < HD; i++) out[i] = kvo_h2f(kvo_f2h(kvo_h2f(sc[i / 32]) * (float) c[i]));
}

/* n rows at once (row stride = the format's bytes): fp32 (f16 = 0) or the fp16-rounded operand (f16 = 1) */
void kvo_dequant_rows(const uint8_t * q, const uint16_t * sc, int bits, int n, float * out, int f16) {
    const size_t rb = (size_t) kvo_row_bytes(bits);
    for (int i = 0; i < n; i++)
        (f16 ? kvo_dequant_f16 : kvo_dequant_f32)(q + (size_t) i * rb, sc + (size_t) i * 8, bits, out + (size_t) i * HD);
}

/* ---------------------------------------------------------------- store of one row (kv_store, :2099-2116) */

/* optional rotation, then the main row in `bits` and (if ring_q) the q8 ring copy of the same rotated values */
void kvo_store_row(const float * vin, int rotate, int bits, uint8_t * main_q, uint16_t * main_s, int8_t * ring_q, uint16_t * ring_s) {
    float v[HD];
    memcpy(v, vin, sizeof v);
    if (rotate) kvo_fwht256(v);
    if (bits == 8) kvo_store_q8(v, (int8_t *) main_q, main_s);
    else kvo_store_qn(v, main_q, main_s, bits);
    if (ring_q) kvo_store_q8(v, ring_q, ring_s);
}

/* ring refill of one row (k_ring_refill, :2488-2517): q8 of the fp32 dequantized main row */
void kvo_ring_refill_row(const uint8_t * main_q, const uint16_t * main_s, int bits, int8_t * ring_q, uint16_t * ring_s) {
    float v[HD];
    kvo_dequant_f32(main_q, main_s, bits, v);
    kvo_store_q8(v, ring_q, ring_s);
}

/* ---------------------------------------------------------------- window / partition geometry */

/* kv_ws (:2118-2126): positions >= ws are read from the q8 ring */
int kvo_ws(int L, int win) {
    if (win <= 0) return 0;
    const int ws = (L + ATT_BUCKET - 1) / ATT_BUCKET - 1 - (win + ATT_BUCKET - 1) / ATT_BUCKET;
    return ws > 0 ? ws * ATT_BUCKET : 0;
}
/* ring rows per kv head (loader.cu:1479-1486) */
int kvo_kvrc(int win) { return win > 0 ? ((win + ATT_BUCKET - 1) / ATT_BUCKET + 1) * ATT_BUCKET + ATP : 0; }
/* attn_dims (:2548-2551) */
void kvo_attn_dims(int L, int * nch, int * cs) {
    int b = (L + ATT_BUCKET - 1) / ATT_BUCKET;
    *cs = ATP * (b > 1 ? b : 1);
    const int n = (L + *cs - 1) / *cs;
    *nch = n > 1 ? n : 1;
}
/* att_cap_T (mk_shared.cuh:288-291) */
int kvo_cap_T(int n, int T) {
    const int lim = ATT_BUCKET * ((n + ATT_BUCKET) / ATT_BUCKET) - n;
    return T < lim ? T : lim;
}

/* ---------------------------------------------------------------- Q preparation (:2873-2880) */

/* the fp16 query row: optional FWHT (K stored rotated), then * 1/16, half_rn */
void kvo_q_prep(const float * qin, int rotate, float * out) {
    float v[HD];
    memcpy(v, qin, sizeof v);
    if (rotate) kvo_fwht256(v);
    for (int i = 0; i < HD; i++) out[i] = kvo_h2f(kvo_f2h(v[i] * 0.0625f));
}

/* ---------------------------------------------------------------- attention */

/*
 * Exact attention in fp64 for one KV head: rows r = 0..R-1 (query row r belongs to token t = r % T, q heads ordered
 * as the reference's r = hh * T + t), K/V as fp32 arrays [L][256] (already dequantized), Q as [R][256].  Row of token
 * t sees positions p <= L - T + t (qwen38_mk.cu:2992-2995).  out [R][256].
 */
void kvo_attn_exact(const float * q, const float * K, const float * V, int L, int T, int R, float * out) {
    double * s = (double *) malloc(sizeof(double) * (size_t) L);
    for (int r = 0; r < R; r++) {
        const int t = r % T, lim = L - T + t;
        double m = -INFINITY;
        for (int p = 0; p <= lim; p++) {
            double a = 0;
            for (int i = 0; i < HD; i++) a += (double) q[(size_t) r * HD + i] * (double) K[(size_t) p * HD + i];
            s[p] = a;
            if (a > m) m = a;
        }
        double l = 0;
        double o[HD];
        for (int i = 0; i < HD; i++) o[i] = 0;
        for (int p = 0; p <= lim; p++) {
            const double e = exp(s[p] - m);
            l += e;
            for (int i = 0; i < HD; i++) o[i] += e * (double) V[(size_t) p * HD + i];
        }
        for (int i = 0; i < HD; i++) out[(size_t) r * HD + i] = (float) (o[i] / l);
    }
    free(s);
}

/*
 * The reference's split-K decode arithmetic for one KV head (attn_core_t :2757-3080 per chunk, attn_combine
 * :4617-4700): chunks of attn_dims(L); per 32-position tile S = sum of fp16 q * fp16 k in fp32; the causal mask;
 * online softmax m_new = max(m, max s), p = expf(s - m_new), alpha = expf(m - m_new), l = l alpha + sum p; P rounded
 * to fp16; O = O alpha + P V in fp32.  Then the combine: M = max m_c, w_c = expf(m_c - M), y = sum w_c O_c / sum w_c l_c.
 * q and K/V are the fp16-valued operands (kvo_q_prep, kvo_dequant_f16).  The MMA's summation order is not restated
 * (sequential here), so this matches the reference to fp32 rounding, not bitwise.
 */
typedef struct {
    const float *q, *K, *V;
    int L, T, R;
    int nch, cs;
    float * part; /* [nch][R][256] */
    float * ml;   /* [nch][R][2] */
    int c_lo, c_hi;
} ChunkJob;

static void attn_chunk_run(const float * q, const float * K, const float * V, int L, int T, int R, int c0, int c1, float * O, float * mlo) {
    float m[48], l[48];
    for (int r = 0; r < R; r++) {
        m[r] = -INFINITY;
        l[r] = 0.f;
        for (int i = 0; i < HD; i++) O[r * HD + i] = 0.f;
    }
    float S[ATP];
    float P[ATP];
    for (int tb = c0; tb < c1; tb += ATP) {
        const int np = (c1 - tb) < ATP ? (c1 - tb) : ATP;
        for (int r = 0; r < R; r++) {
            const int lim = L - T + (r % T);
            const float * qr = q + (size_t) r * HD;
            float mt = -INFINITY;
            for (int j = 0; j < ATP; j++) {
                float a = -INFINITY;
                if (j < np && tb + j <= lim) {
                    const float * kr = K + (size_t) (tb + j) * HD;
                    a = 0.f;
                    for (int i = 0; i < HD; i++) a = fmaf(qr[i], kr[i], a);
                }
                S[j] = a;
                mt = fmaxf(mt, a);
            }
            const float mnew = fmaxf(m[r], mt);
            float al = 1.f, ps = 0.f;
            for (int j = 0; j < ATP; j++) P[j] = 0.f;
            if (mnew != -INFINITY) {
                for (int j = 0; j < ATP; j++) {
                    const float p = expf(S[j] - mnew);
                    ps += p;
                    P[j] = kvo_h2f(kvo_f2h(p));
                }
                al = expf(m[r] - mnew);
            }
            l[r] = fmaf(l[r], al, ps); /* nvcc contracts sL * al + ps */
            m[r] = mnew;
            float * o = O + (size_t) r * HD;
            for (int i = 0; i < HD; i++) o[i] *= al;
            for (int j = 0; j < np; j++) {
                if (P[j] == 0.f) continue;
                const float * vr = V + (size_t) (tb + j) * HD;
                for (int i = 0; i < HD; i++) o[i] = fmaf(P[j], vr[i], o[i]);
            }
        }
    }
    for (int r = 0; r < R; r++) {
        mlo[2 * r] = m[r];
        mlo[2 * r + 1] = l[r];
    }
}

static void * chunk_job_main(void * arg) {
    ChunkJob * j = (ChunkJob *) arg;
    for (int c = j->c_lo; c < j->c_hi; c++) {
        const int c0 = c * j->cs, c1 = (c0 + j->cs) < j->L ? (c0 + j->cs) : j->L;
        attn_chunk_run(j->q, j->K, j->V, j->L, j->T, j->R, c0, c1, j->part + (size_t) c * j->R * HD, j->ml + (size_t) c * j->R * 2);
    }
    return NULL;
}

static void attn_combine_rows(const float * part, const float * ml, int nch, int R, float * out) {
    for (int r = 0; r < R; r++) {
        float M = -INFINITY;
        for (int c = 0; c < nch; c++) M = fmaxf(M, ml[(size_t) c * R * 2 + 2 * r]);
        float den = 0.f;
        float num[HD];
        for (int i = 0; i < HD; i++) num[i] = 0.f;
        for (int c = 0; c < nch; c++) {
            const float mc = ml[(size_t) c * R * 2 + 2 * r];
            const float w = mc == -INFINITY ? 0.f : expf(mc - M);
            den = fmaf(w, ml[(size_t) c * R * 2 + 2 * r + 1], den);
            for (int i = 0; i < HD; i++) num[i] = fmaf(w, part[((size_t) c * R + r) * HD + i], num[i]);
        }
        for (int i = 0; i < HD; i++) out[(size_t) r * HD + i] = num[i] / den;
    }
}

/* nthreads <= 1: single-threaded.  Returns 0, -1 on bad arguments. */
int kvo_attn_chunked(const float * q, const float * K, const float * V, int L, int T, int R, float * out, int nthreads) {
    if (L <= 0 || T <= 0 || R <= 0 || R > 48 || T > L) return -1;
    int nch, cs;
    kvo_attn_dims(L, &nch, &cs);
    float * part = (float *) malloc(sizeof(float) * (size_t) nch * R * HD);
    float * ml = (float *) malloc(sizeof(float) * (size_t) nch * R * 2);
    if (nthreads < 1) nthreads = 1;
    if (nthreads > nch) nthreads = nch;
    ChunkJob jobs[64];
    pthread_t th[64];
    if (nthreads > 64) nthreads = 64;
    for (int i = 0; i < nthreads; i++) {
        jobs[i] = (ChunkJob) {q, K, V, L, T, R, nch, cs, part, ml, nch * i / nthreads, nch * (i + 1) / nthreads};
        if (nthreads > 1) pthread_create(&th[i], NULL, chunk_job_main, &jobs[i]);
        else chunk_job_main(&jobs[i]);
    }
    if (nthreads > 1)
        for (int i = 0; i < nthreads; i++) pthread_join(th[i], NULL);
    attn_combine_rows(part, ml, nch, R, out);
    free(part);
    free(ml);
    return 0;
}

/* ---------------------------------------------------------------- multi-head batch for the CPU baseline */

typedef struct {
    const float *q, *K, *V;
    int L, T, R, nkv;
    float * out;
    int g;
} HeadJob;

static void * head_job_main(void * arg) {
    HeadJob * j = (HeadJob *) arg;
    kvo_attn_chunked(j->q + (size_t) j->g * j->R * HD, j->K + (size_t) j->g * j->L * HD, j->V + (size_t) j->g * j->L * HD, j->L, j->T, j->R,
                     j->out + (size_t) j->g * j->R * HD, 1);
    return NULL;
}

/* nkv heads: q [nkv][R][256], K/V [nkv][L][256], out [nkv][R][256]; threads split (head, chunk) work: with
 * nthreads >= nkv each head gets nthreads / nkv threads over its chunks. */
int kvo_attn_heads(const float * q, const float * K, const float * V, int nkv, int L, int T, int R, float * out, int nthreads) {
    if (nkv <= 0 || nkv > 64) return -1;
    if (nthreads <= nkv) {
        HeadJob jobs[64];
        pthread_t th[64];
        const int nt = nthreads < 1 ? 1 : nthreads;
        for (int g0 = 0; g0 < nkv; g0 += nt) {
            const int n = (nkv - g0) < nt ? (nkv - g0) : nt;
            for (int i = 0; i < n; i++) {
                jobs[i] = (HeadJob) {q, K, V, L, T, R, nkv, out, g0 + i};
                if (n > 1) pthread_create(&th[i], NULL, head_job_main, &jobs[i]);
                else head_job_main(&jobs[i]);
            }
            if (n > 1)
                for (int i = 0; i < n; i++) pthread_join(th[i], NULL);
        }
        return 0;
    }
    for (int g = 0; g < nkv; g++) {
        const int r = kvo_attn_chunked(q + (size_t) g * R * HD, K + (size_t) g * L * HD, V + (size_t) g * L * HD, L, T, R, out + (size_t) g * R * HD,
                                       nthreads);
        if (r) return r;
    }
    return 0;
}

/* ---------------------------------------------------------------- append batch for the CPU baseline */

typedef struct {
    const float * kv; /* [rows][256] */
    int rows, rot, bits, lo, hi;
    uint8_t * mq;
    uint16_t * ms;
    int8_t * rq;
    uint16_t * rs;
} StoreJob;

static void * store_job_main(void * arg) {
    StoreJob * j = (StoreJob *) arg;
    const int rb = kvo_row_bytes(j->bits);
    for (int i = j->lo; i < j->hi; i++)
        kvo_store_row(j->kv + (size_t) i * HD, j->rot, j->bits, j->mq + (size_t) i * rb, j->ms + (size_t) i * 8, j->rq ? j->rq + (size_t) i * HD : NULL,
                      j->rs ? j->rs + (size_t) i * 8 : NULL);
    return NULL;
}

/* store `rows` rows of one side (all with the same format) over nthreads threads */
void kvo_store_rows(const float * kv, int rows, int rot, int bits, uint8_t * mq, uint16_t * ms, int8_t * rq, uint16_t * rs, int nthreads) {
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 64) nthreads = 64;
    if (nthreads > rows) nthreads = rows > 0 ? rows : 1;
    StoreJob jobs[64];
    pthread_t th[64];
    for (int i = 0; i < nthreads; i++) {
        jobs[i] = (StoreJob) {kv, rows, rot, bits, rows * i / nthreads, rows * (i + 1) / nthreads, mq, ms, rq, rs};
        if (nthreads > 1) pthread_create(&th[i], NULL, store_job_main, &jobs[i]);
        else store_job_main(&jobs[i]);
    }
    if (nthreads > 1)
        for (int i = 0; i < nthreads; i++) pthread_join(th[i], NULL);
}

/* ---------------------------------------------------------------- state digest (engine.cu:1444-1456) */

uint64_t kvo_dg_hash(const void * p, size_t nb, uint64_t h) {
    const unsigned char * b = (const unsigned char *) p;
    size_t i = 0;
    for (; i + 8 <= nb; i += 8) {
        uint64_t w;
        memcpy(&w, b + i, 8);
        h = (h ^ w) * 0x100000001b3ULL;
        h ^= h >> 31;
    }
    for (; i < nb; i++) h = (h ^ b[i]) * 0x100000001b3ULL;
    return h;
}
/* one row's digest word: the scales hashed with the values' hash as seed (engine.cu:1487) */
uint64_t kvo_row_digest(const uint8_t * q, int bits, const uint16_t * sc) {
    return kvo_dg_hash(sc, 16, kvo_dg_hash(q, (size_t) kvo_row_bytes(bits), 0xcbf29ce484222325ULL));
}

double kvo_now(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double) ts.tv_sec + 1e-9 * (double) ts.tv_nsec;
}

/* ---------------------------------------------------------------- combine epilogue (qwen38_mk.cu:4686-4688) */
/* the sigmoid output gate */
float kvo_gate(float y, float g) { return y / (1.0f + expf(-g)); }

/* q32_store of one token's output row o[24 * 256] into the o_proj activation units (qwen38_mk.cu:283-307): block
 * j = 8 head + k (32 values, element 32 j + i) -> amax, d = amax / 127 (IEEE division), q = roundf(v / d) (half away from
 * zero; 0 when amax = 0); unit gi = 8 (j >> 3) + 2 ((j >> 1) & 3) + hh for the block's halves hh = i / 16: bytes
 * (j odd ? xb : xa)[gi * 16 + i % 16]; meta[gi] = {half scale of the xa block, of the xb block, int sum of the xa
 * half, of the xb half} (uint16 x 4). */
void kvo_q32_row(const float * o, int8_t * xa, int8_t * xb, uint16_t * meta) {
    for (int j = 0; j < 192; j++) {
        const float * v = o + 32 * j;
        float am = 0.f;
        for (int i = 0; i < 32; i++) am = fmaxf(am, fabsf(v[i]));
        const float d = am / 127.0f;
        int qs[2] = {0, 0};
        const int part = j & 1, gi0 = 8 * (j >> 3) + 2 * ((j >> 1) & 3);
        for (int i = 0; i < 32; i++) {
            const int q = am == 0.0f ? 0 : (int) roundf(v[i] / d);
            const int gi = gi0 + i / 16;
            (part ? xb : xa)[gi * 16 + i % 16] = (int8_t) q;
            qs[i / 16] += q;
        }
        for (int hh = 0; hh < 2; hh++) {
            const int gi = gi0 + hh;
            meta[gi * 4 + part] = kvo_f2h(d);
            meta[gi * 4 + 2 + part] = (uint16_t) (int16_t) qs[hh];
        }
    }
}

/* RoPE text table rows p0 .. p0+n-1: out[(r * 32 + i) * 2 + {0, 1}] = (cos, sin) of p * 1e7^(-2i/64), computed in double
 * and rounded to float (loader.cu:1252-1258, ROPE_BASE mk_shared.cuh:240). */
void kvo_rope_rows(int p0, int n, float * out) {
    for (int r = 0; r < n; r++)
        for (int i = 0; i < 32; i++) {
            const double th = (double) (p0 + r) * pow(10000000.0, -2.0 * i / 64.0);
            out[(r * 32 + i) * 2] = (float) cos(th);
            out[(r * 32 + i) * 2 + 1] = (float) sin(th);
        }
}

/* Q/K prep of one 256-value row (qwen38_mk.cu:2903-2910, rope8 :2623-2636, EPS mk_shared.cuh:239): RMSNorm with eps
 * 1e-6 and weights w, then pair (i, i + 32), i < 32, rotated by rc[i] = (cos, sin): first = a c - b s, second =
 * b c + a s.  The order is the HIP kernels' (qk_prep): 64 partial sums of 4 squares as an FMA chain, an xor-butterfly
 * over the 64 partials, 1 / sqrtf (the reference: rsqrtf, an approximation within 2 ulp), the weight folded into the
 * scale first, the rotation as one FMA over a rounded product. */
void kvo_qk_prep(const float * x, const float * w, const float * rc, float * out) {
    float s[64], t[64], v[HD];
    for (int l = 0; l < 64; l++) {
        const float * a = x + 4 * l;
        s[l] = fmaf(a[3], a[3], fmaf(a[2], a[2], fmaf(a[1], a[1], a[0] * a[0])));
    }
    for (int m = 1; m < 64; m <<= 1) {
        for (int l = 0; l < 64; l++) t[l] = s[l] + s[l ^ m];
        memcpy(s, t, sizeof s);
    }
    const float rs = 1.0f / sqrtf(s[0] / 256.0f + 1e-6f);
    for (int i = 0; i < HD; i++) v[i] = x[i] * (rs * w[i]);
    for (int i = 0; i < 32; i++) {
        const float c = rc[2 * i], sn = rc[2 * i + 1], a = v[i], b = v[i + 32];
        v[i] = fmaf(a, c, -(b * sn));
        v[i + 32] = fmaf(a, sn, b * c);
    }
    memcpy(out, v, sizeof v);
}
