// Split-K decode attention launchers, the L2 prefetch, the combine kernels and prefill attention (gfx950).  The
// decode kernel template is in kv_attn_decode.h.
#include "kv_attn_decode.h"

namespace qkv {

// ------------------------------------------------------------------------------------------------ prefetch
// The first `tiles` tiles of every wave slice of an attention launch's work items copied into LDS and dropped: the
// bytes pass through the L2 of the XCD that workgroup x runs on, and the attention launch with the same arguments puts
// work item x on workgroup x -- the same XCD (workgroups go round-robin over the XCDs by index) -- so its first tile
// copies hit that L2 (or the last-level cache) instead of HBM.  No results: issued ahead of the attention, on another
// stream beside independent work (the reference's pf_l2 in attn_proj, qwen38_mk.cu:2600-2621).
// One workgroup per (sequence, layer, kv head, segment): the launch's n_base work items.  (An attention launch of
// T = 5..8 in two 24-row batches has n_items = 2 n_base; batch b of item x is not item n_base + x, and an index past
// n_base names a layer outside the launch.)  Item x's batches run on workgroups of x's XCD (kv_attn_decode.h), as x does
// here.
template <int KB, int VB>
__global__ __launch_bounds__(256) void k_prefetch(AttnArgs a, int tiles) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const StoreLayout & S = a.S;
    const unsigned st_lds = (unsigned) __builtin_amdgcn_readfirstlane((unsigned) (size_t) (__attribute__((address_space(3))) uint8_t *) smem + wv * STAGE_BYTES);
    for (int item = blockIdx.x; item < a.n_base; item += gridDim.x) {
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

// one (row, 64-dim quarter dq) of the output from the row's segment partials; part / ml / out as in AttnArgs, nseg and
// item0 those of the row's sequence si
__device__ __forceinline__ void combine_split_core(const float * __restrict__ part, const float2 * __restrict__ ml_, float * out, int R, int T,
                                                   int nseq, int nseg, int item0, const CombineRow & cr, int dq, uint8_t * scratch) {
    float4 (*s_num)[16] = reinterpret_cast<float4 (*)[16]>(scratch);        // [AWAVES][16]
    float2 * s_md = reinterpret_cast<float2 *>(scratch + AWAVES * 16 * 16); // [AWAVES]
    const int r = cr.r, g = cr.g, si = cr.si, l = cr.l;
    const size_t head0 = (size_t) item0 + (size_t) (l * NKV + g) * nseg;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, sub = lane >> 4, dl = lane & 15;
    const int slot = 4 * wv + sub, dim = 64 * dq + 4 * dl;
    constexpr int PER = MAX_SEG / 16;
    float2 ml[PER];
    float4 o[PER];
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const int c = slot + 16 * k;
        if (c < nseg) {
            ml[k] = ml_[(head0 + c) * R + r];
            o[k] = *reinterpret_cast<const float4 *>(part + ((head0 + c) * R + r) * HD + dim);
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
        *reinterpret_cast<float4 *>(out + (((size_t) (l * nseq + si) * T + t) * NH + h) * HD + dim) =
            make_float4(y.x / dd, y.y / dd, y.z / dd, y.w / dd);
    }
}

__global__ __launch_bounds__(256) void k_combine(AttnArgs a) {
    __shared__ __attribute__((aligned(16))) uint8_t scratch[AWAVES * 64 * 16 + AWAVES * 8];
    combine_row(a, combine_row_of(a, blockIdx.x), scratch);
}

__global__ __launch_bounds__(256) void k_combine_split(AttnArgs a) {
    __shared__ __attribute__((aligned(16))) uint8_t scratch[AWAVES * 16 * 16 + AWAVES * 8];
    const CombineRow cr = combine_row_of(a, blockIdx.x >> 2);
    const SeqDesc & sd = a.sd[cr.si];
    combine_split_core(a.part, a.ml, a.out, a.R, a.T, a.nseq, sd.nseg, sd.item0, cr, blockIdx.x & 3, scratch);
}

// the same for one sequence, with every argument a scalar: they arrive preloaded in SGPRs (kernel-argument preloading,
// build flags of this file), so the partials' loads issue without a round trip to the argument segment first
__global__ __launch_bounds__(256) void k_combine_split1(const float * part, const float2 * ml, float * out, int R, int T, int nseg, int item0) {
    __shared__ __attribute__((aligned(16))) uint8_t scratch[AWAVES * 16 * 16 + AWAVES * 8];
    int b = blockIdx.x >> 2;
    CombineRow cr;
    cr.r = b % R;
    b /= R;
    cr.g = b % NKV;
    cr.si = 0;
    cr.l = b / NKV;
    combine_split_core(part, ml, out, R, T, 1, nseg, item0, cr, blockIdx.x & 3, scratch);
}

// launches whose rows need the whole row in one workgroup (V stored rotated, gate, o_proj units) use the row form
static bool host_combine_needs_rows(const AttnArgs & a) {
    const unsigned vrot = (a.vrot >> a.layer0) & ((a.nl >= 32 ? 0u : 1u << a.nl) - 1u);
    return vrot || a.gate || a.q32a;
}

hipError_t launch_combine(const AttnArgs & a, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1) {
    const unsigned rows = (unsigned) (a.nl * a.nseq * NKV * a.R);
    if (host_combine_needs_rows(a)) hipExtLaunchKernelGGL(k_combine, dim3(rows), dim3(256), 0, st, ev0, ev1, 0, a);
    else if (a.nseq == 1)
        hipExtLaunchKernelGGL(k_combine_split1, dim3(4 * rows), dim3(256), 0, st, ev0, ev1, 0, (const float *) a.part, (const float2 *) a.ml, a.out,
                              a.R, a.T, a.sd[0].nseg, a.sd[0].item0);
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

// fp16 tile layout in LDS: K and V as [32][SK_LD] (row = position; the consumers read V transposed, read_tr16)
constexpr int SK_LD = HD + 8;
// V rows 560 bytes apart: the 4 rows that one 16-lane group of a transposed read addresses (32 bytes each) start 32
// bytes apart in the banks instead of overlapping (528 bytes: 3.6% slower; 576: 4% slower; 592: the same as 560)
constexpr int SV_LD = HD + 24;
typedef float f32x16 __attribute__((ext_vector_type(16)));

// Prefill attention on 32x32x16 MFMAs: workgroup = (128 query rows, kv head, key segment), row block fastest so the
// workgroups of one segment run side by side; 8 waves.  Waves 0-3 (consumers) hold 32 query
// rows each and run the MFMAs and the softmax on the fp16 tile of buffer i % 2; waves 4-7 (producers) each copy an
// 8-position quarter of the tiles (two tiles in flight) and dequantize exactly what they copied into the other
// buffer.  One barrier per tile hands a buffer over; on each SIMD a producer's VALU work overlaps a consumer's MFMAs.
constexpr int PQ_REGION = 5120;                           // per producer and stage: K rows 2 KB, V rows 2 KB, scales 1 KB
constexpr int PQ_STAGES = 2 * 4 * PQ_REGION;              // two stages of the 4 producers
constexpr int PQ_BUF = ATP * (SK_LD + SV_LD) * 2;        // one fp16 tile: K [32][SK_LD], V [32][SV_LD]
constexpr int PQ_LDS = PQ_STAGES + 2 * PQ_BUF;

typedef __fp16 f16v4 __attribute__((__vector_size__(4 * sizeof(__fp16))));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
// ds_read_b64_tr_b16 at LDS byte address off: in each group of 16 lanes, lane i receives element i % 4 of the 8-byte
// pieces addressed by lanes i / 4 + 4 j, j = 0..3 (as element j)
__device__ __forceinline__ half4 read_tr16(unsigned off) {
    return __builtin_bit_cast(half4, __builtin_amdgcn_ds_read_tr16_b64_v4f16((__attribute__((address_space(3))) f16v4 *) (size_t) off));
}

// Instruction order for an unrolled chain of N LDS fragment reads each feeding one MFMA: the first D reads, then one
// MFMA and the next read in turn, then the last D MFMAs (scheduling groups; no effect on the arithmetic).  Left to
// itself the scheduler reads each fragment just before its MFMA into the same registers, so every MFMA of the chain
// waits a whole LDS round trip.
// K: 3 fragments ahead; V: 2 MFMAs ahead (4 transposed reads).  Measured: K 2 ahead 1.3% slower, V 3 or 4 ahead
// 1.1% and 0.3% slower.
constexpr int PF_K = 3, PF_V = 2;
template <int D, int N, int RPM = 1>
__device__ __forceinline__ void pipeline_reads() {
    if constexpr (D > 0) {
        __builtin_amdgcn_sched_group_barrier(0x100, D * RPM, 0); // DS reads
#pragma unroll
        for (int i = 0; i < N - D; i++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0); // MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, RPM, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, D, 0);
    }
}
static_assert(PQ_LDS >= PF2_ROWS * SK_LD * 2, "query staging inside the tile buffers");

// the 8 positions of quarter pw of tile i: one producer wave's copies (5 instructions, always) into its region
template <int KB, int VB>
__device__ __forceinline__ void pq_issue(const TileSrc & t, int nq, unsigned lds, int lane) {
    constexpr int KRB = 32 * KB, VRB = 32 * VB; // row bytes
#pragma unroll
    for (int j = 0; j < 2; j++) {
        int o = 1024 * j + 16 * lane;
        if (o >= nq * KRB) o = nq * KRB - 16;
        dma16_keep(t.k + o, lds + 1024 * j);
    }
#pragma unroll
    for (int j = 0; j < 2; j++) {
        int o = 1024 * j + 16 * lane;
        if (o >= nq * VRB) o = nq * VRB - 16;
        dma16_keep(t.v + o, lds + 2048 + 1024 * j);
    }
    const int r = min(lane & 7, nq - 1);
    dma16_keep(lane < 8 ? static_cast<const void *>(t.ks + 8 * r) : static_cast<const void *>(t.vs + 8 * r), lds + 4096);
}

// one producer lane: position lane % 8 of its quarter, scale block lane / 8, K and V into the fp16 buffer
template <int KB, int VB>
__device__ __forceinline__ void pq_dequant(const uint8_t * reg, int pw, int lane, _Float16 * sK, _Float16 * sV) {
    const int pl = lane & 7, b = lane >> 3, p = 8 * pw + pl;
    const uint16_t * ksc = reinterpret_cast<const uint16_t *>(reg + 4096);
    half2v o[16];
    dequant_block<KB>(reg + pl * 32 * KB, ksc[pl * 8 + b], b, o);
    uint4 * kd = reinterpret_cast<uint4 *>(sK + p * SK_LD + 32 * b);
#pragma unroll
    for (int k = 0; k < 4; k++) kd[k] = make_uint4(as_u(o[4 * k]), as_u(o[4 * k + 1]), as_u(o[4 * k + 2]), as_u(o[4 * k + 3]));
    dequant_block<VB>(reg + 2048 + pl * 32 * VB, ksc[64 + pl * 8 + b], b, o);
    uint4 * vd = reinterpret_cast<uint4 *>(sV + p * SV_LD + 32 * b);
#pragma unroll
    for (int k = 0; k < 4; k++) vd[k] = make_uint4(as_u(o[4 * k]), as_u(o[4 * k + 1]), as_u(o[4 * k + 2]), as_u(o[4 * k + 3]));
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
    // by value: held in registers, not re-read from the kernel arguments for every tile
    const SideLayout SK = S.side[a.layer][0];
    const SideLayout SV = S.side[a.layer][1];
    const size_t ring0 = (size_t) (a.seq * NKV + g) * S.kvrc;
    const int L = a.L, ws = a.ws;
    auto is_ring = [&](int i) { return S.kvrc > 0 && c0 + ATP * i >= ws; };
    // the producer's tiles are issued in order 0, 1, 2, ..: the page and offset of the next one are tracked (a tile
    // never straddles a page: pages hold a multiple of 32 positions), and a page's physical index is looked up when the
    // previous tile ends the previous page, one tile before its copies are issued
    const int * const pt = S.ptab + (size_t) a.seq * S.pt_stride;
    int nx_lp = c0 / S.page, nx_off = c0 - nx_lp * S.page;
    int nx_phys = ((const_int_p) pt)[nx_lp];
    // producer: the copies of quarter pw of tile i into stage i % 2
    auto issue = [&](int i) {
        const int p0t = c0 + ATP * i, nv = min(ATP, L - p0t);
        const int q0 = min(8 * pw, nv - 1), nq = min(8, nv - q0), p0 = p0t + q0;
        const unsigned lds = (unsigned) __builtin_amdgcn_readfirstlane(lds0 + ((i & 1) * 4 + pw) * PQ_REGION);
        const bool ring = is_ring(i);
        const size_t mr = (size_t) (g * S.n_pages + nx_phys) * S.page + nx_off + q0;
        nx_off += ATP;
        if (nx_off == S.page) {
            nx_off = 0;
            nx_lp++;
            if (i + 1 < ntiles) nx_phys = ((const_int_p) pt)[nx_lp];
        }
        const TileSrc t = tile_src_row<KB, VB>(S.kvrc, SK, SV, !ring || !SK.ring || !SV.ring ? mr : 0, p0, ring0, ring);
        if (ring) pq_issue<8, 8>(t, nq, lds, lane);
        else pq_issue<KB, VB>(t, nq, lds, lane);
    };
    auto dequant = [&](int i) {
        const uint8_t * reg = smem + ((i & 1) * 4 + pw) * PQ_REGION;
        _Float16 * sK = buf0 + (i & 1) * (PQ_BUF / 2);
        _Float16 * sV = sK + ATP * SK_LD;
        if (is_ring(i)) pq_dequant<8, 8>(reg, pw, lane, sK, sV);
        else pq_dequant<KB, VB>(reg, pw, lane, sK, sV);
    };
    // ---- query rows: all 8 waves stage 16 rows each (prep, FWHT for rotated K, * 1/16, fp16), consumers take fragments;
    // loaded 8 rows at a time (independent loads, one wait)
    _Float16 * const qs = reinterpret_cast<_Float16 *>(smem);
    for (int jb = 0; jb < 16; jb += 8) {
        float4 xs[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int r = r0 + 16 * wv + jb + u, t = r / GQA, hh = r - GQA * t;
            xs[u] = r < a.R ? *reinterpret_cast<const float4 *>(a.q + ((size_t) t * NH + GQA * g + hh) * a.qs + 4 * lane)
                            : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
    for (int u = 0; u < 8; u++) {
        const int rl = 16 * wv + jb + u, r = r0 + rl;
        half2v o0 = {(_Float16) 0.f, (_Float16) 0.f}, o1 = o0;
        if (r < a.R) {
            const int t = r / GQA;
            const float4 x = xs[u];
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
    }
    __syncthreads();
    // Both roles pass the same barriers: two after the staging, then one per tile.
    if (producer) {
        // the producers set the pace (their dequantization and fp16 tile writes take longer per tile than a consumer's
        // MFMAs and softmax): on a SIMD shared with a consumer, the arbiter's preference for the older wave (the
        // consumer) would otherwise give the consumer's issue slots first
        __builtin_amdgcn_s_setprio(1);
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
        const _Float16 * const sV = sK + ATP * SK_LD;
        // V operand of O^T += V^T P^T (lane l: dim 32 db + l % 32, the 8 positions of P's k order for half hf) by two
        // transposed reads of 4 positions: lane a = q + 4 j of each 16-lane group g addresses position 16 s2 + 4 hf + j
        // (+ 8 for the second read), dims 32 db + 16 (g & 1) + 4 q .. + 3, and lane i of the group receives dim
        // 32 db + 16 (g & 1) + i of the 4 positions
        const unsigned v_lane = (unsigned) (size_t) (const __attribute__((address_space(3))) _Float16 *) sV +
                                2 * ((4 * hf + ((lane >> 2) & 3)) * SV_LD + 16 * ((lane >> 4) & 1) + 4 * (lane & 3));
        const int p0 = c0 + ATP * i;
        f32x16 sacc;
#pragma unroll
        for (int e = 0; e < 16; e++) sacc[e] = 0.f;
#pragma unroll
        for (int ks = 0; ks < 16; ks++) {
            const half8 ak = *reinterpret_cast<const half8 *>(sK + c * SK_LD + 16 * ks + 8 * hf);
            sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ak, qf[ks], sacc, 0, 0, 0);
        }
        // the K fragments are read PF_K ahead of their MFMAs: each read's LDS latency then hides behind the MFMAs
        // already issued instead of standing between two MFMAs of the chain
        pipeline_reads<PF_K, 16>();
        // fully visible tiles (wave-uniform) skip the causal mask
        float mx = -INFINITY;
        if (p0 + ATP - 1 <= lim_min) {
#pragma unroll
            for (int e = 0; e < 16; e++) {
                sacc[e] = sacc[e] * LOG2E;
                mx = fmaxf(mx, sacc[e]);
            }
        } else {
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const int pos = p0 + 8 * (e >> 2) + 4 * hf + (e & 3);
                sacc[e] = pos <= lim ? sacc[e] * LOG2E : -INFINITY;
                mx = fmaxf(mx, sacc[e]);
            }
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
                const unsigned vo = v_lane + 2 * ((16 * s2) * SV_LD + 32 * db);
                const half8 av = __builtin_shufflevector(read_tr16(vo), read_tr16(vo + 2 * 8 * SV_LD), 0, 1, 2, 3, 4, 5, 6, 7);
                O[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, pb[s2], O[db], 0, 0, 0);
            }
        pipeline_reads<PF_V, 16, 2>(); // (the score registers are free here: the V fragments have room to run further ahead)
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
    // up to 8 segments' partials loaded in one round, then folded in order (the fold is the same sequence of operations
    // as one segment at a time)
    constexpr int RND = 8;
    for (int k0 = 0; k0 < nk; k0 += RND) {
        float2 mls[RND];
        float4 os[RND];
#pragma unroll
        for (int j = 0; j < RND; j++)
            if (k0 + j < nk) {
                const size_t u = (size_t) (g * a.nseg + k0 + j) * a.R + r;
                mls[j] = a.ml[u];
                os[j] = *reinterpret_cast<const float4 *>(a.part + u * HD + 4 * lane);
            }
#pragma unroll
        for (int j = 0; j < RND; j++)
            if (k0 + j < nk) {
                const float2 ml = mls[j];
                const float4 o = os[j];
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
    }
    float v[4] = {num.x / den, num.y / den, num.z / den, num.w / den};
    const int h = GQA * g + hh;
    finish_row(v, a.vrot, a.gate ? a.gate + ((size_t) t * NH + h) * a.gs : nullptr, a.out + ((size_t) t * NH + h) * HD, a.q32a,
               a.q32b, a.q32m, (size_t) t, h);
}

// ------------------------------------------------------------------------------------------------ dispatch

template <int NP>
static AttnKernel pick(int kb, int vb) {
#define QKV_VB(K)                                                                                                      \
    switch (vb) {                                                                                                      \
    case 4: return k_attn<NP, K, 4>;                                                                                   \
    case 5: return k_attn<NP, K, 5>;                                                                                   \
    case 6: return k_attn<NP, K, 6>;                                                                                   \
    case 7: return k_attn<NP, K, 7>;                                                                                   \
    case 8: return k_attn<NP, K, 8>;                                                                                   \
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
    // (the fused append runs in two-per-CU kernels only)
    const bool small = !a.kin && np == 1 && kb + vb <= 11 && (occ == 3 || (occ == 0 && a.n_items > 2 * device_cus()));
    if (a.kin) k = pick_fused(np, a.wide, kb, vb);
    else if (small) k = pick_small(kb, vb);
    else if (np == 1) k = pick<1>(kb, vb);
    else if (np == 2) k = pick<2>(kb, vb);
    else if (np == 3) k = a.wide ? verify_of<false>(kb, vb) : pick<3>(kb, vb);
    if (!k) return hipErrorInvalidValue;
    static thread_local const void * configured[256];
    static thread_local int n_configured = 0;
    bool done = false;
    for (int i = 0; i < n_configured; i++) done |= configured[i] == (const void *) k;
    const int lds = a.wide ? 2 * (ATTN_LDS + a.RP * HD * 2) : (small ? AWAVES * (1024 * (kb + vb) + 1024) : ATTN_LDS) + a.RP * HD * 2;
    if (!done) {
        const hipError_t e = hipFuncSetAttribute((const void *) k, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
        if (e != hipSuccess) return e;
        if (n_configured < 256) configured[n_configured++] = (const void *) k;
    }
    int blocks = a.n_items;
    if (a.wide) blocks = std::min(blocks, device_cus()); // k_verify: persistent, one workgroup per CU
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
    hipLaunchKernelGGL((k_prefetch<KB, VB>), dim3(a.n_base), dim3(256), lds, st, a, tiles);
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
