// Append/evict half of the KV path (gfx950, wave64).
//
// k_append      : new K/V rows -> optional K prep (RMSNorm + RoPE) -> optional 256-point FWHT -> main row in the side's format (q8 or 4..7-bit packed)
//                 and, for sides with a window, the q8 ring copy of the same rotated values (kv_store,
//                 qwen38_mk.cu:2099-2116).  Eviction from the window is ring-slot reuse plus the read-side window
//                 rule: the packed row was written from the same fp32 values, so nothing is requantized later.
// k_ring_refill : after a rewind, ring rows re-stored as q8 of the fp32-dequantized main rows (k_ring_refill,
//                 qwen38_mk.cu:2485-2517).
#include "kv_dev.h"
#include "kv_launch.h"

namespace qkv {

// One wave per row; lane l holds values 4l .. 4l+3.  Rows of the input: [T][nl][NKV][256] (fp16 or fp32).
// The scalar arguments come first: this file is built with kernel-argument preloading (the first 14 dwords arrive in
// SGPRs at wave launch), so the input address and the page-table entry's address (ptab, pt_stride, page: copies of
// S's) need no round trip to the argument segment, and every load of the row issues at once.
__global__ __launch_bounds__(256) void k_append(int seq, int layer0, int nl, int pos, int T, int f16, const void * kin, const void * vin,
                                                const int * ptab, int pt_stride, int page, StoreLayout S, const float * knw,
                                                const float2 * rope) {
    // the row index as a scalar: the side's layout and the page-table entry then come from scalar loads issued at the
    // start, not from vector loads whose waits would put a memory round trip between each step of the row
    const int wave = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (wave >= T * nl * NKV * 2) return;
    const int w = wave & 1;
    int r = wave >> 1;
    const int g = r % NKV;
    r /= NKV;
    const int l = r % nl, t = r / nl;
    const size_t src = ((size_t) (t * nl + l) * NKV + g) * HD;
    const int p = pos + t;
    // every load the row needs, issued before the first wait: the page-table entry of the main row and the side's
    // layout (scalar loads; the page table through the constant address space: no kernel writes it), and the input
    // values; the empty asm after the input load makes the scalar values live while that load is in flight
    const int lp = p / page;
    const int phys = ((const __attribute__((address_space(4))) int *) ptab)[seq * pt_stride + lp];
    const SideLayout sd = S.side[layer0 + l][w];
    const void * in = w ? vin : kin;
    float v[4];
    if (f16) {
        const uint2 x = *reinterpret_cast<const uint2 *>(static_cast<const _Float16 *>(in) + src + 4 * lane_id());
        asm volatile("" ::"s"(phys), "s"(sd.vals), "s"(sd.scs), "s"(sd.ring), "s"(sd.rsc), "s"(sd.bits), "s"(sd.rot), "s"(S.n_pages), "s"(S.kvrc));
        const half2v a = __builtin_bit_cast(half2v, x.x), b = __builtin_bit_cast(half2v, x.y);
        v[0] = (float) a[0];
        v[1] = (float) a[1];
        v[2] = (float) b[0];
        v[3] = (float) b[1];
    } else {
        const float4 x = *reinterpret_cast<const float4 *>(static_cast<const float *>(in) + src + 4 * lane_id());
        asm volatile("" ::"s"(phys), "s"(sd.vals), "s"(sd.scs), "s"(sd.ring), "s"(sd.rsc), "s"(sd.bits), "s"(sd.rot), "s"(S.n_pages), "s"(S.kvrc));
        v[0] = x.x;
        v[1] = x.y;
        v[2] = x.z;
        v[3] = x.w;
    }
    const size_t row = (size_t) (g * S.n_pages + phys) * page + (p - lp * page);
    const size_t rr = S.kvrc > 0 ? ring_row(S, seq, g, p) : 0;
    if (knw && !w) qk_prep(v, knw + (size_t) l * HD, rope + (size_t) p * 32);
    // ring copy: only for the newest kvrc positions of the call (p >= pos + T - kvrc); an older one shares its ring
    // row with a newer position of the same launch and is evicted by it anyway, and writing both would race
    store_row_at(sd, row, rr, p >= pos + T - S.kvrc, v);
}

// One wave per (position, layer, side, kv head) of positions p0 .. p1-1.
__global__ __launch_bounds__(256) void k_ring_refill(StoreLayout S, int seq, int nl, int p0, int n) {
    const int wave = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); // (scalar: the side by scalar loads)
    if (wave >= n * nl * NKV * 2) return;
    const int lane = threadIdx.x & 63;
    const int w = wave & 1;
    int r = wave >> 1;
    const int g = r % NKV;
    r /= NKV;
    const int l = r % nl, p = p0 + r / nl;
    const SideLayout & sd = S.side[l][w];
    if (!sd.ring) return;
    const size_t row = main_row(S, seq, g, p);
    const float d = h2f_bits(sd.scs[row * 8 + (lane >> 3)]);
    float v[4];
    if (sd.bits == 8) {
        const unsigned x = *reinterpret_cast<const unsigned *>(sd.vals + row * HD + 4 * lane);
#pragma unroll
        for (int k = 0; k < 4; k++) v[k] = d * (float) (int8_t) (x >> (8 * k));
    } else {
        const int bits = sd.bits, hb = bits - 4, half = lane & 1, word = lane >> 1, bias = 1 << (bits - 1);
        const uint8_t * rp = sd.vals + row * row_bytes(bits);
        const unsigned W = *reinterpret_cast<const unsigned *>(rp + 4 * word);
        unsigned hi = 0;
        for (int k = 0; k < hb; k++) hi |= (unsigned) rp[128 + word * hb + k] << (8 * k);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int kk = 4 * half + k;
            const unsigned nib = (W >> (8 * k + 4 * half)) & 15u;
            const unsigned hv = hb ? (hi >> (hb * kk)) & ((1u << hb) - 1u) : 0u;
            v[k] = d * (float) ((int) (nib | (hv << 4)) - bias);
        }
    }
    uint16_t rs;
    const unsigned word = quant_q8(v, rs);
    const size_t rr = ring_row(S, seq, g, p);
    *reinterpret_cast<unsigned *>(sd.ring + rr * HD + 4 * lane) = word;
    if ((lane & 7) == 0) sd.rsc[rr * 8 + (lane >> 3)] = rs;
}

hipError_t launch_append(const StoreLayout & S, int seq, int layer0, int nl, int pos, int T, const void * k, const void * v, int f16,
                         hipStream_t st, hipEvent_t ev0, hipEvent_t ev1, const float * knw, const float2 * rope) {
    const int waves = T * nl * NKV * 2;
    hipExtLaunchKernelGGL(k_append, dim3((waves + 3) / 4), dim3(256), 0, st, ev0, ev1, 0, seq, layer0, nl, pos, T, f16, k, v, S.ptab,
                          S.pt_stride, S.page, S, knw, rope);
    return hipGetLastError();
}

hipError_t launch_ring_refill(const StoreLayout & S, int seq, int nl, int p0, int p1, hipStream_t st) {
    const int n = p1 - p0;
    if (n <= 0) return hipSuccess;
    const long long waves = (long long) n * nl * NKV * 2;
    hipLaunchKernelGGL(k_ring_refill, dim3((unsigned) ((waves + 3) / 4)), dim3(256), 0, st, S, seq, nl, p0, n);
    return hipGetLastError();
}

} // namespace qkv
