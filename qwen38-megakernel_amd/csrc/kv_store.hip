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
__global__ __launch_bounds__(256) void k_append(StoreLayout S, int seq, int layer0, int nl, int pos, int T, const void * kin,
                                                const void * vin, int f16, const float * knw, const float2 * rope) {
    // the row index as a scalar: the side's layout and the page-table entry then come from scalar loads issued at the
    // start, not from vector loads whose waits would put a memory round trip between each step of the row
    const int wave = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // the arguments the input address needs, in one round of scalar loads (not one round before the bounds check and
    // another after it)
    asm volatile("" ::"s"(T), "s"(nl), "s"(pos), "s"(kin), "s"(vin), "s"(f16), "s"(S.ptab), "s"(S.pt_stride), "s"(S.page), "s"(S.n_pages),
                 "s"(S.kvrc));
    if (wave >= T * nl * NKV * 2) return;
    const int w = wave & 1;
    int r = wave >> 1;
    const int g = r % NKV;
    r /= NKV;
    const int l = r % nl, t = r / nl;
    const size_t src = ((size_t) (t * nl + l) * NKV + g) * HD;
    const int p = pos + t;
    // every load the row needs, issued before the first wait: the input values, then the page-table entry of the main
    // row and the side's layout (scalar loads, made live by the empty asm while the input load is in flight)
    const void * in = w ? vin : kin;
    uint4 raw; // the lane's 4 values as loaded (fp16: the first 8 bytes)
    if (f16) {
        const uint2 x = *reinterpret_cast<const uint2 *>(static_cast<const _Float16 *>(in) + src + 4 * lane_id());
        raw = make_uint4(x.x, x.y, 0u, 0u);
    } else {
        raw = *reinterpret_cast<const uint4 *>(static_cast<const float *>(in) + src + 4 * lane_id());
    }
    // (the page-table entry through the constant address space: a scalar load; no kernel writes the table)
    const int lp = p / S.page;
    const int phys = ((const __attribute__((address_space(4))) int *) S.ptab)[seq * S.pt_stride + lp];
    const size_t row = (size_t) (g * S.n_pages + phys) * S.page + (p - lp * S.page);
    const size_t rr = S.kvrc > 0 ? ring_row(S, seq, g, p) : 0;
    const SideLayout sd = S.side[layer0 + l][w];
    asm volatile("" ::"s"(sd.vals), "s"(sd.scs), "s"(sd.ring), "s"(sd.rsc), "s"(sd.bits), "s"(sd.rot));
    float v[4];
    if (f16) {
        const half2v a = __builtin_bit_cast(half2v, raw.x), b = __builtin_bit_cast(half2v, raw.y);
        v[0] = (float) a[0];
        v[1] = (float) a[1];
        v[2] = (float) b[0];
        v[3] = (float) b[1];
    } else {
        v[0] = __builtin_bit_cast(float, raw.x);
        v[1] = __builtin_bit_cast(float, raw.y);
        v[2] = __builtin_bit_cast(float, raw.z);
        v[3] = __builtin_bit_cast(float, raw.w);
    }
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
    hipExtLaunchKernelGGL(k_append, dim3((waves + 3) / 4), dim3(256), 0, st, ev0, ev1, 0, S, seq, layer0, nl, pos, T, k, v, f16, knw,
                          rope);
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
