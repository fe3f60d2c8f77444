// Kernel launchers of the KV path (defined in kv_store.hip / kv_attn*.hip), called by the C-ABI host code.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include "kv_layout.h"

namespace qkv {

// one sequence entry of an attention launch
struct SeqDesc {
    int seq;   // store sequence (lane) index
    int L;     // context length after this call's rows: positions 0 .. L-1
    int ws;    // window start: tiles at positions >= ws are read from the q8 ring
    int cs;    // canonical segment length (a function of L's 640-bucket only)
    int nseg;  // segments: ceil(L / cs) <= 128
    int item0; // first work item of this sequence in the launch
    int pbase; // >= 0: the sequence's pages are pbase, pbase + 1, .. (no table lookup); -1: read the page table
    unsigned nseg_m; // magic31(nseg)
};

// ceil(2^31 / d): floor(n / d) = (2 n * magic31(d)) >> 32 exactly for 0 <= n, 1 <= d with n d < 2^31 (div_m)
inline unsigned magic31(int d) { return (unsigned) (((1ull << 31) + (unsigned) d - 1) / (unsigned) d); }

// The scalars a decode workgroup (k_attn) needs before its first tile copy and for its merge, as 52 dwords at offset 0
// of the kernel arguments: the kernel reads them with four scalar loads and one wait, into registers the
// compiler cannot refill from memory later (it would otherwise re-read fields from the argument segment, each re-read
// a round trip under the launch's load, several of them in series before the first copy).
struct AttnHead {
    uint8_t * kvals; // side0[0]: K of slot layer0
    uint16_t * kscs;
    int8_t * kring;
    uint16_t * krsc;
    uint8_t * vvals; // side0[1]: V of slot layer0
    uint16_t * vscs;
    int8_t * vring;
    uint16_t * vrsc;
    const float * q;       // AttnArgs::q, part, ml, S.ptab, qnw, rope
    float * part;
    float2 * ml;
    const int * ptab;
    const float * qnw;
    const float2 * rope;
    int L, ws, cs, nseg, item0, pbase, seq;                                       // sd[0]
    int n_items, n_base, nseq, T, R, layer0, qs, kvrc, page, n_pages, pt_stride; // AttnArgs / S fields of the same names
    unsigned krot;
    unsigned nseg_m, T_m; // magic31(nseg of sd[0]), magic31(T)
    int pad[3];
};
static_assert(sizeof(AttnHead) == 208, "three 16-dword loads and one 4-dword load");

struct AttnArgs {
    AttnHead h;          // the decode kernels' copy of fields below (fill_head); the others read the fields themselves
    SideLayout side0[2]; // K, V layouts of slot layer0 (S.side[layer0])
    StoreLayout S;
    int layer0;          // first slot of the launch
    int nl;              // layers in the launch (all with the same K/V bits)
    int T, R, RP;        // query tokens, query rows per kv head (6 T), rows per batch: 8 (R <= 8), 16 (R <= 16), else 24
    int nseq;
    int n_base;          // (sequence, layer, kv head, segment) work items
    int n_items;         // n_base (wide), else n_base * ceil(R / RP): every item once per row batch (batch-minor)
    int wide;            // R > 24 in one pass (k_verify: persistent 8-wave workgroups, waves 4..7 holding rows 24..47)
    unsigned krot, vrot; // per-slot bit masks: K / V stored rotated
    SeqDesc sd[8];
    const float * q;     // [nl][nseq][T][NH][HD] queries of this launch's layers (fp32, before the 1/16 scale)
    float * out;         // [nl][nseq][T][NH][HD]
    int qs, gs;          // row strides (floats) of q and gate: 256, or 512 for the q_proj layout [.. NH][q 256 | gate 256]
    const float * qnw;   // optional [nl][HD] q-norm weights: q rows get RMSNorm + RoPE (qk_prep) before use
    const float2 * rope; // with qnw: [positions][32] (cos, sin); row t of a sequence of length L is position L - T + t
    const float * gate;  // optional [nl][nseq][T][NH][gs]: out = y / (1 + exp(-gate))
    int8_t * q32a;       // optional o_proj activation units of out: [nl][nseq][T][192][16] int8 (even blocks)
    int8_t * q32b;       // ... (odd blocks)
    uint16_t * q32m;     // ... [nl][nseq][T][192][4]: half scales of the a / b blocks, int sums of the a / b halves
    float * part;        // [item][R][HD] per-segment partial outputs (unnormalised)
    float2 * ml;         // [item][R] per-segment (max in log2 units, sum)
    // fused append (mk_kv_append_attend): the rows of positions L - T .. L - 1 of every sequence, stored inside this
    // launch by the wave whose tiles hold them, before those tiles are copied.  kin / vin [nseq][T][kin_nl][NKV][HD]
    // (fp16 when kin_f16), layer l of the launch at kin_nl index l; nullptr: no append
    const void * kin;
    const void * vin;
    int kin_nl, kin_f16;
};

// AttnHead from the launch's other fields (after they are final)
inline void fill_head(AttnArgs & a) {
    AttnHead & h = a.h;
    h.kvals = a.side0[0].vals;
    h.kscs = a.side0[0].scs;
    h.kring = a.side0[0].ring;
    h.krsc = a.side0[0].rsc;
    h.vvals = a.side0[1].vals;
    h.vscs = a.side0[1].scs;
    h.vring = a.side0[1].ring;
    h.vrsc = a.side0[1].rsc;
    h.q = a.q;
    h.part = a.part;
    h.ml = a.ml;
    h.ptab = a.S.ptab;
    h.qnw = a.qnw;
    h.rope = a.rope;
    const SeqDesc & d = a.sd[0];
    h.L = d.L;
    h.ws = d.ws;
    h.cs = d.cs;
    h.nseg = d.nseg;
    h.item0 = d.item0;
    h.pbase = d.pbase;
    h.seq = d.seq;
    h.n_items = a.n_items;
    h.n_base = a.n_base;
    h.nseq = a.nseq;
    h.T = a.T;
    h.R = a.R;
    h.layer0 = a.layer0;
    h.qs = a.qs;
    h.kvrc = a.S.kvrc;
    h.page = a.S.page;
    h.n_pages = a.S.n_pages;
    h.pt_stride = a.S.pt_stride;
    h.krot = a.krot;
    h.nseg_m = d.nseg_m;
    h.T_m = magic31(a.T);
    h.pad[0] = h.pad[1] = h.pad[2] = 0;
}

// one prefill piece of one layer: query rows r = 6 t + hh (token t = 0 .. Tp-1 at position n0 + t, query head
// 6 g + hh of kv head g), keys in absolute segments of `seg` positions (pf_seg of the piece's bucket)
struct PrefillArgs {
    StoreLayout S;
    int layer, seq;
    int n0, Tp, L, ws; // first query position, rows' tokens, L = n0 + Tp (one 640-bucket), window start of the bucket
    int R, nrb, nseg;  // 6 Tp rows per kv head, ceil(R / PF2_ROWS) row blocks, ceil(L / seg) key segments
    int seg;           // key positions per segment
    int krot, vrot;
    const float * q;   // [Tp][NH][qs]
    int qs;
    const float * qnw; // optional q-norm weights [HD] (the Q prep, table rope)
    const float2 * rope;
    float * out;       // [Tp][NH][HD]
    const float * gate; // optional [Tp][NH][gs]
    int gs;
    int8_t * q32a;     // optional o_proj units [Tp][192][16] (a / b), meta [Tp][192][4]
    int8_t * q32b;
    uint16_t * q32m;
    float * part;      // [NKV][nseg][R][HD] per-segment partial outputs (unnormalised)
    float2 * ml;       // [NKV][nseg][R] (max in log2 units, sum)
};
// key positions per prefill segment: 128 ceil(Lb / 256) with Lb = L rounded up to its 640-bucket: two segments per row
// at most, the same segments for every row of a bucket (every row's result is a function of its position).  A full
// 640-position piece then runs 30 row blocks x 4 kv heads x 2 segments = 240 workgroups, one round on 256 CUs at one
// workgroup per CU; more segments repeat each workgroup's query staging and partial stores (about 4 segments: 9% slower
// on a 16,384-position prompt, about 8: 23%; odd counts leave a partial round: about 3 segments 21% slower; one
// segment uses half the CUs: 39% slower)
inline int pf_seg(int L) {
    const int lb = (L + ATT_BUCKET - 1) / ATT_BUCKET * ATT_BUCKET;
    return 128 * ((lb + 255) / 256);
}
constexpr int PF2_ROWS = 128; // query rows per prefill workgroup (32 per wave)

// canonical segment length: 128 ceil(Lb / 16384) positions with Lb = L rounded up to a 640 bucket: a multiple of 4 tiles,
// so the 4 waves of a workgroup stream the same number of tiles; at most 128 segments per kv head (one layer's 4 heads
// fit the 2 workgroup slots of each of the 256 CUs in one pass) and the same partition for every row count T whose rows
// share one bucket
inline __host__ __device__ int seg_len(int L) {
    const int lb = (L + ATT_BUCKET - 1) / ATT_BUCKET * ATT_BUCKET;
    return ATP * AWAVES * ((lb + 16383) / 16384);
}
constexpr int MAX_SEG = 128;
constexpr int STAGE_BYTES = 2 * 32 * 256 + 1024; // one 32-position tile, widest format (q8 K and V) + its scales
constexpr int ATTN_LDS = AWAVES * STAGE_BYTES;   // one stage per wave (+ the query rows: RP * 512 bytes)

// ev0 / ev1: optional events recorded at the kernel's own start and end (hipExtLaunchKernelGGL: the dispatch packet's
// timestamps, the same the profiler reads), for the store's kernel timing
// knw (optional): [nl][HD] k-norm weights; K rows then get RMSNorm + RoPE (qk_prep, table rope) before quantization
hipError_t launch_append(const StoreLayout & S, int seq, int layer0, int nl, int pos, int T, const void * k, const void * v, int f16,
                         hipStream_t st, hipEvent_t ev0 = nullptr, hipEvent_t ev1 = nullptr, const float * knw = nullptr,
                         const float2 * rope = nullptr);
hipError_t launch_ring_refill(const StoreLayout & S, int seq, int nl, int p0, int p1, hipStream_t st);
// occ: workgroups per CU for one 8-row group of packed formats up to 11 KiB per tile: 0 = three when the launch has more
// work items than two per CU hold, else two; 2 = two; 3 = three
hipError_t launch_attn(const AttnArgs & a, int kb, int vb, int max_blocks, int occ, hipStream_t st, hipEvent_t ev0 = nullptr,
                       hipEvent_t ev1 = nullptr);
// the first `tiles` tiles of every wave slice of the attention launch `a` read into the L2 its workgroups will use
hipError_t launch_prefetch(const AttnArgs & a, int kb, int vb, int tiles, hipStream_t st);
hipError_t launch_combine(const AttnArgs & a, hipStream_t st, hipEvent_t ev0 = nullptr, hipEvent_t ev1 = nullptr);
hipError_t launch_prefill(const PrefillArgs & a, int kb, int vb, hipStream_t st, hipEvent_t ev0 = nullptr, hipEvent_t ev1 = nullptr);

} // namespace qkv
