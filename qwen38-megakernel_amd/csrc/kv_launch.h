// Kernel launchers of the KV path (defined in kv_store.hip / kv_attn*.hip), called by the C-ABI host code.
#pragma once
#include <hip/hip_runtime.h>
#include "kv_layout.h"

namespace qkv {

// one sequence entry of an attention launch
struct SeqDesc {
    int seq;   // store sequence (lane) index
    int L;     // context length after this call's rows: positions 0 .. L-1
    int ws;    // window start: tiles at positions >= ws are read from the q8 ring
    int nseg;  // canonical segments: ceil(L / SEG)
    int item0; // first work item of this sequence in the launch
};

struct AttnArgs {
    StoreLayout S;
    int layer0;    // first slot of the launch
    int nl;        // layers in the launch (all with the same K/V bits)
    int T, R;      // query tokens, query rows per kv head (6 T)
    int RP;        // padded rows (16 per MFMA row group)
    int nseq;
    int n_items;
    SeqDesc sd[8];
    const _Float16 * qh; // [nl][nseq][NKV][RP][256] prepared fp16 queries
    float * part;        // [item][R][256] per-segment partial outputs (unnormalised)
    float2 * ml;         // [item][R] per-segment (max in log2 units, sum)
};

hipError_t launch_append(const StoreLayout & S, int seq, int layer0, int nl, int pos, int T, const void * k, const void * v, int f16,
                         hipStream_t st);
hipError_t launch_ring_refill(const StoreLayout & S, int seq, int nl, int p0, int p1, hipStream_t st);
hipError_t launch_qprep(const float * q, _Float16 * qh, int layer0, int nl, int nseq, int T, int R, int RP, unsigned rotmask, hipStream_t st);
hipError_t launch_attn(const AttnArgs & a, int kb, int vb, int max_blocks, hipStream_t st);
hipError_t launch_combine(const AttnArgs & a, unsigned rotv_mask, float * out, hipStream_t st);

} // namespace qkv
