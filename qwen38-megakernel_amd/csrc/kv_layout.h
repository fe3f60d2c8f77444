// HBM layout of the KV store, shared by the host library and the kernels.
//
// Per attention layer (slot) and side (K = 0, V = 1):
//   packed / main store  vals [NKV][n_pages][page][row_bytes]   row_bytes = 256 * bits / 8
//                        scs  [NKV][n_pages][page][8]           fp16 scales, one per 32 values
//   q8 ring (window)     ring [n_seq][NKV][kvrc][256]           present for low-bit sides when a window is set
//                        rsc  [n_seq][NKV][kvrc][8]
// A sequence's logical position p lives in physical page ptab[seq][p / page], row p % page of it.  With one page per
// sequence and the identity table this is the reference's [kv head][ctx][row] layout (loader.cu:1438-1468).
#pragma once
#include <stdint.h>

namespace qkv {

constexpr int HD = 256;           // head dim
constexpr int NKV = 4;            // kv heads
constexpr int NH = 24;            // query heads (GQA 6)
constexpr int GQA = NH / NKV;
constexpr int ATP = 32;           // positions per attention tile
constexpr int ATT_BUCKET = 640;   // the reference's window / partition bucket (mk_shared.cuh:263-265)
constexpr int AWAVES = 4;         // waves per attention workgroup (tiles of a segment dealt round-robin)
constexpr int MAXT = 8;           // query tokens per call (1 + 7 drafts)
constexpr int MAXR = GQA * MAXT;  // query rows per kv head
constexpr int MAX_LAYERS = 17;    // 16 attention layers + MTP slot
constexpr int MAX_SEQ = 8;        // sequences per attention launch


struct SideLayout {
    uint8_t * vals;
    uint16_t * scs;
    int8_t * ring;  // nullptr: this side has no window ring
    uint16_t * rsc;
    int bits;       // 4..8
    int rot;        // 1: stored Walsh-Hadamard rotated
};

struct StoreLayout {
    SideLayout side[17][2];
    const int * ptab; // [n_seq][pt_stride] physical page of each logical page
    int pt_stride;
    int page;         // positions per page (multiple of 32)
    int n_pages;      // pages in the pool
    int kvrc;         // ring rows per kv head (0: no window)
    int win;          // MK_KV_WIN
    int n_seq;
};

__host__ __device__ inline int row_bytes(int bits) { return 32 * bits; }

} // namespace qkv
