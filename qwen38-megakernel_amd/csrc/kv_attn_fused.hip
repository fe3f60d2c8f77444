// The decode kernels with the fused append (mk_kv_append_attend): k_attn<.., APPEND = true> for every row-group count
// and k_verify<.., APPEND = true>, for every K / V format, in a translation unit of their own so that they compile
// beside the plain kernels.
#include "kv_attn_decode.h"

namespace qkv {

template <int NP>
static AttnKernel fused_of(int kb, int vb) {
#define QKV_VB(K)                                                                                                      \
    switch (vb) {                                                                                                      \
    case 4: return k_attn<NP, K, 4, false, true>;                                                                      \
    case 5: return k_attn<NP, K, 5, false, true>;                                                                      \
    case 6: return k_attn<NP, K, 6, false, true>;                                                                      \
    case 7: return k_attn<NP, K, 7, false, true>;                                                                      \
    case 8: return k_attn<NP, K, 8, false, true>;                                                                      \
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

AttnKernel pick_fused(int np, bool wide, int kb, int vb) {
    if (np == 1) return fused_of<1>(kb, vb);
    if (np == 2) return fused_of<2>(kb, vb);
    if (np == 3) return wide ? verify_of<true>(kb, vb) : fused_of<3>(kb, vb);
    return nullptr;
}

} // namespace qkv
