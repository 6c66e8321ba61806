// Gate/up kernels of the decode / verify window for the weight formats of
// formats.h (IQ2_S, IQ2_XXS, IQ2_XS, IQ3_XXS, IQ4_XS), in their own translation unit so the library's
// kernels compile in parallel.
#include "moe_kern.h"

namespace q4mi {

template <uint32_t TY>
static bool gu_nt(int nt, const MoeArgs &a, uint32_t nu_host) {
    if (nt == 1) return gu_dispatch<TY, 1>(a, nu_host);
    if (nt == 2) return gu_dispatch<TY, 2>(a, nu_host);
    if (nt <= 4) return gu_dispatch<TY, 4>(a, nu_host);
    return gu_dispatch<TY, 8>(a, nu_host);
}

// the reference window's other gate/up formats (win_iq_bb,
// src/q4_rocm.cu:7333-7343): IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ4_XS
bool moe_fmt_gu(uint32_t ty, int nt, const MoeArgs &a, uint32_t nu_host) {
    switch (ty) {
    case Q4MI_T_IQ2_S: return gu_nt<Q4MI_T_IQ2_S>(nt, a, nu_host);
    case Q4MI_T_IQ2_XXS: return gu_nt<Q4MI_T_IQ2_XXS>(nt, a, nu_host);
    case Q4MI_T_IQ2_XS: return gu_nt<Q4MI_T_IQ2_XS>(nt, a, nu_host);
    case Q4MI_T_IQ3_XXS: return gu_nt<Q4MI_T_IQ3_XXS>(nt, a, nu_host);
    case Q4MI_T_IQ4_XS: return gu_nt<Q4MI_T_IQ4_XS>(nt, a, nu_host);
    }
    set_error("moe: gate/up type %u not covered", ty);
    return false;
}

// this translation unit's kernels' timeout word (bits of q4mi_status_text)
uint32_t moe_fmt_status(int clear) {
    uint32_t v = 0, w = 0;
    if (hipMemcpyFromSymbol(&v, HIP_SYMBOL(g_moe_status), sizeof v, 0, hipMemcpyDeviceToHost) !=
        hipSuccess)
        return 0x80000000u;
    if (v && clear)
        (void)hipMemcpyToSymbol(HIP_SYMBOL(g_moe_status), &w, sizeof w, 0, hipMemcpyHostToDevice);
    return v | moe_fmt_status_dn(clear);
}

}  // namespace q4mi
