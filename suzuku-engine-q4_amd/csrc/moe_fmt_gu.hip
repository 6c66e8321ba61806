// Gate/up kernels of the decode / verify window for the weight formats of
// formats.h (IQ2_S), in their own translation unit so the library's
// kernels compile in parallel.
#include "moe_kern.h"

namespace q4mi {

bool moe_fmt_gu(uint32_t ty, int nt, const MoeArgs &a, uint32_t nu_host) {
    if (ty == Q4MI_T_IQ2_S) {
        if (nt == 1) return gu_dispatch<Q4MI_T_IQ2_S, 1>(a, nu_host);
        if (nt == 2) return gu_dispatch<Q4MI_T_IQ2_S, 2>(a, nu_host);
        if (nt <= 4) return gu_dispatch<Q4MI_T_IQ2_S, 4>(a, nu_host);
        return gu_dispatch<Q4MI_T_IQ2_S, 8>(a, nu_host);
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
