// rf_adam8_inst.hip -- instantiates k_adam8 for one (APPLY, MSR, EXACT)
// combination, selected by -DRFI_APPLY / -DRFI_MSR / -DRFI_EXACT.  The build
// compiles this file once per combination, in parallel, and links all of
// them into one library; rf_host.hip picks the instance per call.
#include "rf_device.h"

#if !defined(RFI_APPLY) || !defined(RFI_MSR) || !defined(RFI_EXACT)
#error "build with -DRFI_APPLY=0|1 -DRFI_MSR=0|1 -DRFI_EXACT=0|1"
#endif

#define RF_PICK_NAME2(a, m, e) rf_pick_adam8_a##a##_m##m##_e##e
#define RF_PICK_NAME(a, m, e) RF_PICK_NAME2(a, m, e)

namespace rf {

template <typename PT, typename GT>
static adam_kernel_t pick(bool psr, bool nest)
{
    constexpr bool A = RFI_APPLY != 0, M = RFI_MSR != 0, E = RFI_EXACT != 0;
    if constexpr (A && IS_BF16<PT>) {  // stochastic rounding exists for bf16 params only
        if (psr) return nest ? &k_adam8<PT, GT, A, M, true, true, E> : &k_adam8<PT, GT, A, M, true, false, E>;
    }
    return nest ? &k_adam8<PT, GT, A, M, false, true, E> : &k_adam8<PT, GT, A, M, false, false, E>;
}

// dtype_combo = 2*(param is bf16) + (grad is bf16) for f32/bf16 params and
// grads, 4 for f16 params and grads; -1 = the generic kernel, -2 = its
// instance for lists of full-chunk fallback units only (moment SR plays no
// part there: those are asked of the MSR = 0 instances; null otherwise)
adam_kernel_t RF_PICK_NAME(RFI_APPLY, RFI_MSR, RFI_EXACT)(int dtype_combo, bool psr, bool nest)
{
    constexpr bool A = RFI_APPLY != 0, M = RFI_MSR != 0, E = RFI_EXACT != 0;
    if (dtype_combo == -2) {
        if constexpr (M) {
            return nullptr;
        } else {
            if constexpr (A) {
                if (psr)
                    return nest ? &k_adam8_gen<A, M, true, true, E, true> : &k_adam8_gen<A, M, true, false, E, true>;
            }
            return nest ? &k_adam8_gen<A, M, false, true, E, true> : &k_adam8_gen<A, M, false, false, E, true>;
        }
    }
    if (dtype_combo < 0) {
        if constexpr (A) {
            if (psr) return nest ? &k_adam8_gen<A, M, true, true, E> : &k_adam8_gen<A, M, true, false, E>;
        }
        return nest ? &k_adam8_gen<A, M, false, true, E> : &k_adam8_gen<A, M, false, false, E>;
    }
    switch (dtype_combo) {
        case 4: return pick<_Float16, _Float16>(psr, nest);
        case 3: return pick<uint16_t, uint16_t>(psr, nest);
        case 2: return pick<uint16_t, float>(psr, nest);
        case 1: return pick<float, uint16_t>(psr, nest);
        default: return pick<float, float>(psr, nest);
    }
}

}  // namespace rf
