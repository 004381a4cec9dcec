// kernels_gemv_norm.hip -- the normalised GEMVs of a decode step (M = 1),
// each instantiated for its epilogue (gemv_device.hpp: norm_view).  In a
// source of their own so that they compile in parallel with the generic
// instantiations in kernels_gemv.hip.
#include "gemv_device.hpp"

namespace tlhip {

template <int WT, int NB>
static bool launch_norm_epi_nb(hipStream_t s, const GemvParams& p, int pro) {
    if (pro == PRO_RMS) {
        switch (p.epi) {
            case EPI_SWIGLU_PAIR: launch_norm_shape<WT, NB, PRO_RMS, EPI_SWIGLU_PAIR>(s, p); return true;
            case EPI_QKV_ROPE: launch_norm_shape<WT, NB, PRO_RMS, EPI_QKV_ROPE>(s, p); return true;
            case EPI_ARGMAX: launch_norm_shape<WT, NB, PRO_RMS, EPI_ARGMAX>(s, p); return true;
            default: return false;
        }
    }
    if (pro == PRO_LN) {
        switch (p.epi) {
            case EPI_QKV_ROPE: launch_norm_shape<WT, NB, PRO_LN, EPI_QKV_ROPE>(s, p); return true;
            case EPI_BIAS_GELU: launch_norm_shape<WT, NB, PRO_LN, EPI_BIAS_GELU>(s, p); return true;
            case EPI_ARGMAX: launch_norm_shape<WT, NB, PRO_LN, EPI_ARGMAX>(s, p); return true;
            default: return false;
        }
    }
    return false;
}

template <int WT>
static bool launch_norm_epi_wt(hipStream_t s, const GemvParams& p, int nb, int pro) {
    if (p.M != 1) return false;
    if (nb == 1) return launch_norm_epi_nb<WT, 1>(s, p, pro);
    if (nb == 2) return launch_norm_epi_nb<WT, 2>(s, p, pro);
    return false;
}

bool launch_norm_epi(hipStream_t s, tlhip_dtype wt, const GemvParams& p, int nb, int pro) {
    switch (wt) {
        case TLHIP_Q4_0: return launch_norm_epi_wt<TLHIP_Q4_0>(s, p, nb, pro);
        case TLHIP_Q8_0: return launch_norm_epi_wt<TLHIP_Q8_0>(s, p, nb, pro);
        case TLHIP_Q6_K: return launch_norm_epi_wt<TLHIP_Q6_K>(s, p, nb, pro);
        case TLHIP_F16: return launch_norm_epi_wt<TLHIP_F16>(s, p, nb, pro);
        default: return false;
    }
}

}  // namespace tlhip
