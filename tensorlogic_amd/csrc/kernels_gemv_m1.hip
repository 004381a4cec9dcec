// kernels_gemv_m1.hip -- the single-row GEMV (M = 1, from 1024 rows)
// instantiated for each plain epilogue (gemv_device.hpp: gemv_m1_kernel with
// EPI >= 0).  In a source of their own so that they compile in parallel with
// the generic instantiations in kernels_gemv.hip.
#include "gemv_device.hpp"

namespace tlhip {

template <int WT, int NB, int RI, int FN = 0, int WPB = 4>
static bool launch_m1_epi_nb(hipStream_t s, const Gemv1Params& p) {
    const dim3 grid((unsigned)(((p.N + RI - 1) / RI + WPB - 1) / WPB)), block(WPB * 64);
    const bool b = p.bias != nullptr, r = p.resid != nullptr;
    switch (p.epi) {
        case EPI_STORE: hipLaunchKernelGGL((gemv_m1_kernel<WT, NB, RI, EPI_STORE, FN, WPB>), grid, block, 0, s, p); return true;
        case EPI_BIAS:
            if (!b) return false;
            hipLaunchKernelGGL((gemv_m1_kernel<WT, NB, RI, EPI_BIAS, FN, WPB>), grid, block, 0, s, p);
            return true;
        case EPI_RESID:
            if (!r) return false;
            hipLaunchKernelGGL((gemv_m1_kernel<WT, NB, RI, EPI_RESID, FN, WPB>), grid, block, 0, s, p);
            return true;
        case EPI_BIAS_RESID:
            if (!b || !r) return false;
            hipLaunchKernelGGL((gemv_m1_kernel<WT, NB, RI, EPI_BIAS_RESID, FN, WPB>), grid, block, 0, s, p);
            return true;
        case EPI_BIAS_GELU:
            if (!b) return false;
            hipLaunchKernelGGL((gemv_m1_kernel<WT, NB, RI, EPI_BIAS_GELU, FN, WPB>), grid, block, 0, s, p);
            return true;
        default: return false;
    }
}

// Two rows per wave up to two 64-block passes per row (Q4_0 from 32768 rows:
// four), one row per wave beyond (the shapes launch_m1 picks for M = 1 from
// 1024 rows).  Q4_0, K = 2048, cold weights, measured on MI355X: 65536 rows
// 14.1-14.4 us with four rows per wave against 14.7-14.8 with two (eight
// waves per workgroup: 15.3-15.4 with two rows, 14.4-14.7 with four),
// 32768 rows 8.4-8.5 against 8.8.
template <int WT>
static bool launch_m1_epi_wt(hipStream_t s, const Gemv1Params& p, int nb, int ri) {
    if (ri == 2) {
        switch (nb) {
            case 1:
                if constexpr (WT == TLHIP_Q4_0)
                    if (p.N >= 32768) return launch_m1_epi_nb<WT, 1, 4>(s, p);
                return launch_m1_epi_nb<WT, 1, 2>(s, p);
            case 2:
                // 80 blocks per row (K = 2560): the flat task layout, 4 rows per
                // wave from 8192 rows, 2 below (enough waves to fill the device)
                if (WT != TLHIP_Q6_K && p.K == 80 * 32)
                    return p.N >= 8192 ? launch_m1_epi_nb<WT, 2, 4, 80>(s, p) : launch_m1_epi_nb<WT, 2, 2, 80>(s, p);
                return launch_m1_epi_nb<WT, 2, 2>(s, p);
            default: return false;
        }
    }
    switch (nb) {   // the block counts launch_m1 rounds to
        case 3: return launch_m1_epi_nb<WT, 3, 1>(s, p);
        case 4: return launch_m1_epi_nb<WT, 4, 1>(s, p);
        case 5: return launch_m1_epi_nb<WT, 5, 1>(s, p);   // (K = 10240: 320 blocks, 5 x 64)
        case 6: return launch_m1_epi_nb<WT, 6, 1>(s, p);
        case 7: case 8: return launch_m1_epi_nb<WT, 8, 1>(s, p);
        default: return false;
    }
}

// Two independent single-row GEMVs in one launch: workgroups [0, nA) run
// the first (NBA blocks per lane pass, RIA rows per wave, epilogue EPA,
// task layout FNA), the rest the second.  Phi-2's decode step pairs dense
// [2560 x 2560] + bias + residual with fc2 [2560 x 10240] + bias: the two
// read different rows (attention output, fc1 output), and the residual's
// last addition (x + dense + fc2) is left to the next layer_norm prologue.
template <int WT, int NBA, int RIA, int EPA, int FNA, int NBB, int RIB, int EPB, int FNB>
__global__ __launch_bounds__(256) void gemv_m1_pair_kernel(Gemv1Params pa, Gemv1Params pb, int nA) {
    const int id = (int)blockIdx.x;
    if (id < nA) gemv_m1_body<WT, NBA, RIA, EPA, FNA, 4>(pa, id);
    else gemv_m1_body<WT, NBB, RIB, EPB, FNB, 4>(pb, id - nA);
}

bool launch_m1_pair(hipStream_t s, tlhip_dtype wt, const GemvArgs& d, int epi_d, const GemvArgs& f, int epi_f) {
    // the shapes it is built for: Q8_0, dense [N <= 8192, 2560] + bias + residual
    // (flat layout, 2 rows per wave) and fc2 [N, 10240] + bias (5 passes,
    // one row per wave), one activation row each
    if (wt != TLHIP_Q8_0 || d.M != 1 || f.M != 1 || epi_d != EPI_BIAS_RESID || epi_f != EPI_BIAS) return false;
    if (d.K != 80 * 32 || d.N < 1024 || d.N >= 8192 || !d.bias || !d.resid) return false;
    if (f.K != 5 * 64 * 32 || f.N < 1024 || !f.bias) return false;
    const Gemv1Params pa = {d.x, (const uint8_t*)d.wq, d.wd, d.bias, d.resid, d.y, d.N, d.K, EPI_BIAS_RESID};
    const Gemv1Params pb = {f.x, (const uint8_t*)f.wq, f.wd, f.bias, nullptr, f.y, f.N, f.K, EPI_BIAS};
    const int nA = (d.N + 7) / 8, nB = (f.N + 3) / 4;   // 4 waves x 2 rows / x 1 row
    hipLaunchKernelGGL((gemv_m1_pair_kernel<TLHIP_Q8_0, 2, 2, EPI_BIAS_RESID, 80, 5, 1, EPI_BIAS, 0>),
                       dim3((unsigned)(nA + nB)), dim3(256), 0, s, pa, pb, nA);
    return true;
}

bool launch_m1_epi(hipStream_t s, tlhip_dtype wt, const Gemv1Params& p, int nb, int ri) {
    if (p.N < 1024) return false;
    switch (wt) {
        case TLHIP_Q4_0: return launch_m1_epi_wt<TLHIP_Q4_0>(s, p, nb, ri);
        case TLHIP_Q8_0: return launch_m1_epi_wt<TLHIP_Q8_0>(s, p, nb, ri);
        case TLHIP_Q6_K: return launch_m1_epi_wt<TLHIP_Q6_K>(s, p, nb, ri);
        case TLHIP_F16: return launch_m1_epi_wt<TLHIP_F16>(s, p, nb, ri);
        default: return false;
    }
}

}  // namespace tlhip
