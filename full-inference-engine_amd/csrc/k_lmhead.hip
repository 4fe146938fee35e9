// Instantiations of the fused output layer + streaming pass k_lmhead (lmhead.h).
#include "launchers.h"
#include "lmhead.h"

namespace fie {

template <int DT>
static void lmhead_dt(const KParams& P, const void* hidden, const void* weight, int H, bool vec, bool longh,
                      hipStream_t st)
{
    const int nrb = (P.a.rows + kLhRows - 1) / kLhRows;
    const int grid = 8 * ((P.NT + 7) / 8) * nrb;
    const uint16_t* h = (const uint16_t*)hidden;
    const uint16_t* w = (const uint16_t*)weight;
    if (vec) {
        if (longh) k_lmhead<DT, true, true><<<grid, kLhThreads, 0, st>>>(P, h, w, H, nrb);
        else k_lmhead<DT, true, false><<<grid, kLhThreads, 0, st>>>(P, h, w, H, nrb);
    } else {
        if (longh) k_lmhead<DT, false, true><<<grid, kLhThreads, 0, st>>>(P, h, w, H, nrb);
        else k_lmhead<DT, false, false><<<grid, kLhThreads, 0, st>>>(P, h, w, H, nrb);
    }
}

hipError_t launch_lmhead(const KParams& P, const void* hidden, const void* weight, int H, bool vec, bool longh,
                         hipStream_t st)
{
    if (P.a.dtype == FIE_F16) lmhead_dt<FIE_F16>(P, hidden, weight, H, vec, longh, st);
    else lmhead_dt<FIE_BF16>(P, hidden, weight, H, vec, longh, st);
    return hipGetLastError();
}

}  // namespace fie
