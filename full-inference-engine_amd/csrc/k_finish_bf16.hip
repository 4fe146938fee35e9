// Instantiations of the per-row kernels k_finish / k_deep (finish.h) for FIE_BF16 logits.
#include "finish.h"
#include "launchers.h"

namespace fie {

hipError_t launch_finish_bf16(const KParams& P, bool vec, bool deep, bool wide, hipStream_t st)
{
    if (deep) {
        // one workgroup per queue slot; those past the queued count leave at once
        if (vec) k_deep<FIE_BF16, true><<<P.a.rows, kFinThreads, 0, st>>>(P);
        else k_deep<FIE_BF16, false><<<P.a.rows, kFinThreads, 0, st>>>(P);
    } else if (vec) {
        if (wide) k_finish<FIE_BF16, true, true><<<dim3(P.a.rows, P.helpers ? P.NS + 1 : 1), kFinThreads, 0, st>>>(P);
        else k_finish<FIE_BF16, true, false><<<P.a.rows, kFinThreads, 0, st>>>(P);
    } else {
        if (wide) k_finish<FIE_BF16, false, true><<<dim3(P.a.rows, P.helpers ? P.NS + 1 : 1), kFinThreads, 0, st>>>(P);
        else k_finish<FIE_BF16, false, false><<<P.a.rows, kFinThreads, 0, st>>>(P);
    }
    return hipGetLastError();
}

}  // namespace fie
