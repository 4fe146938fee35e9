// Instantiations of the streaming pass k_scan (scan.h) and its launcher.
#include "launchers.h"

namespace fie {

template <int DT>
static void scan_dt(const KParams& P, bool vec, bool longh, hipStream_t st)
{
    const dim3 grid(P.NS, P.a.rows);
    if (vec) {
        if (longh) k_scan<DT, true, true><<<grid, kScanThreads, 0, st>>>(P);
        else k_scan<DT, true, false><<<grid, kScanThreads, 0, st>>>(P);
    } else {
        if (longh) k_scan<DT, false, true><<<grid, kScanThreads, 0, st>>>(P);
        else k_scan<DT, false, false><<<grid, kScanThreads, 0, st>>>(P);
    }
}

hipError_t launch_scan(const KParams& P, bool vec, bool longh, hipStream_t st)
{
    switch (P.a.dtype) {
    case FIE_F32: scan_dt<FIE_F32>(P, vec, longh, st); break;
    case FIE_F16: scan_dt<FIE_F16>(P, vec, longh, st); break;
    default: scan_dt<FIE_BF16>(P, vec, longh, st); break;
    }
    return hipGetLastError();
}

}  // namespace fie
