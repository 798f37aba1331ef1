// The decode kernels of one head dim: built once per supported head_dim with
// -DPA_HEAD_DIM=<64|128|192|256> (flydsl_amd/build.py), each object defining that
// head dim's launchers, which the C ABI in pa_decode.hip selects at run time.
#include "pa_decode_kernels.h"

#ifndef PA_HEAD_DIM
#error "build with -DPA_HEAD_DIM=<64|128|192|256>"
#endif

namespace pa {

template <>
hipError_t dispatch_partition<PA_HEAD_DIM>(const DecodeParams &p, bool per_token, bool v4, int mtp, int waves,
                                           dim3 grid, hipStream_t s) {
    if (v4)
        return per_token ? dispatch_partition_pt<true, PA_HEAD_DIM, true>(p, mtp, waves, grid, s)
                         : dispatch_partition_pt<false, PA_HEAD_DIM, true>(p, mtp, waves, grid, s);
    return per_token ? dispatch_partition_pt<true, PA_HEAD_DIM, false>(p, mtp, waves, grid, s)
                     : dispatch_partition_pt<false, PA_HEAD_DIM, false>(p, mtp, waves, grid, s);
}

template <>
hipError_t dispatch_worklist<PA_HEAD_DIM>(const WorklistParams &w, bool per_token, bool v4, int mtp, dim3 grid,
                                          hipStream_t s) {
    if (v4)
        return per_token ? dispatch_worklist_pt<true, PA_HEAD_DIM, true>(w, mtp, grid, s)
                         : dispatch_worklist_pt<false, PA_HEAD_DIM, true>(w, mtp, grid, s);
    return per_token ? dispatch_worklist_pt<true, PA_HEAD_DIM, false>(w, mtp, grid, s)
                     : dispatch_worklist_pt<false, PA_HEAD_DIM, false>(w, mtp, grid, s);
}

}  // namespace pa
