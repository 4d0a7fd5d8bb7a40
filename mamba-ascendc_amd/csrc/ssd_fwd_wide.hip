// Variants of the dstate-128 forward k_fwd_wide and their launcher (declared
// in ssd_launch.h).
#define SSD_KERNEL_TEMPLATES_ONLY
#include "ssd_fwd_wide.h"
#include "ssd_launch.h"

namespace ssd {
namespace {

template <bool kSave, bool kGate, bool kSeq, bool kCB>
void run(dim3 grid, hipStream_t st, const FwdParams &kp, const SegParams &sp) {
    hipLaunchKernelGGL((k_fwd_wide<kSave, kGate, kSeq, kCB>), grid, dim3(kWsThreads), 0, st, kp, sp);
}

using Run = void (*)(dim3, hipStream_t, const FwdParams &, const SegParams &);

}  // namespace

void launch_fwd_wide(bool save, bool gate, bool seq, dim3 grid, hipStream_t st, const FwdParams &kp,
                     const SegParams &sp) {
    static const Run fn[16] = {
        run<false, false, false, false>, run<false, false, true, false>, run<false, true, false, false>,
        run<false, true, true, false>,   run<true, false, false, false>, run<true, false, true, false>,
        run<true, true, false, false>,   run<true, true, true, false>,   run<false, false, false, true>,
        run<false, false, true, true>,   run<false, true, false, true>,  run<false, true, true, true>,
        run<true, false, false, true>,   run<true, false, true, true>,   run<true, true, false, true>,
        run<true, true, true, true>,
    };
    fn[(kp.cb ? 8 : 0) + (save ? 4 : 0) + (gate ? 2 : 0) + (seq ? 1 : 0)](grid, st, kp, sp);
}

void launch_chunk_cb(int n, dim3 grid, hipStream_t st, const float *C, const float *B, float *cb, int64_t L,
                     int G, int K) {
    if (n == 128) hipLaunchKernelGGL((k_chunk_cb<128>), grid, dim3(kCbThreads), 0, st, C, B, cb, L, G, K);
    else hipLaunchKernelGGL((k_chunk_cb<64>), grid, dim3(kCbThreads), 0, st, C, B, cb, L, G, K);
}

}  // namespace ssd
