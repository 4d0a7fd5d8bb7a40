// Variants of the dstate-128 forward k_fwd_wide and their launcher (declared
// in ssd_launch.h).
#define SSD_KERNEL_TEMPLATES_ONLY
#include "ssd_fwd_wide.h"
#include "ssd_launch.h"

namespace ssd {
namespace {

template <bool kSave, bool kGate, bool kSeq>
void run(dim3 grid, hipStream_t st, const FwdParams &kp, const SegParams &sp) {
    hipLaunchKernelGGL((k_fwd_wide<kSave, kGate, kSeq>), grid, dim3(kWsThreads), 0, st, kp, sp);
}

using Run = void (*)(dim3, hipStream_t, const FwdParams &, const SegParams &);

}  // namespace

void launch_fwd_wide(bool save, bool gate, bool seq, dim3 grid, hipStream_t st, const FwdParams &kp,
                     const SegParams &sp) {
    static const Run fn[8] = {
        run<false, false, false>, run<false, false, true>, run<false, true, false>, run<false, true, true>,
        run<true, false, false>,  run<true, false, true>,  run<true, true, false>,  run<true, true, true>,
    };
    fn[(save ? 4 : 0) + (gate ? 2 : 0) + (seq ? 1 : 0)](grid, st, kp, sp);
}

}  // namespace ssd
