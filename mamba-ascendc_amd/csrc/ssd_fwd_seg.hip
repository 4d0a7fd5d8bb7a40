// Variants of the fused forward k_fwd_seg, the group-major state pass
// k_fwd_state_group, and their launchers (declared in
// ssd_launch.h); the library's host code is in mamba2_ssd.hip.
#define SSD_KERNEL_TEMPLATES_ONLY
#include "ssd_fwd_fused.h"
#include "ssd_fwd_group.h"
#include "ssd_launch.h"

namespace ssd {
namespace {

template <bool kStateOnly, bool kSave, bool kGate, bool kSeq, bool kLat = false>
void run(dim3 grid, hipStream_t st, const FwdParams &kp, const SegParams &sp) {
    hipLaunchKernelGGL((k_fwd_seg<kStateOnly, kSave, kGate, kSeq, kLat>), grid, dim3(kWsThreads), 0, st,
                       kp, sp);
}

using Run = void (*)(dim3, hipStream_t, const FwdParams &, const SegParams &);

}  // namespace

void launch_fwd_seg(bool state_only, bool save, bool gate, bool seq, dim3 grid, hipStream_t st,
                    const FwdParams &kp, const SegParams &sp, bool latency) {
    if (state_only) {
        if (save)
            (seq ? run<true, true, false, true> : run<true, true, false, false>)(grid, st, kp, sp);
        else
            (seq ? run<true, false, false, true> : run<true, false, false, false>)(grid, st, kp, sp);
        return;
    }
    if (latency && !seq) {
        // the plain, saving and z-gated passes (the packed forms, whose
        // registers are fuller, keep the one form)
        static const Run lat[4] = {
            run<false, false, false, false, true>, run<false, false, true, false, true>,
            run<false, true, false, false, true>, run<false, true, true, false, true>,
        };
        lat[(save ? 2 : 0) + (gate ? 1 : 0)](grid, st, kp, sp);
        return;
    }
    static const Run full[8] = {
        run<false, false, false, false>, run<false, false, false, true>,
        run<false, false, true, false>,  run<false, false, true, true>,
        run<false, true, false, false>,  run<false, true, false, true>,
        run<false, true, true, false>,   run<false, true, true, true>,
    };
    full[(save ? 4 : 0) + (gate ? 2 : 0) + (seq ? 1 : 0)](grid, st, kp, sp);
}

void launch_fwd_state_group(dim3 grid, hipStream_t st, const FwdParams &kp) {
    hipLaunchKernelGGL((k_fwd_state_group<4>), grid, dim3(kWsThreads), 0, st, kp);
}

}  // namespace ssd
