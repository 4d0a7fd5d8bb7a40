// Variants of the chunk backward k_bwd_ws, the reverse state-gradient pass
// k_bwd_dstate_rev and the run pre-pass k_bwd_run_grad for one value of the z
// gate, and their launchers (declared
// in ssd_launch.h).  Built twice, with SSD_BWD_Z=0 and SSD_BWD_Z=1, so the two
// halves compile in parallel.
#define SSD_KERNEL_TEMPLATES_ONLY
#include "ssd_bwd_fused.h"
#include "ssd_launch.h"

#ifndef SSD_BWD_Z
#error "build with -DSSD_BWD_Z=0 or -DSSD_BWD_Z=1"
#endif

#define SSD_CAT2(a, b) a##b
#define SSD_CAT(a, b) SSD_CAT2(a, b)

namespace ssd {
namespace {

constexpr bool kZ = SSD_BWD_Z != 0;

template <int kR, bool kSeq>
void run_ws(dim3 grid, hipStream_t st, const BwdParams &bp, int nseg, int M) {
    hipLaunchKernelGGL((bwd::k_bwd_ws<kZ, kR, kSeq>), grid, dim3(kBwsThreads), 0, st, bp, nseg, M);
}

template <bool kSeq>
void run_rev(dim3 grid, hipStream_t st, const BwdParams &bp, const float *dfinal, float *dinit) {
    hipLaunchKernelGGL((bwd::k_bwd_dstate_rev<kZ, kSeq>), grid, dim3(kWsThreads), 0, st, bp, dfinal, dinit);
}

template <bool kSeq>
void run_grad(dim3 grid, hipStream_t st, const BwdParams &bp, const RevSeg &rs) {
    hipLaunchKernelGGL((bwd::k_bwd_run_grad<kZ, kSeq>), grid, dim3(kWsThreads), 0, st, bp, rs);
}

}  // namespace

void SSD_CAT(launch_bwd_ws_z, SSD_BWD_Z)(int rev_r, bool seq, dim3 grid, hipStream_t st,
                                          const BwdParams &bp, int nseg, int M) {
    switch (rev_r) {
    case 1: (seq ? run_ws<1, true> : run_ws<1, false>)(grid, st, bp, nseg, M); break;
    case 2: (seq ? run_ws<2, true> : run_ws<2, false>)(grid, st, bp, nseg, M); break;
    case 4: (seq ? run_ws<4, true> : run_ws<4, false>)(grid, st, bp, nseg, M); break;
    default: (seq ? run_ws<0, true> : run_ws<0, false>)(grid, st, bp, nseg, M); break;
    }
}

void SSD_CAT(launch_bwd_dstate_rev_z, SSD_BWD_Z)(bool seq, dim3 grid, hipStream_t st, const BwdParams &bp,
                                                  const float *dfinal, float *dinit) {
    (seq ? run_rev<true> : run_rev<false>)(grid, st, bp, dfinal, dinit);
}

void SSD_CAT(launch_bwd_run_grad_z, SSD_BWD_Z)(bool seq, dim3 grid, hipStream_t st, const BwdParams &bp,
                                               const RevSeg &rs) {
    (seq ? run_grad<true> : run_grad<false>)(grid, st, bp, rs);
}

}  // namespace ssd
