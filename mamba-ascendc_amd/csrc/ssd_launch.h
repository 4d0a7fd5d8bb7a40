// Launchers of the templated kernels, each compiled in a translation unit of
// its own (ssd_fwd_seg.hip, ssd_bwd_ws.hip) so the library builds in
// parallel; the host code in mamba2_ssd.hip picks the variant at run time.
// Every launcher only enqueues: the caller checks hipGetLastError().
#pragma once

#include <hip/hip_runtime.h>

#include "ssd_bwd_kernels.h"

namespace ssd {

struct SegParams;

// k_fwd_seg<state_only, save, gate, seq> (state_only excludes gate); latency:
// the full pass's form for grids of at most one workgroup per CU (plain,
// saving and z-gated passes; ignored for the packed ones)
void launch_fwd_seg(bool state_only, bool save, bool gate, bool seq, dim3 grid, hipStream_t st,
                    const FwdParams &kp, const SegParams &sp, bool latency = false);

// k_fwd_state_group<4>: the chunk-start states of one segment per stream,
// one workgroup per (b, g), four heads per group, no sequence ids; grid B G
void launch_fwd_state_group(dim3 grid, hipStream_t st, const FwdParams &kp);

// k_fwd_wide<save, gate, seq, kp.cb != NULL> (dstate 128)
void launch_fwd_wide(bool save, bool gate, bool seq, dim3 grid, hipStream_t st, const FwdParams &kp,
                     const SegParams &sp);

// k_chunk_cb<n>: C . B^T of every (b, g, chunk), grid B G K
void launch_chunk_cb(int n, dim3 grid, hipStream_t st, const float *C, const float *B, float *cb, int64_t L,
                     int G, int K);

// the has_z halves of the two backward launchers, one per translation unit
void launch_bwd_ws_z0(int rev_r, bool seq, dim3 grid, hipStream_t st, const BwdParams &bp, int nseg,
                      int M);
void launch_bwd_ws_z1(int rev_r, bool seq, dim3 grid, hipStream_t st, const BwdParams &bp, int nseg,
                      int M);
void launch_bwd_dstate_rev_z0(bool seq, dim3 grid, hipStream_t st, const BwdParams &bp, const float *dfinal,
                              float *dinit);
void launch_bwd_dstate_rev_z1(bool seq, dim3 grid, hipStream_t st, const BwdParams &bp, const float *dfinal,
                              float *dinit);
void launch_bwd_run_grad_z0(bool seq, dim3 grid, hipStream_t st, const BwdParams &bp, const RevSeg &rs);
void launch_bwd_run_grad_z1(bool seq, dim3 grid, hipStream_t st, const BwdParams &bp, const RevSeg &rs);

// k_bwd_ws<has_z, rev_r, seq> (rev_r 0, 1, 2 or 4)
inline void launch_bwd_ws(bool has_z, int rev_r, bool seq, dim3 grid, hipStream_t st,
                          const BwdParams &bp, int nseg, int M) {
    if (has_z) launch_bwd_ws_z1(rev_r, seq, grid, st, bp, nseg, M);
    else launch_bwd_ws_z0(rev_r, seq, grid, st, bp, nseg, M);
}

// k_bwd_dstate_rev<has_z, seq>, one workgroup per (b, h)
inline void launch_bwd_dstate_rev(bool has_z, bool seq, dim3 grid, hipStream_t st, const BwdParams &bp,
                                  const float *dfinal, float *dinit) {
    if (has_z) launch_bwd_dstate_rev_z1(seq, grid, st, bp, dfinal, dinit);
    else launch_bwd_dstate_rev_z0(seq, grid, st, bp, dfinal, dinit);
}

// k_bwd_run_grad<has_z, seq>, one workgroup per (b, h, run)
inline void launch_bwd_run_grad(bool has_z, bool seq, dim3 grid, hipStream_t st, const BwdParams &bp,
                                const RevSeg &rs) {
    if (has_z) launch_bwd_run_grad_z1(seq, grid, st, bp, rs);
    else launch_bwd_run_grad_z0(seq, grid, st, bp, rs);
}

}  // namespace ssd
