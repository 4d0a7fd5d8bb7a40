// State at the end of every sequence of a packed batch-1 input (varlen
// states).
//
// Sequence i is tokens cu[i] .. cu[i+1] - 1.  With c the logical chunk
// (length CS) holding its last token, c0 = c CS, and a_t = A q_t:
//   out[i] = sum_{t = max(start, c0)}^{end - 1} exp(sum_{t < m < end} a_m) q_t x_t (x) B_t
//            + [start < c0] exp(sum_{c0 <= m < end} a_m) S_c
// where S_c is the state entering chunk c, i.e. the forward's chunk_states at
// the 64-token chunk c0 / 64 (so CS must be a multiple of 64).  These are the
// semantics of the reference's Triton port (mamba_triton_ascend/mamba2/ops/
// triton/ssd_chunk_state.py:700-775, chunk_state_varlen): the initial state
// reaches a sequence only through S_c.
//
// One workgroup per (sequence, head) walks the sequence's tokens in chunk c
// from the last backwards in blocks of 64: wave 0 forms each block's weights
// exp(sum of the later a) q_t with a lane scan, and every thread adds the
// outer products for its float4s of the [P][N] state.  The work is a few
// thousand multiply-adds per token, far below the forward's.
#pragma once

#include "ssd_fwd_kernels.h"

namespace ssd {

constexpr int kVarlenThreads = 256;

#ifndef SSD_KERNEL_TEMPLATES_ONLY
__global__ __launch_bounds__(kVarlenThreads) void k_varlen_states(FwdParams prm, const int32_t *cu,
                                                                   const float *chunk_states,
                                                                   float *out, int CS, int P,
                                                                   int N) {
    __shared__ float s_w[64];
    __shared__ float s_tail; // sum of a over the sequence's tokens in chunk c
    const int i = blockIdx.x, h = blockIdx.y, H = prm.H;
    const int tid = threadIdx.x, lane = tid & 63;
    const int PN = P * N, nv = PN / (4 * kVarlenThreads); // float4s per thread (PN % 1024 == 0)
    const int start = cu[i], end = cu[i + 1];
    float *o = out + ((int64_t)i * H + h) * PN;
    float4 acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    // an empty or out-of-range sequence has the zero state
    const bool valid = start >= 0 && end > start && end <= prm.L;
    const int c0 = valid ? ((end - 1) / CS) * CS : 0;
    const int lo = max(start, c0);
    const float bias = prm.dt_bias ? prm.dt_bias[h] : 0.f;
    const float A = prm.A[h];
    const int g = h / prm.R;
    float tail = 0.f; // wave 0: sum of a over the tokens after the current block
    for (int te = valid ? end : lo; te > lo; te -= 64) {
        const int tb = max(lo, te - 64), nt = te - tb;
        if (tid < 64) {
            // lane l <-> token te - 1 - l (the block reversed)
            float q = 0.f;
            if (lane < nt)
                q = discretize_dt(prm.dt[(int64_t)(te - 1 - lane) * H + h], bias, prm.softplus != 0,
                                  prm.lo, prm.hi);
            const float a = A * q;
            const float incl = wave_inclusive_scan(a);
            s_w[lane] = __expf(tail + incl - a) * q; // exp(sum over the later tokens) q
            tail += readlane_f(incl, 63);
        }
        __syncthreads();
        for (int l = 0; l < nt; ++l) {
            const int t = te - 1 - l;
            const float w = s_w[l];
            const float *xt = prm.x + ((int64_t)t * H + h) * P;
            const float *bt = prm.B + ((int64_t)t * prm.G + g) * N;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                if (j < nv) {
                    const int e = (tid + j * kVarlenThreads) * 4, p = e / N, n = e % N;
                    const float wx = w * xt[p];
                    const float4 bv = *(const float4 *)(bt + n);
                    acc[j].x += wx * bv.x;
                    acc[j].y += wx * bv.y;
                    acc[j].z += wx * bv.z;
                    acc[j].w += wx * bv.w;
                }
            }
        }
        __syncthreads(); // s_w is rewritten by the next block
    }
    if (tid == 0) s_tail = tail;
    __syncthreads();
    const bool carried = valid && start < c0;
    const float dec = __expf(s_tail);
    const float *sc = carried ? chunk_states + ((int64_t)h * prm.K + c0 / 64) * PN : nullptr;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        if (j < nv) {
            const int e = (tid + j * kVarlenThreads) * 4;
            float4 v = acc[j];
            if (carried) {
                const float4 s = *(const float4 *)(sc + e);
                v.x += dec * s.x;
                v.y += dec * s.y;
                v.z += dec * s.z;
                v.w += dec * s.w;
            }
            *(float4 *)(o + e) = v;
        }
    }
}
#endif

}  // namespace ssd
