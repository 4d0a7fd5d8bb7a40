// Single-token decode step of the Mamba-2 SSM (selective state update).
//
// Per (batch b, head h), with the state S [P][N] of the sequence slot
// state_batch_indices[b] (or b) updated in place:
//   q[p]     = softplus?(dt + dt_bias)            (per head, or per (head, p))
//   S[p][n]  = exp(A q) S[p][n] + q[p] x[p] B[n]  (A per head, or per (h, p, n))
//   out[p]   = sum_n S[p][n] C[n] (+ D[p] x[p]) (* silu(z[p]))
// A negative slot index (or one past the last slot) skips the update and
// writes out = 0.
//
// The semantics are those of the reference's decode kernel
// (mamba_triton_ascend/mamba2/ops/triton/selective_state_update.py:22-131,
// including the tied-head-dim case 101-109 and the skipped padding slots
// 58-64); the layout of the work is this file's own: the op streams the
// state once in and once out, so each lane owns four consecutive state
// columns (one 16-byte load and store), the N / 4 lanes of a row reduce
// out[p] with a butterfly of lane shuffles, and a 256-thread workgroup walks
// the rows of one (b, h) 256 / (N / 4) at a time with B, C and the head's
// scalars loaded once.
#pragma once

#include "ssd_device.h"

namespace ssd {

struct SsuParams {
    float *state;
    int64_t state_bstride;     // floats between consecutive state slots
    int64_t nslots;            // slots in `state`
    const float *x, *dt, *A, *B, *C, *D, *z, *dt_bias;
    const int32_t *slot;       // [B] or NULL
    float *out;
    int H, P, N, G, R;
    int lpr;                   // lanes per state row: N / 4 rounded up to a power of two
    int tied;                  // dt [B, H], A [H], dt_bias [H]; else [B, H, P], [H, P, N], [H, P]
    int softplus, has_D, d_per_channel, has_z;
    // element strides (broadcast dimensions have stride 0)
    int64_t x_b, x_h, z_b, z_h, bc_b, bc_g, dt_b, dt_h, dt_p, A_h, A_p, A_n, bias_h, bias_p,
        D_h, D_p;
};

#ifndef SSD_KERNEL_TEMPLATES_ONLY
__global__ __launch_bounds__(256) void k_ssu(SsuParams prm) {
    const int bh = blockIdx.y, b = bh / prm.H, h = bh % prm.H;
    const int tid = threadIdx.x, lpr = prm.lpr;
    const int rows = 256 / lpr;                       // rows per pass of the workgroup
    const int n0 = (tid % lpr) * 4;
    const bool cols = n0 < prm.N;                     // N is a multiple of 4
    const int slot = prm.slot ? prm.slot[b] : b;
    const bool pad = slot < 0 || slot >= prm.nslots;  // padding (or an index past the slots)
    // per (b, h): the group's B and C columns of this lane, the head's scalars
    float4 bv = make_float4(0.f, 0.f, 0.f, 0.f), cv = bv;
    if (cols && !pad) {
        const int64_t bo = b * prm.bc_b + (h / prm.R) * prm.bc_g + n0;
        bv = *(const float4 *)(prm.B + bo);
        cv = *(const float4 *)(prm.C + bo);
    }
    const float dt_h = prm.tied ? prm.dt[b * prm.dt_b + h * prm.dt_h] : 0.f;
    const float bias_h = prm.tied && prm.dt_bias ? prm.dt_bias[h * prm.bias_h] : 0.f;
    const float A_h = prm.tied ? prm.A[h * prm.A_h] : 0.f;
    // workgroup x covers rows x * rows + i * gridDim.x * rows, kBatch passes
    // at a time: every state, x and dt load of the batch is issued before the
    // math, so each thread keeps kBatch rows in flight
    constexpr int kBatch = 4;
    const int stride = gridDim.x * rows;
    for (int p0 = blockIdx.x * rows; p0 < prm.P; p0 += kBatch * stride) {
        float4 sv[kBatch];
        float xv[kBatch], uv[kBatch];
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
            const int p = p0 + i * stride + tid / lpr;
            sv[i] = make_float4(0.f, 0.f, 0.f, 0.f);
            xv[i] = uv[i] = 0.f;
            if (p < prm.P && !pad) {
                xv[i] = prm.x[b * prm.x_b + h * prm.x_h + p];
                uv[i] = prm.tied ? dt_h + bias_h
                                 : prm.dt[b * prm.dt_b + h * prm.dt_h + p * prm.dt_p] +
                                       (prm.dt_bias ? prm.dt_bias[h * prm.bias_h + p * prm.bias_p] : 0.f);
                if (cols)
                    sv[i] = *(const float4 *)(prm.state + slot * prm.state_bstride +
                                              ((int64_t)h * prm.P + p) * prm.N + n0);
            }
        }
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
            const int p = p0 + i * stride + tid / lpr;
            const bool active = p < prm.P;            // whole rows are in or out
            const int64_t xo = ((int64_t)b * prm.H + h) * prm.P + p; // out is contiguous
            if (pad) {
                // no state update, zero output (one lane per row)
                if (active && n0 == 0) prm.out[xo] = 0.f;
                continue;
            }
            const float q = active ? (prm.softplus ? softplus_f(uv[i]) : uv[i]) : 0.f;
            const float x = xv[i];
            float part = 0.f;
            if (active && cols) {
                float *sp = prm.state + slot * prm.state_bstride + ((int64_t)h * prm.P + p) * prm.N + n0;
                const float4 s4 = sv[i];
                float4 dA;
                if (prm.tied) {
                    const float a = __expf(A_h * q);
                    dA = make_float4(a, a, a, a);
                } else {
                    const float *ap = prm.A + h * prm.A_h + p * prm.A_p + n0 * prm.A_n;
                    const float4 av = prm.A_n == 1 ? *(const float4 *)ap
                                                   : make_float4(ap[0], ap[prm.A_n], ap[2 * prm.A_n], ap[3 * prm.A_n]);
                    dA = make_float4(__expf(av.x * q), __expf(av.y * q), __expf(av.z * q), __expf(av.w * q));
                }
                const float qx = q * x;
                const float4 ns = make_float4(s4.x * dA.x + qx * bv.x, s4.y * dA.y + qx * bv.y,
                                              s4.z * dA.z + qx * bv.z, s4.w * dA.w + qx * bv.w);
                *(float4 *)sp = ns;
                part = ns.x * cv.x + ns.y * cv.y + ns.z * cv.z + ns.w * cv.w;
            }
            // sum over the lpr lanes of the row (aligned groups of a power of two):
            // a 16-lane row (N = 64) or two (N = 128) through DPP and the lane
            // swap, other widths through LDS permutes
            if (lpr == 16) {
                part = sum16(part);
            } else if (lpr == 32) {
                part = sum16(part);
                part += xor16_f(part);
            } else {
                for (int o = lpr >> 1; o > 0; o >>= 1) part += __shfl_xor(part, o, 64);
            }
            if (active && n0 == 0) {
                float y = part;
                if (prm.has_D) y += x * prm.D[h * prm.D_h + (prm.d_per_channel ? p * prm.D_p : 0)];
                if (prm.has_z) y *= silu_f(prm.z[b * prm.z_b + h * prm.z_h + p]);
                prm.out[xo] = y;
            }
        }
    }
}
#endif

}  // namespace ssd
