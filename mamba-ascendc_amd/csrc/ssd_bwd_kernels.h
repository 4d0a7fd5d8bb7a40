// Backward kernels of the Mamba-2 SSD hot path (M1 spec: headdim = dstate = 64,
// execution chunk T = 64).
//
// Per (batch b, head h, chunk k), with q the discretised dt, cs the chunk-local
// inclusive cumsum of A*q, S_k the state entering chunk k, gy = dout * silu(z)
// (or dout), decay_t = exp(cs_last - cs_t):
//
//   k_bwd_dstate      : dSoff_k[p][n] = sum_t gy_t[p] exp(cs_t) C_t[n] (and the
//                       chunk log decay cs_last; with packed sequences the
//                       forward's masks: exp(cs_t) only for tokens that read
//                       the entering state, -inf where the state is cut)
//   k_state_pass_bwd  : reverse recurrence over chunks, in place:
//                         dU_k = g_{k+1};  g_k = dSoff_k + exp(cs_last_k) g_{k+1}
//                       with g_K = dfinal_state and dinitial_states = g_0
//   the chunk products, dx, ddt, dB, dC, dz and the dA / ddt_bias / dD
//   partials run in k_bwd_ws (ssd_bwd_fused.h), the fixed-order sums of the
//   partials in k_bwd_finalize_slots.
//
// The equations are the adjoint of the chunked forward in ssd_fwd_kernels.h
// (the same gradient as mamba_ascendc/csrc/ops/mamba2_ssd_bwd/design.md:73-107 and
// mamba_ascendc/csrc/ops/mamba2_ssd_dt_bwd/design.md:61-78); the kernel split
// and layouts are this file's own.
#pragma once

#include "ssd_bf16.h"
#include "ssd_fwd_kernels.h"

namespace ssd {

struct BwdParams {
    const float *x, *dt, *A, *B, *C, *D, *z, *dt_bias, *dout, *pre_gate;
    float *dx, *ddt, *dB, *dC, *dz;
    const float *states;    // [B, H, K, P, N] state entering each chunk
    float *log_decay;       // [B, H, K] chunk sum of A q (written by k_bwd_dstate)
    float *dstates;         // [B, H, K, P, N]: dSoff, then dU (not used by the
                            // reverse fused chunk kernel)
    const int32_t *seq_idx; // [B, L] sequence id of every token (packed sequences), or NULL
    const float *dfinal;    // [B, H, P, N] or NULL (zero)
    float *dinit;           // [B, H, P, N] or NULL
    float *part_dA;         // [B, H, K]
    float *part_dbias;      // [B, H, K]
    float *part_dD;         // [B, H, K, P] (per-channel D) or [B, H, K]
    const float *carry_in;  // [B, H, nseg, P, N] gradient entering each run of the reverse
                            // fused kernel from the right, or NULL (one run: dfinal)
    int64_t L;
    int H, G, R, K;
    int softplus, has_D, d_per_channel, has_z;
    float lo, hi;
};

// Runs of the reverse fused backward: nseg runs of M chunks per (b, h), whose
// own contributions to the gradient entering each run (seg_carry [B, H, nseg,
// P, N]) and log decays (seg_log_decay [B, H, nseg]) the run pre-pass
// k_bwd_run_grad forms.
struct RevSeg {
    int nseg, M;
    float *seg_carry, *seg_log_decay;
};

// q, cs and dq/ddt of the tokens of one chunk, by wave 0.  Returns this lane's cs.
__device__ __forceinline__ float bwd_prologue(const BwdParams &p, int b, int h, int64_t t0, int tv,
                                             float *s_q, float *s_cs, float *s_dqdu) {
    const int lane = threadIdx.x & 63;
    float q = 0.f, a = 0.f, dq = 0.f;
    if (lane < tv) {
        const float bias = p.dt_bias ? p.dt_bias[h] : 0.f;
        const float dtv = p.dt[((int64_t)b * p.L + t0 + lane) * p.H + h];
        q = discretize_dt(dtv, bias, p.softplus != 0, p.lo, p.hi);
        dq = discretize_grad(dtv, bias, p.softplus != 0, p.lo, p.hi);
        a = p.A[h] * q;
    }
    const float cs = wave_inclusive_scan(a);
    s_q[lane] = q;
    s_cs[lane] = cs;
    s_dqdu[lane] = dq;
    return cs;
}


// --------------------------------------------------------------------------
// dSoff_k = (gy * exp(cs))^T C, one workgroup per (k, h, b); split-bf16
// operands (ssd_bf16.h)
// --------------------------------------------------------------------------
#ifndef SSD_KERNEL_TEMPLATES_ONLY
namespace bwd {
__global__ __launch_bounds__(kThreads) void k_bwd_dstate(BwdParams prm) {
    constexpr int P = 64, N = 64, T = 64;
    __shared__ float s_q[T], s_cs[T], s_dqdu[T], s_e[T];
    __shared__ __attribute__((aligned(16))) __bf16 lds[4 * kTile];

    const int k = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int r16 = lane & 15, kq = lane >> 4;
    const int64_t t0 = (int64_t)k * T;
    const int tv = (int)min((int64_t)T, prm.L - t0);
    const int g = h / prm.R;
    const int64_t rowHP = (int64_t)prm.H * P, rowGN = (int64_t)prm.G * N;

    if (w == 0) {
        const float cs = bwd_prologue(prm, b, h, t0, tv, s_q, s_cs, s_dqdu);
        float e = __expf(cs), ld = cs;
        if (prm.seq_idx) {
            // packed sequences: a token reads the entering state only if its id
            // is that of the token before the chunk (0 before the first); the
            // state carries over the chunk only if the chunk ends on that id
            const int32_t *si = prm.seq_idx + (int64_t)b * prm.L + t0;
            const int sid = si[min(lane, tv - 1)];
            const int prev = k > 0 ? si[-1] : 0;
            const int last = __builtin_amdgcn_readlane(sid, T - 1);
            if (sid != prev) e = 0.f;
            if (last != prev) ld = -INFINITY;
        }
        s_e[lane] = e;
        if (lane == T - 1) prm.log_decay[((int64_t)b * prm.H + h) * prm.K + k] = ld;
    }
    __syncthreads();

    const int64_t xo = (((int64_t)b * prm.L + t0) * prm.H + h) * P;
    const float *dout = prm.dout ? prm.dout + xo : nullptr;
    const float *z = prm.has_z ? prm.z + xo : nullptr;
    const float *Cg = prm.C + (((int64_t)b * prm.L + t0) * prm.G + g) * N;
    SplitTile gq = tile_at(lds, 0), ct = tile_at(lds, 1);
    // gq[p][t] = gy_t[p] exp(cs_t);  ct[n][t] = C_t[n]
    stage_cols<false>(gq, [&](int t, int c) {
        if (t >= tv || !dout) return 0.f;
        const int64_t o = (int64_t)t * rowHP + c;
        float v = dout[o];
        if (z) v *= silu_f(z[o]);
        return v * s_e[t];
    });
    stage_cols<false>(ct, [&](int t, int c) { return t < tv ? Cg[(int64_t)t * rowGN + c] : 0.f; });
    __syncthreads();

    f32x4 acc[4];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) acc[nb] = zero4();
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
        const Frag a = frag(gq, 16 * w + r16, ks);
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) acc[nb] = mma3f(a, frag(ct, 16 * nb + r16, ks), acc[nb]);
    }
    float *out = prm.dstates + (((int64_t)b * prm.H + h) * prm.K + k) * (int64_t)(P * N);
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
        for (int r = 0; r < 4; ++r) out[(16 * w + 4 * kq + r) * N + 16 * nb + r16] = acc[nb][r];
}
}  // namespace bwd
#endif

// --------------------------------------------------------------------------
// reverse state passing (elementwise over P*N, serial over chunks, in place)
// --------------------------------------------------------------------------
#ifndef SSD_KERNEL_TEMPLATES_ONLY
__global__ __launch_bounds__(kThreads) void k_state_pass_bwd(float *ds, const float *log_decay,
                                                             const float *dfinal, float *dinit,
                                                             int K, int PN) {
    constexpr int D = kStateRing;
    const int64_t bh = blockIdx.y;
    const int idx = (blockIdx.x * kThreads + threadIdx.x) * 4;
    if (idx >= PN) return;
    float *d = ds + bh * K * (int64_t)PN;
    float4 g = dfinal ? *(const float4 *)(dfinal + bh * PN + idx) : make_float4(0.f, 0.f, 0.f, 0.f);
    // step i handles chunk K - 1 - i; a ring of D steps in flight (step i in
    // slot i % D, loaded D steps before it is used).  The loads are
    // unconditional (exact wait counts): a step past chunk 0 reads through an
    // empty-range resource (zeros, no memory traffic), and its value is never
    // used.  The caller keeps K * PN * 4 below 2^31.
    const float *ld = log_decay + bh * K;
    float4 buf[D];
    float lv[D];
#pragma unroll
    for (int i = 0; i < D; ++i) {
        const int k = max(K - 1 - i, 0);
        buf[i] = buf_load4(buf_rsrc_n(d, i < K ? K * PN * 4 : 0), (k * PN + idx) * 4, 0);
        lv[i] = buf_load(buf_rsrc_n(ld, i < K ? K * 4 : 0), k * 4, 0);
    }
    int i0 = 0;
    for (; i0 + D <= K; i0 += D) {
#pragma unroll
        for (int i = 0; i < D; ++i) {
            const int k = K - 1 - (i0 + i);
            const float dec = __expf(lv[i]);
            *(float4 *)(d + (int64_t)k * PN + idx) = g; // dU_k: the gradient of the state leaving chunk k
            g.x = buf[i].x + dec * g.x;
            g.y = buf[i].y + dec * g.y;
            g.z = buf[i].z + dec * g.z;
            g.w = buf[i].w + dec * g.w;
            const int kn = max(k - D, 0);
            buf[i] = buf_load4(buf_rsrc_n(d, k >= D ? K * PN * 4 : 0), (kn * PN + idx) * 4, 0);
            lv[i] = buf_load(buf_rsrc_n(ld, k >= D ? K * 4 : 0), kn * 4, 0);
        }
    }
#pragma unroll
    for (int i = 0; i < D; ++i) {
        if (i0 + i < K) {
            const int k = K - 1 - (i0 + i);
            const float dec = __expf(lv[i]);
            *(float4 *)(d + (int64_t)k * PN + idx) = g;
            g.x = buf[i].x + dec * g.x;
            g.y = buf[i].y + dec * g.y;
            g.z = buf[i].z + dec * g.z;
            g.w = buf[i].w + dec * g.w;
        }
    }
    if (dinit) *(float4 *)(dinit + bh * PN + idx) = g;
}
#endif

// --------------------------------------------------------------------------
// workgroup sum (256 threads) in a fixed order
// --------------------------------------------------------------------------
__device__ __forceinline__ float block_sum(float v, float *s_tmp) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) s_tmp[w] = v;
    __syncthreads();
    return s_tmp[0] + s_tmp[1] + s_tmp[2] + s_tmp[3];
}

}  // namespace ssd
