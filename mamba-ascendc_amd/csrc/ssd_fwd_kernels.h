// Chunk-parallel forward pieces of the Mamba-2 SSD hot path, and the generic
// token recurrence for shapes outside the MFMA kernels.
//
// Execution chunk T = 64 tokens.  Per (batch b, head h, chunk k), with q the
// discretised dt, a = A*q and cs the chunk-local inclusive cumsum of a:
//
//   k_chunk_state : U[k][p][n] = sum_t q_t x_t[p] exp(cs_last - cs_t) B_t[n]
//                   chunk_log_decay[k] = cs_last   (the backward's state
//                   recompute when the forward's chunk states are not passed)
//   k_state_pass  : S_start[k] = S ; S = exp(cs_last[k]) S + U[k]  (in place;
//                   also over segments of the fused forward and as the
//                   standalone state-passing op)
//
// The math is that of mamba_ascendc/csrc/ops/mamba2_ssd_fwd/design.md:10-20 and
// the chunked decomposition of mamba_torch/ssd_reference.py:113-189; the
// blocking, layouts and precision scheme are this file's own.
#pragma once

#include "ssd_device.h"

namespace ssd {

constexpr int kChunk = 64;    // execution chunk
constexpr int kThreads = 256; // 4 waves per workgroup

struct FwdParams {
    const float *x, *dt, *A, *B, *C, *D, *z, *dt_bias, *init;
    float *out, *final_state;
    float *pre_gate;        // [B, L, H, P] y + D x before the z gate, or NULL
    float *states;          // [B, H, K, P, N]: chunk states, then states at chunk starts
    float *chunk_log_decay; // [B, H, K]
    float *chunk_states;    // [B, H, K, P, N] state entering each chunk (fused forward), or NULL
    const int32_t *seq_idx; // [B, L] sequence id of every token (packed sequences), or NULL
    int64_t L;
    int H, G, R, K;         // heads, groups, heads per group, chunks
    int hdiv;               // the fused kernels see a head of dim 64 m as m heads of dim 64
                            // (H, R counted that way); dt, A, dt_bias and a per-head D are
                            // indexed by h / hdiv, dt's token stride is H / hdiv
    int softplus, has_D, d_per_channel, has_z;
    float lo, hi;
    const float *cb;        // [B, G, K, 64, 64] C_t . B_s of every chunk (k_chunk_cb), read by
                            // k_fwd_wide<.., kCB = true>; NULL otherwise
};

// Chunk-local q and cs for (b, h, chunk k) by wave 0: s_q[t], s_cs[t].
// Returns this lane's cs.
__device__ __forceinline__ float chunk_prologue(const FwdParams &p, int b, int h, int64_t t0,
                                               int tv, float *s_q, float *s_cs) {
    const int lane = threadIdx.x & 63;
    float q = 0.f, a = 0.f;
    if (lane < tv) {
        const float bias = p.dt_bias ? p.dt_bias[h] : 0.f;
        q = discretize_dt(p.dt[((int64_t)b * p.L + t0 + lane) * p.H + h], bias, p.softplus != 0,
                          p.lo, p.hi);
        a = p.A[h] * q;
    }
    const float cs = wave_inclusive_scan(a);
    s_q[lane] = q;
    s_cs[lane] = cs;
    return cs;
}

// --------------------------------------------------------------------------
// chunk states
// --------------------------------------------------------------------------
template <int P, int N>
__global__ __launch_bounds__(kThreads) void k_chunk_state(FwdParams prm) {
    constexpr int T = kChunk;
    constexpr int XS = T + 8; // LDS row stride in halves of the [row][t] tiles
    __shared__ float s_q[T], s_cs[T], s_w[T];
    __shared__ __attribute__((aligned(16))) _Float16 xh[P * XS], xl[P * XS];
    __shared__ __attribute__((aligned(16))) _Float16 bh[N * XS], bl[N * XS];

    const int k = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t t0 = (int64_t)k * T;
    const int tv = (int)min((int64_t)T, prm.L - t0);
    const int g = h / prm.R;

    if (wave == 0) {
        const float cs = chunk_prologue(prm, b, h, t0, tv, s_q, s_cs);
        const float last = readlane_f(cs, T - 1);
        s_w[lane] = s_q[lane] * __expf(last - cs);
        if (lane == 0) prm.chunk_log_decay[((int64_t)b * prm.H + h) * prm.K + k] = last;
    }
    __syncthreads();

    // x_t[p] * q_t * exp(cs_last - cs_t), transposed to [p][t]
    {
        constexpr int TPC = kThreads / P; // threads per column
        constexpr int TT = T / TPC;       // tokens per thread
        const int pc = tid % P, tb = tid / P;
        const float *xb = prm.x + (((int64_t)b * prm.L + t0) * prm.H + h) * P + pc;
#pragma unroll
        for (int i0 = 0; i0 < TT; i0 += 8) {
            half8 vh, vl;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int t = tb * TT + i0 + i;
                const float v = t < tv ? xb[(int64_t)t * prm.H * P] * s_w[t] : 0.f;
                _Float16 a, c;
                split_f16(v, a, c);
                vh[i] = a;
                vl[i] = c;
            }
            *(half8 *)&xh[pc * XS + tb * TT + i0] = vh;
            *(half8 *)&xl[pc * XS + tb * TT + i0] = vl;
        }
    }
    // B_t[n] transposed to [n][t]
    {
        constexpr int TPC = kThreads / N;
        constexpr int TT = T / TPC;
        const int nc = tid % N, tb = tid / N;
        const float *bb = prm.B + (((int64_t)b * prm.L + t0) * prm.G + g) * N + nc;
#pragma unroll
        for (int i0 = 0; i0 < TT; i0 += 8) {
            half8 vh, vl;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int t = tb * TT + i0 + i;
                const float v = t < tv ? bb[(int64_t)t * prm.G * N] : 0.f;
                _Float16 a, c;
                split_f16(v, a, c);
                vh[i] = a;
                vl[i] = c;
            }
            *(half8 *)&bh[nc * XS + tb * TT + i0] = vh;
            *(half8 *)&bl[nc * XS + tb * TT + i0] = vl;
        }
    }
    __syncthreads();

    const int r16 = lane & 15, kq = lane >> 4;
    float *U = prm.states + (((int64_t)b * prm.H + h) * prm.K + k) * (int64_t)(P * N);
    for (int pb = wave; pb < P / 16; pb += 4) {
        f32x4 acc[N / 16];
#pragma unroll
        for (int nb = 0; nb < N / 16; ++nb) acc[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < T / 32; ++ks) {
            const half8 ah = *(const half8 *)&xh[(pb * 16 + r16) * XS + ks * 32 + kq * 8];
            const half8 al = *(const half8 *)&xl[(pb * 16 + r16) * XS + ks * 32 + kq * 8];
#pragma unroll
            for (int nb = 0; nb < N / 16; ++nb) {
                const half8 b_h = *(const half8 *)&bh[(nb * 16 + r16) * XS + ks * 32 + kq * 8];
                const half8 b_l = *(const half8 *)&bl[(nb * 16 + r16) * XS + ks * 32 + kq * 8];
                acc[nb] = mma3(ah, al, b_h, b_l, acc[nb]);
            }
        }
#pragma unroll
        for (int nb = 0; nb < N / 16; ++nb)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                U[(pb * 16 + kq * 4 + r) * N + nb * 16 + r16] = acc[nb][r];
    }
}

// --------------------------------------------------------------------------
// state passing (elementwise over P*N, serial over chunks)
// --------------------------------------------------------------------------
constexpr int kStateRing = 16;  // chunks in flight per thread in k_state_pass (and _bwd)

// Four consecutive chunk-state elements (element offset `elem`) as fp32: the
// chunk states of the stage op come in fp32 or, as the reference's op also
// takes them, in fp16 (8-byte loads, widened exactly).
template <typename Tin>
__device__ __forceinline__ float4 load_state4(__amdgpu_buffer_rsrc_t r, int elem) {
    if constexpr (sizeof(Tin) == 2) {
        typedef uint32_t u2 __attribute__((ext_vector_type(2)));
        const u2 v = __builtin_bit_cast(u2, __builtin_amdgcn_raw_buffer_load_b64(r, elem * 2, 0, 0));
        const half4 h = __builtin_bit_cast(half4, v);
        return make_float4((float)h[0], (float)h[1], (float)h[2], (float)h[3]);
    } else {
        return buf_load4(r, elem * 4, 0);
    }
}

// S_start[k] = S ; S = exp(log_decay[k]) S + U[k] over the K chunks of one
// (b, h) stream (blockIdx.y), four state elements per thread.
template <typename Tin>
__device__ __forceinline__ void state_pass_body(const Tin *chunk_states, const float *log_decay, const float *init,
                                                float *states_start, float *final_state, int K, int PN) {
    constexpr int D = kStateRing;
    const int64_t bh = blockIdx.y;
    const int idx = (blockIdx.x * kThreads + threadIdx.x) * 4;
    if (idx >= PN) return;
    const Tin *u = chunk_states + bh * K * (int64_t)PN;
    float *so = states_start + bh * K * (int64_t)PN + idx;
    const float *ld = log_decay + bh * K;
    float4 s = init ? *(const float4 *)(init + bh * PN + idx) : make_float4(0.f, 0.f, 0.f, 0.f);
    // a ring of D chunks in flight: chunk k sits in slot k % D and is loaded
    // D chunks before it is used.  The loads are unconditional: chunks past K
    // read through a resource whose range ends at chunk K (zeros, no memory
    // traffic), so every round issues the same loads and the wait counts
    // stay exact.
    auto rsrc_from = [&](int k) {
        const int64_t left = (int64_t)(K - k) * PN * (int64_t)sizeof(Tin);
        return buf_rsrc_n(u + (int64_t)k * PN, (int)(left < 0 ? 0 : (left > 0x7fffffff ? 0x7fffffff : left)));
    };
    // the log decays ride in the same ring (every lane reads the chunk's one value)
    const auto rl = buf_rsrc_n(ld, K * 4);
    float4 buf[D];
    float lv[D];
    {
        const auto r = rsrc_from(0);
#pragma unroll
        for (int i = 0; i < D; ++i) {
            buf[i] = load_state4<Tin>(r, i * PN + idx);
            lv[i] = buf_load(rl, 0, i * 4);
        }
    }
    int k0 = 0;
    for (; k0 + D <= K; k0 += D) {
        const auto r = rsrc_from(k0 + D);
#pragma unroll
        for (int i = 0; i < D; ++i) {
            const float dec = __expf(lv[i]);
            *(float4 *)(so + (int64_t)(k0 + i) * PN) = s;
            s.x = dec * s.x + buf[i].x;
            s.y = dec * s.y + buf[i].y;
            s.z = dec * s.z + buf[i].z;
            s.w = dec * s.w + buf[i].w;
            buf[i] = load_state4<Tin>(r, i * PN + idx);
            lv[i] = buf_load(rl, 0, (k0 + D + i) * 4);
        }
    }
#pragma unroll
    for (int i = 0; i < D; ++i) {
        if (k0 + i < K) {
            const float dec = __expf(lv[i]);
            *(float4 *)(so + (int64_t)(k0 + i) * PN) = s;
            s.x = dec * s.x + buf[i].x;
            s.y = dec * s.y + buf[i].y;
            s.z = dec * s.z + buf[i].z;
            s.w = dec * s.w + buf[i].w;
        }
    }
    if (final_state) *(float4 *)(final_state + bh * PN + idx) = s;
}

#ifndef SSD_KERNEL_TEMPLATES_ONLY
__global__ __launch_bounds__(kThreads) void k_state_pass(const float *chunk_states, const float *log_decay,
                                                         const float *init, float *states_start,
                                                         float *final_state, int K, int PN) {
    state_pass_body(chunk_states, log_decay, init, states_start, final_state, K, PN);
}

// The same with fp16 chunk states (fp32 states out).
__global__ __launch_bounds__(kThreads) void k_state_pass_f16(const _Float16 *chunk_states, const float *log_decay,
                                                             const float *init, float *states_start,
                                                             float *final_state, int K, int PN) {
    state_pass_body(chunk_states, log_decay, init, states_start, final_state, K, PN);
}
#endif

// --------------------------------------------------------------------------
// zero-padding copy: dst[o][r][c] = (r < rs && c < cs) ? src[o][r][c] : 0 for
// r < rd, c < cd (a [outer, rs, cs] array into [outer, rd, cd]; with rd <= rs
// and cd <= cs it cuts the padding off again).  Grid-stride over dst.
// --------------------------------------------------------------------------
#ifndef SSD_KERNEL_TEMPLATES_ONLY
constexpr int kPadThreads = 256;
__global__ __launch_bounds__(kPadThreads) void k_pad_copy(const float *src, int64_t outer, int rs, int cs,
                                                          float *dst, int rd, int cd) {
    const int64_t total = outer * rd * cd;
    for (int64_t i = (int64_t)blockIdx.x * kPadThreads + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * kPadThreads) {
        const int c = (int)(i % cd);
        const int64_t orow = i / cd;
        const int r = (int)(orow % rd);
        const int64_t o = orow / rd;
        dst[i] = (r < rs && c < cs) ? src[(o * rs + r) * cs + c] : 0.f;
    }
}
#endif

// --------------------------------------------------------------------------
// dst[i] = src ? src[i] : 0 for i < n (grid-stride): the states of an empty
// sequence (its initial state, or zero) written by a kernel, so the forward
// issues no memset or memcpy nodes (a caller may capture it in a graph).
// --------------------------------------------------------------------------
#ifndef SSD_KERNEL_TEMPLATES_ONLY
__global__ __launch_bounds__(kPadThreads) void k_copy_or_zero(const float *src, float *dst, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * kPadThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kPadThreads)
        dst[i] = src ? src[i] : 0.f;
}
#endif

// --------------------------------------------------------------------------
// generic token recurrence (any headdim / dstate <= 256); one wave per (b,h,p)
// --------------------------------------------------------------------------
#ifndef SSD_KERNEL_TEMPLATES_ONLY
__global__ __launch_bounds__(64) void k_generic_fwd(FwdParams prm, int P, int N) {
    const int pc = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int lane = threadIdx.x;
    const int g = h / prm.R;
    float S[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int n = lane + 64 * i;
        S[i] = (n < N && prm.init) ? prm.init[(((int64_t)b * prm.H + h) * P + pc) * N + n] : 0.f;
    }
    const float bias = prm.dt_bias ? prm.dt_bias[h] : 0.f;
    const float A = prm.A[h];
    for (int64_t t = 0; t < prm.L; ++t) {
        const float q = discretize_dt(prm.dt[((int64_t)b * prm.L + t) * prm.H + h], bias,
                                      prm.softplus != 0, prm.lo, prm.hi);
        const float a = expf(A * q);
        const int64_t row = (((int64_t)b * prm.L + t) * prm.H + h) * P;
        const float xv = prm.x[row + pc];
        const float v = xv * q;
        const float *Bt = prm.B + (((int64_t)b * prm.L + t) * prm.G + g) * N;
        const float *Ct = prm.C + (((int64_t)b * prm.L + t) * prm.G + g) * N;
        float part = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int n = lane + 64 * i;
            if (n < N) {
                S[i] = a * S[i] + v * Bt[n];
                part += S[i] * Ct[n];
            }
        }
        float y = wave_sum(part);
        if (lane == 0) {
            if (prm.has_D) y += (prm.d_per_channel ? prm.D[h * P + pc] : prm.D[h]) * xv;
            if (prm.pre_gate) prm.pre_gate[row + pc] = y;
            if (prm.has_z) y *= silu_f(prm.z[row + pc]);
            prm.out[row + pc] = y;
        }
    }
    if (prm.final_state) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int n = lane + 64 * i;
            if (n < N) prm.final_state[(((int64_t)b * prm.H + h) * P + pc) * N + n] = S[i];
        }
    }
}
#endif

}  // namespace ssd
