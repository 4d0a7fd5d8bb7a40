// Forward kernels of the Mamba-2 SSD hot path (chunk-parallel form).
//
// Execution chunk T = 64 tokens.  Per (batch b, head h, chunk k), with q the
// discretised dt, a = A*q and cs the chunk-local inclusive cumsum of a:
//
//   k_chunk_state : U[k][p][n] = sum_t q_t x_t[p] exp(cs_last - cs_t) B_t[n]
//                   chunk_log_decay[k] = cs_last
//   k_state_pass  : S_start[k] = S ; S = exp(cs_last[k]) S + U[k]  (in place)
//   k_chunk_scan  : y_t = sum_{s<=t} (C_t.B_s) exp(cs_t - cs_s) q_s x_s
//                         + exp(cs_t) C_t . S_start[k]          (+ D x, * silu z)
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
    int64_t L;
    int H, G, R, K;         // heads, groups, heads per group, chunks
    int softplus, has_D, d_per_channel, has_z;
    float lo, hi;
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
        const float last = __shfl(cs, T - 1, 64);
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
constexpr int kStateDepth = 8;

__global__ __launch_bounds__(kThreads) void k_state_pass(const float *chunk_states,
                                                         const float *log_decay,
                                                         const float *init, float *states_start,
                                                         float *final_state, int K, int PN) {
    const int64_t bh = blockIdx.y;
    const int idx = (blockIdx.x * kThreads + threadIdx.x) * 4;
    if (idx >= PN) return;
    const float *u = chunk_states + bh * K * (int64_t)PN + idx;
    float *so = states_start + bh * K * (int64_t)PN + idx;
    const float *ld = log_decay + bh * K;
    float4 s = init ? *(const float4 *)(init + bh * PN + idx) : make_float4(0.f, 0.f, 0.f, 0.f);
    for (int k0 = 0; k0 < K; k0 += kStateDepth) {
        float4 buf[kStateDepth];
        float dec[kStateDepth];
#pragma unroll
        for (int i = 0; i < kStateDepth; ++i) {
            if (k0 + i < K) {
                buf[i] = *(const float4 *)(u + (int64_t)(k0 + i) * PN);
                dec[i] = __expf(ld[k0 + i]);
            }
        }
#pragma unroll
        for (int i = 0; i < kStateDepth; ++i) {
            if (k0 + i < K) {
                *(float4 *)(so + (int64_t)(k0 + i) * PN) = s;
                s.x = dec[i] * s.x + buf[i].x;
                s.y = dec[i] * s.y + buf[i].y;
                s.z = dec[i] * s.z + buf[i].z;
                s.w = dec[i] * s.w + buf[i].w;
            }
        }
    }
    if (final_state) *(float4 *)(final_state + bh * PN + idx) = s;
}

// --------------------------------------------------------------------------
// chunk scan: y = (C B^T o decay) (x q) + exp(cs) C S_start, + D x, * silu(z)
// --------------------------------------------------------------------------
template <int P, int N>
__global__ __launch_bounds__(kThreads) void k_chunk_scan(FwdParams prm) {
    constexpr int T = kChunk;
    constexpr int NS = N + 8; // row stride (halves) of [row][n] tiles
    constexpr int XS = T + 8; // row stride (halves) of the [p][perm(s)] tile
    __shared__ float s_q[T], s_cs[T];
    __shared__ __attribute__((aligned(16))) _Float16 bsh[T * NS], bsl[T * NS];
    __shared__ __attribute__((aligned(16))) _Float16 ssh[P * NS], ssl[P * NS];
    __shared__ __attribute__((aligned(16))) _Float16 xph[P * XS], xpl[P * XS];

    const int k = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int64_t t0 = (int64_t)k * T;
    const int tv = (int)min((int64_t)T, prm.L - t0);
    const int g = h / prm.R;

    if (w == 0) chunk_prologue(prm, b, h, t0, tv, s_q, s_cs);

    // B rows [s][n]
    for (int i = tid; i < T * N / 4; i += kThreads) {
        const int t = i / (N / 4), n4 = (i % (N / 4)) * 4;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (t < tv) v = *(const float4 *)(prm.B + (((int64_t)b * prm.L + t0 + t) * prm.G + g) * N + n4);
        half4 vh, vl;
        split4(v, vh, vl);
        *(half4 *)&bsh[t * NS + n4] = vh;
        *(half4 *)&bsl[t * NS + n4] = vl;
    }
    // S_start rows [p][n]
    {
        const float *S = prm.states + (((int64_t)b * prm.H + h) * prm.K + k) * (int64_t)(P * N);
        for (int i = tid; i < P * N / 4; i += kThreads) {
            const int pr = i / (N / 4), n4 = (i % (N / 4)) * 4;
            const float4 v = *(const float4 *)(S + pr * N + n4);
            half4 vh, vl;
            split4(v, vh, vl);
            *(half4 *)&ssh[pr * NS + n4] = vh;
            *(half4 *)&ssl[pr * NS + n4] = vl;
        }
    }
    __syncthreads(); // s_q visible
    // x_s[p] * q_s transposed to [p][perm(s)]: thread writes one 8-slot run
    {
        constexpr int TPC = kThreads / P;
        const int pc = tid % P, tb = tid / P;
        const float *xb = prm.x + (((int64_t)b * prm.L + t0) * prm.H + h) * P + pc;
        for (int run = tb; run < T / 8; run += TPC) {
            const int m = run >> 2, j = run & 3; // slab m, lane group j
            half8 vh, vl;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int s = m * 32 + (i < 4 ? 4 * j + i : 16 + 4 * j + (i - 4));
                const float v = s < tv ? xb[(int64_t)s * prm.H * P] * s_q[s] : 0.f;
                _Float16 a, c;
                split_f16(v, a, c);
                vh[i] = a;
                vl[i] = c;
            }
            *(half8 *)&xph[pc * XS + m * 32 + j * 8] = vh;
            *(half8 *)&xpl[pc * XS + m * 32 + j * 8] = vl;
        }
    }
    __syncthreads();

    const int r16 = lane & 15, kq = lane >> 4;
    const int t_lane = w * 16 + r16; // C row owned by this lane as an operand

    // C rows of this wave's 16-token block, split, in operand layout
    half8 ch[N / 32], cl[N / 32];
    {
        const float *crow = prm.C + (((int64_t)b * prm.L + t0 + t_lane) * prm.G + g) * N;
#pragma unroll
        for (int ks = 0; ks < N / 32; ++ks) {
            float4 v0 = make_float4(0.f, 0.f, 0.f, 0.f), v1 = v0;
            if (t_lane < tv) {
                v0 = *(const float4 *)(crow + ks * 32 + kq * 8);
                v1 = *(const float4 *)(crow + ks * 32 + kq * 8 + 4);
            }
            const float vv[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                _Float16 a, c;
                split_f16(vv[i], a, c);
                ch[ks][i] = a;
                cl[ks][i] = c;
            }
        }
    }

    // y_off = C . S_start^T, rows scaled by exp(cs_t)
    f32x4 acc[P / 16];
#pragma unroll
    for (int pb = 0; pb < P / 16; ++pb) {
        acc[pb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < N / 32; ++ks) {
            const half8 sh = *(const half8 *)&ssh[(pb * 16 + r16) * NS + ks * 32 + kq * 8];
            const half8 sl = *(const half8 *)&ssl[(pb * 16 + r16) * NS + ks * 32 + kq * 8];
            acc[pb] = mma3(ch[ks], cl[ks], sh, sl, acc[pb]);
        }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const float e = __expf(s_cs[w * 16 + kq * 4 + r]);
#pragma unroll
        for (int pb = 0; pb < P / 16; ++pb) acc[pb][r] *= e;
    }

    // (C B^T)^T tiles for source blocks sigma <= w:
    // cbt[sigma][r] = C_t . B_s with t = 16 w + r16, s = 16 sigma + 4 kq + r
    f32x4 cbt[T / 16];
#pragma unroll
    for (int sg = 0; sg < T / 16; ++sg) {
        cbt[sg] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (sg <= w) {
#pragma unroll
            for (int ks = 0; ks < N / 32; ++ks) {
                const half8 b_h = *(const half8 *)&bsh[(sg * 16 + r16) * NS + ks * 32 + kq * 8];
                const half8 b_l = *(const half8 *)&bsl[(sg * 16 + r16) * NS + ks * 32 + kq * 8];
                cbt[sg] = mma3(b_h, b_l, ch[ks], cl[ks], cbt[sg]);
            }
        }
    }

    // y_diag: W[t][s] = cbt * exp(cs_t - cs_s) on s <= t, fed as the A operand
    // with the k permutation of perm32 (no LDS round trip)
    const float cs_t = s_cs[t_lane];
#pragma unroll
    for (int m = 0; m < T / 32; ++m) {
        if (2 * m <= w) {
            half8 wh, wl;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int s0 = m * 32 + 4 * kq + r, s1 = s0 + 16;
                const float v0 = (s0 <= t_lane) ? cbt[2 * m][r] * __expf(cs_t - s_cs[s0]) : 0.f;
                const float v1 = (2 * m + 1 <= w && s1 <= t_lane)
                                     ? cbt[2 * m + 1][r] * __expf(cs_t - s_cs[s1])
                                     : 0.f;
                _Float16 a, c;
                split_f16(v0, a, c);
                wh[r] = a;
                wl[r] = c;
                split_f16(v1, a, c);
                wh[4 + r] = a;
                wl[4 + r] = c;
            }
#pragma unroll
            for (int pb = 0; pb < P / 16; ++pb) {
                const half8 xh_ = *(const half8 *)&xph[(pb * 16 + r16) * XS + m * 32 + kq * 8];
                const half8 xl_ = *(const half8 *)&xpl[(pb * 16 + r16) * XS + m * 32 + kq * 8];
                acc[pb] = mma3(wh, wl, xh_, xl_, acc[pb]);
            }
        }
    }

    // epilogue: + D x, * silu(z), store
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int t = w * 16 + kq * 4 + r;
        if (t >= tv) continue;
        const int64_t row = (((int64_t)b * prm.L + t0 + t) * prm.H + h) * P;
#pragma unroll
        for (int pb = 0; pb < P / 16; ++pb) {
            const int pc = pb * 16 + r16;
            float v = acc[pb][r];
            if (prm.has_D) {
                const float d = prm.d_per_channel ? prm.D[h * P + pc] : prm.D[h];
                v += d * prm.x[row + pc];
            }
            if (prm.pre_gate) prm.pre_gate[row + pc] = v;
            if (prm.has_z) v *= silu_f(prm.z[row + pc]);
            prm.out[row + pc] = v;
        }
    }
}

// --------------------------------------------------------------------------
// generic token recurrence (any headdim / dstate <= 256); one wave per (b,h,p)
// --------------------------------------------------------------------------
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

}  // namespace ssd
