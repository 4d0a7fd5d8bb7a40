// Backward kernels of the Mamba-2 SSD hot path (M1 spec: headdim = dstate = 64,
// execution chunk T = 64).
//
// Per (batch b, head h, chunk k), with q the discretised dt, cs the chunk-local
// inclusive cumsum of A*q, S_k the state entering chunk k, gy = dout * silu(z)
// (or dout), decay_t = exp(cs_last - cs_t):
//
//   k_bwd_dstate      : dSoff_k[p][n] = sum_t gy_t[p] exp(cs_t) C_t[n]
//   k_state_pass_bwd  : reverse recurrence over chunks, in place:
//                         dU_k = g_{k+1};  g_k = dSoff_k + exp(cs_last_k) g_{k+1}
//                       with g_K = dfinal_state and dinitial_states = g_0
//   k_bwd_chunk       : one workgroup per (b, group g, k) walks the heads of the
//                       group, so dB and dC are summed over heads in a fixed
//                       order in registers (deterministic, no atomics):
//       W[t][s]  = (C_t . B_s) exp(cs_t - cs_s) [s <= t]
//       dW[t][s] = gy_t . xdt_s                               (xdt = x q)
//       dxdt     = W^T gy + decay * (B dU^T)
//       dC      += (dW o exp-mask) B + exp(cs) * (gy S)
//       dB      += (dW o exp-mask)^T C + decay * (xdt dU)
//       dcs_t    = rowsum(dW o W)_t - colsum(dW o W)_t + sum_n dC_off[t][n] C_t[n]
//                  - decay_t r_t,   r_t = xdt_t . (B dU^T)_t
//       dcs_last+= sum_t decay_t r_t + exp(cs_last) sum(dU o S_k)
//       da       = reverse cumsum of dcs;  dq = A da + x . dxdt
//       dx       = q dxdt + D gy;  ddt = dq * dq/ddt;  dz = dout ypre silu'(z)
//     plus per-(b, h, k) partial sums of dA, ddt_bias and dD.
//   k_bwd_finalize    : fixed-order sums of those partials over (b, k).
//
// The equations are the adjoint of the chunked forward in ssd_fwd_kernels.h
// (the same gradient as mamba_ascendc/csrc/ops/mamba2_ssd_bwd/design.md:73-107 and
// mamba_ascendc/csrc/ops/mamba2_ssd_dt_bwd/design.md:61-78); the kernel split,
// layouts and register chaining are this file's own.
#pragma once

#include "ssd_fwd_kernels.h"

namespace ssd {

struct BwdParams {
    const float *x, *dt, *A, *B, *C, *D, *z, *dt_bias, *dout, *pre_gate;
    float *dx, *ddt, *dB, *dC, *dz;
    const float *states;    // [B, H, K, P, N] state entering each chunk
    const float *log_decay; // [B, H, K] chunk sum of A q
    float *dstates;         // [B, H, K, P, N]: dSoff, then dU
    float *part_dA;         // [B, H, K]
    float *part_dbias;      // [B, H, K]
    float *part_dD;         // [B, H, K, P] (per-channel D) or [B, H, K]
    int64_t L;
    int H, G, R, K;
    int softplus, has_D, d_per_channel, has_z;
    float lo, hi;
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

__device__ __forceinline__ float sigmoid_f(float v) { return 1.f / (1.f + __expf(-v)); }

// --------------------------------------------------------------------------
// dSoff_k = (gy * exp(cs))^T C, one workgroup per (k, h, b)
// --------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void k_bwd_dstate(BwdParams prm) {
    constexpr int P = 64, N = 64, T = 64;
    __shared__ float s_q[T], s_cs[T], s_dqdu[T], s_e[T];
    __shared__ __attribute__((aligned(16))) _Float16 lds[4 * kTile];

    const int k = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int r16 = lane & 15, kq = lane >> 4;
    const int64_t t0 = (int64_t)k * T;
    const int tv = (int)min((int64_t)T, prm.L - t0);
    const int g = h / prm.R;
    const int64_t rowHP = (int64_t)prm.H * P, rowGN = (int64_t)prm.G * N;

    if (w == 0) {
        const float cs = bwd_prologue(prm, b, h, t0, tv, s_q, s_cs, s_dqdu);
        s_e[lane] = __expf(cs);
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

// --------------------------------------------------------------------------
// reverse state passing (elementwise over P*N, serial over chunks, in place)
// --------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void k_state_pass_bwd(float *ds, const float *log_decay,
                                                             const float *dfinal, float *dinit,
                                                             int K, int PN) {
    const int64_t bh = blockIdx.y;
    const int idx = (blockIdx.x * kThreads + threadIdx.x) * 4;
    if (idx >= PN) return;
    float *d = ds + bh * K * (int64_t)PN + idx;
    const float *ld = log_decay + bh * K;
    float4 g = dfinal ? *(const float4 *)(dfinal + bh * PN + idx) : make_float4(0.f, 0.f, 0.f, 0.f);
    for (int k0 = K - 1; k0 >= 0; k0 -= kStateDepth) {
        float4 buf[kStateDepth];
        float dec[kStateDepth];
#pragma unroll
        for (int i = 0; i < kStateDepth; ++i) {
            const int kk = k0 - i;
            if (kk >= 0) {
                buf[i] = *(const float4 *)(d + (int64_t)kk * PN);
                dec[i] = __expf(ld[kk]);
            }
        }
#pragma unroll
        for (int i = 0; i < kStateDepth; ++i) {
            const int kk = k0 - i;
            if (kk >= 0) {
                *(float4 *)(d + (int64_t)kk * PN) = g;
                g.x = buf[i].x + dec[i] * g.x;
                g.y = buf[i].y + dec[i] * g.y;
                g.z = buf[i].z + dec[i] * g.z;
                g.w = buf[i].w + dec[i] * g.w;
            }
        }
    }
    if (dinit) *(float4 *)(dinit + bh * PN + idx) = g;
}

// --------------------------------------------------------------------------
// chunk backward, one workgroup per (k, g, b), heads of the group in order
// --------------------------------------------------------------------------
// C_t . B_s is formed once per (b, g, k) into an fp32 LDS tile and read back
// per head in both orientations; global tiles are read through buffer
// resources (per-lane VGPR offset + wave-uniform SGPR offset); every barrier
// orders LDS only (the kernel shares nothing else between waves).  Exponents
// are taken in the log2 domain (cs2 = cumsum of A q log2(e)).
__global__ __launch_bounds__(kThreads) void k_bwd_chunk(BwdParams prm) {
    constexpr int T = 64, P = 64, N = 64, CBS = 68; // CBS: fp32 row stride of s_cb
    __shared__ __attribute__((aligned(16))) _Float16 lds[6 * kTile]; // three split tiles
    __shared__ __attribute__((aligned(16))) float s_cb[T * CBS];   // C_t . B_s at [t][s], s-block <= t-block
    __shared__ float s_q[T], s_cs[T], s_dqdu[T], s_dte[T], s_ecs[T];
    __shared__ float s_dcs1[T], s_goff[T], s_rdte[T], s_da[T], s_ddt[T];
    __shared__ float s_red[4], s_dD[4][P];

    const int k = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
    const int r16 = lane & 15, kq = lane >> 4;
    const int own = 16 * w + r16; // operand row owned by this lane
    const int c = lane;           // staged column of this lane
    const int64_t t0 = (int64_t)k * T;
    const int tv = (int)min((int64_t)T, prm.L - t0);
    const bool full = tv == T;
    const int H = prm.H, G = prm.G;
    const int rowHP4 = H * P * 4, rowGN4 = G * N * 4; // token strides, bytes
    const auto rB = buf_rsrc(prm.B + (((int64_t)b * prm.L + t0) * G + g) * N);
    const auto rC = buf_rsrc(prm.C + (((int64_t)b * prm.L + t0) * G + g) * N);
    const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);

    SplitTile tA = tile_at(lds, 0), tB = tile_at(lds, 1), tC = tile_at(lds, 2);

    // token-major staging of a 64 x 64 tile: lane (tid / 16, tid % 16) reads
    // float4 rows tid / 16 + 16 j; f maps (value, token, column) -> value
    const int rt = tid >> 4, rc4 = (tid & 15) * 4;
    auto stage_rows_buf = [&](SplitTile d, __amdgpu_buffer_rsrc_t r, int row4, auto f) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int t = rt + 16 * j;
            float4 v = (full || t < tv) ? buf_load4(r, rt * row4 + rc4 * 4, 16 * j * row4) : z4;
            v = f(v, t, rc4);
            half4 vh, vl;
            split4(v, vh, vl);
            *(half4 *)&d.hi[t * kTS + rc4] = vh;
            *(half4 *)&d.lo[t * kTS + rc4] = vl;
        }
    };
    // column staging in perm order: tile[c][slot] = f(value of token(slot), token)
    auto stage_cols_buf = [&](SplitTile d, __amdgpu_buffer_rsrc_t r, int row4, auto f) {
#pragma unroll
        for (int rr = 0; rr < 2; ++rr) {
            const int run = w + 4 * rr;
            float v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int t = perm_token(run * 8 + i); // wave-uniform
                v[i] = t < tv ? f(buf_load(r, 4 * c + t * row4, 0), t) : 0.f;
            }
            const Frag fr = pack_frag(v);
            *(half8 *)&d.hi[c * kTS + run * 8] = fr.h;
            *(half8 *)&d.lo[c * kTS + run * 8] = fr.l;
        }
    };
    auto ident4 = [](float4 v, int, int) { return v; };
    auto ident1 = [](float v, int) { return v; };

    // ---- group prologue: C.B^T into s_cb, B own-row operand
    stage_rows_buf(tA, rB, rowGN4, ident4);
    stage_rows_buf(tB, rC, rowGN4, ident4);
    lds_barrier();
    Frag Bown[2];
    {
        Frag Cown[2];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            Bown[ks] = frag(tA, own, ks);
            Cown[ks] = frag(tB, own, ks);
        }
        // rows t = 16 w + 4 kq + i, columns s = 16 j + r16, for s-blocks j <= w
        for (int j = 0; j <= w; ++j) {
            f32x4 cb = zero4();
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) cb = mma3f(Cown[ks], frag(tA, 16 * j + r16, ks), cb);
#pragma unroll
            for (int i = 0; i < 4; ++i) s_cb[(16 * w + 4 * kq + i) * CBS + 16 * j + r16] = cb[i];
        }
    }
    f32x4 dBa[4], dCa[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        dBa[i] = zero4();
        dCa[i] = zero4();
    }
    const float bias0 = 0.f;
    (void)bias0;

    for (int rh = 0; rh < prm.R; ++rh) {
        const int h = g * prm.R + rh;
        lds_barrier(); // previous readers of the tiles and per-token arrays are done
        if (w == 0) {
            float q = 0.f, a = 0.f, dq = 0.f;
            if (lane < tv) {
                const float bias = prm.dt_bias ? prm.dt_bias[h] : 0.f;
                const float dtv = prm.dt[((int64_t)b * prm.L + t0 + lane) * H + h];
                q = discretize_dt(dtv, bias, prm.softplus != 0, prm.lo, prm.hi);
                dq = discretize_grad(dtv, bias, prm.softplus != 0, prm.lo, prm.hi);
                a = prm.A[h] * kLog2e * q;
            }
            const float cs = wave_inclusive_scan(a); // log2 units
            const float last = readlane_f(cs, T - 1);
            s_q[lane] = q;
            s_cs[lane] = cs;
            s_dqdu[lane] = dq;
            s_dte[lane] = exp2_f(last - cs);
            s_ecs[lane] = exp2_f(cs);
        }
        lds_barrier();
        const int64_t xo = (((int64_t)b * prm.L + t0) * H + h) * P;
        const auto rX = buf_rsrc(prm.x + xo);
        const bool has_dout = prm.dout != nullptr;
        const auto rDo = buf_rsrc(has_dout ? prm.dout + xo : prm.x + xo);
        const auto rZ = buf_rsrc(prm.has_z ? prm.z + xo : prm.x + xo);

        // ---- phase 1: dW in both orientations, W and the decay masks
        stage_rows_buf(tA, rDo, rowHP4, [&](float4 v, int t, int c4) {
            if (!has_dout) return z4;
            if (prm.has_z) {
                const float4 zz = (full || t < tv) ? buf_load4(rZ, rt * rowHP4 + c4 * 4, (t - rt) * rowHP4) : z4;
                v.x *= silu_f(zz.x);
                v.y *= silu_f(zz.y);
                v.z *= silu_f(zz.z);
                v.w *= silu_f(zz.w);
            }
            return v;
        });
        stage_rows_buf(tB, rX, rowHP4, [&](float4 v, int t, int) {
            const float q = s_q[t];
            return make_float4(v.x * q, v.y * q, v.z * q, v.w * q);
        });
        lds_barrier();
        Frag GYo[2], XDo[2];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            GYo[ks] = frag(tA, own, ks);
            XDo[ks] = frag(tB, own, ks);
        }
        Frag WS[2], DCT[2], DCS[2];
        {
            const float cs_own = s_cs[own];
            // T orientation (t = own, s = 16 j + 4 kq + i, s-blocks j <= w):
            // dW[t][s], then dCB = dW * exp2(cs_t - cs_s) and rowsum(dW o W)
            float rows = 0.f;
            {
                float dct[2][8];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    f32x4 dw = zero4();
                    float4 cb = z4;
                    if (j <= w) {
#pragma unroll
                        for (int ks = 0; ks < 2; ++ks) dw = mma3f(frag(tB, 16 * j + r16, ks), GYo[ks], dw);
                        cb = *(const float4 *)&s_cb[own * CBS + 16 * j + 4 * kq];
                    }
                    const float cbv[4] = {cb.x, cb.y, cb.z, cb.w};
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int u = 16 * j + 4 * kq + i;
                        const float e = (j <= w && u <= own) ? exp2_f(cs_own - s_cs[u]) : 0.f;
                        rows += dw[i] * cbv[i] * e;
                        dct[j >> 1][(j & 1) * 4 + i] = dw[i] * e;
                    }
                }
                DCT[0] = pack_frag(dct[0]);
                DCT[1] = pack_frag(dct[1]);
            }
            // S orientation (s = own, t = 16 j + 4 kq + i, t-blocks j >= w):
            // W[t][s], dCB, colsum(dW o W)
            float cols = 0.f;
            {
                float ws[2][8], dcs_[2][8];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    f32x4 dw = zero4();
                    if (j >= w)
#pragma unroll
                        for (int ks = 0; ks < 2; ++ks) dw = mma3f(frag(tA, 16 * j + r16, ks), XDo[ks], dw);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int u = 16 * j + 4 * kq + i;
                        const float cbS = j >= w ? s_cb[u * CBS + own] : 0.f;
                        const float e = (j >= w && own <= u) ? exp2_f(s_cs[u] - cs_own) : 0.f;
                        const float wsv = cbS * e;
                        cols += dw[i] * wsv;
                        ws[j >> 1][(j & 1) * 4 + i] = wsv;
                        dcs_[j >> 1][(j & 1) * 4 + i] = dw[i] * e;
                    }
                }
                WS[0] = pack_frag(ws[0]);
                WS[1] = pack_frag(ws[1]);
                DCS[0] = pack_frag(dcs_[0]);
                DCS[1] = pack_frag(dcs_[1]);
            }
            rows = sum_kq(rows);
            cols = sum_kq(cols);
            if (kq == 0) s_dcs1[own] = rows - cols;
        }
        lds_barrier(); // phase-1 tiles consumed

        // ---- phase 2a: the token-contracted products
        stage_cols_buf(tA, rDo, rowHP4, [&](float v, int t) {
            if (!has_dout) return 0.f;
            if (prm.has_z) v *= silu_f(buf_load(rZ, 4 * c, t * rowHP4));
            return v;
        });
        stage_cols_buf(tB, rB, rowGN4, ident1);
        stage_cols_buf(tC, rC, rowGN4, ident1);
        lds_barrier();
        f32x4 dxa[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) dxa[i] = zero4();
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            if (2 * m + 1 >= w) {
#pragma unroll
                for (int pb = 0; pb < 4; ++pb) dxa[pb] = mma3f(WS[m], frag(tA, 16 * pb + r16, m), dxa[pb]);
#pragma unroll
                for (int nb = 0; nb < 4; ++nb) dBa[nb] = mma3f(DCS[m], frag(tC, 16 * nb + r16, m), dBa[nb]);
            }
            if (2 * m <= w) {
#pragma unroll
                for (int nb = 0; nb < 4; ++nb) dCa[nb] = mma3f(DCT[m], frag(tB, 16 * nb + r16, m), dCa[nb]);
            }
        }
        lds_barrier();

        // ---- phase 2b: the state-side products
        const int64_t so = (((int64_t)b * H + h) * prm.K + k) * (int64_t)(P * N);
        const auto rS = buf_rsrc(prm.states + so);
        const auto rU = buf_rsrc(prm.dstates + so);
        float sdu = 0.f;
        {
            // tA[n][p] = S[p][n], tB[n][p] = dU[p][n] (same thread mapping)
#pragma unroll
            for (int rr = 0; rr < 2; ++rr) {
                const int run = w + 4 * rr;
                float sv[8], dv[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const int p = run * 8 + i;
                    sv[i] = buf_load(rS, 4 * c, p * N * 4);
                    dv[i] = buf_load(rU, 4 * c, p * N * 4);
                    sdu += sv[i] * dv[i];
                }
                const Frag fs = pack_frag(sv), fd = pack_frag(dv);
                *(half8 *)&tA.hi[c * kTS + run * 8] = fs.h;
                *(half8 *)&tA.lo[c * kTS + run * 8] = fs.l;
                *(half8 *)&tB.hi[c * kTS + run * 8] = fd.h;
                *(half8 *)&tB.lo[c * kTS + run * 8] = fd.l;
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) { // tC[p][n] = dU rows
            const int p = rt + 16 * j;
            const float4 v = buf_load4(rU, rt * N * 4 + rc4 * 4, 16 * j * N * 4);
            half4 vh, vl;
            split4(v, vh, vl);
            *(half4 *)&tC.hi[p * kTS + rc4] = vh;
            *(half4 *)&tC.lo[p * kTS + rc4] = vl;
        }
        sdu = wave_sum(sdu);
        if (lane == 0) s_red[w] = sdu;
        lds_barrier();
        {
            // one product at a time keeps a single 16-register temporary live
            const int vrowx = (16 * w + 4 * kq) * rowHP4 + 4 * r16; // row t = 16 w + 4 kq (+ r)
            const int vrowc = (16 * w + 4 * kq) * rowGN4 + 4 * r16;
            float rpart[4] = {0.f, 0.f, 0.f, 0.f}, gpart[4] = {0.f, 0.f, 0.f, 0.f};
            {
                f32x4 xs[4]; // [t][p] = B_t . dU[p]
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    xs[i] = zero4();
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks) xs[i] = mma3f(Bown[ks], frag(tC, 16 * i + r16, ks), xs[i]);
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int t = 16 * w + 4 * kq + r;
                    const bool valid = full || t < tv;
                    const float dte = s_dte[t], q = s_q[t];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float xv = valid ? buf_load(rX, vrowx + r * rowHP4 + 64 * i, 0) : 0.f;
                        rpart[r] += xv * q * xs[i][r];
                        dxa[i][r] += xs[i][r] * dte;
                    }
                }
            }
            {
                f32x4 bs[4]; // [t][n] = xdt_t . dU[:, n]
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    bs[i] = zero4();
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks) bs[i] = mma3f(XDo[ks], frag(tB, 16 * i + r16, ks), bs[i]);
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float dte = s_dte[16 * w + 4 * kq + r];
#pragma unroll
                    for (int i = 0; i < 4; ++i) dBa[i][r] += bs[i][r] * dte;
                }
            }
            {
                f32x4 co[4]; // [t][n] = gy_t . S[:, n]
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    co[i] = zero4();
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks) co[i] = mma3f(GYo[ks], frag(tA, 16 * i + r16, ks), co[i]);
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int t = 16 * w + 4 * kq + r;
                    const bool valid = full || t < tv;
                    const float ecs = s_ecs[t];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float dco = co[i][r] * ecs;
                        dCa[i][r] += dco;
                        const float cv = valid ? buf_load(rC, vrowc + r * rowGN4 + 64 * i, 0) : 0.f;
                        gpart[r] += dco * cv;
                    }
                }
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = 16 * w + 4 * kq + r;
                const float rp = sum16(rpart[r]), gp = sum16(gpart[r]);
                if (r16 == 0) {
                    s_goff[t] = gp;
                    s_rdte[t] = rp * s_dte[t];
                }
            }
        }
        lds_barrier();

        // ---- dcs -> da (reverse cumsum), dA partial
        if (w == 0) {
            const float sdu_tot = s_red[0] + s_red[1] + s_red[2] + s_red[3];
            const float rd = s_rdte[lane];
            const float rd_tot = wave_sum(rd);
            float dcs = s_dcs1[lane] + s_goff[lane] - rd;
            if (lane == T - 1) dcs += rd_tot + exp2_f(s_cs[T - 1]) * sdu_tot;
            const float da = wave_suffix_scan(dcs);
            s_da[lane] = da;
            const float dA_p = wave_sum(da * s_q[lane]);
            if (lane == 0) prm.part_dA[((int64_t)b * H + h) * prm.K + k] = dA_p;
        }
        lds_barrier();

        // ---- epilogue: dx, ddt, dz and the D partial
        {
            const float Ah = prm.A[h];
            float dDp[4] = {0.f, 0.f, 0.f, 0.f};
            const auto rPg = buf_rsrc(prm.has_z ? prm.pre_gate + xo : prm.x + xo);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = 16 * w + 4 * kq + r;
                const bool valid = full || t < tv;
                const float q = s_q[t];
                float dqp = 0.f;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int cc = 16 * i + r16;
                    const int vo = (16 * w + 4 * kq + r) * rowHP4 + 4 * r16 + 64 * i, uo = 0;
                    const float xv = valid ? buf_load(rX, vo, uo) : 0.f;
                    const float dov = (valid && has_dout) ? buf_load(rDo, vo, uo) : 0.f;
                    float gyv = dov;
                    if (prm.has_z && valid) {
                        const float zv = buf_load(rZ, vo, uo), sg = sigmoid_f(zv);
                        gyv = dov * zv * sg;
                        prm.dz[xo + (int64_t)t * H * P + cc] = dov * buf_load(rPg, vo, uo) * sg * (1.f + zv * (1.f - sg));
                    }
                    const float dxdt = dxa[i][r];
                    dqp += xv * dxdt;
                    float dxv = q * dxdt;
                    if (prm.has_D) {
                        const float Dv = prm.d_per_channel ? prm.D[h * P + cc] : prm.D[h];
                        dxv += Dv * gyv;
                        dDp[i] += gyv * xv;
                    }
                    if (valid) prm.dx[xo + (int64_t)t * H * P + cc] = dxv;
                }
                dqp = sum16(dqp);
                if (r16 == 0) {
                    float ddtv = 0.f;
                    if (valid) {
                        ddtv = (Ah * s_da[t] + dqp) * s_dqdu[t];
                        prm.ddt[((int64_t)b * prm.L + t0 + t) * H + h] = ddtv;
                    }
                    s_ddt[t] = ddtv;
                }
            }
            if (prm.has_D) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float v = sum_kq(dDp[i]);
                    if (kq == 0) s_dD[w][16 * i + r16] = v;
                }
            }
        }
        lds_barrier();
        if (w == 0) {
            const int64_t pi = ((int64_t)b * H + h) * prm.K + k;
            const float db = wave_sum(s_ddt[lane]);
            if (lane == 0) prm.part_dbias[pi] = db;
            if (prm.has_D) {
                const float v = s_dD[0][lane] + s_dD[1][lane] + s_dD[2][lane] + s_dD[3][lane];
                if (prm.d_per_channel) {
                    prm.part_dD[pi * P + lane] = v;
                } else {
                    const float tot = wave_sum(v);
                    if (lane == 0) prm.part_dD[pi] = tot;
                }
            }
        }
    }

    // ---- group outputs
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int t = 16 * w + 4 * kq + r;
        if (t >= tv) continue;
        const int64_t o = (((int64_t)b * prm.L + t0 + t) * G + g) * N;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            prm.dB[o + 16 * i + r16] = dBa[i][r];
            prm.dC[o + 16 * i + r16] = dCa[i][r];
        }
    }
}

// --------------------------------------------------------------------------
// fixed-order reductions of the per-chunk partials, one workgroup per head
// --------------------------------------------------------------------------
__device__ __forceinline__ float block_sum(float v, float *s_tmp) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) s_tmp[w] = v;
    __syncthreads();
    return s_tmp[0] + s_tmp[1] + s_tmp[2] + s_tmp[3];
}

__global__ __launch_bounds__(kThreads) void k_bwd_finalize(const float *part_dA,
                                                           const float *part_dbias,
                                                           const float *part_dD, float *dA,
                                                           float *ddt_bias, float *dD, int B,
                                                           int H, int K, int P, int has_D,
                                                           int d_per_channel) {
    __shared__ float s_tmp[4];
    __shared__ float s_col[4][64];
    const int h = blockIdx.x, tid = threadIdx.x;
    const int n = B * K;
    float a = 0.f, db = 0.f, dd = 0.f;
    for (int i = tid; i < n; i += kThreads) {
        const int bb = i / K, kk = i % K;
        const int64_t pi = ((int64_t)bb * H + h) * K + kk;
        a += part_dA[pi];
        db += part_dbias[pi];
        if (has_D && !d_per_channel) dd += part_dD[pi];
    }
    a = block_sum(a, s_tmp);
    if (tid == 0) dA[h] = a;
    db = block_sum(db, s_tmp);
    if (tid == 0 && ddt_bias) ddt_bias[h] = db;
    if (has_D && !d_per_channel) {
        dd = block_sum(dd, s_tmp);
        if (tid == 0) dD[h] = dd;
    }
    if (has_D && d_per_channel) {
        // column p = tid % 64 summed over (b, k) by 4 thread groups, then combined
        for (int p0 = 0; p0 < P; p0 += 64) {
            const int p = p0 + (tid & 63), grp = tid >> 6;
            float v = 0.f;
            if (p < P)
                for (int i = grp; i < n; i += 4) {
                    const int bb = i / K, kk = i % K;
                    v += part_dD[(((int64_t)bb * H + h) * K + kk) * P + p];
                }
            s_col[grp][tid & 63] = v;
            __syncthreads();
            if (grp == 0 && p < P)
                dD[h * P + p] = s_col[0][tid] + s_col[1][tid] + s_col[2][tid] + s_col[3][tid];
            __syncthreads();
        }
    }
}

}  // namespace ssd
