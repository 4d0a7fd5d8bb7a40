// Group-major state pass of the forward (headdim = dstate = 64): the state
// entering every chunk, for the backward's recompute of the chunk states when
// the forward did not keep them.
//
// The state-only form of k_fwd_seg walks one (b, h) stream per workgroup, so
// the R heads of a group read the group's B rows each on their own; they
// drift apart over a pass and B comes from HBM several times (C3: about 2.8x,
// 1.20x the pass's algorithmic bytes).  Here one workgroup walks the R heads
// of a (b, g) stream: per chunk it loads B once and runs R steps, one per
// head (x of that head staged as T2, B decay q of that head as T3, the state
// update U = T3^T T2 of that head), double buffered by step parity, with the
// R states in the consumers' registers.  The staging, scales, products and
// update are those of the state-only k_fwd_seg, step for step, so the chunk
// states are bitwise equal.  Four heads' states take the consumers to 160
// VGPRs, so one workgroup runs per CU; the producers keep a chunk of loads in
// flight instead (a ring of four head steps).  C3: 1.003 ms and 5.11 GB
// (1.05x the algorithmic bytes) against 1.075 ms and 5.85 GB for the
// per-head pass.  Used for one segment per stream without sequence ids,
// R = 4, and at least as many (b, g) streams as CUs.
//
// The math is that of mamba_torch/ssd_reference.py:113-189 (chunk states and
// the inter-chunk recurrence).
#pragma once

#include "ssd_fwd_fused.h"

namespace ssd {

template <int kR>
__global__ __attribute__((amdgpu_flat_work_group_size(1, kWsThreads), amdgpu_waves_per_eu(2))) void
k_fwd_state_group(FwdParams prm) {
    constexpr int T = 64, P = 64, N = 64;
    constexpr int64_t PN = (int64_t)P * N;
    // T2(s), T3(s) of step parity s (split fp16, rows kTS halves apart)
    __shared__ __attribute__((aligned(16))) _Float16 lds[8 * kTile];
    struct StepTok {
        float cs_last[2]; // log2 decay of the step's chunk and head
        int sexp[2];      // eN: T3 holds B dec q 2^-eN, the scale of the state leaving the chunk
    };
    __shared__ StepTok s_tok;
    __shared__ __attribute__((aligned(16))) float s_smax[kR][4]; // |entering state| max per head and consumer wave

    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const bool producer = wave >= 4;
    const int w = wave & 3;
    const int r16 = lane & 15, kq = lane >> 4;
    auto T2 = [&](int s) { return tile_at(lds, 2 * s); };
    auto T3 = [&](int s) { return tile_at(lds, 2 * s + 1); };

    const int bg = blockIdx.x, g = bg % prm.G, b = bg / prm.G;
    const int H = prm.H, G = prm.G, K = prm.K;
    const int NS = K * kR; // steps: chunk n / kR, head g kR + n % kR
    const bool s0_nonzero = prm.init != nullptr;

    // ------------------------------------------------------------ producers
    // A ring of four step slots (a chunk ahead): rows rt + 16 j (columns
    // c4 .. c4 + 3) of x of the step's head, of B (read for real only on a
    // chunk's first step; the other steps read through an empty-range
    // resource, so every step issues the same loads), dt of token `lane`.
    // Step n sits in slot n % 4, the slot of its head.
    if (producer) {
        constexpr int kDepth = 4;
        const int pt = tid - 4 * kWave;
        const int rt = pt >> 4, c4 = (pt & 15) * 4;
        const int rowHP4 = H * P * 4, rowGN4 = G * N * 4;
        int xrow_off[4], brow_off[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            xrow_off[j] = (rt + 16 * j) * rowHP4;
            brow_off[j] = (rt + 16 * j) * rowGN4;
        }
        const int Hr = H / prm.hdiv;
        const int dt_off = lane * Hr * 4;
        float Ah2[kR], bias[kR];
        int p_eS[kR];
#pragma unroll
        for (int r = 0; r < kR; ++r) {
            const int hr = (g * kR + r) / prm.hdiv;
            Ah2[r] = prm.A[hr] * kLog2e;
            bias[r] = prm.dt_bias ? prm.dt_bias[hr] : 0.f;
            p_eS[r] = kZeroState;
        }
        float4 xr[kDepth][4], br[kDepth][4], bcur[4];
        float dtr[kDepth];
        // loads of step n into slot sl (n past the end: empty ranges)
        auto p_load = [&](int n, auto r_c, auto sl_c) {
            constexpr int r = decltype(r_c)::value, sl = decltype(sl_c)::value;
            const bool real = n < NS;
            const int k = real ? n / kR : 0, h = g * kR + r, hr = h / prm.hdiv;
            const int64_t t0 = (int64_t)k * T;
            const int tv = (int)min((int64_t)T, prm.L - t0);
            const auto rx = buf_rsrc_n(prm.x + (((int64_t)b * prm.L + t0) * H + h) * P, real ? 0x7fffffff : 0);
            const auto rb = buf_rsrc_n(prm.B + (((int64_t)b * prm.L + t0) * G + g) * N,
                                       (real && r == 0) ? 0x7fffffff : 0);
            const int xlast = (tv - 1) * rowHP4, blast = (tv - 1) * rowGN4;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                // x is read once: non-temporal, so the B rows stay in L2
                xr[sl][j] = buf_load4_nt(rx, min(xrow_off[j], xlast) + c4 * 4, 0);
                br[sl][j] = buf_load4(rb, min(brow_off[j], blast) + c4 * 4, 0);
            }
            const auto rdt = buf_rsrc(prm.dt + ((int64_t)b * prm.L + t0) * Hr + hr);
            dtr[sl] = buf_load(rdt, min(dt_off, (tv - 1) * Hr * 4), 0);
        };
        auto put = [&](SplitTile d, int row, float4 v) {
            half4 vh, vl;
            split4(v, vh, vl);
            *(half4 *)&d.hi[row * kTS + c4] = vh;
            *(half4 *)&d.lo[row * kTS + c4] = vl;
        };
        // stage step n (chunk k, head r) into parity s = n % 2 from slot sl = n % 4
        auto p_stage = [&](int n, auto r_c, auto sl_c) {
            constexpr int r = decltype(r_c)::value, sl = decltype(sl_c)::value, s = sl & 1;
            const int k = n / kR;
            const int tv = (int)min((int64_t)T, prm.L - (int64_t)k * T); // <= 0 past the end
            float q = 0.f;
            if (lane < tv) q = discretize_dt(dtr[sl], bias[r], prm.softplus != 0, prm.lo, prm.hi);
            const float sq = wave_inclusive_scan(q);
            const float cs = opaque_f(Ah2[r] * sq);
            const float cs_last = readlane_f(cs, T - 1);
            const int ek = chunk_q_exp(readlane_f(sq, T - 1), wave_max(fabsf(q)));
            const float dec = exp2_f(cs_last - cs);
            const int eN = next_state_exp(p_eS[r], ek, cs_last, false);
            p_eS[r] = eN;
            if (w == 0 && lane == 0) {
                StepTok *tk = opaque_lds_t(&s_tok);
                tk->cs_last[s] = cs_last;
                tk->sexp[s] = eN;
            }
            const float qn = __builtin_amdgcn_ldexpf(q, -eN);
            if (r == 0) {
#pragma unroll
                for (int j = 0; j < 4; ++j) bcur[j] = br[sl][j];
            }
            const SplitTile t2 = T2(s), t3 = T3(s);
            float drs[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) drs[j] = __shfl(dec * qn, rt + 16 * j, kWave);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int row = rt + 16 * j;
                const float dr = drs[j];
                const float4 bv = bcur[j];
                put(t2, row, xr[sl][j]);
                put(t3, row, make_float4(bv.x * dr, bv.y * dr, bv.z * dr, bv.w * dr));
            }
        };
        using I0 = std::integral_constant<int, 0>;
        using I1 = std::integral_constant<int, 1>;
        using I2 = std::integral_constant<int, 2>;
        using I3 = std::integral_constant<int, 3>;
        static_assert(kR == 4, "the unrolled head steps below assume four heads per group");
        p_load(0, I0{}, I0{});
        p_load(1, I1{}, I1{});
        p_load(2, I2{}, I2{});
        p_load(3, I3{}, I3{});
        if (s0_nonzero) {
            lds_barrier(); // the consumers' maxima of the entering states
#pragma unroll
            for (int r = 0; r < kR; ++r) p_eS[r] = state_exp_of(s_smax[r]);
        }
        p_stage(0, I0{}, I0{});
        p_load(4, I0{}, I0{});
        lds_barrier();
        // iteration n stages step n + 1 (slot (n + 1) % 4) and loads step
        // n + 5 into that slot; past the end it stages zeros no consumer reads
        for (int k = 0; k < K; ++k) {
            const int n = k * kR;
            p_stage(n + 1, I1{}, I1{});
            p_load(n + 5, I1{}, I1{});
            lds_barrier();
            p_stage(n + 2, I2{}, I2{});
            p_load(n + 6, I2{}, I2{});
            lds_barrier();
            p_stage(n + 3, I3{}, I3{});
            p_load(n + 7, I3{}, I3{});
            lds_barrier();
            p_stage(n + 4, I0{}, I0{});
            p_load(n + 8, I0{}, I0{});
            lds_barrier();
        }
        return;
    }

    // ------------------------------------------------------------ consumers
    // wave W keeps n-block W of every head's state: Sr[r][i] = S[p = 16 i + l % 16][n = 16 W + 4 (l / 16) + e]
    auto consumer = [&](auto wave_c) {
        constexpr int W = decltype(wave_c)::value;
        auto toff = [&](int i) { return (16 * i + r16) * N + 16 * W + 4 * kq; };
        typedef unsigned v4u __attribute__((ext_vector_type(4)));
        const int st_off = toff(0) * 4; // bytes; tile i adds 16 i rows
        f32x4 Sr[kR][4];
        int eS[kR];
#pragma unroll
        for (int r = 0; r < kR; ++r) {
            const float *s0 = prm.init ? prm.init + ((int64_t)b * H + g * kR + r) * PN : nullptr;
            eS[r] = kZeroState;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (s0) {
                    const float4 v = *(const float4 *)(s0 + toff(i));
                    Sr[r][i] = f32x4{v.x, v.y, v.z, v.w};
                } else {
                    Sr[r][i] = zero4();
                }
            }
        }
        if (s0_nonzero) {
#pragma unroll
            for (int r = 0; r < kR; ++r) {
                float m = 0.f;
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int e = 0; e < 4; ++e) m = fmaxf(m, fabsf(Sr[r][i][e]));
                m = wave_max(m);
                if (lane == 0) s_smax[r][W] = m;
            }
            lds_barrier();
#pragma unroll
            for (int r = 0; r < kR; ++r) {
                eS[r] = state_exp_of(s_smax[r]);
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int e = 0; e < 4; ++e) Sr[r][i][e] = __builtin_amdgcn_ldexpf(Sr[r][i][e], -eS[r]);
            }
        }
        lds_barrier();
        auto step = [&](int k, auto r_c) {
            constexpr int r = decltype(r_c)::value, s = r & 1;
            const int h = g * kR + r;
            // saved for the backward: the state entering chunk k, through a
            // buffer resource (one lane offset for every head and tile, the
            // chunk's base in scalar registers)
            const auto rst = buf_rsrc(prm.chunk_states + (((int64_t)b * H + h) * K + k) * PN);
            const float f = __builtin_amdgcn_ldexpf(1.f, eS[r]);
#pragma unroll
            for (int i = 0; i < 4; ++i)
                __builtin_amdgcn_raw_buffer_store_b128(
                    __builtin_bit_cast(v4u, make_float4(Sr[r][i][0] * f, Sr[r][i][1] * f, Sr[r][i][2] * f,
                                                        Sr[r][i][3] * f)),
                    rst, st_off, 16 * i * N * 4, 0);
            f32x4 U[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) U[i] = zero4();
            const SplitTile t2 = T2(s), t3 = T3(s);
#pragma unroll
            for (int m = 0; m < 2; ++m) {
                const Frag a3 = frag_tp_s<kTS>(t3, m, 16 * W);
#pragma unroll
                for (int i = 0; i < 4; ++i) U[i] = mma3f(a3, frag_tp_s<kTS>(t2, m, 16 * i), U[i]);
            }
            const int eN = s_tok.sexp[s];
            const float alpha = __builtin_amdgcn_ldexpf(exp2_f(s_tok.cs_last[s]), eS[r] - eN);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int e = 0; e < 4; ++e) Sr[r][i][e] = alpha * Sr[r][i][e] + U[i][e];
            eS[r] = eN;
            lds_barrier(); // parity s is free, parity s ^ 1 is staged
        };
        for (int k = 0; k < K; ++k) {
            step(k, std::integral_constant<int, 0>{});
            step(k, std::integral_constant<int, 1>{});
            step(k, std::integral_constant<int, 2>{});
            step(k, std::integral_constant<int, 3>{});
        }
    };
    switch (w) {
    case 0: consumer(std::integral_constant<int, 0>{}); break;
    case 1: consumer(std::integral_constant<int, 1>{}); break;
    case 2: consumer(std::integral_constant<int, 2>{}); break;
    default: consumer(std::integral_constant<int, 3>{}); break;
    }
}

}  // namespace ssd
