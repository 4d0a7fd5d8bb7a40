// Warp-specialized chunk backward of the Mamba-2 SSD hot path (M1 spec:
// headdim = dstate = 64, execution chunk T = 64).
//
// One workgroup owns one (batch b, group g, run of chunks) and walks its
// (chunk, head) steps in order: for each chunk, the R heads of the group.
// dB and dC of a chunk are sums over the group's heads; they stay in the
// consumer registers across the chunk's heads and are written once, so the
// reduction order is fixed (deterministic, no atomics).
//
// Roles: waves 4..7 (producers) load the global tiles of the next steps into
// registers and stage them into LDS as split fp16; waves 0..3 (consumers) own
// 16 token rows each and run the products.  Each tile is kept in LDS once,
// token-major (rows = the tile's leading index); operands that contract over
// that index are read with the gfx950 transposing LDS read (ds_read_b64_tr_b16)
// instead of a second, transposed copy.
//
// Per step (head h of chunk k), with xdt = q x, gy = dout (* silu z),
// cs the chunk cumsum of A q, W[t][s] = (C_t . B_s) exp(cs_t - cs_s) [s <= t],
// dCB = dW o exp-mask, S the state entering the chunk, dU = dL/d(state leaving):
//   phase A (tiles x, gy, B, C):
//     dW[t][s] = gy_t . xdt_s in both orientations, W, dCB, the dcs row/col sums,
//     dxdt  = W^T gy,  dC += dCB B,  dB += dCB^T C
//   phase B (tiles S, dU):
//     dxdt += decay (B dU^T),  dC += exp(cs) (gy S),  dB += decay q (x dU),
//     dcs  += g_off - decay r  (g_off = sum_n dC_off C, r = xdt . (B dU^T))
//   epilogue (run at the start of the next step's phase A, once every wave's
//   dcs is in LDS): da = reverse cumsum of dcs (+ the chunk-end terms),
//     dq = A da + x . dxdt, ddt = dq dq/ddt, dx = q dxdt + D gy, dz,
//     and per-(b, h, k, wave) partials of dA, ddt_bias and dD.
// The LDS tiles are single-buffered: producers stage S, dU of step n while
// consumers run phase A(n), and x, gy (and B, C of a new chunk) of step n + 1
// while consumers run phase B(n); two workgroup barriers per step separate
// the phases.  Producer registers hold the global loads one step ahead.
//
// The gradient is that of mamba_ascendc/csrc/ops/mamba2_ssd_bwd/design.md:73-107
// and mamba_ascendc/csrc/ops/mamba2_ssd_dt_bwd/design.md:61-78; the fusion,
// role split and layouts are this file's own.
#pragma once

#include <type_traits>

#include "ssd_bf16.h"
#include "ssd_bwd_kernels.h"
#include "ssd_fwd_fused.h"

namespace ssd {

constexpr int kBwsThreads = 512;  // 4 consumer + 4 producer waves
constexpr int kBwsSlots = 4;      // partial sums per (b, h, k): one per consumer wave

// The chunk kernels below use split-bf16 operands (ssd_bf16.h): the upstream
// gradient of a mean-reduced loss is far below fp16's range.
namespace bwd {

// kRevR = 0: steps in chunk order, the state gradients dU_k read from
// prm.dstates.  kRevR = R (1, 2 or 4 heads per group): chunks from last to
// first, and the producers carry each head's state gradient g in registers
// (the reverse recurrence of k_bwd_dstate_rev fused in), so no dU reaches HBM:
//   dU_k = g;   g <- dSoff_k + exp(cs_last_k) g,   dSoff_k = (gy exp(cs))^T C,
// starting from dfinal_state and ending at dinitial_states.  With nseg > 1
// runs per stream, run sg starts from prm.carry_in (the gradient entering it
// from the right, given by the run pre-pass k_bwd_run_grad and the recurrence
// over runs) and only run 0 writes dinitial_states.
//
// kSeq: packed sequences (prm.seq_idx), the forward's masks in adjoint form:
// W (and so dW, dCB and their dcs terms) only between equal ids, the state
// terms through s_dte (tokens that enter the state leaving the chunk) and
// s_ecs (tokens that read the state entering it), and the carry of the
// state across the chunk (alpha and the chunk-end dcs term) through s_carry.
template <bool kHasZ, int kRevR = 0, bool kSeq = false>
__global__ __launch_bounds__(kBwsThreads) void k_bwd_ws(BwdParams prm, int nseg, int M) {
    static_assert(kRevR == 0 || kRevR == 1 || kRevR == 2 || kRevR == 4, "heads per group");
    constexpr bool kRev = kRevR > 0;
    // reverse pass with the z gate: z and pre_gate are loaded after the first
    // barrier of a step instead of half a step ahead (register pressure)
    constexpr bool kLateZ = kHasZ && kRev;
    // rows of every tile interleaved (trow), except in the z-gated form,
    // whose registers the slot arithmetic would spill
    constexpr bool kIl = !kHasZ;
    using Tile = SplitTileT<kIl>;
    constexpr int T = 64, P = 64, N = 64;
    constexpr int TS = kSeq ? T : 1;
    // x and gy tiles double buffered by step parity (the epilogue of step n
    // still reads them while step n + 1 runs); S, dU, B, C single
    __shared__ __attribute__((aligned(16))) __bf16 lds[16 * kTile];
    // The per-token arrays are aligned above the tile array so the LDS layout
    // places them first, below 64 KB: their lane addresses then share one
    // base register with 16-bit immediate offsets instead of one register each.
    // Per-token (and per-channel D) values of a step written by the dt
    // prologue, double buffered by step parity; one struct, so the writing
    // wave addresses every member from one base (see the prologue).
    // bT[t] = exp2(cs of the last token of t's 16-token block - cs_t) and
    // bS[t] = exp2(cs_t - cs of the first token of its block): the decay
    // masks of phase A's off-diagonal blocks factor through block bounds,
    // one exp2 per block and lane instead of one per element (both factors
    // have the sign of the whole exponent, so neither overflows where the
    // product does not)
    struct StepTok {
        float q[2][T], cs[2][T], dqdu[2][T], dte[2][T], ecs[2][T], bT[2][T], bS[2][T], D[2][P];
        int sid[2][TS];  // kSeq: token ids
        float carry[2];  // kSeq: 1 where the state carries over
        float A[2];
    };
    __shared__ __attribute__((aligned(32))) StepTok s_tok;
    auto &s_q = s_tok.q, &s_cs = s_tok.cs, &s_dqdu = s_tok.dqdu, &s_dte = s_tok.dte, &s_ecs = s_tok.ecs,
         &s_D = s_tok.D, &s_bT = s_tok.bT, &s_bS = s_tok.bS;
    auto &s_sid = s_tok.sid;
    auto &s_carry = s_tok.carry, &s_A = s_tok.A;
    __shared__ __attribute__((aligned(32))) float s_dcs[2][T], s_rd[2][T];
    __shared__ __attribute__((aligned(32))) float s_sdu[2][4];
    __shared__ __attribute__((aligned(32))) float s_da[4][T]; // epilogue: da of a step, per consumer wave

    // tiles: x(par) = 0 + par, gy(par) = 2 + par, S 4, dU 5, B 6, C 7 (the
    // roles address them through copies of `lds` the optimizer cannot see
    // through)
    const Tile St = tile_at<kIl>(lds, 4), Ut = tile_at<kIl>(lds, 5);

    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const int r16 = lane & 15, kq = lane >> 4;
    // unit = (b * G + g) * nseg + sg.  With one run per stream each XCD takes
    // blocks of eight consecutive groups (xcd_unit), so the ddt and dt rows
    // the 32 heads of a token share (one 128-byte line) pass through one L2:
    // C3 backward 0.4 % faster than with the groups of a line on eight XCDs.
    // With several runs per stream (C4) the same blocks ran 1.5-2 % slower
    // than consecutive workgroups on consecutive units, and the forward 4 %
    // slower, which keeps one group per block.
    const int ub = nseg == 1 ? xcd_unit(blockIdx.x, (int)gridDim.x, prm.R < 32 ? 32 / prm.R : 1) : (int)blockIdx.x;
    const int sg = ub % nseg, bg = ub / nseg;
    const int g = bg % prm.G, b = bg / prm.G;
    const int R = kRev ? kRevR : prm.R, H = prm.H, G = prm.G, K = prm.K;
    const int kbeg = sg * M, kend = min(kbeg + M, K);
    const int NS = (kend - kbeg) * R;
    if (NS <= 0) return;
    const int rowHP4 = H * P * 4, rowGN4 = G * N * 4; // token strides, bytes
    auto tvalid = [&](int k) __attribute__((always_inline)) { return (int)min((int64_t)T, prm.L - (int64_t)k * T); };
    // chunk of step n: the run in order, or (kRev) from its last chunk back
    auto chunk_of = [&](int n) __attribute__((always_inline)) { return kRev ? kend - 1 - n / R : kbeg + n / R; };

    // ------------------------------------------------------------ producers
    // Every step issues the same global loads, unconditionally (rows past the
    // sequence end re-read its last row and are zeroed when staged; steps past
    // the run re-read its last step), so the load counts the compiler tracks
    // are exact and a stage waits only for the loads it consumes, which were
    // issued a step earlier.  The producers also write dz, which needs no
    // product: dz = dout pre_gate silu'(z).
    if (wave >= 4) {
        const int pt = tid - 4 * kWave, pw = wave - 4;
        const int rt = pt >> 4, c4 = (pt & 15) * 4; // rows rt + 16 j, columns c4 .. c4 + 3
        const bool has_dout = prm.dout != nullptr;
        const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
        float4 xr[4], gr[4], zr[4], pr[4], sr[4], ur[4], br[4], cr[4];
        float dtr = 0.f, Ahr = 0.f, biasr = 0.f, Dr = 0.f;
        int sidr = 0, sprv = 0; // kSeq: id of token `lane`, id of the token before the chunk
        const float *dtb = prm.dt_bias ? prm.dt_bias : prm.A; // read unconditionally
        const float *Dp = prm.has_D ? prm.D : prm.A;
        // z and pre_gate of step n (the z gate)
        auto load_zp = [&](int n) __attribute__((always_inline)) {
            n = min(n, NS - 1);
            const int k = chunk_of(n), h = g * R + n % R, tv = tvalid(k);
            const int64_t xo = (((int64_t)b * prm.L + (int64_t)k * T) * H + h) * P;
            const auto rz = buf_rsrc(prm.z + xo);
            const auto rp = buf_rsrc(prm.pre_gate + xo);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int lo = min(rt + 16 * j, tv - 1) * rowHP4 + c4 * 4;
                zr[j] = buf_load4(rz, lo, 0);
                pr[j] = buf_load4(rp, lo, 0);
            }
        };
        auto load_xg = [&](int n) __attribute__((always_inline)) {
            n = min(n, NS - 1);
            const int k = chunk_of(n), h = g * R + n % R, tv = tvalid(k);
            const int64_t xo = (((int64_t)b * prm.L + (int64_t)k * T) * H + h) * P;
            const auto rx = buf_rsrc(prm.x + xo);
            const auto rd = buf_rsrc(has_dout ? prm.dout + xo : prm.x + xo);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int lo = min(rt + 16 * j, tv - 1) * rowHP4 + c4 * 4;
                xr[j] = buf_load4(rx, lo, 0);
                gr[j] = buf_load4(rd, lo, 0);
            }
            if (kHasZ && !kLateZ) load_zp(n);
            dtr = prm.dt[((int64_t)b * prm.L + (int64_t)k * T + min(lane, tv - 1)) * H + h];
            if (kSeq) {
                const int32_t *si = prm.seq_idx + (int64_t)b * prm.L + (int64_t)k * T;
                sidr = si[min(lane, tv - 1)];
                const int pv = si[k > 0 ? -1 : 0]; // read unconditionally, 0 before the first chunk
                sprv = k > 0 ? pv : 0;
            }
            Dr = Dp[prm.has_D && prm.d_per_channel ? h * P + lane : h];
            Ahr = prm.A[h];
            biasr = dtb[h];
        };
        // B, C of the chunk of step n, read for real only when step n starts
        // a chunk (the only steps whose B, C get staged); the other steps
        // issue the same loads through an empty-range resource
        auto load_bc = [&](int n) __attribute__((always_inline)) {
            const int range = (n < NS && n % R == 0) ? 0x7fffffff : 0;
            n = min(n, NS - 1);
            const int k = chunk_of(n), tv = tvalid(k);
            const int64_t o = (((int64_t)b * prm.L + (int64_t)k * T) * G + g) * N;
            const auto rb = buf_rsrc_n(prm.B + o, range), rc = buf_rsrc_n(prm.C + o, range);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int lo = min(rt + 16 * j, tv - 1) * rowGN4 + c4 * 4;
                br[j] = buf_load4(rb, lo, 0);
                cr[j] = buf_load4(rc, lo, 0);
            }
        };
        // kRev: the state-gradient carries of the group's heads, and S in the
        // same MFMA accumulator layout: gc[r][pb][i] = g[p][n] of head g R + r,
        // p = 16 pb + l % 16, n = 16 pw + 4 (l / 16) + i
        f32x4 gc[kRev ? kRevR : 1][4];
        const int acc_off = (r16 * N + 16 * pw + 4 * kq) * 4; // bytes, + 16 pb rows
        if constexpr (kRev) {
#pragma unroll
            for (int rr = 0; rr < kRevR; ++rr) {
                // the gradient of the state leaving the run's last chunk: the
                // segment recurrence's (segmented) or dfinal_state
                const int64_t bh = (int64_t)b * H + g * R + rr;
                const float *cin = prm.carry_in ? prm.carry_in + (bh * nseg + sg) * (P * N)
                                                : (prm.dfinal ? prm.dfinal + bh * (P * N) : nullptr);
#pragma unroll
                for (int pb = 0; pb < 4; ++pb) {
                    gc[rr][pb] = zero4();
                    if (cin) {
                        const float4 v = *(const float4 *)((const char *)cin + acc_off + 16 * pb * N * 4);
                        gc[rr][pb] = f32x4{v.x, v.y, v.z, v.w};
                    }
                }
            }
        }
        auto load_su = [&](int n) __attribute__((always_inline)) {
            n = min(n, NS - 1);
            const int k = chunk_of(n), h = g * R + n % R;
            const int64_t so = (((int64_t)b * H + h) * K + k) * (int64_t)(P * N);
            const auto rs = buf_rsrc(prm.states + so);
            if constexpr (kRev) {
#pragma unroll
                for (int pb = 0; pb < 4; ++pb) sr[pb] = buf_load4(rs, acc_off, 16 * pb * N * 4);
            } else {
                const auto ru = buf_rsrc(prm.dstates + so);
                const int lo = (rt * N + c4) * 4;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    sr[j] = buf_load4(rs, lo, 16 * j * N * 4);
                    ur[j] = buf_load4(ru, lo, 16 * j * N * 4);
                }
            }
        };
        auto put = [&](Tile d, int row, float4 v) __attribute__((always_inline)) {
            store_split4(d, row, c4, v);
        };
        auto stage_xg = [&](int n) __attribute__((always_inline)) {
            const int par = n & 1, k = chunk_of(n), h = g * R + n % R, tv = tvalid(k);
            const int64_t xo = (((int64_t)b * prm.L + (int64_t)k * T) * H + h) * P;
            __bf16 *lp = opaque_lds_t(lds);
            const Tile xt = tile_at<kIl>(lp, par), gt = tile_at<kIl>(lp, 2 + par);
            const auto rdz = buf_rsrc(kHasZ ? prm.dz + xo : prm.x + xo);
            float4 dD4 = z4; // sum over this lane's rows of x gy, columns c4 .. c4 + 3
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int row = rt + 16 * j;
                const bool ok = row < tv;
                const float4 xv = ok ? xr[j] : z4;
                put(xt, row, xv);
                const float4 dv = (ok && has_dout) ? gr[j] : z4;
                float4 v = dv;
                if (kHasZ) {
                    const float zz[4] = {zr[j].x, zr[j].y, zr[j].z, zr[j].w};
                    const float pp[4] = {pr[j].x, pr[j].y, pr[j].z, pr[j].w};
                    const float dd[4] = {dv.x, dv.y, dv.z, dv.w};
                    float gv[4], dzv[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float sgm = sigmoid_f(zz[i]);
                        gv[i] = dd[i] * zz[i] * sgm;
                        dzv[i] = dd[i] * pp[i] * sgm * (1.f + zz[i] * (1.f - sgm));
                    }
                    v = make_float4(gv[0], gv[1], gv[2], gv[3]);
                    if (ok)
                        __builtin_amdgcn_raw_buffer_store_b128(
                            __builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned,
                                               make_float4(dzv[0], dzv[1], dzv[2], dzv[3])),
                            rdz, (rt * H * P + c4) * 4, 16 * j * rowHP4, 0);
                }
                put(gt, row, v);
                dD4.x += xv.x * v.x;
                dD4.y += xv.y * v.y;
                dD4.z += xv.z * v.z;
                dD4.w += xv.w * v.w;
            }
            // dD partials of this wave's rows: slot pw of (b, h, k)
            if (prm.has_D) {
                const int64_t bhk = ((int64_t)b * H + h) * K + k;
                if (prm.d_per_channel) {
                    const float4 t4 = make_float4(sum_kq(dD4.x), sum_kq(dD4.y), sum_kq(dD4.z), sum_kq(dD4.w));
                    if (lane < 16) *(float4 *)(prm.part_dD + (bhk * kBwsSlots + pw) * P + c4) = t4;
                } else {
                    const float tot = wave_sum(dD4.x + dD4.y + dD4.z + dD4.w);
                    if (lane == 0) prm.part_dD[bhk * kBwsSlots + pw] = tot;
                }
            }
            if (pw == 0) {
                float q = 0.f, a = 0.f, dq = 0.f;
                const float bias = prm.dt_bias ? biasr : 0.f;
                if (lane < tv) {
                    q = discretize_dt(dtr, bias, prm.softplus != 0, prm.lo, prm.hi);
                    dq = discretize_grad(dtr, bias, prm.softplus != 0, prm.lo, prm.hi);
                    a = Ahr * kLog2e * q;
                }
                const float cs = wave_inclusive_scan(a); // log2 units
                const float last = readlane_f(cs, T - 1);
                float into = 1.f, reads = 1.f;
                // every member from one base the optimizer cannot split into
                // per-array registers (those were held across the step loop
                // and spilled, and each reload waited for the prefetches)
                StepTok *tk = opaque_lds_t(&s_tok);
                if (kSeq) {
                    const int e_end = __builtin_amdgcn_readlane(sidr, T - 1); // rows past the end repeat the last id
                    into = (sidr == e_end && e_end >= 0) ? 1.f : 0.f;
                    reads = sidr == sprv ? 1.f : 0.f;
                    tk->sid[par][lane] = sidr;
                    if (lane == 0) tk->carry[par] = e_end == sprv ? 1.f : 0.f;
                }
                tk->q[par][lane] = q;
                tk->cs[par][lane] = cs;
                tk->dqdu[par][lane] = dq;
                tk->dte[par][lane] = exp2_f(last - cs) * into;
                tk->ecs[par][lane] = exp2_f(cs) * reads;
                // cs of the last and the first lane of the lane's 16-lane
                // block: DPP row_newbcast 15 and 0 (no LDS round trip)
                tk->bT[par][lane] = exp2_f(dpp_f<0x15F>(cs) - cs);
                tk->bS[par][lane] = exp2_f(cs - dpp_f<0x150>(cs));
                tk->D[par][lane] = prm.has_D ? Dr : 0.f;
                if (lane == 0) tk->A[par] = Ahr;
            }
        };
        auto stage_bc = [&](int n) __attribute__((always_inline)) {
            const int tv = tvalid(chunk_of(min(n, NS - 1)));
            __bf16 *lp = opaque_lds_t(lds);
            const Tile bt = tile_at<kIl>(lp, 6), ct = tile_at<kIl>(lp, 7);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const bool ok = rt + 16 * j < tv;
                put(bt, rt + 16 * j, ok ? br[j] : z4);
                put(ct, rt + 16 * j, ok ? cr[j] : z4);
            }
        };
        auto stage_su = [&](int n) __attribute__((always_inline)) {
            float sdu = 0.f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                put(St, rt + 16 * j, sr[j]);
                put(Ut, rt + 16 * j, ur[j]);
                sdu += sr[j].x * ur[j].x + sr[j].y * ur[j].y + sr[j].z * ur[j].z + sr[j].w * ur[j].w;
            }
            sdu = wave_sum(sdu);
            if (lane == 0) s_sdu[n & 1][pw] = sdu;
        };
        // kRev, step n of head slot rr: stage S and dU = the carry, then fold
        // this chunk into the carry, g <- dSoff + exp2(cs_last) g, with
        // dSoff^T[n][p] = sum_t (exp2(cs_t) C_t[n]) gy_t[p] from the C and gy
        // tiles the consumers read in the same phase
        auto put_acc = [&](Tile d, int pb, f32x4 v) __attribute__((always_inline)) {
            store_split4(d, 16 * pb + r16, 16 * pw + 4 * kq, make_float4(v[0], v[1], v[2], v[3]));
        };
        auto stage_su_rev = [&](int n, auto slot_c) __attribute__((always_inline)) {
            constexpr int rr = decltype(slot_c)::value;
            const int par = n & 1;
            __bf16 *lp = opaque_lds_t(lds);
            const Tile st_ = tile_at<kIl>(lp, 4), ut = tile_at<kIl>(lp, 5), ct = tile_at<kIl>(lp, 7);
            float sdu = 0.f;
#pragma unroll
            for (int pb = 0; pb < 4; ++pb) {
                const f32x4 sv = f32x4{sr[pb].x, sr[pb].y, sr[pb].z, sr[pb].w};
                put_acc(st_, pb, sv);
                put_acc(ut, pb, gc[rr][pb]);
#pragma unroll
                for (int i = 0; i < 4; ++i) sdu += sv[i] * gc[rr][pb][i];
            }
            sdu = wave_sum(sdu);
            if (lane == 0) s_sdu[par][pw] = sdu;
            // A operand: C^T rows 16 pw + l % 16 in the perm32 token order, each
            // token scaled by exp2(cs_t)
            Frag ae[2];
#pragma unroll
            for (int m = 0; m < 2; ++m) {
                const Frag f = frag_tp(ct, m, 16 * pw);
                const float4 e0 = *(const float4 *)&s_ecs[par][32 * m + 4 * kq];
                const float4 e1 = *(const float4 *)&s_ecs[par][32 * m + 16 + 4 * kq];
                const float ev[8] = {e0.x, e0.y, e0.z, e0.w, e1.x, e1.y, e1.z, e1.w};
                float v[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) v[j] = ((float)f.h[j] + (float)f.l[j]) * ev[j];
                ae[m] = pack_frag(v);
            }
            const Tile gt = tile_at<kIl>(lp, 2 + par);
            const float alpha = kSeq ? exp2_f(s_cs[par][T - 1]) * s_carry[par] : exp2_f(s_cs[par][T - 1]);
#pragma unroll
            for (int pb = 0; pb < 4; ++pb) {
                f32x4 d = zero4();
#pragma unroll
                for (int m = 0; m < 2; ++m) d = mma3f(ae[m], frag_tp(gt, m, 16 * pb), d);
#pragma unroll
                for (int i = 0; i < 4; ++i) gc[rr][pb][i] = d[i] + alpha * gc[rr][pb][i];
                // one p-block's operands in flight at a time: the carries of
                // every head are live here
                __builtin_amdgcn_sched_barrier(0);
            }
        };

        load_xg(0);
        if (kLateZ) load_zp(0);
        load_bc(0);
        load_su(0);
        stage_xg(0);
        stage_bc(0);
        if (!kRev) {
            load_xg(1);
            load_bc(1);
        }
        lds_barrier();
        // every step: two barriers, as in the consumer loop
        auto step_rest = [&](int n) __attribute__((always_inline)) {
            load_su(n + 1);
            lds_barrier();
            if (n + 1 < NS) {
                stage_xg(n + 1);
                if ((n + 1) % R == 0) stage_bc(n + 1);
            }
            load_xg(n + 2);
            load_bc(n + 2);
            lds_barrier();
        };
        if constexpr (kRev) {
            // one chunk (its kRevR heads) per round, so each head's carry is a
            // fixed register slot.  The tiles of step n + 1 are loaded after
            // the carry update of step n and staged once the consumers leave
            // phase A (half a step of latency cover, which keeps those
            // registers free while the carries and the dSoff operands are
            // live); B, C only by the step before a chunk's first.
            auto rev_step = [&](int n, auto pos_c) __attribute__((always_inline)) {
                constexpr int pos = decltype(pos_c)::value;
                stage_su_rev(n, pos_c);
                load_su(n + 1);
                load_xg(n + 1);
                if constexpr ((pos + 1) % kRevR == 0) load_bc(n + 1);
                lds_barrier();
                if constexpr (kLateZ) {
                    // the z gate: B, C staged first and z, pre_gate loaded only
                    // now (covered by the consumers' phase B), so their
                    // registers are not live beside the carries and the
                    // other step's loads; both unconditional (past the end
                    // they only restage tiles no consumer reads)
                    if constexpr ((pos + 1) % kRevR == 0) stage_bc(n + 1);
                    load_zp(n + 1);
                    if (n + 1 < NS) stage_xg(n + 1);
                } else {
                    if (n + 1 < NS) {
                        stage_xg(n + 1);
                        if constexpr ((pos + 1) % kRevR == 0) stage_bc(n + 1);
                    }
                }
                lds_barrier();
            };
            using I0 = std::integral_constant<int, 0>;
            using I1 = std::integral_constant<int, 1>;
            using I2 = std::integral_constant<int, 2>;
            using I3 = std::integral_constant<int, 3>;
            for (int n0 = 0; n0 < NS; n0 += kRevR) {
                rev_step(n0, I0{});
                if constexpr (kRevR >= 2) rev_step(n0 + 1, I1{});
                if constexpr (kRevR == 4) {
                    rev_step(n0 + 2, I2{});
                    rev_step(n0 + 3, I3{});
                }
            }
            // the carries of the first run now hold the gradients of the initial states
            if (prm.dinit && sg == 0) {
#pragma unroll
                for (int rr = 0; rr < kRevR; ++rr)
#pragma unroll
                    for (int pb = 0; pb < 4; ++pb)
                        *(float4 *)((char *)(prm.dinit + ((int64_t)b * H + g * R + rr) * (P * N)) +
                                    acc_off + 16 * pb * N * 4) =
                            make_float4(gc[rr][pb][0], gc[rr][pb][1], gc[rr][pb][2], gc[rr][pb][3]);
            }
        } else {
            for (int n = 0; n < NS; ++n) {
                stage_su(n);
                step_rest(n);
            }
        }
        return;
    }

    // ------------------------------------------------------------ consumers
    // No global loads: every operand comes from LDS, every output is a store.
    // The products that end in per-token outputs are formed transposed
    // (operands swapped), so each lane owns token `own` and channels
    // 16 blk + 4 (l / 16) + 0..3 of every 16-channel block: per-token factors
    // are per-lane scalars, the sums over channels a 4-lane reduction, and
    // the dx, dB, dC rows leave as 16-byte stores.
    auto consumer = [&](auto wave_c) __attribute__((always_inline)) {
        constexpr int W = decltype(wave_c)::value;
        const int own = 16 * W + r16; // token of this lane (its operand row)
        const int cq = 4 * kq;        // first of its 4 channels in each 16-channel block
        // dxa[pb][i] = dxdt[own][16 pb + cq + i]; dBa, dCa likewise over n
        f32x4 dBa[4], dCa[4], dxa[4];
        // x[own][16 pb + cq + i] of the step, read in phase B and kept for the
        // step's epilogue (at the start of the next step)
        f32x4 xk[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            dBa[i] = zero4();
            dCa[i] = zero4();
        }

        // epilogue of step n (dxa holds its dxdt)
        auto epilogue = [&](int n) __attribute__((always_inline)) {
            const int k = chunk_of(n), h = g * R + n % R, par = n & 1;
            const int64_t t0 = (int64_t)k * T;
            const int tv = tvalid(k);
            const int64_t bhk = ((int64_t)b * H + h) * K + k;
            // the chunk-end terms join the last token's dcs (branch-free: every
            // lane forms them from wave-uniform values)
            const float rd_tot = wave_sum(s_rd[par][lane]);
            const float4 sdu4 = *(const float4 *)&s_sdu[par][0];
            const float carry = kSeq ? s_carry[par] : 1.f;
            const float tail = rd_tot + carry * exp2_f(s_cs[par][T - 1]) * (sdu4.x + sdu4.y + sdu4.z + sdu4.w);
            const float v = s_dcs[par][lane] + (lane == T - 1 ? tail : 0.f);
            const float da = wave_suffix_scan(v);
            if (W == 0) {
                const float dA_p = wave_sum(da * s_q[par][lane]);
                if (lane == 0) prm.part_dA[bhk] = dA_p;
            }
            const float Ah = s_A[par];
            const int64_t xo = (((int64_t)b * prm.L + t0) * H + h) * P;
            f32x4 xa[4], ga[4], Dv[4];
            __bf16 *le = opaque_lds_t(lds);
#pragma unroll
            for (int pb = 0; pb < 4; ++pb) {
                xa[pb] = xk[pb];
                ga[pb] = zero4();
                Dv[pb] = zero4();
            }
            if (prm.has_D) {
                // D gy joins dx (wave-uniform: without D neither is read)
#pragma unroll
                for (int pb = 0; pb < 4; ++pb) {
                    ga[pb] = tile_row4(tile_at<kIl>(le, 2 + par), own, 16 * pb + cq);
                    // s_D holds D per channel (a scalar D repeated)
                    const float4 d4 = *(const float4 *)&s_D[par][16 * pb + cq];
                    Dv[pb] = f32x4{d4.x, d4.y, d4.z, d4.w};
                }
            }
            // da of token own: through this wave's LDS row (written and read
            // back by the same wave, so no barrier)
            s_da[W][lane] = da;
            const float da_o = s_da[W][own];
            const float q_o = s_q[par][own], u_o = s_dqdu[par][own];
            float dqp = 0.f;
#pragma unroll
            for (int pb = 0; pb < 4; ++pb)
#pragma unroll
                for (int i = 0; i < 4; ++i) dqp += xa[pb][i] * dxa[pb][i];
            dqp = sum_kq(dqp);
            const bool valid = own < tv;
            const float ddt = valid ? (Ah * da_o + dqp) * u_o : 0.f;
            // stores through buffer resources: a per-lane row offset plus
            // immediate offsets instead of 64-bit addresses
            if (valid) {
                if (kq == 0)
                    buf_store(buf_rsrc(prm.ddt + ((int64_t)b * prm.L + t0) * H + h), own * H * 4, 0, ddt);
                const auto rdx = buf_rsrc(prm.dx + xo);
#pragma unroll
                for (int pb = 0; pb < 4; ++pb) {
                    f32x4 o;
#pragma unroll
                    for (int i = 0; i < 4; ++i) o[i] = q_o * dxa[pb][i] + Dv[pb][i] * ga[pb][i];
                    __builtin_amdgcn_raw_buffer_store_b128(
                        __builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned, o), rdx,
                        own * rowHP4 + (16 * pb + cq) * 4, 0, 0);
                }
            }
            const float dbias = wave_sum(kq == 0 ? ddt : 0.f);
            if (lane == 0) prm.part_dbias[bhk * kBwsSlots + W] = dbias;
        };

        // kRev: C . B^T of the chunk in both orientations (the blocks of
        // phase A), formed on a chunk's first head step and reused by its
        // other heads (B and C stay staged for the whole chunk)
        f32x4 cbT[4], cbS[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            cbT[j] = zero4();
            cbS[j] = zero4();
        }
        lds_barrier(); // first tiles staged
        for (int n = 0; n < NS; ++n) {
            const int k = chunk_of(n), r = n % R, par = n & 1;
            const bool form_cb = !kRev || r == 0;
            if (n > 0) epilogue(n - 1);
            __bf16 *la = opaque_lds_t(lds);
            const Tile xt = tile_at<kIl>(la, par), gt = tile_at<kIl>(la, 2 + par);
            const Tile Bt = tile_at<kIl>(la, 6), Ct = tile_at<kIl>(la, 7);

            // ---------------- phase A: x, gy, B, C
            const float *q_ = s_q[par], *cs_ = s_cs[par], *bT_ = s_bT[par], *bS_ = s_bS[par];
            Frag Bo[2];
            f32x4 ca[4];
            {
                Frag Co[2], Go[2], Xo[2];
#pragma unroll
                for (int ks = 0; ks < 2; ++ks) {
                    Bo[ks] = frag(Bt, own, ks);
                    Co[ks] = frag(Ct, own, ks);
                    Go[ks] = frag(gt, own, ks);
                    Xo[ks] = frag(xt, own, ks);
                }
                const float cs_own = cs_[own], q_own = q_[own];
                const int sid_own = kSeq ? s_sid[par][own] : 0;
                Frag DCT[2], DCS[2], WS[2];
                float rows = 0.f, cols = 0.f;
                {
                    // T orientation: t = own, s = 16 j + 4 kq + i, s-blocks j <= W
                    float dct[2][8];
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        if (j <= W) {
                            f32x4 dw = zero4();
                            if (form_cb) {
                                f32x4 cbn = zero4();
#pragma unroll
                                for (int ks = 0; ks < 2; ++ks) cbn = mma3f(frag(Bt, 16 * j + r16, ks), Co[ks], cbn);
                                cbT[j] = cbn;
                            }
                            const f32x4 cb = cbT[j];
#pragma unroll
                            for (int ks = 0; ks < 2; ++ks) dw = mma3f(frag(xt, 16 * j + r16, ks), Go[ks], dw);
                            const float4 qv = *(const float4 *)&q_[16 * j + 4 * kq];
                            // exp2(cs_own - cs_s): per element on the diagonal block,
                            // else exp2(cs_own - cs_end(j)) bT[s]
                            const float4 cv = *(const float4 *)&(j < W ? bT_ : cs_)[16 * j + 4 * kq];
                            const float aj = j < W ? exp2_f(cs_own - cs_[16 * j + 15]) : 0.f;
                            const float qa[4] = {qv.x, qv.y, qv.z, qv.w}, cva[4] = {cv.x, cv.y, cv.z, cv.w};
                            int sva[4] = {0, 0, 0, 0};
                            if (kSeq) {
                                const int4 sv = *(const int4 *)&s_sid[par][16 * j + 4 * kq];
                                sva[0] = sv.x, sva[1] = sv.y, sva[2] = sv.z, sva[3] = sv.w;
                            }
#pragma unroll
                            for (int i = 0; i < 4; ++i) {
                                const bool in = (j < W || 4 * kq + i <= r16) && (!kSeq || sva[i] == sid_own);
                                const float e = in ? (j < W ? aj * cva[i] : exp2_f(cs_own - cva[i])) : 0.f;
                                const float dwv = dw[i] * qa[i];
                                rows += dwv * cb[i] * e;
                                dct[j >> 1][(j & 1) * 4 + i] = dwv * e;
                            }
                        } else {
#pragma unroll
                            for (int i = 0; i < 4; ++i) dct[j >> 1][(j & 1) * 4 + i] = 0.f;
                        }
                    }
                    DCT[0] = pack_frag(dct[0]);
                    DCT[1] = pack_frag(dct[1]);
                }
                {
                    // S orientation: s = own, t = 16 j + 4 kq + i, t-blocks j >= W
                    float ws[2][8], dcs[2][8];
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        if (j >= W) {
                            f32x4 dw = zero4();
                            if (form_cb) {
                                f32x4 cbn = zero4();
#pragma unroll
                                for (int ks = 0; ks < 2; ++ks) cbn = mma3f(frag(Ct, 16 * j + r16, ks), Bo[ks], cbn);
                                cbS[j] = cbn;
                            }
                            const f32x4 cb = cbS[j];
#pragma unroll
                            for (int ks = 0; ks < 2; ++ks) dw = mma3f(frag(gt, 16 * j + r16, ks), Xo[ks], dw);
                            // exp2(cs_t - cs_own): per element on the diagonal block,
                            // else exp2(cs_start(j) - cs_own) bS[t]
                            const float4 cv = *(const float4 *)&(j > W ? bS_ : cs_)[16 * j + 4 * kq];
                            const float aj = j > W ? exp2_f(cs_[16 * j] - cs_own) : 0.f;
                            const float cva[4] = {cv.x, cv.y, cv.z, cv.w};
                            int sva[4] = {0, 0, 0, 0};
                            if (kSeq) {
                                const int4 sv = *(const int4 *)&s_sid[par][16 * j + 4 * kq];
                                sva[0] = sv.x, sva[1] = sv.y, sva[2] = sv.z, sva[3] = sv.w;
                            }
#pragma unroll
                            for (int i = 0; i < 4; ++i) {
                                const bool in = (j > W || r16 <= 4 * kq + i) && (!kSeq || sva[i] == sid_own);
                                const float e = in ? (j > W ? aj * cva[i] : exp2_f(cva[i] - cs_own)) : 0.f;
                                const float dwv = dw[i] * q_own, wsv = cb[i] * e;
                                cols += dwv * wsv;
                                ws[j >> 1][(j & 1) * 4 + i] = wsv;
                                dcs[j >> 1][(j & 1) * 4 + i] = dwv * e;
                            }
                        } else {
#pragma unroll
                            for (int i = 0; i < 4; ++i) {
                                ws[j >> 1][(j & 1) * 4 + i] = 0.f;
                                dcs[j >> 1][(j & 1) * 4 + i] = 0.f;
                            }
                        }
                    }
                    WS[0] = pack_frag(ws[0]);
                    WS[1] = pack_frag(ws[1]);
                    DCS[0] = pack_frag(dcs[0]);
                    DCS[1] = pack_frag(dcs[1]);
                }
                rows = sum_kq(rows);
                cols = sum_kq(cols);
                if (kq == 0) s_dcs[par][own] = rows - cols;

                // dxdt^T = gy^T W (column s = own)
#pragma unroll
                for (int pb = 0; pb < 4; ++pb) dxa[pb] = zero4();
#pragma unroll
                for (int m = 0; m < 2; ++m)
                    if (2 * m + 1 >= W)
#pragma unroll
                        for (int pb = 0; pb < 4; ++pb) dxa[pb] = mma3f(frag_tp(gt, m, 16 * pb), WS[m], dxa[pb]);
                // dC^T += B^T dCB^T (column t = own), dB^T += C^T dCB (column s = own)
#pragma unroll
                for (int m = 0; m < 2; ++m) {
                    if (2 * m <= W)
#pragma unroll
                        for (int nb = 0; nb < 4; ++nb) dCa[nb] = mma3f(frag_tp(Bt, m, 16 * nb), DCT[m], dCa[nb]);
                    if (2 * m + 1 >= W)
#pragma unroll
                        for (int nb = 0; nb < 4; ++nb) dBa[nb] = mma3f(frag_tp(Ct, m, 16 * nb), DCS[m], dBa[nb]);
                }
                // C[own][.] for phase B (the producers may restage C then)
#pragma unroll
                for (int nb = 0; nb < 4; ++nb) ca[nb] = tile_row4(Ct, own, 16 * nb + cq);
            }
            lds_barrier(); // S, dU staged; B, C of the next chunk may now be staged

            // ---------------- phase B: S, dU (x, gy of this step are still in LDS)
            __bf16 *lb = opaque_lds_t(lds);
            const Tile xb = tile_at<kIl>(lb, par), gb = tile_at<kIl>(lb, 2 + par);
            const Tile St = tile_at<kIl>(lb, 4), Ut = tile_at<kIl>(lb, 5);
            const float q_o = s_q[par][own], dte_o = s_dte[par][own], ecs_o = s_ecs[par][own];
            float rpart = 0.f, gpart = 0.f;
            {
                // (B dU^T)^T: [p][t]
#pragma unroll
                for (int pb = 0; pb < 4; ++pb) {
                    f32x4 rm = zero4();
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks) rm = mma3f(frag(Ut, 16 * pb + r16, ks), Bo[ks], rm);
                    xk[pb] = tile_row4(xb, own, 16 * pb + cq);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        dxa[pb][i] += dte_o * rm[i];
                        rpart += xk[pb][i] * rm[i];
                    }
                }
            }
            {
                // (gy S)^T: [n][t]
                Frag Go[2];
#pragma unroll
                for (int ks = 0; ks < 2; ++ks) Go[ks] = frag(gb, own, ks);
#pragma unroll
                for (int nb = 0; nb < 4; ++nb) {
                    f32x4 co = zero4();
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks) co = mma3f(frag_tn(St, ks, 16 * nb), Go[ks], co);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float vv = ecs_o * co[i];
                        dCa[nb][i] += vv;
                        gpart += vv * ca[nb][i];
                    }
                }
            }
            {
                // (x dU)^T: [n][t]
                Frag Xo[2];
#pragma unroll
                for (int ks = 0; ks < 2; ++ks) Xo[ks] = frag(xb, own, ks);
                const float sq = dte_o * q_o;
#pragma unroll
                for (int nb = 0; nb < 4; ++nb) {
                    f32x4 bs = zero4();
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks) bs = mma3f(frag_tn(Ut, ks, 16 * nb), Xo[ks], bs);
#pragma unroll
                    for (int i = 0; i < 4; ++i) dBa[nb][i] += sq * bs[i];
                }
            }
            {
                const float rd = sum_kq(rpart) * q_o * dte_o;
                const float gp = sum_kq(gpart);
                if (kq == 0) {
                    s_dcs[par][own] += gp - rd;
                    s_rd[par][own] = rd;
                }
            }
            if (r == R - 1) {
                const int64_t t0 = (int64_t)k * T;
                if (own < tvalid(k)) {
                    const int64_t o = (((int64_t)b * prm.L + t0) * G + g) * N;
                    const auto rdB = buf_rsrc(prm.dB + o), rdC = buf_rsrc(prm.dC + o);
                    typedef __attribute__((ext_vector_type(4))) unsigned u4;
#pragma unroll
                    for (int nb = 0; nb < 4; ++nb) {
                        const int off = own * rowGN4 + (16 * nb + cq) * 4;
                        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, dBa[nb]), rdB, off, 0, 0);
                        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, dCa[nb]), rdC, off, 0, 0);
                    }
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    dBa[i] = zero4();
                    dCa[i] = zero4();
                }
            }
            lds_barrier(); // S, dU free; x, gy of step n + 1 staged
        }
        epilogue(NS - 1);
    };
    switch (wave) {
    case 0: consumer(std::integral_constant<int, 0>{}); break;
    case 1: consumer(std::integral_constant<int, 1>{}); break;
    case 2: consumer(std::integral_constant<int, 2>{}); break;
    default: consumer(std::integral_constant<int, 3>{}); break;
    }
}

// Reverse state-gradient pass: one workgroup per (b, h) walks the stream's
// chunks from last to first with the state gradient g in registers:
//   dU_k = g;   g <- dSoff_k + exp(cs_last_k) g,   dSoff_k = (gy exp(cs))^T C
// starting from g = dfinal_state; dU_k goes to prm.dstates and the final g is
// dinitial_states (the per-chunk dS_off never reaches HBM).  Step i handles
// chunk K - 1 - i; the R heads of a group sit on one XCD, so C of a chunk is
// read from HBM once into its L2.  Producer waves stage gy exp(cs) and C of the next step
// (token-major, split bf16) while the consumer waves run the product
// dSoff^T[n][p] = sum_t C[t][n] (gy exp(cs))[t][p], read transposed from LDS.
// The recurrence is that of mamba_ascendc/csrc/ops/mamba2_ssd_state_passing_bwd
// (state_passing_bwd/design.md:44-61) with the dS_off product fused in.
// kSeq: packed sequences, exp(cs_t) only for tokens that read the entering
// state and the carry only where the state is not cut (as in k_bwd_ws).
template <bool kHasZ, bool kSeq>
__global__ __launch_bounds__(kWsThreads) void k_bwd_dstate_rev(BwdParams prm, const float *dfinal,
                                                                float *dinit) {
    constexpr int T = 64, P = 64, N = 64;
    __shared__ __attribute__((aligned(16))) __bf16 lds[8 * kTile]; // GE(s), CT(s), s = 0, 1
    __shared__ float s_alpha[2];

    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const int w = wave & 3, r16 = lane & 15, kq = lane >> 4;
    auto GE = [&](int s) { return tile_at(lds, 2 * s); };
    auto CT = [&](int s) { return tile_at(lds, 2 * s + 1); };
    // unit = (b * G + g) * R + r
    const int u = xcd_unit(blockIdx.x, (int)gridDim.x, prm.R);
    const int bg = u / prm.R;
    const int g = bg % prm.G, b = bg / prm.G, h = g * prm.R + u % prm.R;
    const int H = prm.H, G = prm.G, K = prm.K;
    const int nsteps = K;
    const int rowHP4 = H * P * 4, rowGN4 = G * N * 4;
    auto tvalid = [&](int k) { return (int)min((int64_t)T, prm.L - (int64_t)k * T); };

    if (wave >= 4) {
        // ---------------------------------------------------------- producers
        // ring of kDepth register slots; step i uses slot i % kDepth
        constexpr int kDepth = 3;
        const int pt = tid - 4 * kWave;
        const int rt = pt >> 4, c4 = (pt & 15) * 4; // rows rt + 16 j, columns c4 .. c4 + 3
        const bool has_dout = prm.dout != nullptr;
        const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
        float4 gr[kDepth][4], zr[kDepth][4], cr[kDepth][4];
        float dtr[kDepth];
        int sidr[kDepth], sprv[kDepth]; // kSeq: id of token `lane`, id of the token before the chunk
        // unconditional loads (exact wait counts): rows past the sequence end
        // re-read its last row (zeroed when staged), steps past chunk 0 read
        // through an empty-range resource (zeros, no traffic)
        auto p_load = [&](int i, auto slot_c) {
            constexpr int sl = decltype(slot_c)::value;
            const bool real = i < nsteps;
            const int k = real ? K - 1 - i : 0, tv = tvalid(k);
            const int range = real ? 0x7fffffff : 0;
            const int64_t t0 = (int64_t)k * T;
            const int64_t xo = (((int64_t)b * prm.L + t0) * H + h) * P;
            const auto rd = buf_rsrc_n(has_dout ? prm.dout + xo : prm.x + xo, range);
            const auto rz = buf_rsrc_n(kHasZ ? prm.z + xo : prm.x + xo, range);
            const auto rc = buf_rsrc_n(prm.C + (((int64_t)b * prm.L + t0) * G + g) * N, range);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int row = min(rt + 16 * j, tv - 1);
                gr[sl][j] = buf_load4(rd, row * rowHP4 + c4 * 4, 0);
                if (kHasZ) zr[sl][j] = buf_load4(rz, row * rowHP4 + c4 * 4, 0);
                cr[sl][j] = buf_load4(rc, row * rowGN4 + c4 * 4, 0);
            }
            dtr[sl] = prm.dt[((int64_t)b * prm.L + t0 + min(lane, tv - 1)) * H + h];
            if (kSeq) {
                const int32_t *si = prm.seq_idx + (int64_t)b * prm.L + t0;
                sidr[sl] = si[min(lane, tv - 1)];
                const int pv = si[t0 > 0 ? -1 : 0]; // read unconditionally, 0 before the first chunk
                sprv[sl] = t0 > 0 ? pv : 0;
            }
        };
        auto put = [&](SplitTile d, int row, float4 v) { store_split4(d, row, c4, v); };
        auto p_stage = [&](int i, int s, auto slot_c) {
            constexpr int sl = decltype(slot_c)::value;
            const bool real = i < nsteps;
            const int tv = real ? tvalid(K - 1 - i) : 0; // nothing valid past chunk 0
            const float Ah2 = prm.A[h] * kLog2e;
            const float bias = prm.dt_bias ? prm.dt_bias[h] : 0.f;
            float a = 0.f;
            if (lane < tv) a = Ah2 * discretize_dt(dtr[sl], bias, prm.softplus != 0, prm.lo, prm.hi);
            const float cs = wave_inclusive_scan(a); // log2 units
            const float cs_last = readlane_f(cs, T - 1);
            float reads = 1.f, carry = 1.f;
            if (kSeq) {
                const int e_end = __builtin_amdgcn_readlane(sidr[sl], T - 1);
                reads = sidr[sl] == sprv[sl] ? 1.f : 0.f;
                carry = e_end == sprv[sl] ? 1.f : 0.f;
            }
            if (w == 0 && lane == 0) s_alpha[s] = exp2_f(cs_last) * carry;
            const float ecs = exp2_f(cs) * reads;
            const SplitTile ge = GE(s), ct = CT(s);
            // the four permutes issued back to back, ahead of every tile
            // write: one wait for all of them instead of one each
            float es[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) es[j] = __shfl(ecs, rt + 16 * j, kWave);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int row = rt + 16 * j;
                const bool ok = row < tv;
                const float e = es[j];
                float4 v = (ok && has_dout) ? gr[sl][j] : z4;
                if (kHasZ) {
                    v.x *= silu_f(zr[sl][j].x);
                    v.y *= silu_f(zr[sl][j].y);
                    v.z *= silu_f(zr[sl][j].z);
                    v.w *= silu_f(zr[sl][j].w);
                }
                put(ge, row, make_float4(v.x * e, v.y * e, v.z * e, v.w * e));
                put(ct, row, ok ? cr[sl][j] : z4);
            }
        };
        using S0 = std::integral_constant<int, 0>;
        using S1 = std::integral_constant<int, 1>;
        using S2 = std::integral_constant<int, 2>;
        static_assert(kDepth == 3, "the unrolled ring below assumes three slots");
        p_load(0, S0{});
        p_load(1, S1{});
        p_load(2, S2{});
        p_stage(0, 0, S0{});
        p_load(3, S0{});
        lds_barrier();
        // past the last step this stages zeros that no consumer reads
        auto p_iter = [&](int i, auto slot_next) {
            p_stage(i + 1, (i + 1) & 1, slot_next);
            p_load(i + 1 + kDepth, slot_next);
            lds_barrier();
        };
        // whole rounds of the ring, then the 0..2 remaining steps
        int i0 = 0;
        for (; i0 + kDepth <= nsteps; i0 += kDepth) {
            p_iter(i0, S1{});
            p_iter(i0 + 1, S2{});
            p_iter(i0 + 2, S0{});
        }
        if (i0 < nsteps) p_iter(i0, S1{});
        if (i0 + 1 < nsteps) p_iter(i0 + 1, S2{});
        return;
    }

    // -------------------------------------------------------------- consumers
    // g[p = 16 pb + l % 16][n = 16 w + 4 (l / 16) + i] in gs[pb][i]
    f32x4 gs[4];
    const int goff = (r16 * N + 16 * w + 4 * kq); // + 16 pb N
    const int64_t bh = (int64_t)b * H + h;
#pragma unroll
    for (int pb = 0; pb < 4; ++pb) {
        gs[pb] = zero4();
        if (dfinal) {
            const float4 v = *(const float4 *)(dfinal + bh * (P * N) + goff + 16 * pb * N);
            gs[pb] = f32x4{v.x, v.y, v.z, v.w};
        }
    }
    lds_barrier();
    for (int i = 0; i < nsteps; ++i) {
        const int k = K - 1 - i, s = i & 1;
        float *du = prm.dstates + ((bh * K + k) * (P * N));
#pragma unroll
        for (int pb = 0; pb < 4; ++pb)
            *(float4 *)(du + goff + 16 * pb * N) = make_float4(gs[pb][0], gs[pb][1], gs[pb][2], gs[pb][3]);
        const SplitTile ge = GE(s), ct = CT(s);
        f32x4 U[4];
#pragma unroll
        for (int pb = 0; pb < 4; ++pb) U[pb] = zero4();
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const Frag a = frag_tn(ct, ks, 16 * w);
#pragma unroll
            for (int pb = 0; pb < 4; ++pb) U[pb] = mma3f(a, frag_tn(ge, ks, 16 * pb), U[pb]);
        }
        const float alpha = s_alpha[s];
#pragma unroll
        for (int pb = 0; pb < 4; ++pb)
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) gs[pb][ii] = alpha * gs[pb][ii] + U[pb][ii];
        lds_barrier(); // buffer s is free, buffer s ^ 1 is staged
    }
    if (dinit) {
#pragma unroll
        for (int pb = 0; pb < 4; ++pb)
            *(float4 *)(dinit + bh * (P * N) + goff + 16 * pb * N) =
                make_float4(gs[pb][0], gs[pb][1], gs[pb][2], gs[pb][3]);
    }
}

// Segment pre-pass of the reverse fused backward, one workgroup per (b, h,
// run of M chunks): the gradient the run's own tokens send to the state
// entering it, and the run's log decay,
//   c[p][n] = sum_t exp2(CS_t) gy_t[p] C_t[n],   CS_t = log2 decay from the
//   run's start through token t,
// the closed form of k_bwd_dstate_rev's recurrence g <- dSoff_k +
// exp2(cs_last_k) g over the run (from its last chunk, g = 0) with the
// decays folded into the staged operand.  Chunks go in pairs, both staged at
// once by all eight waves (the loads of the whole pair in flight together,
// the next pair's issued before this pair's products), so a run of one or two
// chunks is a single pass: the recurrence's chunk-by-chunk steps through a
// register ring are latency-bound at one or two chunks per head.  The 16
// output tiles go two to a wave (n-block wave % 4, p-blocks 2 (wave / 4) and
// 2 (wave / 4) + 1); the same operands, fragments and split-bf16 products
// as the recurrence's.
template <bool kHasZ, bool kSeq>
__global__ __launch_bounds__(kWsThreads, 2) void k_bwd_run_grad(BwdParams prm, RevSeg rs) {
    constexpr int T = 64, P = 64, N = 64;
    __shared__ __attribute__((aligned(16))) __bf16 lds[8 * kTile]; // GE(c), CT(c) of the pair's chunk c
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const int r16 = lane & 15, kq = lane >> 4;
    auto GE = [&](int c) { return tile_at(lds, 2 * c); };
    auto CT = [&](int c) { return tile_at(lds, 2 * c + 1); };
    // unit = ((b * G + g) * nseg + sg) * R + r: the R heads of a group's run
    // on one XCD, so C of the run reaches one L2
    const int R = prm.R;
    const int u = xcd_unit(blockIdx.x, (int)gridDim.x, R);
    const int r = u % R, sg = (u / R) % rs.nseg, bg = u / (R * rs.nseg);
    const int g = bg % prm.G, b = bg / prm.G, h = g * R + r;
    const int H = prm.H, G = prm.G, K = prm.K;
    const int kbeg = sg * rs.M, kend = min(kbeg + rs.M, K);
    const int rowHP4 = H * P * 4, rowGN4 = G * N * 4;
    const bool has_dout = prm.dout != nullptr;
    const float Ah2 = prm.A[h] * kLog2e;
    const float bias = prm.dt_bias ? prm.dt_bias[h] : 0.f;
    // staging: this thread's chunk of the pair, rows rt + 16 j, columns c4 .. c4 + 3
    const int cpair = tid >> 8, pt = tid & 255;
    const int rt = pt >> 4, c4 = (pt & 15) * 4;
    auto tvalid = [&](int k) { return k < kend ? (int)min((int64_t)T, prm.L - (int64_t)k * T) : 0; };

    float4 gr[4], zr[4], cr[4];
    float dtr[2];
    int sidr[2], sprv[2];
    // unconditional loads (exact wait counts): rows past the sequence end
    // re-read its last row and chunks past the run read through an
    // empty-range resource (zeros); both are zeroed when staged
    auto load = [&](int k0) {
        const int k = k0 + cpair;
        const bool real = k < kend;
        const int kk = real ? k : kbeg, tv = (int)min((int64_t)T, prm.L - (int64_t)kk * T);
        const int range = real ? 0x7fffffff : 0;
        const int64_t t0 = (int64_t)kk * T;
        const int64_t xo = (((int64_t)b * prm.L + t0) * H + h) * P;
        const auto rd = buf_rsrc_n(has_dout ? prm.dout + xo : prm.x + xo, range);
        const auto rz = buf_rsrc_n(kHasZ ? prm.z + xo : prm.x + xo, range);
        const auto rc = buf_rsrc_n(prm.C + (((int64_t)b * prm.L + t0) * G + g) * N, range);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int row = min(rt + 16 * j, tv - 1);
            gr[j] = buf_load4(rd, row * rowHP4 + c4 * 4, 0);
            if (kHasZ) zr[j] = buf_load4(rz, row * rowHP4 + c4 * 4, 0);
            cr[j] = buf_load4(rc, row * rowGN4 + c4 * 4, 0);
        }
        // dt (and ids) of token `lane` of both chunks, for every wave's scans
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const int kc = k0 + c < kend ? k0 + c : kbeg;
            const int64_t tc = (int64_t)kc * T;
            const int tvc = (int)min((int64_t)T, prm.L - tc);
            dtr[c] = prm.dt[((int64_t)b * prm.L + tc + min(lane, tvc - 1)) * H + h];
            if (kSeq) {
                const int32_t *si = prm.seq_idx + (int64_t)b * prm.L + tc;
                sidr[c] = si[min(lane, tvc - 1)];
                const int pv = si[tc > 0 ? -1 : 0]; // read unconditionally, 0 before the first chunk
                sprv[c] = tc > 0 ? pv : 0;
            }
        }
    };

    // output tiles g[p = 16 pb + l % 16][n = 16 nb + 4 (l / 16) + i]
    const int nb = wave & 3, pb0 = 2 * (wave >> 2);
    f32x4 acc[2] = {zero4(), zero4()};
    float off = 0.f;   // log2 decay from the run's start to the pair's first token
    float keep = 1.f;  // kSeq: 0 once the state is cut inside the run
    bool cut = false;
    load(kbeg);
    for (int k0 = kbeg; k0 < kend; k0 += 2) {
        // per-token log2 decays of both chunks (every wave, lane = token)
        float cs[2], last[2], reads[2] = {1.f, 1.f}, carry[2] = {1.f, 1.f};
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const int tv = tvalid(k0 + c);
            float a = 0.f;
            if (lane < tv) a = Ah2 * discretize_dt(dtr[c], bias, prm.softplus != 0, prm.lo, prm.hi);
            cs[c] = wave_inclusive_scan(a);
            last[c] = readlane_f(cs[c], T - 1);
            if (kSeq && k0 + c < kend) {
                const int e_end = __builtin_amdgcn_readlane(sidr[c], T - 1);
                reads[c] = sidr[c] == sprv[c] ? 1.f : 0.f;
                carry[c] = e_end == sprv[c] ? 1.f : 0.f;
            }
        }
        // exp2(CS_t) of this thread's chunk, times the kSeq masks
        const float base = cpair ? off + last[0] : off;
        const float mask = kSeq ? (cpair ? keep * carry[0] : keep) * (cpair ? reads[1] : reads[0]) : 1.f;
        const float ecs = exp2_f(base + (cpair ? cs[1] : cs[0])) * mask;
        float es[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) es[j] = __shfl(ecs, rt + 16 * j, kWave);
        __builtin_amdgcn_sched_barrier(0);
        const int tv = tvalid(k0 + cpair);
        const SplitTile ge = GE(cpair), ct = CT(cpair);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int row = rt + 16 * j;
            const bool ok = row < tv;
            const float e = es[j];
            float4 v = (ok && has_dout) ? gr[j] : make_float4(0.f, 0.f, 0.f, 0.f);
            if (kHasZ) {
                v.x *= silu_f(zr[j].x);
                v.y *= silu_f(zr[j].y);
                v.z *= silu_f(zr[j].z);
                v.w *= silu_f(zr[j].w);
            }
            store_split4(ge, row, c4, make_float4(v.x * e, v.y * e, v.z * e, v.w * e));
            store_split4(ct, row, c4, ok ? cr[j] : make_float4(0.f, 0.f, 0.f, 0.f));
        }
        off += last[0] + last[1];
        if (kSeq) {
            keep *= carry[0] * carry[1];
            cut = cut || carry[0] == 0.f || carry[1] == 0.f;
        }
        // the next pair's loads fly under this pair's products
        if (k0 + 2 < kend) load(k0 + 2);
        lds_barrier();
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const Frag a = frag_tn(CT(c), ks, 16 * nb);
#pragma unroll
                for (int i = 0; i < 2; ++i) acc[i] = mma3f(a, frag_tn(GE(c), ks, 16 * (pb0 + i)), acc[i]);
            }
        lds_barrier(); // the tiles are free for the next pair
    }
    const int64_t bh = (int64_t)b * H + h;
    float *dst = rs.seg_carry + (bh * rs.nseg + sg) * (P * N);
#pragma unroll
    for (int i = 0; i < 2; ++i)
        *(float4 *)(dst + (16 * (pb0 + i) + r16) * N + 16 * nb + 4 * kq) = make_float4(acc[i][0], acc[i][1], acc[i][2], acc[i][3]);
    if (tid == 0) rs.seg_log_decay[bh * rs.nseg + sg] = cut ? -INFINITY : off * kLn2;
}

}  // namespace bwd

// fixed-order reductions of the per-chunk partials, one workgroup per head:
// dA from [B, H, K], ddt_bias and dD from [B, H, K, slots] (dD per channel:
// [B, H, K, slots, P])
#ifndef SSD_KERNEL_TEMPLATES_ONLY
__global__ __launch_bounds__(kThreads) void k_bwd_finalize_slots(
    const float *part_dA, const float *part_dbias, const float *part_dD, float *dA, float *ddt_bias,
    float *dD, int B, int H, int K, int P, int slots, int has_D, int d_per_channel) {
    __shared__ float s_tmp[4];
    __shared__ float s_col[4][64];
    const int h = blockIdx.x, tid = threadIdx.x;
    const int n1 = B * K, ks = K * slots, n4 = B * ks;
    float a = 0.f, db = 0.f, dd = 0.f;
    for (int i = tid; i < n1; i += kThreads) a += part_dA[((int64_t)(i / K) * H + h) * K + i % K];
    for (int i = tid; i < n4; i += kThreads) {
        const int64_t pi = ((int64_t)(i / ks) * H + h) * ks + i % ks;
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
        for (int p0 = 0; p0 < P; p0 += 64) {
            const int p = p0 + (tid & 63), grp = tid >> 6;
            float v = 0.f;
            if (p < P)
                for (int i = grp; i < n4; i += 4) {
                    const int64_t pi = ((int64_t)(i / ks) * H + h) * ks + i % ks;
                    v += part_dD[pi * P + p];
                }
            s_col[grp][tid & 63] = v;
            __syncthreads();
            if (grp == 0 && p < P)
                dD[h * P + p] = s_col[0][tid] + s_col[1][tid] + s_col[2][tid] + s_col[3][tid];
            __syncthreads();
        }
    }
}
#endif

}  // namespace ssd
