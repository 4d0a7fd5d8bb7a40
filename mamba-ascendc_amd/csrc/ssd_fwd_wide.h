// Fused forward for dstate N = 128 (headdim 64): one workgroup per
// (batch b, head h, channel half ph, segment), 32 channels of the head and all
// 128 state columns.
//
// The two channel halves of a head are independent problems: the state rows
// p, the output channels p and the x columns p of one half never meet the
// other half's, while C . B^T (over all 128 columns) is the same for both, so
// each workgroup forms it in full.  Each workgroup therefore writes its own
// channels of `out` (with D x, pre_gate and the z gate) directly, reads its
// half of every x row, and B and C come from HBM once per head group: the two
// halves of a head, like the R heads of a group, run on consecutive workgroups
// of one XCD (xcd_unit), so the second reader finds them in that XCD's L2.
//
// Per 64-token chunk, as in k_fwd_seg (q = discretised dt, cs = chunk-local
// cumsum of A q in log2 units, decay_t = exp2(cs_last - cs_t)):
//   y_t[p] = exp2(cs_t) C_t . S[p] + sum_{s <= t} (C_t . B_s) exp2(cs_t - cs_s) q_s x_s[p]
//   S[p]  <- exp2(cs_last) S[p] + sum_t B_t (decay_t q_t x_t[p])
// Tiles (split fp16, LDS, double buffered by chunk parity s):
//   T1 = B [t][n], 64 x 128      (A operand of C.B^T, rows s; and, read
//                                 transposed, the A operand of U^T)
//   T2 = x [t][p], 64 x 32       (x^T operand of the W product, transposed
//                                 reads; and the x of the D x term)
//   T3 = decay q x [t][p], 64 x 32  (B operand of U^T, transposed reads)
//   T4 = S [p][n], 32 x 128      (A operand of the C.S term)
// and, in registers, C_t for the lane's own token row.  The state of wave W is
// its two 16-column blocks n in {16 W.., 64 + 16 W..} for the 32 rows p, held
// in the accumulator layout of U^T.
//
// Long sequences with few streams are cut into segments exactly as for
// k_fwd_seg: the state-only pass of k_fwd_seg (two 64-column halves) gives each
// pre-segment's contribution in the same [B, H, nseg, P, N] layout, and this
// kernel starts each segment from the state entering it, folded from those
// contributions in its prologue (fold_entry) or read from the boundary states
// of the segment recurrence (k_state_pass) when there are many.
//
// kCB: with many heads per group the 2 R workgroups of a group's chunk read
// C . B^T from k_chunk_cb's per-chunk products instead of each forming it.
//
// The math is that of mamba_ascendc/csrc/ops/mamba2_ssd_fwd/design.md:10-20 and
// the chunked decomposition of mamba_torch/ssd_reference.py:113-189; the
// fusion, blocking and layouts are this file's own.
#pragma once

#include <type_traits>

#include "ssd_fwd_fused.h"

namespace ssd {

namespace wide {
constexpr int kT = 64, kPC = 32, kNC = 128;
constexpr int kS1 = kNC + 8;  // row stride (halves) of the 128-wide tiles T1, T4
constexpr int kS2 = kPC + 8;  // row stride of the 32-wide tiles T2, T3
constexpr int kA1 = kT * kS1, kA2 = kT * kS2, kA4 = kPC * kS1;  // halves per array
// offsets (halves) of the arrays of buffer s: T1 hi, lo | T2 hi, lo | T3 hi, lo | T4 hi, lo
constexpr int kBuf = 2 * (kA1 + 2 * kA2 + kA4);
__device__ __forceinline__ SplitTile T1(_Float16 *b, int s) { return {b + s * kBuf, b + s * kBuf + kA1}; }
__device__ __forceinline__ SplitTile T2(_Float16 *b, int s) {
    return {b + s * kBuf + 2 * kA1, b + s * kBuf + 2 * kA1 + kA2};
}
__device__ __forceinline__ SplitTile T3(_Float16 *b, int s) {
    return {b + s * kBuf + 2 * kA1 + 2 * kA2, b + s * kBuf + 2 * kA1 + 3 * kA2};
}
__device__ __forceinline__ SplitTile T4(_Float16 *b, int s) {
    return {b + s * kBuf + 2 * kA1 + 4 * kA2, b + s * kBuf + 2 * kA1 + 4 * kA2 + kA4};
}
}  // namespace wide

// C_t . B_s of one 64-token chunk of one (b, g):
// cb[((b G + g) K + k) 64 + t][s] = sum_n C[t][n] B[s][n] for the blocks
// s <= t (16-token blocks; the others are never read), rows past the sequence
// end zero.  Every workgroup of the group's heads (2 R of them in k_fwd_wide)
// reads it instead of forming the product itself.  The operands are split
// fp16 exactly as in k_fwd_wide's own product (same fragments, same MFMA
// order), so both give the same bits.  One workgroup (4 waves) per (b, g, k);
// wave W forms the blocks of tokens t in 16 W .. 16 W + 15.
constexpr int kCbThreads = 256;
template <int kN>
__global__ __launch_bounds__(kCbThreads) void k_chunk_cb(const float *C, const float *B, float *cb, int64_t L,
                                                         int G, int K) {
    constexpr int T = 64, kS = kN + 8; // row stride (halves)
    __shared__ __attribute__((aligned(16))) _Float16 lds[4 * T * kS];
    const SplitTile tb{lds, lds + T * kS}, tc{lds + 2 * T * kS, lds + 3 * T * kS};
    const int64_t id = blockIdx.x; // (b G + g) K + k
    const int k = (int)(id % K);
    const int64_t bg = id / K;
    const int g = (int)(bg % G);
    const int64_t b = bg / G;
    const int64_t t0 = (int64_t)k * T;
    const int tv = (int)min((int64_t)T, L - t0);
    const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
    // every load issued before the first is used: rows past the sequence end
    // re-read its last row and are zeroed when staged
    constexpr int kIt = T * kN / 4 / kCbThreads;
    static_assert(kIt * kCbThreads * 4 == T * kN, "whole rows per pass");
    float4 vb[kIt], vc[kIt];
#pragma unroll
    for (int i = 0; i < kIt; ++i) {
        const int e = threadIdx.x + i * kCbThreads, row = e / (kN / 4), c4 = (e % (kN / 4)) * 4;
        const int64_t o = ((b * L + t0 + min(row, tv - 1)) * G + g) * kN + c4;
        vb[i] = *(const float4 *)(B + o);
        vc[i] = *(const float4 *)(C + o);
    }
#pragma unroll
    for (int i = 0; i < kIt; ++i) {
        const int e = threadIdx.x + i * kCbThreads, row = e / (kN / 4), c4 = (e % (kN / 4)) * 4;
        store_split4(tb, row * kS + c4, row < tv ? vb[i] : z4);
        store_split4(tc, row * kS + c4, row < tv ? vc[i] : z4);
    }
    __syncthreads();
    const int W = wave_id(), lane = threadIdx.x & 63, r16 = lane & 15, kq = lane >> 4;
    const int own = 16 * W + r16;
    Frag Co[kN / 32];
#pragma unroll
    for (int ks = 0; ks < kN / 32; ++ks) Co[ks] = frag_s<kS>(tc, own, ks);
    float *dst = cb + id * (T * T);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        if (j > W) break;
        f32x4 acc = zero4();
#pragma unroll
        for (int ks = 0; ks < kN / 32; ++ks) acc = mma3f(frag_s<kS>(tb, 16 * j + r16, ks), Co[ks], acc);
        *(float4 *)(dst + own * T + 16 * j + 4 * kq) = make_float4(acc[0], acc[1], acc[2], acc[3]);
    }
}

// Ownership of a workgroup's 32 x 128 state (16 tiles of 16 x 16: p-block
// pb = 0, 1, n-block nb = 0..7) over the four consumer waves.  Wave W forms
// the causal C . B^T blocks j <= W of its token rows (over 128 columns), so
// the later waves carry more of the mask work; its own tiles are n-blocks W
// and W + 4, and a split (c0, c1, c2, c3) other than (4, 4, 4, 4) hands tiles
// of the later waves to the earlier ones (with them their U products, state
// update and T4 staging).  Measured (A/B, three interleaved runs, k_fwd_wide
// average): C2 4444 0.0540 ms, 6532 0.0523, 7531 0.0523, 5533 0.0534; C5
// (C . B^T precomputed, so less to balance) 0.1716, 0.1731, 0.1744, 0.1730.
struct WideTileMap {
    int n[4];
    int nb[4][8], pb[4][8];
    int nd[4], dnb[4][8], tix[4][8]; // distinct n-blocks of a wave, and each tile's index among them
};
constexpr WideTileMap make_wide_tiles(int c0, int c1, int c2, int c3) {
    WideTileMap m{};
    const int want[4] = {c0, c1, c2, c3};
    int snb[16] = {}, spb[16] = {}, ns = 0;
    for (int w = 0; w < 4; ++w)
        for (int i = 0; i < 4; ++i) {
            const int nb = w + 4 * (i >> 1), pb = i & 1;
            if (i < want[w]) {
                m.nb[w][m.n[w]] = nb;
                m.pb[w][m.n[w]] = pb;
                ++m.n[w];
            } else {
                snb[ns] = nb;
                spb[ns] = pb;
                ++ns;
            }
        }
    int t = 0;
    for (int w = 0; w < 4; ++w)
        while (m.n[w] < want[w] && t < ns) {
            m.nb[w][m.n[w]] = snb[t];
            m.pb[w][m.n[w]] = spb[t];
            ++m.n[w];
            ++t;
        }
    for (int w = 0; w < 4; ++w)
        for (int i = 0; i < m.n[w]; ++i) {
            int j = 0;
            while (j < m.nd[w] && m.dnb[w][j] != m.nb[w][i]) ++j;
            if (j == m.nd[w]) m.dnb[w][m.nd[w]++] = m.nb[w][i];
            m.tix[w][i] = j;
        }
    return m;
}
constexpr WideTileMap kWideTiles = make_wide_tiles(6, 5, 3, 2);

// kSave: also write the state entering every chunk to prm.chunk_states (the
// varlen states read them).  kGate: the z gate.  kSeq: packed sequences.
// kCB: C . B^T of each chunk comes from prm.cb (k_chunk_cb) instead of
// being formed here (the 2 R workgroups of a group would each form it).
template <bool kSave = false, bool kGate = false, bool kSeq = false, bool kCB = false>
__global__ __launch_bounds__(kWsThreads) void k_fwd_wide(FwdParams prm, SegParams sp) {
    using namespace wide;
    constexpr int T = kT, P = 64, NS = kNC;
    constexpr int TS = kSeq ? T : 1;
    __shared__ __attribute__((aligned(16))) _Float16 lds[2 * kBuf];
    struct ChunkTok {
        float cs[2][T], q[2][T];
        // q_s 2^-ek exp2(cs_e - cs_s), e the last token of s's 16-token block:
        // the blocks below the diagonal take exp2(cs_t - cs_s) q_s as
        // exp2(cs_t - cs_e) times this (both factors <= 1)
        float gq[2][T];
        int sid[2][TS];
        float off[2][TS];
        float carry[2];
        int mixed[2];
        int qexp[2]; // ek: q holds q 2^-ek
        int qe[2][TS]; // kSeq: q of token t holds q 2^-qe[t] (ek of its id)
        int sexp[2]; // eN: T3 holds x dec q 2^-eN, the scale of the state leaving the chunk
    };
    __shared__ __attribute__((aligned(16))) ChunkTok s_tok;
    __shared__ __attribute__((aligned(16))) float s_smax[4]; // |entering state| maximum per consumer wave
    auto &s_cs = s_tok.cs, &s_q = s_tok.q;
    auto &s_sid = s_tok.sid;
    auto &s_off = s_tok.off;
    auto &s_carry = s_tok.carry;
    auto &s_mixed = s_tok.mixed;
    __shared__ __attribute__((aligned(16))) float s_Dv[kPC]; // D of this half's channels

    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const bool producer = wave >= 4;
    const int w = wave & 3;
    const int r16 = lane & 15, kq = lane >> 4;

    // unit = (((b * G + g) * nseg + sg) * R + r) * 2 + ph
    const int u = xcd_unit(blockIdx.x, (int)gridDim.x, 2 * prm.R);
    const int ph = u & 1;
    const int r = (u >> 1) % prm.R;
    const int sg = (u / (2 * prm.R)) % sp.nseg;
    const int bg = u / (2 * prm.R * sp.nseg);
    const int g = bg % prm.G, b = bg / prm.G;
    const int h = g * prm.R + r;
    const int H = prm.H, G = prm.G;
    const int p0 = kPC * ph; // first channel of this half
    const int64_t PNS = (int64_t)P * NS;
    const int kbeg = sg * sp.M, kend = min(kbeg + sp.M, prm.K);

    // ------------------------------------------------------------ producer
    // Ring of kDepth register slots with the loads of the next kDepth chunks:
    // x rows xrow + 32 j (columns p0 + cx .. + 3) and B rows brow + 8 j
    // (columns cb .. cb + 3) of that chunk, and dt of token `lane`.
    constexpr int kDepth = 3;
    const int pt = tid - 4 * kWave;
    const int xrow = pt >> 3, cx = (pt & 7) * 4;   // x: 8 threads per 32-column row
    const int brow = pt >> 5, cb = (pt & 31) * 4;  // B: 32 threads per 128-column row
    float4 xr[kDepth][2], br[kDepth][8];
    float dtr[kDepth];
    int p_eS = kZeroState; // exponent of the state entering the chunk being staged
    int sidr[kDepth], sprv[kDepth];
    const int rowHP4 = (int)((int64_t)H * P * 4), rowGN4 = (int)((int64_t)G * NS * 4); // token strides, bytes
    const int hr = h / prm.hdiv, Hr = H / prm.hdiv;
    const int xrow_off = xrow * rowHP4, brow_off = brow * rowGN4; // bytes
    const int dt_off = lane * Hr * 4;                             // dt of token `lane`, bytes
    const float Ah2 = prm.A[hr] * kLog2e;
    const float bias = prm.dt_bias ? prm.dt_bias[hr] : 0.f;
    auto p_load = [&](int k, auto slot_c) {
        constexpr int sl = decltype(slot_c)::value;
        const bool real = k < kend;
        const int64_t t0 = (int64_t)(real ? k : kbeg) * T;
        const int tv = (int)min((int64_t)T, prm.L - t0);
        const int range = real ? 0x7fffffff : 0;
        const auto rx = buf_rsrc_n(prm.x + (((int64_t)b * prm.L + t0) * H + h) * P + p0, range);
        const auto rb = buf_rsrc_n(prm.B + (((int64_t)b * prm.L + t0) * G + g) * NS, range);
        // row offsets clamped to the last valid row: min of the lane's
        // precomputed offsets and the chunk's last-row offset
        const int xlast = (tv - 1) * rowHP4, blast = (tv - 1) * rowGN4;
#pragma unroll
        for (int j = 0; j < 2; ++j) xr[sl][j] = buf_load4(rx, min(xrow_off + 32 * j * rowHP4, xlast) + cx * 4, 0);
#pragma unroll
        for (int j = 0; j < 8; ++j) br[sl][j] = buf_load4(rb, min(brow_off + 8 * j * rowGN4, blast) + cb * 4, 0);
        const auto rdt = buf_rsrc(prm.dt + ((int64_t)b * prm.L + t0) * Hr + hr);
        dtr[sl] = buf_load(rdt, min(dt_off, (tv - 1) * Hr * 4), 0);
        if (kSeq) {
            const int32_t *si = prm.seq_idx + (int64_t)b * prm.L + t0;
            sidr[sl] = si[min(lane, tv - 1)];
            const int pv = si[t0 > 0 ? -1 : 0];
            sprv[sl] = t0 > 0 ? pv : 0;
        }
    };
    auto p_stage = [&](int k, int s, auto slot_c) {
        constexpr int sl = decltype(slot_c)::value;
        const int tv = (int)min((int64_t)T, prm.L - (int64_t)k * T);
        float q = 0.f;
        if (lane < tv) q = discretize_dt(dtr[sl], bias, prm.softplus != 0, prm.lo, prm.hi);
        const float sq = wave_inclusive_scan(q); // prefix sums of q
        const float cs = opaque_f(Ah2 * sq);               // log2 units
        const float cs_last = readlane_f(cs, T - 1);
        int ek = chunk_q_exp(readlane_f(sq, T - 1), wave_max(fabsf(q))); // kSeq: that of the id leaving the chunk
        int ek_tok = ek; // exponent of the token's q (kSeq: that of its id)
        ChunkTok *tk = opaque_lds_t(&s_tok);
        if (w == 0) tk->cs[s][lane] = cs;
        float dec = exp2_f(cs_last - cs);
        bool cut = false; // kSeq: the state does not carry over the chunk
        if (kSeq) {
            const int sid = sidr[sl], e_end = __builtin_amdgcn_readlane(sid, T - 1), e_prev = sprv[sl];
            if (sid != e_end || e_end < 0) dec = 0.f;
            const bool mixed = __ballot(sid != e_end) != 0;
            if (mixed) { // wave-uniform
                ek_tok = id_q_exp(sid, q);
                ek = __builtin_amdgcn_readlane(ek_tok, T - 1);
            }
            if (w == 0) {
                tk->sid[s][lane] = sid;
                tk->off[s][lane] = sid == e_prev ? 1.f : 0.f;
                tk->qe[s][lane] = ek_tok;
                if (lane == 0) {
                    tk->carry[s] = e_end == e_prev ? 1.f : 0.f;
                    tk->mixed[s] = mixed ? 1 : 0;
                }
            }
            cut = e_end != e_prev;
        }
        if (w == 0) {
            const float qs = __builtin_amdgcn_ldexpf(q, -ek_tok);
            tk->q[s][lane] = qs;
            tk->gq[s][lane] = exp2_f(dpp_f<0x15F>(cs) - cs) * qs;
        }
        // the state leaving the chunk is held as S 2^-eN: every producer wave
        // runs this recurrence, and the consumers take eN from LDS
        const int eN = next_state_exp(p_eS, ek, cs_last, cut);
        p_eS = eN;
        if (w == 0 && lane == 0) {
            tk->qexp[s] = ek;
            tk->sexp[s] = eN;
        }
        const float qn = __builtin_amdgcn_ldexpf(q, -eN);
        _Float16 *lp = opaque_lds(lds);
        const SplitTile t1 = T1(lp, s), t2 = T2(lp, s), t3 = T3(lp, s);
        // both permutes issued ahead of every tile write: one wait for both
        float drs[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) drs[j] = __shfl(dec * qn, xrow + 32 * j, kWave);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int row = xrow + 32 * j;
            const float dr = drs[j];
            const float4 xv = xr[sl][j];
            store_split4(t2, row * kS2 + cx, xv);
            store_split4(t3, row * kS2 + cx, make_float4(xv.x * dr, xv.y * dr, xv.z * dr, xv.w * dr));
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) store_split4(t1, (brow + 8 * j) * kS1 + cb, br[sl][j]);
    };

    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    using S2 = std::integral_constant<int, 2>;
    static_assert(kDepth == 3, "the unrolled ring below assumes three slots");
    // the entering state can be nonzero: its magnitude sets its first scale,
    // through one more barrier in both roles (wave-uniform)
    const bool s0_nonzero = sp.seg_in != nullptr || prm.init != nullptr;
    if (producer) {
        p_load(kbeg, S0{});
        p_load(kbeg + 1, S1{});
        p_load(kbeg + 2, S2{});
        if (s0_nonzero) {
            lds_barrier(); // the consumers' maxima of the entering state
            p_eS = state_exp_of(s_smax);
        }
        p_stage(kbeg, 0, S0{});
        p_load(kbeg + 3, S0{});
        lds_barrier();
        auto p_iter = [&](int k, auto slot_next) {
            const int s = (k - kbeg) & 1;
            p_stage(k + 1, s ^ 1, slot_next);
            p_load(k + 1 + kDepth, slot_next);
            lds_barrier();
        };
        int k0 = kbeg;
        for (; k0 + kDepth <= kend; k0 += kDepth) {
            p_iter(k0, S1{});
            p_iter(k0 + 1, S2{});
            p_iter(k0 + 2, S0{});
        }
        if (k0 < kend) p_iter(k0, S1{});
        if (k0 + 1 < kend) p_iter(k0 + 1, S2{});
        return;
    }

    // ------------------------------------------------------------ consumers
    auto consumer = [&](auto wave_c) {
        constexpr int W = decltype(wave_c)::value;
        const int own = 16 * W + r16; // token row of this lane
        // Sr[i][r] = S[p0 + 16 tpb(i) + l % 16][n = 16 tnb(i) + 4 (l / 16) + r]
        // 2^-eS for this wave's NT tiles (eS = kZeroState while the state is
        // zero; every consumer wave forms the same eS, and the producers the
        // same sequence)
        constexpr int NT = kWideTiles.n[W];
        auto tnb = [](int i) { return kWideTiles.nb[W][i]; };
        auto tpb = [](int i) { return kWideTiles.pb[W][i]; };
        // offset of tile i's four values within a [P, NS] state
        auto toff = [&](int i) { return (p0 + 16 * tpb(i) + r16) * NS + 16 * tnb(i) + 4 * kq; };
        f32x4 Sr[NT];
        int eS = kZeroState;
        // C row `own` of the next chunk (128 columns: k-steps ks = 0..3, each
        // 8 (l / 16) + 0..7 of its 32 columns), loaded one chunk ahead; past
        // the segment end an empty-range read
        float4 cr[8];
        auto c_load = [&](int k) {
            const bool real = k < kend;
            const int64_t t0 = (int64_t)(real ? k : kbeg) * T;
            const int tv = (int)min((int64_t)T, prm.L - t0);
            const auto rc = buf_rsrc_n(prm.C + (((int64_t)b * prm.L + t0) * G + g) * NS, real ? 0x7fffffff : 0);
            const int vo = (min(own, tv - 1) * G * NS + 8 * kq) * 4;
#pragma unroll
            for (int j = 0; j < 8; ++j) cr[j] = buf_load4(rc, vo + (32 * (j >> 1) + 4 * (j & 1)) * 4, 0);
        };
        // kCB: this lane's C . B^T values of the next chunk, (t = own,
        // s = 16 j + 4 (l / 16) + 0..3) for s-blocks j <= W
        float4 cbr[4];
        auto cb_load = [&](int k) {
            if (!kCB) return;
            const bool real = k < kend;
            const auto rcb = buf_rsrc_n(prm.cb + (((int64_t)b * G + g) * prm.K + (real ? k : kbeg)) * (T * T),
                                        real ? T * T * 4 : 0);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (j <= W) cbr[j] = buf_load4(rcb, (own * T + 16 * j + 4 * kq) * 4, 0);
        };
        float4 zr[2];
        auto z_load = [&](int k) {
            if (!kGate) return;
            const bool real = k < kend;
            const int64_t t0 = (int64_t)(real ? k : kbeg) * T;
            const int tv = (int)min((int64_t)T, prm.L - t0);
            const auto rz = buf_rsrc_n(prm.z + (((int64_t)b * prm.L + t0) * H + h) * P + p0, real ? 0x7fffffff : 0);
            const int vo = (min(own, tv - 1) * H * P + 4 * kq) * 4;
#pragma unroll
            for (int pb = 0; pb < 2; ++pb) zr[pb] = buf_load4(rz, vo + 64 * pb, 0);
        };
        auto write_T4 = [&](int s) {
            const SplitTile t4 = T4(opaque_lds(lds), s);
#pragma unroll
            for (int i = 0; i < NT; ++i)
                store_split4(t4, (16 * tpb(i) + r16) * kS1 + 16 * tnb(i) + 4 * kq,
                             make_float4(Sr[i][0], Sr[i][1], Sr[i][2], Sr[i][3]));
        };

        {
            const float *s0 = nullptr;
            const int64_t bh = (int64_t)b * H + h;
            if (sp.seg_in && sp.seg_in_log_decay) {
                fold_entry(Sr, sp.seg_in + bh * sp.seg_in_n * PNS, sp.seg_in_log_decay + bh * sp.seg_in_n,
                           sg * sp.in_mult, PNS, prm.init ? prm.init + bh * PNS : nullptr, toff);
            } else {
                if (sp.seg_in)
                    s0 = sp.seg_in + (bh * sp.seg_in_n + sg * sp.in_mult) * PNS;
                else if (prm.init)
                    s0 = prm.init + bh * PNS;
#pragma unroll
                for (int i = 0; i < NT; ++i) {
                    if (s0) {
                        const float4 v = *(const float4 *)(s0 + toff(i));
                        Sr[i] = f32x4{v.x, v.y, v.z, v.w};
                    } else {
                        Sr[i] = zero4();
                    }
                }
            }
            if (s0_nonzero) {
                // the entering state's largest magnitude over the four
                // consumer waves sets its scale (one more barrier, matched by
                // the producers, which read the same maxima)
                float m = 0.f;
#pragma unroll
                for (int i = 0; i < NT; ++i)
#pragma unroll
                    for (int r = 0; r < 4; ++r) m = fmaxf(m, fabsf(Sr[i][r]));
                m = wave_max(m);
                if (lane == 0) s_smax[W] = m;
                lds_barrier();
                eS = state_exp_of(s_smax);
#pragma unroll
                for (int i = 0; i < NT; ++i)
#pragma unroll
                    for (int r = 0; r < 4; ++r) Sr[i][r] = __builtin_amdgcn_ldexpf(Sr[i][r], -eS);
            }
            write_T4(0);
            c_load(kbeg);
            cb_load(kbeg);
            z_load(kbeg);
            if (W == 0 && lane < kPC) {
                const float dv = prm.has_D ? prm.D[prm.d_per_channel ? h * P + p0 + lane : hr] : 0.f;
                s_Dv[lane] = dv;
            }
        }
        lds_barrier();

        auto iter = [&](int k, auto full_c) {
            constexpr bool kFull = decltype(full_c)::value;
            const int s = (k - kbeg) & 1;
            const int64_t t0 = (int64_t)k * T;
            const int tv = (int)min((int64_t)T, prm.L - t0);
            const float cs_last = s_cs[s][T - 1];
            // scales: q by 2^-ek, the state leaving the chunk by 2^-eN, the
            // chunk's products of y by 2^-eo
            const int eN = s_tok.sexp[s];
            // kSeq: the exponents of the lane's own row; a row that does not
            // read the entering state takes no part of its scale
            const int ek = kSeq ? s_tok.qe[s][own] : s_tok.qexp[s];
            int eo = max(ek, eS - kMaxShift);
            if (kSeq && s_off[s][own] == 0.f) eo = ek;
            if (kSave) {
                float *cst = prm.chunk_states + (((int64_t)b * H + h) * prm.K + k) * PNS;
                const float f = __builtin_amdgcn_ldexpf(1.f, eS);
#pragma unroll
                for (int i = 0; i < NT; ++i)
                    *(float4 *)(cst + toff(i)) = make_float4(Sr[i][0] * f, Sr[i][1] * f, Sr[i][2] * f, Sr[i][3] * f);
            }
            Frag Cown[4];
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const float4 v0 = cr[2 * ks], v1 = cr[2 * ks + 1];
                const float vv[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
                Cown[ks] = pack_frag(vv);
            }
            float4 cbv[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) cbv[j] = kCB ? cbr[j] : make_float4(0.f, 0.f, 0.f, 0.f);
            c_load(k + 1);
            cb_load(k + 1);
            _Float16 *la = opaque_lds(lds);
            const SplitTile t1 = T1(la, s), t4 = T4(la, s);
            const float cs_own = s_cs[s][own];
            // W in the output's scale 2^-eo: q 2^-ek times 2^(ek - eo), an exact
            // shift of the exponent argument (0 unless the state outweighs the
            // chunk by 2^kMaxShift)
            const float cs_w = cs_own + (float)(ek - eo);

            // W^T tiles: C_t . B_s exp2(cs_t - cs_s) q_s, s <= t, t = own
            Frag WT[2];
            {
                float wv[2][8];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if (j > W) { // above the diagonal: zero (compile-time)
#pragma unroll
                        for (int i = 0; i < 4; ++i) wv[j >> 1][(j & 1) * 4 + i] = 0.f;
                        continue;
                    }
                    f32x4 cb = zero4();
                    if (kCB) {
                        cb = f32x4{cbv[j].x, cbv[j].y, cbv[j].z, cbv[j].w};
                    } else {
#pragma unroll
                        for (int ks = 0; ks < 4; ++ks)
                            cb = mma3f(frag_s<kS1>(t1, 16 * j + r16, ks), Cown[ks], cb);
                    }
                    if (j < W) {
                        // below the diagonal: one exponential per block (the
                        // decay from the block's last token to t)
                        const float fe = exp2_f(cs_w - s_cs[s][16 * j + 15]);
                        const float4 gv = *(const float4 *)&s_tok.gq[s][16 * j + 4 * kq];
                        const float ga[4] = {gv.x, gv.y, gv.z, gv.w};
#pragma unroll
                        for (int i = 0; i < 4; ++i) wv[j >> 1][(j & 1) * 4 + i] = cb[i] * (fe * ga[i]);
                        continue;
                    }
                    // the diagonal block: cs and q of tokens 16 j + 4 kq .. + 3
                    // read unconditionally and the causal zeros selected per
                    // lane (a conditional read becomes a divergent branch that
                    // drains every LDS read in flight)
                    const float4 csv = *(const float4 *)&s_cs[s][16 * j + 4 * kq];
                    const float4 qv = *(const float4 *)&s_q[s][16 * j + 4 * kq];
                    const float csa[4] = {csv.x, csv.y, csv.z, csv.w}, qa[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float e = exp2_f(cs_w - csa[i]) * qa[i];
                        wv[j >> 1][(j & 1) * 4 + i] = (4 * kq + i <= r16) ? cb[i] * e : 0.f;
                    }
                }
                if (kSeq && s_mixed[s]) {
                    const int sid_own = s_sid[s][own];
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int4 sv = *(const int4 *)&s_sid[s][16 * j + 4 * kq];
                        const int sva[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            if (sva[i] != sid_own) wv[j >> 1][(j & 1) * 4 + i] = 0.f;
                    }
                }
                WT[0] = pack_frag(wv[0]);
                WT[1] = pack_frag(wv[1]);
            }
            // 2^-eo y^T[p][t]: exp2(cs_t) S C_t + sum_s W[t][s] q_s x_s, p in this
            // half (S held as S 2^-eS, W built in the scale 2^-eo)
            f32x4 acc[2];
#pragma unroll
            for (int pb = 0; pb < 2; ++pb) {
                acc[pb] = zero4();
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) acc[pb] = mma3f(frag_s<kS1>(t4, 16 * pb + r16, ks), Cown[ks], acc[pb]);
            }
            const float ecs = __builtin_amdgcn_ldexpf(kSeq ? exp2_f(cs_own) * s_off[s][own] : exp2_f(cs_own),
                                                      eS - eo);
#pragma unroll
            for (int pb = 0; pb < 2; ++pb)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[pb][i] *= ecs;
            _Float16 *lb = opaque_lds(lds);
            const SplitTile t2 = T2(lb, s), t3 = T3(lb, s), t1b = T1(lb, s);
#pragma unroll
            for (int m = 0; m < 2; ++m) {
                if (2 * m <= W)
#pragma unroll
                    for (int pb = 0; pb < 2; ++pb)
                        acc[pb] = mma3f(frag_tp_s<kS2>(t2, m, 16 * pb), WT[m], acc[pb]);
            }
            {
                const float f = __builtin_amdgcn_ldexpf(1.f, eo);
#pragma unroll
                for (int pb = 0; pb < 2; ++pb)
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[pb][i] *= f;
            }
            if (kFull || own < tv) {
                const int64_t row = (((int64_t)b * prm.L + t0 + own) * H + h) * P + p0;
                // one wave-uniform branch per feature for the whole row
                f32x4 v[2] = {acc[0], acc[1]};
                if (prm.has_D) {
#pragma unroll
                    for (int pb = 0; pb < 2; ++pb) {
                        const int p = 16 * pb + 4 * kq;
                        const f32x4 xa = tile_row4_s<kS2>(t2, own, p);
                        const float4 d = *(const float4 *)&s_Dv[p];
                        v[pb][0] += d.x * xa[0];
                        v[pb][1] += d.y * xa[1];
                        v[pb][2] += d.z * xa[2];
                        v[pb][3] += d.w * xa[3];
                    }
                }
                if (prm.pre_gate) {
#pragma unroll
                    for (int pb = 0; pb < 2; ++pb)
                        *(float4 *)(prm.pre_gate + row + 16 * pb + 4 * kq) =
                            make_float4(v[pb][0], v[pb][1], v[pb][2], v[pb][3]);
                }
#pragma unroll
                for (int pb = 0; pb < 2; ++pb) {
                    if (kGate) {
                        const float4 zv = zr[pb];
                        v[pb][0] *= silu_f(zv.x);
                        v[pb][1] *= silu_f(zv.y);
                        v[pb][2] *= silu_f(zv.z);
                        v[pb][3] *= silu_f(zv.w);
                    }
                    *(float4 *)(prm.out + row + 16 * pb + 4 * kq) =
                        make_float4(v[pb][0], v[pb][1], v[pb][2], v[pb][3]);
                }
            }
            z_load(k + 1);
            // U^T[n][p] = sum_t B[t][n] (decay q x)[t][p]; S <- exp2(cs_last) S + U
            f32x4 U[NT];
#pragma unroll
            for (int i = 0; i < NT; ++i) U[i] = zero4();
#pragma unroll
            for (int m = 0; m < 2; ++m) {
                Frag f3[2];
#pragma unroll
                for (int pb = 0; pb < 2; ++pb) f3[pb] = frag_tp_s<kS2>(t3, m, 16 * pb);
                // the B operand of each n-block this wave's tiles use
                constexpr int ND = kWideTiles.nd[W];
                Frag a1[ND];
#pragma unroll
                for (int j = 0; j < ND; ++j) a1[j] = frag_tp_s<kS1>(t1b, m, 16 * kWideTiles.dnb[W][j]);
#pragma unroll
                for (int i = 0; i < NT; ++i) U[i] = mma3f(a1[kWideTiles.tix[W][i]], f3[tpb(i)], U[i]);
            }
            // S' 2^-eN = exp2(cs_last) 2^(eS - eN) (S 2^-eS) + U 2^-eN (T3's scale)
            const float alpha = __builtin_amdgcn_ldexpf(kSeq ? exp2_f(cs_last) * s_carry[s] : exp2_f(cs_last),
                                                        eS - eN);
#pragma unroll
            for (int i = 0; i < NT; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) Sr[i][r] = alpha * Sr[i][r] + U[i][r];
            eS = eN;
            write_T4(s ^ 1);
            lds_barrier(); // buffer s is free, buffer s ^ 1 and T4(s ^ 1) are complete
        };
        const int kfull = (int)min((int64_t)kend, prm.L / T);
        int k = kbeg;
        for (; k < kfull; ++k) iter(k, std::true_type{});
        if (k < kend) iter(k, std::false_type{});

        if (sp.write_final && sg == sp.nseg - 1 && prm.final_state) {
            float *dst = prm.final_state + ((int64_t)b * H + h) * PNS;
            const float f = __builtin_amdgcn_ldexpf(1.f, eS);
#pragma unroll
            for (int i = 0; i < NT; ++i)
                *(float4 *)(dst + toff(i)) = make_float4(Sr[i][0] * f, Sr[i][1] * f, Sr[i][2] * f, Sr[i][3] * f);
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
