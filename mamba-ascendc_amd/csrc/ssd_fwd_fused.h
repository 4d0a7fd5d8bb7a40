// Fused forward of the Mamba-2 SSD hot path for headdim = dstate = 64.
//
// One workgroup owns one (batch b, head h, segment) and walks the segment's
// 64-token chunks in order, carrying the 64 x 64 state S in registers, so the
// per-chunk states never go through HBM.  Per chunk (q = discretised dt,
// cs = chunk-local cumsum of A q, decay_t = exp(cs_last - cs_t)):
//
//   y_t = exp(cs_t) C_t . S + sum_{s <= t} (C_t . B_s) exp(cs_t - cs_s) q_s x_s
//         (+ D x_t, * silu(z_t))
//   S  <- exp(cs_last) S + sum_t decay_t q_t x_t (x) B_t
//
// dstate N = 128: the full pass is k_fwd_wide (ssd_fwd_wide.h); the
// state-only pass below runs two independent 64-column halves of the state
// (nsplit = 2), one workgroup each, since a state contribution splits by
// columns.
//
// Long sequences with few (b, h) streams are cut into segments so the grid
// still fills the GPU: a state-only pass (kStateOnly) computes the state
// contribution from zero and the total log decay of each pre-segment (the
// segments cut finer), and the full pass starts each segment from the state
// entering it: either folded from those contributions in its own prologue
// (fold_entry, sp.seg_in_log_decay) or, with many pre-segments, from the
// recurrence k_state_pass ran over them.  With one segment per stream the
// full pass alone does everything and needs no workspace.
//
// Exponentials are taken in the log2 domain: the chunk cumsum is formed over
// A q log2(e), so every decay factor is a single exp2 of a difference.
//
// Packed sequences (kSeq, per-token ids seq_idx): with e_k the id of chunk
// k's last token and e_{-1} = 0, C_t . B_s counts only for equal ids, token s
// enters the state only if its id is e_k >= 0, the state carries over chunk k
// only if e_k == e_{k-1}, and token t reads the state entering its chunk only
// if its id is e_{k-1} (the masks of the reference's Triton port:
// mamba_triton_ascend/mamba2/ops/triton/ssd_bmm.py:159-161,
// ssd_chunk_state.py:208-231, ssd_state_passing.py:62-72,
// ssd_chunk_scan.py:375-376).  The producers turn the ids into the three
// per-token / per-chunk factors; a segment whose state is cut reports a log
// decay of -inf, so the fold (or the segment recurrence) drops the state
// before it.
//
// Tiles (split fp16, LDS, all stored row-major in their first index), for
// the chunk being processed:
//   T1 = B [t][n]          (A operand of C.B^T, rows s)
//   T2 = x [t][p]          (A operand of y^T and B operand of U^T, both
//                           contracting over t: transposed reads; also the
//                           x of the D x term, so x is read from HBM once)
//   T3 = decay q B [t][n]  (A operand of U^T, transposed reads)
//   T4 = S [p][n]          (A operand of the C.S term)
// with q_s folded into the W^T tiles instead of into x.
// and, in registers, C_t for the lane's own token row t = 16 w + l % 16.
// Outputs are produced transposed (y^T[p][t], U^T[n][p]) so that the C.B^T
// tiles feed the next product straight from registers (see perm32; the
// transposed reads of T2 use the same k order) and S stays in the
// accumulator layout of U^T.  Producers fill the tiles from 16-byte row loads
// (nine loads per chunk and lane, so three chunks of loads stay within the
// 63 outstanding vector-memory operations a wave can track).
//
// The math is that of mamba_ascendc/csrc/ops/mamba2_ssd_fwd/design.md:10-20 and
// the chunked decomposition of mamba_torch/ssd_reference.py:113-189; the
// fusion, blocking and layouts are this file's own.
#pragma once

#include <type_traits>

#include "ssd_fwd_kernels.h"

namespace ssd {

struct SegParams {
    int nseg;              // segments per (b, h) stream
    int M;                 // chunks per segment (the last one may be shorter)
    float *seg_state;      // [B, H, nseg, P, N] segment contributions (state-only pass)
    float *seg_log_decay;  // [B, H, nseg]
    const float *seg_in;   // [B, H, seg_in_n, P, N] states at the segment-pass boundaries, or
                           // NULL; segment sg starts from entry sg * in_mult
    const float *seg_in_log_decay; // [B, H, seg_in_n] non-NULL: seg_in holds the state-only
                           // pass's contributions (from a zero state) and segment sg folds
                           // entries 0 .. sg * in_mult - 1 onto the initial states itself
    int seg_in_n, in_mult;
    int write_final;       // the last segment writes final_state
    int nsplit;            // 64-column state halves per head: 1 (N = 64) or 2 (N = 128,
                           // state-only pass; the full pass of N = 128 is k_fwd_wide)
};

constexpr int kXcds = 8; // MI355X: workgroups go round-robin over 8 XCDs

// Workgroup id -> work unit, in blocks of R consecutive units per XCD: with
// R the units of one group, the heads of a group share an XCD (consecutive
// workgroups of an XCD walk the heads of one group, so B and C of a chunk are
// read from HBM once into that XCD's L2).  Ids past the last full block of
// kXcds * R map to themselves.  With fewer units than one such block (many
// heads per group, one round), each XCD takes a contiguous run of
// total / kXcds units instead (the heads of one segment of a group, so B and
// C of a chunk reach a few XCDs' L2 rather than all eight).
__device__ __forceinline__ int xcd_unit(int id, int total, int R) {
    const int span = kXcds * R;
    if (total < span) return total % kXcds ? id : (id % kXcds) * (total / kXcds) + id / kXcds;
    const int main = (total / span) * span;
    if (id >= main) return id;
    const int x = id % kXcds, n = id / kXcds;
    return R * ((n / R) * kXcds + x) + n % R;
}

constexpr int kWsThreads = 512; // 4 producer + 4 consumer waves

// Ownership of the state in the full pass: the 16 tiles (16 x 16 blocks,
// n-block nb, p-block pb) of S, and with them the U products, the state
// update and the T4 staging, over the four consumer waves.  Wave W also forms
// the causal C.B^T blocks j <= W of its token rows, so the later waves carry
// more of the mask work; a split (c0, c1, c2, c3) other than (4, 4, 4, 4)
// hands tiles of the later waves' n-blocks to the earlier waves.  Measured
// at C3 (plain forward, one box, A/B): 4444 1.342 ms, 5533 1.335, 5542 1.329,
// 6532 1.326; at C4 0.0330 -> 0.0325 ms.  A phase-timestamp probe of one
// workgroup put wave 3's mask phase at 2.5x wave 0's and wave 0 idle at the
// barrier for a quarter of the step, but moving tiles gains far less than
// that imbalance: the waves also contend for the CU's LDS, VALU issue and
// vector-memory paths (each 20-40 % busy).  The z-gate and packed-sequence
// variants keep 4444 (6532 spills 12-24 bytes there).
struct TileMap {
    int n[4];
    int nb[4][8], pb[4][8];
};
constexpr TileMap make_tiles(int c0, int c1, int c2, int c3) {
    TileMap m{};
    const int want[4] = {c0, c1, c2, c3};
    int snb[16] = {}, spb[16] = {}, ns = 0;
    for (int w = 0; w < 4; ++w)
        for (int p = 0; p < 4; ++p) {
            if (p < want[w]) {
                m.nb[w][m.n[w]] = w;
                m.pb[w][m.n[w]] = p;
                ++m.n[w];
            } else {
                snb[ns] = w;
                spb[ns] = p;
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
    return m;
}
constexpr TileMap kTilesEven = make_tiles(4, 4, 4, 4);
constexpr TileMap kTilesShifted = make_tiles(6, 5, 3, 2);

// State entering segment sg when the segment recurrence is folded into the
// full pass (sp.seg_in_log_decay non-NULL): with U_j the contribution of
// pre-segment j (from a zero state) and ld_j its log decay,
//   S = sum_{j < J} exp(ld_{j+1} + .. + ld_{J-1}) U_j + exp(ld_0 + .. + ld_{J-1}) init,
// J = sg * in_mult, every term an independent load (no chain of dependent
// steps).  `off(i)` is the element offset of this thread's float4 i within a
// [P, N] state; U points at pre-segment 0 of the stream, init at the stream's
// initial state or NULL.
template <int kN, typename Off>
__device__ __forceinline__ void fold_entry(f32x4 (&acc)[kN], const float *U, const float *ld, int J,
                                          int64_t PNS, const float *init, Off off) {
#pragma unroll
    for (int i = 0; i < kN; ++i) acc[i] = zero4();
    float lw = 0.f; // log weight of entry j: the decays after it
#pragma unroll 2
    for (int j = J - 1; j >= 0; --j) {
        const float wj = __expf(lw);
#pragma unroll
        for (int i = 0; i < kN; ++i) {
            const float4 v = *(const float4 *)(U + j * PNS + off(i));
            acc[i][0] += wj * v.x;
            acc[i][1] += wj * v.y;
            acc[i][2] += wj * v.z;
            acc[i][3] += wj * v.w;
        }
        lw += ld[j];
    }
    if (init) {
        const float wi = __expf(lw);
#pragma unroll
        for (int i = 0; i < kN; ++i) {
            const float4 v = *(const float4 *)(init + off(i));
            acc[i][0] += wi * v.x;
            acc[i][1] += wi * v.y;
            acc[i][2] += wi * v.z;
            acc[i][3] += wi * v.w;
        }
    }
}

// kSave: also write the state entering every chunk to prm.chunk_states; with
// kStateOnly, a state pass that starts each segment from its entering state
// (sp.seg_in, or the initial states) and writes only those chunk states (the
// backward's recompute of the states it was not given).
// kGate: the z gate (prm.has_z), whose z rows the consumers prefetch a chunk ahead.
// kSeq: packed sequences (prm.seq_idx).
// kLat: the latency form of the C.S products, for grids of at most one
// workgroup per CU (each workgroup's step latency is then the kernel time).
template <bool kStateOnly, bool kSave = false, bool kGate = false, bool kSeq = false, bool kLat = false>
__global__ __launch_bounds__(kWsThreads) void k_fwd_seg(FwdParams prm, SegParams sp) {
    constexpr int T = 64, P = 64, N = 64;
    constexpr int TS = kSeq ? T : 1; // per-token sequence arrays (kSeq only)
    // stage tiles, double buffered by chunk parity s: full pass T1(s), T2(s),
    // T3(s) = tiles 3 s .. 3 s + 2 and T4(s) = tile 6 + s; state-only pass
    // T2(s), T3(s) = tiles 2 s, 2 s + 1
    constexpr int kTiles = kStateOnly ? 4 : 8;
    // full pass: T1..T3 rows kXS = 80 halves apart, T4 rows kTS = 72 apart
    // (80 for all eight would not fit in LDS).  At 80 the 16-byte operand
    // reads of T1 and the transposing reads of T2, T3 are free of LDS bank
    // conflicts (two-way at 72): C3 forward 0.9 % faster.  The state-only
    // pass keeps 72, so two of its workgroups share a CU, and so do the z
    // gate and the saving packed pass, whose registers the extra address
    // offsets crowd (the gate 1 % slower at 80; the other spilled).
    constexpr int kXS = (kStateOnly || kGate || (kSave && kSeq)) ? kTS : 80, kXTile = 64 * kXS;
    constexpr int kXTiles = kStateOnly ? 4 : 6;
    __shared__ __attribute__((aligned(16))) _Float16 lds[2 * kXTiles * kXTile + 2 * (kTiles - kXTiles) * kTile];
    // Per-token values of a chunk written by the producers' dt prologue, by
    // chunk parity; one struct, so the writing wave addresses every member
    // from one base (see the prologue).
    struct ChunkTok {
        float cs[2][T], q[2][T];
        // q_s 2^-ek exp2(cs_e - cs_s), e the last token of s's 16-token block:
        // the blocks below the diagonal take exp2(cs_t - cs_s) q_s as
        // exp2(cs_t - cs_e) times this (both factors <= 1)
        float gq[2][T];
        // kSeq: token ids, 1 where the token reads the entering state
        int sid[2][TS];
        float off[2][TS];
        float carry[2]; // kSeq: 1 where the state carries over the chunk
        int mixed[2];   // kSeq: the chunk holds more than one id (C.B^T needs the id mask)
        int qexp[2];    // ek: q holds q 2^-ek
        int qe[2][TS];  // kSeq: q of token t holds q 2^-qe[t] (ek of its id)
        int sexp[2];    // eN: T3 holds B dec q 2^-eN, the scale of the state leaving the chunk
    };
    __shared__ __attribute__((aligned(16))) ChunkTok s_tok;
    __shared__ __attribute__((aligned(16))) float s_smax[4]; // |entering state| maximum per consumer wave
    auto &s_cs = s_tok.cs, &s_q = s_tok.q;
    auto &s_sid = s_tok.sid;
    auto &s_off = s_tok.off;
    auto &s_carry = s_tok.carry;
    auto &s_mixed = s_tok.mixed;
    __shared__ __attribute__((aligned(16))) float s_Dv[P]; // D per channel (a scalar D repeated)

    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const bool producer = wave >= 4;
    const int w = wave & 3; // index of the wave within its role
    const int r16 = lane & 15, kq = lane >> 4;

    auto xtile = [&](int i) { return SplitTile{lds + (2 * i) * kXTile, lds + (2 * i + 1) * kXTile}; };
    auto T1 = [&](int s) { return xtile(3 * s); };
    auto T2 = [&](int s) { return xtile(kStateOnly ? 2 * s : 3 * s + 1); };
    auto T3 = [&](int s) { return xtile(kStateOnly ? 2 * s + 1 : 3 * s + 2); };
    auto T4 = [&](int s) { return tile_at(lds + 2 * kXTiles * kXTile, s); };

    // unit = (((b * G + g) * nseg + sg) * R + r) * nsplit + nh: the column
    // halves of a head next to each other, so the second reads the head's x
    // rows from the L2 the first filled
    const int u = xcd_unit(blockIdx.x, (int)gridDim.x, prm.R * sp.nsplit);
    const int nh = u % sp.nsplit;
    const int r = (u / sp.nsplit) % prm.R;
    const int sg = (u / (prm.R * sp.nsplit)) % sp.nseg;
    const int bg = u / (prm.R * sp.nsplit * sp.nseg);
    const int g = bg % prm.G, b = bg / prm.G;
    const int h = g * prm.R + r;
    const int H = prm.H, G = prm.G;
    // NS: dstate (row stride of B, C and of every state); this unit's
    // columns start at n0
    const int NS = N * sp.nsplit, n0 = N * nh;
    const int64_t rowHP = (int64_t)H * P, rowGN = (int64_t)G * NS;
    const int64_t PNS = (int64_t)P * NS;
    const int kbeg = sg * sp.M, kend = min(kbeg + sp.M, prm.K);

    // ------------------------------------------------------------ producer
    // A ring of kDepth register slots holds, for the next kDepth chunks, rows
    // rt + 16 j (columns c4 .. c4 + 3) of x and B and dt of token `lane`, so
    // each chunk's loads are issued kDepth iterations before it is staged.
    // Slot of chunk k: (k - kbeg) % kDepth.
    constexpr int kDepth = 3;
    const int pt = tid - 4 * kWave;
    const int rt = pt >> 4, c4 = (pt & 15) * 4;
    float4 xr[kDepth][4], br[kDepth][4];
    float dtr[kDepth];
    int p_eS = kZeroState; // exponent of the state entering the chunk being staged
    int sidr[kDepth], sprv[kDepth]; // kSeq: id of token `lane`, id of the token before the chunk
    const int rowHP4 = (int)(rowHP * 4), rowGN4 = (int)(rowGN * 4); // token strides, bytes
    int xrow_off[4], brow_off[4]; // byte offsets of rows rt + 16 j
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        xrow_off[j] = (rt + 16 * j) * rowHP4;
        brow_off[j] = (rt + 16 * j) * rowGN4;
    }
    const int hr = h / prm.hdiv, Hr = H / prm.hdiv;                      // the real head
    const int dt_off = lane * Hr * 4;                                    // dt of token `lane`, bytes
    const float Ah2 = prm.A[hr] * kLog2e;                                // A in log2 units
    const float bias = prm.dt_bias ? prm.dt_bias[hr] : 0.f;
    // Loads are issued unconditionally, so the wait counts the compiler
    // derives are exact: rows past the sequence end re-read its last row
    // (their q is 0, so they add nothing), and chunks past the segment read
    // through an empty-range resource (all zeros, no memory traffic).
    auto p_load = [&](int k, auto slot_c) {
        constexpr int sl = decltype(slot_c)::value;
        const bool real = k < kend;
        const int64_t t0 = (int64_t)(real ? k : kbeg) * T;
        const int tv = (int)min((int64_t)T, prm.L - t0);
        const int range = real ? 0x7fffffff : 0;
        const auto rx = buf_rsrc_n(prm.x + (((int64_t)b * prm.L + t0) * H + h) * P, range);
        const auto rb = buf_rsrc_n(prm.B + (((int64_t)b * prm.L + t0) * G + g) * NS + n0, range);
        // row offsets clamped to the last valid row: min of the lane's
        // precomputed offsets and the chunk's last-row offset (no per-chunk
        // multiplies)
        const int xlast = (tv - 1) * rowHP4, blast = (tv - 1) * rowGN4;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            // the backward's recompute pass (two workgroups per CU, four
            // rounds at C3) reads x non-temporally, so the B rows the group's
            // other heads read stay in L2 (2 % faster there; the segment
            // pre-passes of few streams ran 10 % slower with it)
            const int xo = min(xrow_off[j], xlast) + c4 * 4;
            xr[sl][j] = (kStateOnly && kSave) ? buf_load4_nt(rx, xo, 0) : buf_load4(rx, xo, 0);
            br[sl][j] = buf_load4(rb, min(brow_off[j], blast) + c4 * 4, 0);
        }
        const auto rdt = buf_rsrc(prm.dt + ((int64_t)b * prm.L + t0) * Hr + hr);
        dtr[sl] = buf_load(rdt, min(dt_off, (tv - 1) * Hr * 4), 0);
        if (kSeq) {
            const int32_t *si = prm.seq_idx + (int64_t)b * prm.L + t0;
            sidr[sl] = si[min(lane, tv - 1)];
            const int pv = si[t0 > 0 ? -1 : 0]; // read unconditionally, 0 before the first chunk
            sprv[sl] = t0 > 0 ? pv : 0;
        }
    };
    auto put = [&](SplitTile d, int row, float4 v) {
        half4 vh, vl;
        split4(v, vh, vl);
        *(half4 *)&d.hi[row * kXS + c4] = vh;
        *(half4 *)&d.lo[row * kXS + c4] = vl;
    };
    // discretise (lane = token), cumsum in log2 units, fill the stage tiles
    auto p_stage = [&](int k, int s, auto slot_c) {
        constexpr int sl = decltype(slot_c)::value;
        const int tv = (int)min((int64_t)T, prm.L - (int64_t)k * T); // <= 0 past the end
        float q = 0.f;
        if (lane < tv) q = discretize_dt(dtr[sl], bias, prm.softplus != 0, prm.lo, prm.hi);
        const float sq = wave_inclusive_scan(q); // prefix sums of q
        const float cs = opaque_f(Ah2 * sq);               // log2 units
        const float cs_last = readlane_f(cs, T - 1);
        int ek = chunk_q_exp(readlane_f(sq, T - 1), wave_max(fabsf(q))); // kSeq: that of the id leaving the chunk
        int ek_tok = ek; // exponent of the token's q (kSeq: that of its id)
        // every member from one base the optimizer cannot split into
        // per-array address registers
        ChunkTok *tk = opaque_lds_t(&s_tok);
        if (w == 0) tk->cs[s][lane] = cs;
        float dec = exp2_f(cs_last - cs);
        bool cut = false; // kSeq: the state does not carry over the chunk
        if (kSeq) {
            // rows past the sequence end repeat its last token's id
            const int sid = sidr[sl], e_end = __builtin_amdgcn_readlane(sid, T - 1), e_prev = sprv[sl];
            if (sid != e_end || e_end < 0) dec = 0.f; // not part of the state leaving the chunk
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
            if (!kStateOnly) tk->gq[s][lane] = exp2_f(dpp_f<0x15F>(cs) - cs) * qs;
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
        const SplitTile t1 = T1(s), t2 = T2(s), t3 = T3(s);
        // the four permutes issued back to back, ahead of every tile write:
        // one wait for all of them instead of one each
        float drs[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) drs[j] = __shfl(dec * qn, rt + 16 * j, kWave);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int row = rt + 16 * j;
            const float dr = drs[j];
            const float4 xv = xr[sl][j], bv = br[sl][j];
            put(t2, row, xv);
            put(t3, row, make_float4(bv.x * dr, bv.y * dr, bv.z * dr, bv.w * dr));
            if (!kStateOnly) put(t1, row, bv);
        }
    };

    // the entering state can be nonzero: its magnitude sets its first scale,
    // through one more barrier in both roles (wave-uniform)
    const bool s0_nonzero = (!kStateOnly || kSave) && (sp.seg_in != nullptr || prm.init != nullptr);

    // ------------------------------------------------------------ producer role
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    using S2 = std::integral_constant<int, 2>;
    static_assert(kDepth == 3, "the unrolled ring below assumes three slots");
    // The two roles run separate loops with the same number of barriers (one
    // after the prologue, one per chunk), so the compiler can give the
    // producer's load ring and the consumer's state the same registers.
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
        // stage chunk k + 1 into the other buffer while the consumers work
        // on chunk k; chunk k + 1 sits in slot (k + 1 - kbeg) % 3.  Past the
        // segment end this stages zeros that no consumer reads.
        auto p_iter = [&](int k, auto slot_next) {
            const int s = (k - kbeg) & 1;
            p_stage(k + 1, s ^ 1, slot_next);
            p_load(k + 1 + kDepth, slot_next);
            lds_barrier();
        };
        // whole rounds of the ring, then the 0..2 remaining chunks: every
        // path into the loop's back edge has issued the same loads
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

    // ------------------------------------------------------------ consumer role
    // One straight-line copy per consumer wave: with the wave index a
    // compile-time constant, the causal tile skips are static and the
    // products of a chunk form one basic block the scheduler can interleave.
    auto consumer = [&](auto wave_c) {
        constexpr int W = decltype(wave_c)::value;
        const int own = 16 * W + r16; // token row of this lane
        // state: Sr[i][r] = S[p = 16 tpb(i) + l % 16][n = 16 tnb(i) + 4 (l / 16) + r]
        // 2^-eS for this wave's NT tiles (eS = kZeroState while the state is
        // zero; every consumer wave forms the same eS, and the producers the
        // same sequence).  The state-only pass keeps n-block W.
        constexpr TileMap tm = (kGate || kSeq) ? kTilesEven : kTilesShifted;
        constexpr int NT = kStateOnly ? 4 : tm.n[W];
        auto tnb = [](int i) { return kStateOnly ? W : tm.nb[W][i]; };
        auto tpb = [](int i) { return kStateOnly ? i : tm.pb[W][i]; };
        // offset of tile i's four values within a [P, NS] state
        auto toff = [&](int i) { return (16 * tpb(i) + r16) * NS + 16 * tnb(i) + 4 * kq; };
        f32x4 Sr[NT];
        int eS = kZeroState;
        // C row `own` of the next two chunks: chunk k in cr[(k - kbeg) & 1],
        // loaded two chunks ahead
        float4 cr[2][4];
        // C row `own` of chunk k (rows past the sequence end re-read its last
        // row: they only feed outputs that are not stored); past the segment
        // end an empty-range read, so the load count per chunk is fixed
        auto c_load = [&](int k, auto slot_c) {
            constexpr int sl = decltype(slot_c)::value;
            const bool real = k < kend;
            const int64_t t0 = (int64_t)(real ? k : kbeg) * T;
            const int tv = (int)min((int64_t)T, prm.L - t0);
            const auto rc = buf_rsrc_n(prm.C + (((int64_t)b * prm.L + t0) * G + g) * NS + n0,
                                       real ? 0x7fffffff : 0);
            const int vo = (min(own, tv - 1) * G * NS + 8 * kq) * 4;
    #pragma unroll
            for (int j = 0; j < 4; ++j) cr[sl][j] = buf_load4(rc, vo + (32 * (j >> 1) + 4 * (j & 1)) * 4, 0);
        };
        using C0 = std::integral_constant<int, 0>;
        using C1 = std::integral_constant<int, 1>;
        // z of row `own` for the next chunk's gate, loaded one chunk ahead (an
        // empty-range read without z or past the segment end)
        float4 zr[4];
        auto z_load = [&](int k) {
            if (!kGate) return;
            const bool real = k < kend;
            const int64_t t0 = (int64_t)(real ? k : kbeg) * T;
            const int tv = (int)min((int64_t)T, prm.L - t0);
            const auto rz = buf_rsrc_n(prm.z + (((int64_t)b * prm.L + t0) * H + h) * P,
                                       real ? 0x7fffffff : 0);
            const int vo = (min(own, tv - 1) * H * P + 4 * kq) * 4;
    #pragma unroll
            for (int pb = 0; pb < 4; ++pb) zr[pb] = buf_load4(rz, vo + 64 * pb, 0);
        };
        auto write_T4 = [&](int s) {
            const SplitTile t4 = T4(s);
    #pragma unroll
            for (int i = 0; i < NT; ++i) {
                half4 hh, ll;
                split4(make_float4(Sr[i][0], Sr[i][1], Sr[i][2], Sr[i][3]), hh, ll);
                *(half4 *)&t4.hi[(16 * tpb(i) + r16) * kTS + 16 * tnb(i) + 4 * kq] = hh;
                *(half4 *)&t4.lo[(16 * tpb(i) + r16) * kTS + 16 * tnb(i) + 4 * kq] = ll;
            }
        };

        {
            const float *s0 = nullptr;
            const int64_t bh = (int64_t)b * H + h;
            if ((!kStateOnly || kSave) && sp.seg_in && sp.seg_in_log_decay) {
                fold_entry(Sr, sp.seg_in + bh * sp.seg_in_n * PNS + n0, sp.seg_in_log_decay + bh * sp.seg_in_n,
                           sg * sp.in_mult, PNS, prm.init ? prm.init + bh * PNS + n0 : nullptr, toff);
            } else {
                if (!kStateOnly || kSave) {
                    if (sp.seg_in)
                        s0 = sp.seg_in + (bh * sp.seg_in_n + sg * sp.in_mult) * PNS + n0;
                    else if (prm.init)
                        s0 = prm.init + bh * PNS + n0;
                }
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
            if (!kStateOnly) {
                write_T4(0);
                c_load(kbeg, C0{});
                c_load(kbeg + 1, C1{});
                z_load(kbeg);
                if (W == 0) {
                    const float dv = prm.has_D ? prm.D[prm.d_per_channel ? h * P + lane : hr] : 0.f;
                    s_Dv[lane] = dv;
                }
            }
        }
        lds_barrier();

        float log_decay_sum = 0.f;
        float seg_carry = 1.f; // kSeq: 0 once the state is cut inside the segment
        // full chunks store unconditionally (a fixed number of stores per
        // chunk keeps the C-row prefetch wait exact); only the last chunk of
        // the sequence can be partial
        auto iter = [&](int k, auto full_c, auto slot_c) {
            constexpr bool kFull = decltype(full_c)::value;
            constexpr int sl = decltype(slot_c)::value;
            const int s = (k - kbeg) & 1;
            const int64_t t0 = (int64_t)k * T;
            const int tv = (int)min((int64_t)T, prm.L - t0);
            const float cs_last = s_cs[s][T - 1];
            log_decay_sum += cs_last;
            // scales: q by 2^-ek, the state leaving the chunk by 2^-eN, the
            // chunk's products of y by 2^-eo
            const int eN = s_tok.sexp[s];
            // kSeq: the exponents of the lane's own row; a row that does not
            // read the entering state takes no part of its scale
            const int ek = kSeq ? s_tok.qe[s][own] : s_tok.qexp[s];
            int eo = max(ek, eS - kMaxShift);
            if (kSeq && s_off[s][own] == 0.f) eo = ek;
            if (kSave) {
                // saved for the backward: the state entering chunk k
                float *cst = prm.chunk_states + (((int64_t)b * H + h) * prm.K + k) * PNS + n0;
                const float f = __builtin_amdgcn_ldexpf(1.f, eS);
    #pragma unroll
                for (int i = 0; i < NT; ++i)
                    *(float4 *)(cst + toff(i)) = make_float4(Sr[i][0] * f, Sr[i][1] * f, Sr[i][2] * f, Sr[i][3] * f);
            }
            const SplitTile t2 = T2(s), t3 = T3(s);
            f32x4 U[NT];
    #pragma unroll
            for (int i = 0; i < NT; ++i) U[i] = zero4();
            if (!kStateOnly) {
                Frag Cown[2];
    #pragma unroll
                for (int ks = 0; ks < 2; ++ks) {
                    const float4 v0 = cr[sl][2 * ks], v1 = cr[sl][2 * ks + 1];
                    const float vv[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
                    Cown[ks] = pack_frag(vv);
                }
                c_load(k + 2, slot_c);
                const SplitTile t1 = T1(s), t4 = T4(s);
                const float cs_own = s_cs[s][own];
                // W in the output's scale 2^-eo: q 2^-ek times 2^(ek - eo), an
                // exact shift of the exponent argument (0 unless the state
                // outweighs the chunk by 2^kMaxShift)
                const float cs_w = cs_own + (float)(ek - eo);

                // W^T tiles: C_t . B_s exp2(cs_t - cs_s), s <= t, t = own
                Frag WT[2];
                f32x4 acc[4];
                {
                    float wv[2][8];
                    f32x4 cbs[4];
    #pragma unroll
                    for (int j = 0; j <= W; ++j) {
                        cbs[j] = zero4();
    #pragma unroll
                        for (int ks = 0; ks < 2; ++ks)
                            cbs[j] = mma3f(frag_s<kXS>(t1, 16 * j + r16, ks), Cown[ks], cbs[j]);
                    }
                    // the C.S products issued between C.B^T and the mask
                    // arithmetic, a scheduling phase of their own (C3 0.7 %
                    // faster; without this fence the scheduler interleaves
                    // them with the mask, C3 3.5 % slower)
                    __builtin_amdgcn_sched_barrier(0);
                    if constexpr (kLat) {
                        // latency form: the T4 fragments of p-block pb + 1 read
                        // while pb's products run, the order pinned by the
                        // groups below (left alone, the scheduler issues each
                        // read just before its product and waits for it).  C4
                        // (one round of 256 workgroups) 0.0327 -> 0.0312 ms; at
                        // C3 (8 rounds per CU, the CU's LDS and issue shared by
                        // the waves) 1.344 -> 1.358 ms, so many-round grids keep
                        // the serial form.  Same products in the same order.
                        Frag f4[2][2];
                        f4[0][0] = frag(t4, r16, 0);
                        f4[0][1] = frag(t4, r16, 1);
    #pragma unroll
                        for (int pb = 0; pb < 4; ++pb) {
                            if (pb < 3) {
                                f4[(pb + 1) & 1][0] = frag(t4, 16 * (pb + 1) + r16, 0);
                                f4[(pb + 1) & 1][1] = frag(t4, 16 * (pb + 1) + r16, 1);
                            }
                            acc[pb] = mma3f(f4[pb & 1][0], Cown[0], zero4());
                            acc[pb] = mma3f(f4[pb & 1][1], Cown[1], acc[pb]);
                        }
                        __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);  // reads of p-blocks 0, 1
                        __builtin_amdgcn_sched_group_barrier(0x008, 6, 0);  // products of p-block 0
                        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);  // reads of p-block 2
                        __builtin_amdgcn_sched_group_barrier(0x008, 6, 0);  // p-block 1
                        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);  // reads of p-block 3
                        __builtin_amdgcn_sched_group_barrier(0x008, 12, 0); // p-blocks 2, 3
                    } else {
    #pragma unroll
                        for (int pb = 0; pb < 4; ++pb) {
                            acc[pb] = zero4();
    #pragma unroll
                            for (int ks = 0; ks < 2; ++ks)
                                acc[pb] = mma3f(frag(t4, 16 * pb + r16, ks), Cown[ks], acc[pb]);
                        }
                    }
    #pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        if (j > W) { // above the diagonal: zero (compile-time)
    #pragma unroll
                            for (int i = 0; i < 4; ++i) wv[j >> 1][(j & 1) * 4 + i] = 0.f;
                            continue;
                        }
                        const f32x4 cb = cbs[j];
                        if (j < W) {
                            // below the diagonal: one exponential per block
                            // (the decay from the block's last token to t)
                            const float fe = exp2_f(cs_w - s_cs[s][16 * j + 15]);
                            const float4 gv = *(const float4 *)&s_tok.gq[s][16 * j + 4 * kq];
                            const float ga[4] = {gv.x, gv.y, gv.z, gv.w};
    #pragma unroll
                            for (int i = 0; i < 4; ++i) wv[j >> 1][(j & 1) * 4 + i] = cb[i] * (fe * ga[i]);
                            continue;
                        }
                        // the diagonal block: cs and q of tokens 16 j + 4 kq
                        // .. + 3, read unconditionally (two 16-byte reads),
                        // and the causal zeros selected per lane: a
                        // conditional read would become a divergent branch
                        // that drains every LDS read in flight
                        const float4 csv = *(const float4 *)&s_cs[s][16 * j + 4 * kq];
                        const float4 qv = *(const float4 *)&s_q[s][16 * j + 4 * kq];
                        const float csa[4] = {csv.x, csv.y, csv.z, csv.w}, qa[4] = {qv.x, qv.y, qv.z, qv.w};
    #pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const float e = exp2_f(cs_w - csa[i]) * qa[i];
                            wv[j >> 1][(j & 1) * 4 + i] = (4 * kq + i <= r16) ? cb[i] * e : 0.f;
                        }
                    }
                    // packed sequences: C_t . B_s only between equal ids, applied
                    // only to chunks that hold a sequence boundary (wave-uniform)
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
                // the mask chain (C.B^T, C.S, exponentials, W^T split) is
                // scheduled as a phase of its own, ahead of the W.x and U
                // products: interleaving them in one block ran the C3 forward
                // 5 % slower, this fence 1.3 % faster than a branchy mask
                __builtin_amdgcn_sched_barrier(0);
                // 2^-eo y^T[p][t]: exp2(cs_t) S C_t + sum_s W[t][s] q_s x_s (S held
                // as S 2^-eS, W built in the scale 2^-eo; acc holds S C_t)
                const float ecs = __builtin_amdgcn_ldexpf(kSeq ? exp2_f(cs_own) * s_off[s][own] : exp2_f(cs_own),
                                                          eS - eo);
    #pragma unroll
                for (int pb = 0; pb < 4; ++pb)
    #pragma unroll
                    for (int i = 0; i < 4; ++i) acc[pb][i] *= ecs;
                // each x fragment feeds both y^T (W part) and U^T; the
                // decayed-B fragment of every n-block this wave's tiles use
    #pragma unroll
                for (int m = 0; m < 2; ++m) {
                    Frag a3[4];
    #pragma unroll
                    for (int i = 0; i < NT; ++i) a3[tnb(i)] = frag_tp_s<kXS>(t3, m, 16 * tnb(i));
    #pragma unroll
                    for (int pb = 0; pb < 4; ++pb) {
                        const Frag f2 = frag_tp_s<kXS>(t2, m, 16 * pb);
                        if (2 * m <= W) acc[pb] = mma3f(f2, WT[m], acc[pb]);
    #pragma unroll
                        for (int i = 0; i < NT; ++i)
                            if (tpb(i) == pb) U[i] = mma3f(a3[tnb(i)], f2, U[i]);
                    }
                }
                {
                    const float f = __builtin_amdgcn_ldexpf(1.f, eo);
    #pragma unroll
                    for (int pb = 0; pb < 4; ++pb)
    #pragma unroll
                        for (int i = 0; i < 4; ++i) acc[pb][i] *= f;
                }
                if (kFull || own < tv) {
                    const int64_t row = (((int64_t)b * prm.L + t0 + own) * H + h) * P;
                    // one wave-uniform branch per feature for the whole row
                    // (not one per 16-channel block, which splits the step
                    // into small blocks the scheduler cannot overlap)
                    f32x4 v[4];
    #pragma unroll
                    for (int pb = 0; pb < 4; ++pb) v[pb] = acc[pb];
                    if (prm.has_D) {
    #pragma unroll
                        for (int pb = 0; pb < 4; ++pb) {
                            const int p = 16 * pb + 4 * kq;
                            const f32x4 xa = tile_row4_s<kXS>(t2, own, p); // x from the staged tile
                            const float4 d = *(const float4 *)&s_Dv[p];
                            v[pb][0] += d.x * xa[0];
                            v[pb][1] += d.y * xa[1];
                            v[pb][2] += d.z * xa[2];
                            v[pb][3] += d.w * xa[3];
                        }
                    }
                    if (prm.pre_gate) {
    #pragma unroll
                        for (int pb = 0; pb < 4; ++pb)
                            *(float4 *)(prm.pre_gate + row + 16 * pb + 4 * kq) =
                                make_float4(v[pb][0], v[pb][1], v[pb][2], v[pb][3]);
                    }
    #pragma unroll
                    for (int pb = 0; pb < 4; ++pb) {
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
            }
            // S <- exp2(cs_last) S + U, U^T[n][p] = T3 x T2 (the full pass forms
            // U together with y)
            {
                if (kStateOnly) {
    #pragma unroll
                    for (int m = 0; m < 2; ++m) {
                        const Frag a3 = frag_tp_s<kXS>(t3, m, 16 * W);
    #pragma unroll
                        for (int i = 0; i < NT; ++i) U[i] = mma3f(a3, frag_tp_s<kXS>(t2, m, 16 * tpb(i)), U[i]);
                    }
                }
                // S' 2^-eN = exp2(cs_last) 2^(eS - eN) (S 2^-eS) + U 2^-eN (T3's scale)
                const float alpha = __builtin_amdgcn_ldexpf(kSeq ? exp2_f(cs_last) * s_carry[s] : exp2_f(cs_last),
                                                            eS - eN);
                if (kSeq) seg_carry *= s_carry[s];
    #pragma unroll
                for (int i = 0; i < NT; ++i)
    #pragma unroll
                    for (int r = 0; r < 4; ++r) Sr[i][r] = alpha * Sr[i][r] + U[i][r];
                eS = eN;
            }
            if (!kStateOnly) write_T4(s ^ 1);
            lds_barrier(); // buffer s is free, buffer s ^ 1 and T4(s ^ 1) are complete
        };
        const int kfull = (int)min((int64_t)kend, prm.L / T);
        int k = kbeg;
        for (; k + 2 <= kfull; k += 2) {
            iter(k, std::true_type{}, C0{});
            iter(k + 1, std::true_type{}, C1{});
        }
        if (k < kfull) {
            iter(k, std::true_type{}, C0{});
            if (k + 1 < kend) iter(k + 1, std::false_type{}, C1{});
        } else if (k < kend) {
            iter(k, std::false_type{}, C0{});
        }

        float *dst = nullptr;
        if (kStateOnly && !kSave) {
            const int64_t si = ((int64_t)b * H + h) * sp.nseg + sg;
            dst = sp.seg_state + si * PNS + n0;
            // natural units; -inf (a factor of 0) where the state was cut
            if (tid == 0 && nh == 0)
                sp.seg_log_decay[si] = seg_carry > 0.f ? log_decay_sum * kLn2 : -INFINITY;
        } else if (sp.write_final && sg == sp.nseg - 1 && prm.final_state) {
            dst = prm.final_state + ((int64_t)b * H + h) * PNS + n0;
        }
        if (dst) {
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
