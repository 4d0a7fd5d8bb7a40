// Device helpers shared by the Mamba-2 SSD kernels (gfx950 / CDNA4).
//
// Precision scheme of the forward kernels: every contraction runs on the
// fp16 matrix cores with fp32 accumulation, but each fp32 operand v is carried
// as an unevaluated sum hi + lo of two fp16 values (hi = fp16(v),
// lo = fp16(v - hi), see split2), and a product is formed from three MFMAs:
// hi*hi + hi*lo + lo*hi.  This keeps about 21 bits of operand precision, which
// is what the fp32 contract needs: one fp16 product per contraction misses the
// 2e-2 max-abs bound by 3-10x on the BASELINE shapes (outputs in the hundreds),
// one bf16 product by 25-90x.  The backward kernels split into bf16 instead
// (ssd_bf16.h): their operands scale with the upstream gradient, which a
// mean-reduced loss makes smaller than fp16's normal range.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ssd {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// One 16x16x32 fp16 MFMA: D = A(16x32) * B(32x16) + C.
// Operand lane layout: lane l supplies row (A) / column (B) l % 16 and eight
// consecutive k values of group l / 16.  Only the row/column assignment and
// the output layout matter for correctness: A and B share the k assignment,
// so any fixed permutation of k applied to both leaves the product unchanged.
// Output: acc[r] of lane l holds D[4 * (l / 16) + r][l % 16].
__device__ __forceinline__ f32x4 mfma16(half8 a, half8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Split-precision product accumulate: (ah + al)(bh + bl) without the al*bl term.
__device__ __forceinline__ f32x4 mma3(half8 ah, half8 al, half8 bh, half8 bl, f32x4 c) {
    c = mfma16(al, bh, c);
    c = mfma16(ah, bl, c);
    c = mfma16(ah, bh, c);
    return c;
}

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

// Split two fp32 values into fp16 (hi, lo) pairs with hi + lo ~= v.
// hi comes from ONE packed conversion (round toward zero) and lo is formed
// against that very register.  Writing hi = (_Float16)v; lo = v - (float)hi
// lets the compiler convert v twice (a packed v_cvt_pk_f16_f32 for the stored
// hi, a scalar v_cvt_f16_f32 for the subtraction); on a rounding tie the two
// disagree and hi + lo is off by one fp16 ulp.  With hi truncated, |lo| <
// ulp16(v) and the pair keeps about 21 significant bits.
// lo = fp16(v - hi) is one mixed-precision FMA per value (fp16 hi and fp32 v
// in, fp16 out, round to nearest even): v - hi is exact in fp32, so the
// result equals converting that difference, in half the instructions of
// convert-back, subtract and convert.  The compiler does not form these
// itself, and it cannot see the register writes inside an asm block when it
// spaces dependent instructions: kMfma ends the block with the two wait states
// an MFMA reading a VALU result needs (the s_nop 1 the compiler puts between
// its own conversions and such an MFMA), for operands packed straight into an
// MFMA; values bound for LDS need none.
template <bool kMfma = false>
__device__ __forceinline__ void split2(float a, float b, half2v &hi, half2v &lo) {
    const uint32_t h = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(a, b));
    uint32_t l;
    if (kMfma)
        asm("v_fma_mixlo_f16 %0, -%1, 1.0, %2 op_sel_hi:[1,0,0]\n\t"
            "v_fma_mixhi_f16 %0, -%1, 1.0, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
            "s_nop 1"
            : "=&v"(l)
            : "v"(h), "v"(a), "v"(b));
    else
        asm("v_fma_mixlo_f16 %0, -%1, 1.0, %2 op_sel_hi:[1,0,0]\n\t"
            "v_fma_mixhi_f16 %0, -%1, 1.0, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
            : "=&v"(l)
            : "v"(h), "v"(a), "v"(b));
    hi = __builtin_bit_cast(half2v, h);
    lo = __builtin_bit_cast(half2v, l);
}

__device__ __forceinline__ void split_f16(float v, _Float16 &hi, _Float16 &lo) {
    half2v h, l;
    split2(v, 0.f, h, l);
    hi = h[0];
    lo = l[0];
}

__device__ __forceinline__ void split4(float4 v, half4 &hi, half4 &lo) {
    half2v h0, l0, h1, l1;
    split2(v.x, v.y, h0, l0);
    split2(v.z, v.w, h1, l1);
    hi = half4{h0[0], h0[1], h1[0], h1[1]};
    lo = half4{l0[0], l0[1], l1[0], l1[1]};
}

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// 2^v on the transcendental unit (one v_exp_f32, about 1 ulp).
__device__ __forceinline__ float exp2_f(float v) { return __builtin_amdgcn_exp2f(v); }

// 1 / v on the transcendental unit (v_rcp_f32, about 1 ulp).
__device__ __forceinline__ float rcp_f(float v) { return __builtin_amdgcn_rcpf(v); }

// torch.nn.functional.softplus with beta = 1, threshold = 20, as
// max(u, 0) + ln(1 + e) with e = e^-|u|, using hardware exp2/log2: a handful
// of instructions instead of the libm expf/log1pf chains.  ln(1 + e) is
// evaluated as log1p: with w = fl(1 + e), ln(w) * e / (w - 1) (w - 1 is exact)
// cancels the rounding of w, and where w rounds to 1 the term is e itself, so
// a very negative u keeps its relative accuracy (softplus(-20) = 2.06e-9, not 0).
__device__ __forceinline__ float softplus_f(float u) {
    if (u > 20.f) return u;
    const float e = exp2_f(-fabsf(u) * kLog2e);
    const float w = 1.f + e;
    const float l = w == 1.f ? e : kLn2 * __builtin_amdgcn_logf(w) * (e * rcp_f(w - 1.f));
    return fmaxf(u, 0.f) + l;
}

__device__ __forceinline__ float sigmoid_f(float v) { return rcp_f(1.f + exp2_f(-v * kLog2e)); }

// q = clamp(softplus(dt + bias) or dt + bias, lo, hi)
__device__ __forceinline__ float discretize_dt(float dt, float bias, bool softplus, float lo,
                                               float hi) {
    float u = dt + bias;
    float pre = softplus ? softplus_f(u) : u;
    return fminf(fmaxf(pre, lo), hi);
}

// d q / d dt for the same chain (the clamp passes the gradient on its closed
// interval, softplus contributes sigmoid(u)).
__device__ __forceinline__ float discretize_grad(float dt, float bias, bool softplus, float lo,
                                                 float hi) {
    float u = dt + bias;
    float pre = softplus ? softplus_f(u) : u;
    float g = (pre >= lo && pre <= hi) ? 1.f : 0.f;
    if (softplus) g *= sigmoid_f(u);
    return g;
}

__device__ __forceinline__ float silu_f(float z) { return z * sigmoid_f(z); }

// Lane shift / broadcast of a wave through DPP (register crossbar, no LDS
// round trip); lanes without a source, or outside row_mask, read 0.
template <int kCtrl, int kRowMask = 0xf>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl,
                                                                 kRowMask, 0xf, false));
}

// Inclusive prefix sum across the 64 lanes of a wave: Hillis-Steele within
// each row of 16 lanes (row_shr 1, 2, 4, 8), then the row totals are carried
// with row_bcast:15 (rows 1, 3) and row_bcast:31 (rows 2, 3).
__device__ __forceinline__ float wave_inclusive_scan(float v) {
    v += dpp_f<0x111>(v);
    v += dpp_f<0x112>(v);
    v += dpp_f<0x114>(v);
    v += dpp_f<0x118>(v);
    v += dpp_f<0x142, 0xa>(v);
    v += dpp_f<0x143, 0xc>(v);
    return v;
}

// v of lane l ^ 16 and of lane l ^ 32, through the gfx950 lane-swap
// instructions (v_permlane16_swap / v_permlane32_swap exchange odd and even
// 16-lane rows / the two 32-lane halves of two registers).  Swapping a
// register with itself leaves, in every lane, its own value in one result
// and its partner's in the other; the partner's is the one whose bits differ
// (if they are equal, either is right), which does not depend on which
// result receives which rows.
__device__ __forceinline__ float xor16_f(float v) {
    const unsigned u = __builtin_bit_cast(unsigned, v);
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return __builtin_bit_cast(float, r[0] == u ? r[1] : r[0]);
}
__device__ __forceinline__ float xor32_f(float v) {
    const unsigned u = __builtin_bit_cast(unsigned, v);
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __builtin_bit_cast(float, r[0] == u ? r[1] : r[0]);
}
// v[l] + v[l ^ 16] (resp. ^ 32): addition commutes, so both lanes of a pair
// form the same sum.  (The two results of the swap are not used directly:
// when both operands are one value the compiler may give the instruction a
// single register, which then holds the partner's value in both results.)
__device__ __forceinline__ float add_xor16(float v) { return v + xor16_f(v); }
__device__ __forceinline__ float add_xor32(float v) { return v + xor32_f(v); }

// Sum over the 16 lanes of each row (DPP quad_perm [1,0,3,2], [2,3,0,1],
// row_half_mirror, row_mirror); every lane of the row gets the sum.
__device__ __forceinline__ float sum16(float v) {
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    v += dpp_f<0x141>(v);
    v += dpp_f<0x140>(v);
    return v;
}

// Sum over the 4 lanes that share l % 16.
__device__ __forceinline__ float sum_kq(float v) { return add_xor32(add_xor16(v)); }

// Sum over the 64 lanes, in every lane.
__device__ __forceinline__ float wave_sum(float v) { return sum_kq(sum16(v)); }

// Maximum over the 64 lanes, in every lane (the pattern of wave_sum).
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    v = fmaxf(v, dpp_f<0x140>(v));
    v = fmaxf(v, xor16_f(v));
    return fmaxf(v, xor32_f(v));
}

// Binary exponent e of v = m 2^e, m in [1, 2), clamped to [-126, 126]:
// 2^-e scales v into [1, 2), and 2^e and 2^-e are finite.  v = 0 gives -1
// (frexp's exponent of zero is 0); callers that can see a zero either do not
// care (any scale holds zero exactly) or test for it first.
__device__ __forceinline__ int scale_exp(float v) {
    return min(max(__builtin_amdgcn_frexp_expf(v) - 1, -126), 126);
}

// Power-of-two scales of the fused forwards' split-fp16 operands.  q enters
// W and the state update, and the state scales with it, so for tiny q
// (softplus of a very negative dt) those operands would fall into fp16's
// subnormal range and lose their low bits.  A chunk's q is scaled by 2^-ek
// with its sum in [8, 16) (mean in [1/8, 1/4)), unless that would lift its
// largest |q| to 1 or more: then ek puts the largest |q| in [1/2, 1).  Every
// scaled |q| is therefore below 1, so a scaled operand (x or B times the
// decayed, scaled q) never exceeds the magnitude of the raw x or B row that
// fp16 must already hold (a chunk dominated by one token would otherwise lift
// it to nearly 16 and overflow fp16 at |x| of a few thousand).  The state
// leaving the chunk is held as S 2^-eN:
//   eN = ek                                  where the state is cut (packed sequences),
//   eN = min(max(ek, eS + floor(cs_last)), 126)  otherwise,
// with eS the exponent of the state entering the chunk and cs_last its log2
// decay, since |S'| <= 2^(eS + cs_last) |S 2^-eS| + 2^ek |U 2^-ek|.  All
// scales are exact powers of two and none raises an operand above its raw
// magnitude, so they change results only where fp16 would have lost bits
// (tiny q lifted out of the subnormal range) or overflowed.
__device__ __forceinline__ int chunk_q_exp(float q_sum, float q_max) {
    return max(max(scale_exp(q_sum) - 3, scale_exp(q_max) + 1), -126);
}
__device__ __forceinline__ int next_state_exp(int eS, int ek, float cs_last, bool cut) {
    return cut ? ek : min(max(ek, eS + (int)floorf(fmaxf(cs_last, -512.f))), 126);
}
// Packed sequences: a chunk that holds several ids scales each id's tokens
// by its own sum (the sequences need not share a magnitude of q), so every
// token of one id gets the same exponent, chunk_q_exp of the q sum and the
// largest q over the chunk's tokens of that id.  One pass per distinct id (wave-uniform); the
// loop starts from the active lanes, so it ends whatever the exec mask.
__device__ __forceinline__ int id_q_exp(int sid, float q) {
    int e = 0;
    uint64_t left = __ballot(1);
    while (left) {
        const int id = __builtin_amdgcn_readlane(sid, __builtin_ctzll(left));
        const bool mine = sid == id;
        const float sum = wave_sum(mine ? q : 0.f), top = wave_max(mine ? fabsf(q) : 0.f);
        if (mine) e = chunk_q_exp(sum, top);
        left &= ~__ballot(mine);
    }
    return e;
}

// Exponent of a state known to be zero (any scale holds it exactly; far
// below every exponent the rules above produce).
constexpr int kZeroState = -1000;

// Exponent of a state from the largest magnitudes its four consumer waves
// hold (an LDS array of four floats).
__device__ __forceinline__ int state_exp_of(const float *wave_max4) {
    const float4 m4 = *(const float4 *)wave_max4;
    const float m = fmaxf(fmaxf(m4.x, m4.y), fmaxf(m4.z, m4.w));
    return m > 0.f ? scale_exp(m) : kZeroState;
}
// A chunk's products are formed in the state's scale when the state
// outweighs them by more than 2^kMaxShift (they then hold below 2^-kMaxShift
// of the output).
constexpr int kMaxShift = 60;

// v of lane 63 - l (row_mirror within the row, then the row order reversed).
__device__ __forceinline__ float reverse_lanes(float v) {
    return xor32_f(xor16_f(dpp_f<0x140>(v)));
}

// Suffix (reverse inclusive) sum across the 64 lanes of a wave.
__device__ __forceinline__ float wave_suffix_scan(float v) {
    return reverse_lanes(wave_inclusive_scan(reverse_lanes(v)));
}

// Position of token s (0..31 inside a 32-token slab) in the k-permuted operand
// order produced by taking C*B^T from MFMA output tiles: output lane group j
// holds rows 4j..4j+3 of two consecutive 16-row tiles, which become k slots
// 8j..8j+3 and 8j+4..8j+7 of the next product.
__device__ __forceinline__ int perm32(int s) {
    return 8 * ((s & 15) >> 2) + 4 * (s >> 4) + (s & 3);
}

// Inverse of perm32 over a whole 64-slot row: the token stored at slot `pos`.
__device__ __forceinline__ int perm_token(int pos) {
    const int m = pos >> 5, j = (pos >> 3) & 3, i = pos & 7;
    return 32 * m + (i < 4 ? 4 * j + i : 16 + 4 * j + (i - 4));
}

// ---------------------------------------------------------------------------
// 64 x 64 split tiles in LDS.  A tile is two arrays (hi, lo) of 64 rows with a
// padded row stride of kTS halves; operand reads are 16-byte half8 loads of
// row r16 at column 32 * ks + 8 * kq, the MFMA operand layout above.
// ---------------------------------------------------------------------------
constexpr int kTS = 72;           // row stride (halves): 64 + 8 of padding
constexpr int kTile = 64 * kTS;   // halves per array

struct SplitTile {
    _Float16 *hi, *lo;
};

__device__ __forceinline__ SplitTile tile_at(_Float16 *base, int i) {
    return SplitTile{base + (2 * i) * kTile, base + (2 * i + 1) * kTile};
}

// Column-major staging: tile[c][slot] = f(t, c) with t = the token of `slot`
// (perm_token order when PERM, else slot itself).  Thread c = tid % 64 reads
// one column, so for each token the 64 lanes of a wave read 64 consecutive
// floats of a row.
template <bool PERM, class F>
__device__ __forceinline__ void stage_cols(SplitTile d, F f) {
    const int c = threadIdx.x & 63, tb = threadIdx.x >> 6;
#pragma unroll
    for (int run = tb; run < 8; run += 4) {
        half8 vh, vl;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int slot = run * 8 + i;
            const int t = PERM ? perm_token(slot) : slot;
            _Float16 a, b;
            split_f16(f(t, c), a, b);
            vh[i] = a;
            vl[i] = b;
        }
        *(half8 *)&d.hi[c * kTS + run * 8] = vh;
        *(half8 *)&d.lo[c * kTS + run * 8] = vl;
    }
}

// Operand fragment of row `row`, k-step ks (32 columns) from a split tile.
struct Frag {
    half8 h, l;
};

// Row `row`, k-step ks of a split tile with a row stride of kS halves (the
// 64-wide tiles use kTS; wider or narrower tiles pass their own stride).
template <int kS>
__device__ __forceinline__ Frag frag_s(SplitTile s, int row, int ks) {
    const int kq = (threadIdx.x & 63) >> 4;
    Frag f;
    f.h = *(const half8 *)&s.hi[row * kS + ks * 32 + kq * 8];
    f.l = *(const half8 *)&s.lo[row * kS + ks * 32 + kq * 8];
    return f;
}

__device__ __forceinline__ Frag frag(SplitTile s, int row, int ks) { return frag_s<kTS>(s, row, ks); }

__device__ __forceinline__ f32x4 mma3f(Frag a, Frag b, f32x4 c) { return mma3(a.h, a.l, b.h, b.l, c); }

// Pack eight fp32 values into a split operand fragment.
__device__ __forceinline__ Frag pack_frag(const float (&v)[8]) {
    Frag f;
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
        half2v h, l;
        split2<true>(v[i], v[i + 1], h, l);
        f.h[i] = h[0];
        f.h[i + 1] = h[1];
        f.l[i] = l[0];
        f.l[i + 1] = l[1];
    }
    return f;
}

__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

// ds_read_b64_tr_b16 on a split-tile array stored with the contraction index
// along rows (tile[k][c]).  Each 16-lane group names rows k0..k0+3 (k0 may
// differ between groups); lane l receives tile[k0 + e][c0 + l % 16], e = 0..3.
template <int kS>
__device__ __forceinline__ half4 tr4_s(const _Float16 *arr, int k0, int c0) {
    const int m = threadIdx.x & 15;
    typedef short v4s __attribute__((ext_vector_type(4)));
    auto p = (__attribute__((address_space(3))) v4s *)(arr + (k0 + (m >> 2)) * kS + c0 + 4 * (m & 3));
    return __builtin_bit_cast(half4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(p));
}

__device__ __forceinline__ half4 tr4(const _Float16 *arr, int k0, int c0) { return tr4_s<kTS>(arr, k0, c0); }

// The LDS array base as a value the optimizer cannot see through.  Tiles
// past the first 64 KB of LDS cannot use the 16-bit immediate offset of the
// ds instructions, so every (array, row, k-step) address there becomes a
// register of its own; derived from this base, those addresses are formed
// next to their use in each phase instead of being hoisted out of the step
// loop and held (spilled) for its whole length.
__device__ __forceinline__ _Float16 *opaque_lds(_Float16 *p) {
    typedef __attribute__((address_space(3))) _Float16 *lptr;
    uint32_t a = (uint32_t)(uintptr_t)(lptr)p;
    asm volatile("" : "+s"(a));
    return (_Float16 *)(lptr)(uintptr_t)a;
}

// v as a value the optimizer cannot see through: the product that forms it is
// rounded once, and no later difference is contracted with it into an FMA.
// The forward kernels form the chunk cumsum this way, so the per-token values
// derived from it (decays, scales) get the same bits in every kernel that
// forms them, whatever each kernel's other uses of the cumsum let the
// compiler fuse.
__device__ __forceinline__ float opaque_f(float v) {
    asm volatile("" : "+v"(v));
    return v;
}

// The same for any LDS object (a struct of small arrays, say).
template <class X>
__device__ __forceinline__ X *opaque_lds_t(X *p) {
    typedef __attribute__((address_space(3))) X *lptr;
    uint32_t a = (uint32_t)(uintptr_t)(lptr)p;
    asm volatile("" : "+s"(a));
    return (X *)(lptr)(uintptr_t)a;
}

__device__ __forceinline__ half8 cat8(half4 a, half4 b) {
    return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Operand of columns c0 .. c0 + 15 contracting over the tile's rows in
// natural order (k = 32 ks + 8 (l / 16) + 0..7).
__device__ __forceinline__ Frag frag_tn(SplitTile s, int ks, int c0) {
    const int k0 = 32 * ks + 8 * ((threadIdx.x & 63) >> 4);
    Frag f;
    f.h = cat8(tr4(s.hi, k0, c0), tr4(s.hi, k0 + 4, c0));
    f.l = cat8(tr4(s.lo, k0, c0), tr4(s.lo, k0 + 4, c0));
    return f;
}

// The same in the k order of operands taken from MFMA outputs (perm32):
// slots 0..3 are rows 32 m + 4 (l / 16) + 0..3, slots 4..7 rows 32 m + 16 + ...
template <int kS>
__device__ __forceinline__ Frag frag_tp_s(SplitTile s, int m, int c0) {
    const int k0 = 32 * m + 4 * ((threadIdx.x & 63) >> 4);
    Frag f;
    f.h = cat8(tr4_s<kS>(s.hi, k0, c0), tr4_s<kS>(s.hi, k0 + 16, c0));
    f.l = cat8(tr4_s<kS>(s.lo, k0, c0), tr4_s<kS>(s.lo, k0 + 16, c0));
    return f;
}

__device__ __forceinline__ Frag frag_tp(SplitTile s, int m, int c0) { return frag_tp_s<kTS>(s, m, c0); }

// fp32 hi + lo of four split values: one mixed-precision FMA each
// (hi * 1 + lo with both fp16 operands widened, exact, rounded once to fp32),
// instead of two conversions and an add.  Its results feed VALU arithmetic
// only (an MFMA or DPP reader would need the wait states split2<true> adds).
__device__ __forceinline__ f32x4 join4(half4 h, half4 l) {
    typedef uint32_t u2 __attribute__((ext_vector_type(2)));
    const u2 hb = __builtin_bit_cast(u2, h), lb = __builtin_bit_cast(u2, l);
    float a, b, c, d;
    asm("v_fma_mix_f32 %0, %4, 1.0, %6 op_sel_hi:[1,0,1]\n\t"
        "v_fma_mix_f32 %1, %4, 1.0, %6 op_sel:[1,0,1] op_sel_hi:[1,0,1]\n\t"
        "v_fma_mix_f32 %2, %5, 1.0, %7 op_sel_hi:[1,0,1]\n\t"
        "v_fma_mix_f32 %3, %5, 1.0, %7 op_sel:[1,0,1] op_sel_hi:[1,0,1]"
        : "=&v"(a), "=&v"(b), "=&v"(c), "=&v"(d)
        : "v"(hb[0]), "v"(hb[1]), "v"(lb[0]), "v"(lb[1]));
    return f32x4{a, b, c, d};
}

// fp32 values of tile[row][c0 .. c0 + 3] (one 8-byte read of each half).
template <int kS>
__device__ __forceinline__ f32x4 tile_row4_s(SplitTile s, int row, int c0) {
    return join4(*(const half4 *)&s.hi[row * kS + c0], *(const half4 *)&s.lo[row * kS + c0]);
}

__device__ __forceinline__ f32x4 tile_row4(SplitTile s, int row, int c0) { return tile_row4_s<kTS>(s, row, c0); }

// tile[idx .. idx + 3] = v (both halves)
__device__ __forceinline__ void store_split4(SplitTile d, int idx, float4 v) {
    half4 vh, vl;
    split4(v, vh, vl);
    *(half4 *)&d.hi[idx] = vh;
    *(half4 *)&d.lo[idx] = vl;
}

// Value of v in lane `lane` (which must be the same for the whole wave).
__device__ __forceinline__ float readlane_f(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Workgroup barrier that orders LDS accesses only.  __syncthreads() also
// waits for every outstanding global load of the wave, which would stall on
// a prefetch issued just before it; this one leaves such loads in flight.
// Use it only where the workgroup shares data through LDS alone.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Raw buffer resource over `p` (gfx9 descriptor: no stride, no swizzle,
// 32-bit data format).  Loads through it take a per-lane byte offset in a
// VGPR and a wave-uniform byte offset in an SGPR, so a column of a tile
// costs one VGPR offset instead of a 64-bit address per element.  Range
// checking is not relied on: callers guard every access themselves.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void *p) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, 0x7fffffff,
                                             0x00020000);
}

// The same with a byte range: a load whose offset lies outside [0, nbytes)
// returns 0 without touching memory.  nbytes = 0 gives a resource every load
// of which returns 0, used to issue a fixed number of loads per pipeline step
// past the end of a run (the wait counts then stay exact).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc_n(const void *p, int nbytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, nbytes, 0x00020000);
}

// The builtin returns the raw 32 bits (unsigned); reinterpret, do not convert.
__device__ __forceinline__ float buf_load(__amdgpu_buffer_rsrc_t r, int lane_bytes, int uniform_bytes) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, lane_bytes, uniform_bytes, 0));
}

__device__ __forceinline__ void buf_store(__amdgpu_buffer_rsrc_t r, int lane_bytes, int uniform_bytes, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), r, lane_bytes, uniform_bytes, 0);
}

__device__ __forceinline__ float4 buf_load4(__amdgpu_buffer_rsrc_t r, int lane_bytes, int uniform_bytes) {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, lane_bytes, uniform_bytes, 0));
}

// The same marked non-temporal (cache-policy bit nt): data read once, which
// should not displace lines other workgroups still read from L2.
__device__ __forceinline__ float4 buf_load4_nt(__amdgpu_buffer_rsrc_t r, int lane_bytes, int uniform_bytes) {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, lane_bytes, uniform_bytes, 2));
}

// The wave index as a wave-uniform (scalar) value.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

}  // namespace ssd
