// Split-bf16 operands of the backward kernels (namespace ssd::bwd).
//
// The backward's operands scale with the upstream gradient, and for a
// mean-reduced loss that is O(1 / numel): about 1e-7 per element at
// [8,4096,256,64].  fp16's 5-bit exponent cannot hold such values (its normal
// range starts at 6.1e-5 and its subnormals stop at 6e-8), so a split-fp16
// product of them keeps only a few bits.  Here every fp32 operand v is carried
// as hi + lo with hi = bf16(v) and lo = bf16(v - hi), both rounded to nearest
// even by v_cvt_pk_bf16_f32 (v - hi is exact in fp32): about 17 significant
// bits over the whole fp32 exponent range.  A product is hi*hi + hi*lo +
// lo*hi on the bf16 matrix cores (v_mfma_f32_16x16x32_bf16, the rate of the
// fp16 one), fp32 accumulate.
//
// The tile layouts, operand fragments and lane mappings are those of the split
// fp16 tiles in ssd_device.h (16-bit elements, kTS-element rows, the same
// transposing LDS read); only the element type and the conversions differ.  The
// backward kernels are declared inside this namespace, so their SplitTile,
// Frag, frag, pack_frag, ... are these.
#pragma once

#include "ssd_device.h"

namespace ssd {
namespace bwd {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// (ah + al)(bh + bl) without the al*bl term
__device__ __forceinline__ f32x4 mma3(bf16x8 ah, bf16x8 al, bf16x8 bh, bf16x8 bl, f32x4 c) {
    c = mfma16(al, bh, c);
    c = mfma16(ah, bl, c);
    c = mfma16(ah, bh, c);
    return c;
}

// fp32 value of the bf16 in the low / high half of a packed pair
__device__ __forceinline__ float bf_lo_f32(uint32_t pair) { return __builtin_bit_cast(float, pair << 16); }
__device__ __forceinline__ float bf_hi_f32(uint32_t pair) { return __builtin_bit_cast(float, pair & 0xffff0000u); }

// Split two fp32 values into bf16 (hi, lo) pairs with hi + lo ~= v.
__device__ __forceinline__ void split2(float a, float b, bf16x2 &hi, bf16x2 &lo) {
    const f32x2 v = {a, b};
    hi = __builtin_convertvector(v, bf16x2);
    const uint32_t hb = __builtin_bit_cast(uint32_t, hi);
    const f32x2 r = {a - bf_lo_f32(hb), b - bf_hi_f32(hb)};
    lo = __builtin_convertvector(r, bf16x2);
}

__device__ __forceinline__ void split4(float4 v, bf16x4 &hi, bf16x4 &lo) {
    bf16x2 h0, l0, h1, l1;
    split2(v.x, v.y, h0, l0);
    split2(v.z, v.w, h1, l1);
    hi = bf16x4{h0[0], h0[1], h1[0], h1[1]};
    lo = bf16x4{l0[0], l0[1], l1[0], l1[1]};
}

// A split tile whose rows are stored interleaved (kIl, see trow) or in order;
// every accessor below takes the row order from the tile's type, so the
// writers and readers of one kernel agree by construction.
template <bool kIl>
struct SplitTileT {
    __bf16 *hi, *lo;
};
using SplitTile = SplitTileT<true>;

// Slot of tile row r: inside each 16-row block the rows are interleaved,
// row r at slot 2 (r % 8) + (r / 8) % 2.  At the kTS-element (144-byte) row
// stride, the eight rows a transposing read (ds_read_b64_tr_b16, frag_tp)
// gathers per 32 lanes then fall on eight disjoint 8-bank spans (measured: 0
// bank-conflict cycles per instruction, 2 with rows in order); the 16-byte
// operand reads, the natural-order transposing reads and the row writes keep
// their conflict counts, since each touches a whole 16-row block or a single
// row.  The per-lane slot arithmetic costs registers: the z-gated reverse
// backward at four heads per group, already at 256 VGPRs, spills 4 of them
// with it (C3 full-feature backward 4.33-4.43 ms against 4.24-4.25 ms with
// rows in order, while the plain and packed ones gain 1 % and 3 %), so that
// kernel keeps its rows in order (kIl = false).
template <bool kIl>
__device__ __forceinline__ int trow(int r) {
    return kIl ? ((r & ~15) | ((r & 7) << 1) | ((r >> 3) & 1)) : r;
}

template <bool kIl = true>
__device__ __forceinline__ SplitTileT<kIl> tile_at(__bf16 *base, int i) {
    return SplitTileT<kIl>{base + (2 * i) * kTile, base + (2 * i + 1) * kTile};
}

// tile[row][c0 .. c0 + 3] = v (both halves)
template <bool kIl>
__device__ __forceinline__ void store_split4(SplitTileT<kIl> d, int row, int c0, float4 v) {
    bf16x4 vh, vl;
    split4(v, vh, vl);
    const int idx = trow<kIl>(row) * kTS + c0;
    *(bf16x4 *)&d.hi[idx] = vh;
    *(bf16x4 *)&d.lo[idx] = vl;
}

struct Frag {
    bf16x8 h, l;
};

template <bool kIl>
__device__ __forceinline__ Frag frag(SplitTileT<kIl> s, int row, int ks) {
    const int kq = (threadIdx.x & 63) >> 4;
    Frag f;
    const int idx = trow<kIl>(row) * kTS + ks * 32 + kq * 8;
    f.h = *(const bf16x8 *)&s.hi[idx];
    f.l = *(const bf16x8 *)&s.lo[idx];
    return f;
}

__device__ __forceinline__ f32x4 mma3f(Frag a, Frag b, f32x4 c) { return mma3(a.h, a.l, b.h, b.l, c); }

__device__ __forceinline__ Frag pack_frag(const float (&v)[8]) {
    Frag f;
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
        bf16x2 h, l;
        split2(v[i], v[i + 1], h, l);
        f.h[i] = h[0];
        f.h[i + 1] = h[1];
        f.l[i] = l[0];
        f.l[i + 1] = l[1];
    }
    return f;
}

// ds_read_b64_tr_b16 (the lane mapping of ssd::tr4)
template <bool kIl>
__device__ __forceinline__ bf16x4 tr4(const __bf16 *arr, int k0, int c0) {
    const int m = threadIdx.x & 15;
    typedef short v4s __attribute__((ext_vector_type(4)));
    auto p = (__attribute__((address_space(3))) v4s *)(arr + trow<kIl>(k0 + (m >> 2)) * kTS + c0 + 4 * (m & 3));
    return __builtin_bit_cast(bf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(p));
}

__device__ __forceinline__ bf16x8 cat8(bf16x4 a, bf16x4 b) {
    return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
}

// operand of columns c0 .. c0 + 15 contracting over the tile's rows (natural k order)
template <bool kIl>
__device__ __forceinline__ Frag frag_tn(SplitTileT<kIl> s, int ks, int c0) {
    const int k0 = 32 * ks + 8 * ((threadIdx.x & 63) >> 4);
    Frag f;
    f.h = cat8(tr4<kIl>(s.hi, k0, c0), tr4<kIl>(s.hi, k0 + 4, c0));
    f.l = cat8(tr4<kIl>(s.lo, k0, c0), tr4<kIl>(s.lo, k0 + 4, c0));
    return f;
}

// the same in the perm32 k order of operands taken from MFMA outputs
template <bool kIl>
__device__ __forceinline__ Frag frag_tp(SplitTileT<kIl> s, int m, int c0) {
    const int k0 = 32 * m + 4 * ((threadIdx.x & 63) >> 4);
    Frag f;
    f.h = cat8(tr4<kIl>(s.hi, k0, c0), tr4<kIl>(s.hi, k0 + 16, c0));
    f.l = cat8(tr4<kIl>(s.lo, k0, c0), tr4<kIl>(s.lo, k0 + 16, c0));
    return f;
}

// fp32 hi + lo of four split values
__device__ __forceinline__ f32x4 join4(bf16x4 h, bf16x4 l) {
    typedef uint32_t u2 __attribute__((ext_vector_type(2)));
    const u2 hb = __builtin_bit_cast(u2, h), lb = __builtin_bit_cast(u2, l);
    return f32x4{bf_lo_f32(hb[0]) + bf_lo_f32(lb[0]), bf_hi_f32(hb[0]) + bf_hi_f32(lb[0]),
                 bf_lo_f32(hb[1]) + bf_lo_f32(lb[1]), bf_hi_f32(hb[1]) + bf_hi_f32(lb[1])};
}

// fp32 values of tile[row][c0 .. c0 + 3]
template <bool kIl>
__device__ __forceinline__ f32x4 tile_row4(SplitTileT<kIl> s, int row, int c0) {
    const int idx = trow<kIl>(row) * kTS + c0;
    return join4(*(const bf16x4 *)&s.hi[idx], *(const bf16x4 *)&s.lo[idx]);
}

// column-major staging, tile[c][slot] = f(t, c) (ssd::stage_cols for this element type)
template <bool PERM, bool kIl, class F>
__device__ __forceinline__ void stage_cols(SplitTileT<kIl> d, F f) {
    const int c = threadIdx.x & 63, tb = threadIdx.x >> 6;
#pragma unroll
    for (int run = tb; run < 8; run += 4) {
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int slot = run * 8 + i;
            v[i] = f(PERM ? perm_token(slot) : slot, c);
        }
        const Frag p = pack_frag(v);
        *(bf16x8 *)&d.hi[trow<kIl>(c) * kTS + run * 8] = p.h;
        *(bf16x8 *)&d.lo[trow<kIl>(c) * kTS + run * 8] = p.l;
    }
}

}  // namespace bwd
}  // namespace ssd
