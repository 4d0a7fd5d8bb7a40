// Device helpers shared by the Mamba-2 SSD kernels (gfx950 / CDNA4).
//
// Precision scheme: every contraction runs on the fp16 matrix cores with
// fp32 accumulation, but each fp32 operand v is carried as an unevaluated sum
// hi + lo of two fp16 values (hi = fp16(v), lo = fp16(v - hi)), and a product
// is formed from three MFMAs: hi*hi + hi*lo + lo*hi.  This keeps about 22 bits
// of operand precision, which is what the fp32 public contract needs (plain
// fp16 or bf16 operands miss a 2e-2 max-abs bound by one to two orders of
// magnitude on long sequences with slow decay).
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

__device__ __forceinline__ void split_f16(float v, _Float16 &hi, _Float16 &lo) {
    hi = (_Float16)v;
    lo = (_Float16)(v - (float)hi);
}

__device__ __forceinline__ void split4(float4 v, half4 &hi, half4 &lo) {
    const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const _Float16 h = (_Float16)vv[i];
        hi[i] = h;
        lo[i] = (_Float16)(vv[i] - (float)h);
    }
}

__device__ __forceinline__ float softplus_f(float u) {
    // torch.nn.functional.softplus with beta = 1, threshold = 20
    return u > 20.f ? u : log1pf(expf(u));
}

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
    if (softplus) g *= 1.f / (1.f + expf(-u));
    return g;
}

__device__ __forceinline__ float silu_f(float z) { return z / (1.f + expf(-z)); }

// Inclusive prefix sum across the 64 lanes of a wave.
__device__ __forceinline__ float wave_inclusive_scan(float v) {
    const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
        float o = __shfl_up(v, off, kWave);
        if (lane >= off) v += o;
    }
    return v;
}

// Suffix (reverse inclusive) sum across the 64 lanes of a wave.
__device__ __forceinline__ float wave_suffix_scan(float v) {
    const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
        float o = __shfl_down(v, off, kWave);
        if (lane + off < kWave) v += o;
    }
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// Position of token s (0..31 inside a 32-token slab) in the k-permuted operand
// order produced by taking C*B^T from MFMA output tiles: output lane group j
// holds rows 4j..4j+3 of two consecutive 16-row tiles, which become k slots
// 8j..8j+3 and 8j+4..8j+7 of the next product.
__device__ __forceinline__ int perm32(int s) {
    return 8 * ((s & 15) >> 2) + 4 * (s >> 4) + (s & 3);
}

}  // namespace ssd
