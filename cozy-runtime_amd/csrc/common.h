// Shared device helpers for the gfx950 kernels: vector types, 16-bit float conversions, the
// OCP E4M3 and E8M0 encoders, and the MFMA wrappers. Every conversion here rounds exactly as
// torch's CPU casts do, so kernel outputs can be compared bit for bit with the CPU law.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cozyq {

typedef int32_t i32x2 __attribute__((ext_vector_type(2)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kMaxK = 32768;
constexpr float kE4m3Max = 448.0f;
constexpr float kScaleFloor = 1e-12f;

__host__ __device__ __forceinline__ uint32_t bits_of(float f) { return __builtin_bit_cast(uint32_t, f); }
__host__ __device__ __forceinline__ float float_of(uint32_t u) { return __builtin_bit_cast(float, u); }

// 16-bit activations: bf16 widens by a shift, fp16 by the hardware conversion (exact).
template <bool kHalf>
__device__ __forceinline__ float widen(uint16_t h) {
    if constexpr (kHalf) {
        return static_cast<float>(__builtin_bit_cast(_Float16, h));
    } else {
        return float_of(static_cast<uint32_t>(h) << 16);
    }
}

// float32 -> bf16, round to nearest even; NaN -> 0x7FC0 (c10::BFloat16's rule).
__host__ __device__ __forceinline__ uint16_t bf16_rn(float f) {
    uint32_t u = bits_of(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

template <bool kHalf>
__device__ __forceinline__ uint16_t narrow(float f) {
    if constexpr (kHalf) {
        // The float32 value is materialized first: otherwise the backend folds the producing
        // multiply into v_fma_mix*_f16, rounding once where the CPU law rounds to float32 and
        // then to fp16.
        asm volatile("" : "+v"(f));
        return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));  // v_cvt_f16_f32: RNE
    } else {
        return bf16_rn(f);
    }
}

// float32 -> OCP E4M3FN byte, round to nearest even, subnormals in 2^-9 steps, |v| >= 480 and
// NaN -> 0x7F with the sign kept: torch's `.to(float8_e4m3fn)` (callers clamp to ±448 first).
__host__ __device__ __forceinline__ uint8_t e4m3_rn(float v) {
    const uint32_t u = bits_of(v);
    const uint32_t sign = (u >> 24) & 0x80u;
    const uint32_t mag = u & 0x7fffffffu;
    if (mag >= 0x43f00000u) return static_cast<uint8_t>(sign | 0x7fu);  // >= 480, inf, NaN
    if (mag < 0x3c800000u) {                                                // < 2^-6: subnormal
        // |v|·2^9 is exact (a power-of-two scale of a value below 8); rint rounds half to even.
        const float units = __builtin_rintf(float_of(mag) * 512.0f);
        return static_cast<uint8_t>(sign | static_cast<uint32_t>(units));
    }
    // Normal: keep 3 mantissa bits, round to nearest even at bit 20; a carry bumps the exponent.
    const uint32_t kept = (mag + 0x7ffffu + ((mag >> 20) & 1u)) >> 20;
    return static_cast<uint8_t>(sign | (kept - (120u << 3)));
}

// x from the lane that DPP control kCtrl names (every lane active).
template <int kCtrl>
__device__ __forceinline__ float dpp_move(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), kCtrl, 0xF, 0xF, false));
}

// The maximum over a wave, uniform: each 16-lane row's by DPP (quad swaps, then rotations of the
// row by 4 and 8 lanes), then the four rows' read from lanes 0, 16, 32 and 48. No LDS round trip
// (the ds_bpermute shuffles it replaces wait on the LDS crossbar); a maximum is exact in any order.
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_move<0xB1>(v));   // quad_perm 1,0,3,2
    v = fmaxf(v, dpp_move<0x4E>(v));   // quad_perm 2,3,0,1
    v = fmaxf(v, dpp_move<0x124>(v));  // row_ror:4
    v = fmaxf(v, dpp_move<0x128>(v));  // row_ror:8
    const int b = __builtin_bit_cast(int, v);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// IEEE 754-2019 maximum (v_maximum3_f32 on gfx950): a NaN operand gives NaN, as torch's amax
// does, where fmaxf would drop it.
__device__ __forceinline__ float nan_max(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float nan_min(float a, float b) { return __builtin_elementwise_minimum(a, b); }

// wave_max with NaN propagated: the wave's maximum, or NaN if any lane holds one.
__device__ __forceinline__ float wave_max_nan(float v) {
    v = nan_max(v, dpp_move<0xB1>(v));
    v = nan_max(v, dpp_move<0x4E>(v));
    v = nan_max(v, dpp_move<0x124>(v));
    v = nan_max(v, dpp_move<0x128>(v));
    const int b = __builtin_bit_cast(int, v);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
    return nan_max(nan_max(r0, r1), nan_max(r2, r3));
}

// The sum over a wave of a value that is zero outside lanes 0-3, 20-23, 40-43 and 60-63: the
// diagonal of a 16x16 MFMA result (lane l holds rows 4·(l/16) + r of column l%16), one quad of
// each 16-lane row. Each quad is summed by two DPP quad swaps, then the four quad sums are read
// from lanes 0, 20, 40 and 60: no LDS round trip (six shuffles through ds_bpermute measured
// ~0.45 us of the fp8 decode's 10.9). The result is uniform; float sums run in the fixed order
// ((q0 + q1) + q2) + q3, the same for every call.
template <typename T>
__device__ __forceinline__ T diagonal_sum(T v) {
    v += __builtin_bit_cast(T, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));  // quad_perm 1,0,3,2
    v += __builtin_bit_cast(T, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));  // quad_perm 2,3,0,1
    const int b = __builtin_bit_cast(int, v);
    const T q0 = __builtin_bit_cast(T, __builtin_amdgcn_readlane(b, 0));
    const T q1 = __builtin_bit_cast(T, __builtin_amdgcn_readlane(b, 20));
    const T q2 = __builtin_bit_cast(T, __builtin_amdgcn_readlane(b, 40));
    const T q3 = __builtin_bit_cast(T, __builtin_amdgcn_readlane(b, 60));
    return ((q0 + q1) + q2) + q3;
}

// x / s for s > 0, rounded to nearest even, given r = RN(1/s): q = RN(x·r) is within an ulp of
// x / s, the remainder x − q·s is exact on the FMA, and one correction q + rem·r rounds to
// RN(x / s) (Markstein's theorem; quotients that underflow excepted, which every caller here maps
// to code 0 anyway). The sign is x's, as a true division's is (the correction turns −0 into +0).
// Held against IEEE division by the GPU tests.
__device__ __forceinline__ float div_rn(float x, float s, float r) {
    const float q = x * r;
    const float rem = __builtin_fmaf(-q, s, x);
    return __builtin_copysignf(__builtin_fmaf(rem, r, q), x);
}

// Four float32 values (each within ±448) -> four OCP E4M3 bytes, first in the low byte, on
// gfx950's v_cvt_pk_fp8_f32 (round to nearest even: bit-identical to `e4m3_rn` there, checked
// exhaustively near every rounding boundary by the GPU tests).
__device__ __forceinline__ uint32_t e4m3x4(float a, float b, float c, float d) {
    const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
    return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true));
}

// E4M3FN byte -> float32 (exact); S.1111.111 is NaN (E4M3FN has no infinities).
__device__ __forceinline__ float e4m3_value(uint32_t b) {
    if ((b & 0x7fu) == 0x7fu) return __builtin_nanf("");
    const uint32_t sign = (b & 0x80u) << 24;
    const uint32_t e = (b >> 3) & 0xfu, m = b & 7u;
    if (e == 0) return float_of(sign | bits_of(static_cast<float>(m) * 0.001953125f));  // m·2^-9
    return float_of(sign | ((e + 120u) << 23) | (m << 20));
}

// The MX block exponent byte of a block maximum: clamp(ceil(log2(amax / 448)) + 127, 0, 254),
// 0 for amax == 0 (internal/encoding/leaves.py:1417-1421), with the ceiling of the log taken
// exactly from the quotient's bits rather than from a log2 routine.
__host__ __device__ __forceinline__ uint8_t mx_byte(float amax) {
    if (!(amax > 0.0f)) return 0;  // exponent -127 -> byte 0
    const float v = amax / kE4m3Max;
    const uint32_t u = bits_of(v);
    const int biased = static_cast<int>((u >> 23) & 0xffu);
    const uint32_t man = u & 0x7fffffu;
    int e;
    if (biased == 0) {  // subnormal quotient: v = man · 2^-149
        const int msb = 31 - __builtin_clz(man);
        e = (man & (man - 1)) ? msb - 148 : msb - 149;
    } else {
        e = (man == 0) ? biased - 127 : biased - 126;
    }
    int b = e + 127;
    b = b < 0 ? 0 : (b > 254 ? 254 : b);
    return static_cast<uint8_t>(b);
}

// 2^(byte - 127) as float32 by construction; byte 0 is 2^-127 (formats.py:577-585).
__device__ __forceinline__ float e8m0_value(uint32_t b) {
    return b == 0 ? float_of(1u << 22) : float_of(b << 23);
}

// tanh-GELU, 0.5·y·(1 + tanh(u)) with u = 0.79788456·(y + 0.044715·y³), as y / (1 + e^(-2u)):
// e^(-2u) = 2^(y·(c1 + c2·y²)) with c1 = -2·log2(e)·0.79788456 and c2 = 0.044715·c1. Every GEMM
// tile shares this one sequence, so their GELU outputs agree bit for bit.
__device__ __forceinline__ float gelu_tanh(float y) {
    const float t = __builtin_fmaf(-0.10294324f, y * y, -2.3022082f);
    return y * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(y * t));
}

// ---------------------------------------------------------------------------------- MFMA
// D(16x16) += A(16xK)·B(Kx16). Lane l supplies row l%16 of A and column l%16 of B, its K
// slice chosen by l/16; both operands loaded with the same pattern pair every k correctly.
// The result's lane l holds rows 4·(l/16)+r (r = 0..3) of column l%16.
// f8f6f4 (K = 128, 32 bytes a lane): lane group g = l/16 holds k in [16g, 16g+16) in bytes
// 0..15 and k in [64+16g, 64+16g+16) in bytes 16..31, and the E8M0 scale of K block κ
// (k in [32κ, 32κ+32)) of row (column) i is lane i + 16κ's (measured on gfx950 by the probe
// tests). A lane group therefore loads 16-byte chunks g and g+4 of a 128-byte K step.

__device__ __forceinline__ i32x4 mfma_i8(i32x4 a, i32x4 b, i32x4 c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// e4m3 x e4m3, K = 128 per call (format code 0 for both operands), float32 accumulate.
__device__ __forceinline__ f32x4 mfma_f8(i32x8 a, i32x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

// The same with an E8M0 scale per lane for each operand (its 32-element K block).
__device__ __forceinline__ f32x4 mfma_f8_scaled(i32x8 a, i32x8 b, f32x4 c, int sa, int sb) {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, sa, 0, sb);
}

// The 32x32 form, K = 64 per call: lane l supplies row (column) l%32, lane group g = l/32
// holds k in [16g, 16g+16) in bytes 0..15 and k in [32+16g, 32+16g+16) in bytes 16..31, and
// the E8M0 scale of K block κ of row i is lane i + 32κ's; result register r of lane l is row
// 8·(r/4) + 4·(l/32) + r%4 of column l%32 (measured on gfx950 by the probe tests).
__device__ __forceinline__ f32x16 mfma_f8_32(i32x8 a, i32x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

template <int kSelA = 0, int kSelB = 0>
__device__ __forceinline__ f32x16 mfma_f8_32_scaled(i32x8 a, i32x8 b, f32x16 c, int sa, int sb) {
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, kSelA, sa, kSelB, sb);
}

__device__ __forceinline__ f32x4 mfma_bf16(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// ------------------------------------------------------------------ waits and LDS-DMA
// LDS pointers for buffer_load ... lds (the LDS-DMA loads: 64 lanes x 16 bytes land contiguous
// at the uniform base the pointer gives, lane l at +16l).
typedef __attribute__((address_space(3))) void LdsPtr;

// s_waitcnt with only vmcnt <= N (expcnt and lgkmcnt left unconstrained): gfx9 encoding.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// s_waitcnt lgkmcnt(0) alone.
__device__ __forceinline__ void wait_lgkmcnt0() {
    __builtin_amdgcn_s_waitcnt(0xF | (0x3 << 14) | (0x7 << 4));
}

// Keeps the compiler from moving memory operations across the waits and barriers around it.
__device__ __forceinline__ void fence() { asm volatile("" ::: "memory"); }

// A GEMV epilogue's operands for a wave's rows nw .. nw + kRows - 1: the weight's row scales and
// the bias, for loading with the activation, before the weight stream. Loaded after it (where
// they are used), every wave's end waits out one more memory round trip. Rows past N read zeros.
template <int kRows, bool kBias>
struct RowEpilogue {
    float ws[kRows];
    uint16_t bias[kRows];
};

template <int kRows, bool kBias>
__device__ __forceinline__ RowEpilogue<kRows, kBias> row_epilogue(const float* ws, const uint16_t* bias, int nw, int N) {
    RowEpilogue<kRows, kBias> e;
    const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(ws), 0, 4 * N, 0x00020000);
#pragma unroll
    for (int i = 0; i < kRows; ++i)
        e.ws[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(sr, 4 * (nw + i), 0, 0));
    if constexpr (kBias) {
        const __amdgpu_buffer_rsrc_t br =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(bias), 0, 2 * N, 0x00020000);
#pragma unroll
        for (int i = 0; i < kRows; ++i) e.bias[i] = __builtin_amdgcn_raw_buffer_load_b16(br, 2 * (nw + i), 0, 0);
    }
    return e;
}

}  // namespace cozyq
