// Decode of the stored weight formats into a float destination: the reference's `decoded_float`
// providers (internal/encoding/formats.py:438-868) and its svdq.nvfp4 decode core
// (internal/decode_schemes.py:434-489), each element formed in float32 by the reference's
// sequence of roundings and rounded once into f32, bf16 or f16 (internal/decode_cores.py:
// 196-230,354-372).
//
// Three kernels, all bound by HBM (one read of the codes, one write of the destination):
// - `table_kernel`: element = value(code) · scale, with a second-level factor (× after, or ÷
//   into the scale) and a per-column factor after. Codes are int8, E4M3, E5M2 or packed E2M1;
//   the scale grid is one value, one per row or column, or row blocks of 16/32 stored row-major
//   or in cuBLAS's 128x4 tiles. One thread takes a run of 16 elements of a row with one 16-byte
//   load when the rows are whole runs; other shapes take one element per thread.
// - `convrot_kernel`: int8.convrot's exact int32 Hadamard over each 4^k group. A lane holds 64
//   consecutive elements: the three innermost radix-4 digits are transformed in registers,
//   digits 3-5 across lanes (DPP quad and row permutes, then ds_bpermute across rows), and the
//   digits of 16384- and 65536-element groups across the waves of one workgroup through LDS.
//   Every partial sum is an integer below 127·4^8 < 2^24, so the order of the stages does not
//   change the result.
// - `svdq_decode_kernel`: the nvfp4 value · channel scale · smoothing, plus up·down added term
//   by term in rank order.
#include "common.h"
#include "kernels.h"

namespace cozyq {
namespace {

// ----------------------------------------------------------------------- element values

// E5M2 is the top byte of an IEEE half: widening is exact, infinities and NaN included.
__device__ __forceinline__ float e5m2_value(uint32_t b) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(b << 8)));
}

// E2M1 nibble: bit 3 the sign, bits 2-1 the exponent (bias 1), bit 0 the mantissa; magnitudes
// 0, 0.5, 1, 1.5, 2, 3, 4, 6 (internal/encoding/formats.py:755-759), built from the bits.
__device__ __forceinline__ float e2m1_value(uint32_t nib) {
    const uint32_t m = nib & 7u, sign = (nib & 8u) << 28;
    const uint32_t mag = m < 2 ? (m ? 0x3f000000u : 0u) : (((m >> 1) + 126u) << 23) | ((m & 1u) << 22);
    return float_of(sign | mag);
}

// An E8M0 byte's value with 255 as NaN (internal/encoding/formats.py:577-585).
__device__ __forceinline__ float e8m0_decoded(uint32_t b) {
    return b == 255u ? __builtin_nanf("") : e8m0_value(b);
}

// Element `idx` of a scale-like part of dtype `type` (kNumF32 ... kNumE4m3) as float32; every
// conversion is exact.
__device__ __forceinline__ float num_at(const void* p, int type, int64_t idx) {
    switch (type) {
        case kNumF32: return static_cast<const float*>(p)[idx];
        case kNumBf16: return widen<false>(static_cast<const uint16_t*>(p)[idx]);
        case kNumF16: return widen<true>(static_cast<const uint16_t*>(p)[idx]);
        case kNumE8m0: return e8m0_decoded(static_cast<const uint8_t*>(p)[idx]);
        default: return e4m3_value(static_cast<const uint8_t*>(p)[idx]);
    }
}

template <int kCode>
__device__ __forceinline__ float code_value(uint32_t c) {
    if constexpr (kCode == kCodeI8) return static_cast<float>(static_cast<int8_t>(c));
    else if constexpr (kCode == kCodeE4m3) return e4m3_value(c);
    else if constexpr (kCode == kCodeE5m2) return e5m2_value(c);
    else return e2m1_value(c);
}

// float32 → the destination's bits, round to nearest even (decode_cores.round_into).
template <int kOut>
__device__ __forceinline__ void store_one(void* out, int64_t idx, float v) {
    if constexpr (kOut == kNumF32) static_cast<float*>(out)[idx] = v;
    else static_cast<uint16_t*>(out)[idx] = narrow<kOut == kNumF16>(v);
}

template <int kOut>
__device__ __forceinline__ void store16(void* out, int64_t idx, const float (&v)[16]) {
    if constexpr (kOut == kNumF32) {
        float4* dst = reinterpret_cast<float4*>(static_cast<float*>(out) + idx);
#pragma unroll
        for (int k = 0; k < 4; ++k) dst[k] = make_float4(v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]);
    } else {
        uint32_t w[8];
#pragma unroll
        for (int k = 0; k < 8; ++k)
            w[k] = narrow<kOut == kNumF16>(v[2 * k]) | (static_cast<uint32_t>(narrow<kOut == kNumF16>(v[2 * k + 1])) << 16);
        uint4* dst = reinterpret_cast<uint4*>(static_cast<uint16_t*>(out) + idx);
        dst[0] = make_uint4(w[0], w[1], w[2], w[3]);
        dst[1] = make_uint4(w[4], w[5], w[6], w[7]);
    }
}

// ------------------------------------------------------------------------ table decode

// Scale-grid index of element (i, j) (internal/decode_cores.py:335-351).
__device__ __forceinline__ int64_t grid_index(const TableDecode& a, int64_t i, int64_t j) {
    switch (a.grid) {
        case kGridTensor: return 0;
        case kGridRow: return i;
        case kGridCol: return j;
        default: {
            const int64_t w = (a.cols + a.block - 1) / a.block, b = j / a.block;
            if (!a.tiled) return i * w + b;
            return ((i >> 7) * ((w + 3) >> 2) + (b >> 2)) * 512 + (i & 31) * 16 + ((i & 127) >> 5) * 4 + (b & 3);
        }
    }
}

// value · s, then · g (multiply), or value · (s / g) (divide); then · p (formats.py:762-783,
// decode_cores.py:214-228).
__device__ __forceinline__ float table_law(int second, float v, float s, float g) {
    if (second == kSecondDivide) s = s / g;
    v = v * s;
    if (second == kSecondMultiply) v = v * g;
    return v;
}

// Runs of 16 elements: rows are whole runs (cols % 16 == 0), the parts 16-byte aligned (8 for
// packed E2M1) and the block size, if any, a multiple of 16, so a run has one block scale.
template <int kCode, int kOut>
__global__ __launch_bounds__(256) void table_run_kernel(TableDecode a) {
    const int64_t e = blockIdx.y;
    const int64_t runs = a.rows * a.cols / 16;
    const int64_t run = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (run >= runs) return;
    const int64_t i = run / (a.cols / 16), j0 = (run % (a.cols / 16)) * 16;
    const uint8_t* weight = a.weight + e * a.weight_stride;
    const void* scale = static_cast<const uint8_t*>(a.scale) + e * a.scale_stride * a.scale_size;
    const float g = a.second ? a.scale_2[e * a.scale_2_step] : 1.0f;
    uint32_t c[16];
    if constexpr (kCode == kCodeE2m1) {
        const uint2 raw = *reinterpret_cast<const uint2*>(weight + run * 8);
        const uint32_t lo_first = a.high_first ? 0u : 1u;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t byte = ((k < 4 ? raw.x : raw.y) >> (8 * (k & 3))) & 0xffu;
            c[2 * k] = lo_first ? (byte & 15u) : (byte >> 4);
            c[2 * k + 1] = lo_first ? (byte >> 4) : (byte & 15u);
        }
    } else {
        const uint4 raw = *reinterpret_cast<const uint4*>(weight + run * 16);
        const uint32_t w4[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int k = 0; k < 16; ++k) c[k] = (w4[k >> 2] >> (8 * (k & 3))) & 0xffu;
    }
    float v[16];
    if (a.grid == kGridCol) {
#pragma unroll
        for (int k = 0; k < 16; ++k)
            v[k] = table_law(a.second, code_value<kCode>(c[k]), num_at(scale, a.scale_type, j0 + k), g);
    } else {
        const float s = num_at(scale, a.scale_type, grid_index(a, i, j0));
#pragma unroll
        for (int k = 0; k < 16; ++k) v[k] = table_law(a.second, code_value<kCode>(c[k]), s, g);
    }
    if (a.post_mode == kPostOne) {
        const float p = num_at(a.post, a.post_type, 0);
#pragma unroll
        for (int k = 0; k < 16; ++k) v[k] = v[k] * p;
    } else if (a.post_mode == kPostColumn) {
#pragma unroll
        for (int k = 0; k < 16; ++k) v[k] = v[k] * num_at(a.post, a.post_type, j0 + k);
    }
    store16<kOut>(a.out, e * a.out_stride + run * 16, v);
}

// Any shape and alignment: one element per thread, grid-stride.
template <int kCode, int kOut>
__global__ __launch_bounds__(256) void table_elem_kernel(TableDecode a) {
    const int64_t e = blockIdx.y;
    const int64_t total = a.rows * a.cols;
    const uint8_t* weight = a.weight + e * a.weight_stride;
    const void* scale = static_cast<const uint8_t*>(a.scale) + e * a.scale_stride * a.scale_size;
    const float g = a.second ? a.scale_2[e * a.scale_2_step] : 1.0f;
    for (int64_t x = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; x < total;
         x += static_cast<int64_t>(gridDim.x) * 256) {
        const int64_t i = x / a.cols, j = x - i * a.cols;
        uint32_t c;
        if constexpr (kCode == kCodeE2m1) {
            const uint32_t byte = weight[x >> 1];
            const bool high = ((x & 1) != 0) != (a.high_first != 0);
            c = high ? byte >> 4 : byte & 15u;
        } else {
            c = weight[x];
        }
        float v = table_law(a.second, code_value<kCode>(c), num_at(scale, a.scale_type, grid_index(a, i, j)), g);
        if (a.post_mode == kPostOne) v = v * num_at(a.post, a.post_type, 0);
        else if (a.post_mode == kPostColumn) v = v * num_at(a.post, a.post_type, j);
        store_one<kOut>(a.out, e * a.out_stride + x, v);
    }
}

template <int kCode, int kOut>
hipError_t launch_table(const TableDecode& a, int matrices, hipStream_t s) {
    const int64_t total = a.rows * a.cols;
    const int64_t align = kCode == kCodeE2m1 ? 8 : 16;
    const int out_size = kOut == kNumF32 ? 4 : 2;
    const bool runs = a.cols % 16 == 0 && (a.grid != kGridBlocks || a.block % 16 == 0) &&
                      reinterpret_cast<uintptr_t>(a.weight) % align == 0 &&
                      reinterpret_cast<uintptr_t>(a.out) % 16 == 0 && a.weight_stride % align == 0 &&
                      (a.out_stride * out_size) % 16 == 0;
    if (runs) {
        const int64_t blocks = (total / 16 + 255) / 256;
        hipLaunchKernelGGL((table_run_kernel<kCode, kOut>), dim3(static_cast<uint32_t>(blocks), matrices),
                           dim3(256), 0, s, a);
    } else {
        const int64_t blocks = std::min<int64_t>((total + 255) / 256, 65536);
        hipLaunchKernelGGL((table_elem_kernel<kCode, kOut>), dim3(static_cast<uint32_t>(blocks), matrices),
                           dim3(256), 0, s, a);
    }
    return hipGetLastError();
}

template <int kCode>
hipError_t table_out(const TableDecode& a, int out_type, int matrices, hipStream_t s) {
    switch (out_type) {
        case kNumF32: return launch_table<kCode, kNumF32>(a, matrices, s);
        case kNumBf16: return launch_table<kCode, kNumBf16>(a, matrices, s);
        default: return launch_table<kCode, kNumF16>(a, matrices, s);
    }
}

// ---------------------------------------------------------------------- int8.convrot

template <int kCtrl>
__device__ __forceinline__ int dpp(int v) {
    return __builtin_amdgcn_mov_dpp(v, kCtrl, 0xf, 0xf, false);
}

// The regular H4 on four values a, b, c, d: (a+b+c−d, a+b−c+d, a−b+c+d, −a+b+c+d)
// (internal/encoding/formats.py:667-671). Output j is Σ − 2·v[3 − j].
__device__ __forceinline__ void h4(int& a, int& b, int& c, int& d) {
    const int ab = a + b, amb = a - b, cd = c + d, cmd = c - d;
    a = ab + cmd;
    b = ab - cmd;
    c = amb + cd;
    d = cd - amb;
}

// Digit at lane bits 0-1: partners lane^1, lane^2 and lane^3 (= lane with digit 3 − j) by DPP
// quad permutes.
__device__ __forceinline__ int h4_quad(int v) {
    const int t = v + dpp<0xB1>(v);  // quad_perm [1,0,3,2]: lane ^ 1
    const int s = t + dpp<0x4E>(t);  // quad_perm [2,3,0,1]: lane ^ 2
    return s - 2 * dpp<0x1B>(v);     // quad_perm [3,2,1,0]: lane ^ 3
}

// Digit at lane bits 2-3: the sum by row rotations of 4 and 8 lanes, the partner lane ^ 12 by a
// row mirror (lane ^ 15) then quad_perm [3,2,1,0] (lane ^ 3).
__device__ __forceinline__ int h4_row(int v) {
    const int t = v + dpp<0x124>(v);  // row_ror:4
    const int s = t + dpp<0x128>(t);  // row_ror:8
    return s - 2 * dpp<0x1B>(dpp<0x140>(v));
}

// Digit at lane bits 4-5: across the wave's four rows by ds_bpermute.
__device__ __forceinline__ int h4_wave(int v, int lane) {
    const int t = v + __builtin_amdgcn_ds_bpermute((lane ^ 16) << 2, v);
    const int s = t + __builtin_amdgcn_ds_bpermute((lane ^ 32) << 2, t);
    return s - 2 * __builtin_amdgcn_ds_bpermute((lane ^ 48) << 2, v);
}

constexpr int convrot_waves(int digits) { return digits <= 6 ? 4 : (1 << (2 * (digits - 6))); }

// 64 elements a lane, `kDigits` radix-4 digits (group size 4^kDigits). For kDigits ≤ 6 the
// workgroup's four waves take independent 4096-element chunks of the flattened matrix; for 7
// and 8 a workgroup of 4 or 16 waves takes one group. total % 64 == 0, `w` and `out` 16-byte
// aligned (checked by the launcher).
template <int kDigits, int kOut>
__global__ __launch_bounds__(64 * convrot_waves(kDigits)) __attribute__((amdgpu_waves_per_eu(4, 8)))
void convrot_kernel(
    const int8_t* w, const void* scale, int scale_type, void* out, int64_t total, int64_t cols) {
    constexpr int kWaves = convrot_waves(kDigits);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t block_base = static_cast<int64_t>(blockIdx.x) * (4096 * kWaves);
    const int64_t base = block_base + 64 * static_cast<int64_t>(threadIdx.x);
    const bool active = base < total;

    // Bounded loads: the resource covers this workgroup's span of the matrix only.
    const int64_t span = std::min<int64_t>(total - block_base, 4096 * kWaves);
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t*>(w + block_base), 0, static_cast<int>(span), 0x00020000);
    int v[64];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const i32x4 raw = active ? __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, 64 * threadIdx.x + 16 * k, 0, 0))
                                 : i32x4{0, 0, 0, 0};
#pragma unroll
        for (int b = 0; b < 16; ++b) v[16 * k + b] = static_cast<int8_t>((raw[b >> 2] >> (8 * (b & 3))) & 0xff);
    }

    // Digits 0-2: in registers (index r = 16·d2 + 4·d1 + d0).
#pragma unroll
    for (int d = 0; d < (kDigits < 3 ? kDigits : 3); ++d) {
        const int st = 1 << (2 * d);
#pragma unroll
        for (int r = 0; r < 64; ++r)
            if (((r / st) & 3) == 0) h4(v[r], v[r + st], v[r + 2 * st], v[r + 3 * st]);
    }
    if constexpr (kDigits > 3) {
#pragma unroll
        for (int r = 0; r < 64; ++r) {
            v[r] = h4_quad(v[r]);
            // Materialized here: sunk past a branch, the sums would keep three permuted
            // copies of every register alive across it.
            asm volatile("" : "+v"(v[r]));
        }
    }
    if constexpr (kDigits > 4) {
#pragma unroll
        for (int r = 0; r < 64; ++r) {
            v[r] = h4_row(v[r]);
            // Materialized here: sunk past a branch, the sums would keep three permuted
            // copies of every register alive across it.
            asm volatile("" : "+v"(v[r]));
        }
    }
    if constexpr (kDigits > 5) {
#pragma unroll
        for (int r = 0; r < 64; ++r) {
            v[r] = h4_wave(v[r], lane);
            // Materialized here: sunk past a branch, the sums would keep three permuted
            // copies of every register alive across it.
            asm volatile("" : "+v"(v[r]));
        }
    }
    if constexpr (kDigits > 6) {
        // Digits 6-7: across waves, 16 registers at a time through LDS.
        __shared__ i32x4 lds[kWaves * 64 * 4];
#pragma unroll
        for (int d = 6; d < kDigits; ++d) {
            const int q = 2 * (d - 6);
            const int w1 = wave ^ (1 << q), w2 = wave ^ (2 << q), w3 = wave ^ (3 << q);
#pragma unroll
            for (int pass = 0; pass < 4; ++pass) {
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int r = 16 * pass + 4 * k;
                    lds[(wave * 64 + lane) * 4 + k] = i32x4{v[r], v[r + 1], v[r + 2], v[r + 3]};
                }
                __syncthreads();
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const i32x4 p1 = lds[(w1 * 64 + lane) * 4 + k];
                    const i32x4 p2 = lds[(w2 * 64 + lane) * 4 + k];
                    const i32x4 p3 = lds[(w3 * 64 + lane) * 4 + k];
#pragma unroll
                    for (int b = 0; b < 4; ++b) {
                        int& x = v[16 * pass + 4 * k + b];
                        x = x + p1[b] + p2[b] + p3[b] - 2 * p3[b];
                        asm volatile("" : "+v"(x));
                    }
                }
                __syncthreads();
            }
        }
    }

    if (!active) return;
    constexpr float kInv = 1.0f / static_cast<float>(1 << kDigits);  // 1/√(4^k), exact
    constexpr int kGroup = 1 << (2 * kDigits);
    float s = num_at(scale, scale_type, base / cols);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        float run[16];
#pragma unroll
        for (int b = 0; b < 16; ++b) {
            const int r = 16 * k + b;
            if constexpr (kGroup < 64) {  // groups of 4 or 16 may start a new row inside the lane
                if (r % kGroup == 0 && r > 0) s = num_at(scale, scale_type, (base + r) / cols);
            }
            run[b] = (static_cast<float>(v[r]) * s) * kInv;
        }
        store16<kOut>(out, base + 16 * k, run);
    }
}

// Groups of 4 or 16 on any shape or alignment: one thread a group.
template <int kDigits, int kOut>
__global__ __launch_bounds__(256) void convrot_group_kernel(const int8_t* w, const void* scale,
                                                            int scale_type, void* out, int64_t total,
                                                            int64_t cols) {
    constexpr int kGroup = 1 << (2 * kDigits);
    const int64_t groups = total / kGroup;
    for (int64_t g = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; g < groups;
         g += static_cast<int64_t>(gridDim.x) * 256) {
        int v[kGroup];
#pragma unroll
        for (int r = 0; r < kGroup; ++r) v[r] = w[g * kGroup + r];
#pragma unroll
        for (int d = 0; d < kDigits; ++d) {
            const int st = 1 << (2 * d);
#pragma unroll
            for (int r = 0; r < kGroup; ++r)
                if (((r / st) & 3) == 0) h4(v[r], v[r + st], v[r + 2 * st], v[r + 3 * st]);
        }
        const float s = num_at(scale, scale_type, g * kGroup / cols);
        constexpr float kInv = 1.0f / static_cast<float>(1 << kDigits);
#pragma unroll
        for (int r = 0; r < kGroup; ++r) store_one<kOut>(out, g * kGroup + r, (static_cast<float>(v[r]) * s) * kInv);
    }
}

template <int kDigits, int kOut>
hipError_t launch_convrot(const int8_t* w, const void* scale, int scale_type, void* out, int64_t rows,
                          int64_t cols, hipStream_t s) {
    const int64_t total = rows * cols;
    const bool lanes = total % 64 == 0 && reinterpret_cast<uintptr_t>(w) % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(out) % 16 == 0;
    if constexpr (kDigits <= 2) {
        if (!lanes) {
            const int64_t blocks = std::min<int64_t>((total / (1 << (2 * kDigits)) + 255) / 256, 65536);
            hipLaunchKernelGGL((convrot_group_kernel<kDigits, kOut>), dim3(static_cast<uint32_t>(blocks)),
                               dim3(256), 0, s, w, scale, scale_type, out, total, cols);
            return hipGetLastError();
        }
    } else {
        if (!lanes) return hipErrorInvalidValue;  // groups of 64 and more: the caller aligns
    }
    constexpr int kWaves = convrot_waves(kDigits);
    const int64_t blocks = (total + 4096 * kWaves - 1) / (4096 * kWaves);
    hipLaunchKernelGGL((convrot_kernel<kDigits, kOut>), dim3(static_cast<uint32_t>(blocks)), dim3(64 * kWaves),
                       0, s, w, scale, scale_type, out, total, cols);
    return hipGetLastError();
}

template <int kOut>
hipError_t convrot_digits(const int8_t* w, const void* scale, int scale_type, void* out, int64_t rows,
                          int64_t cols, int digits, hipStream_t s) {
    switch (digits) {
        case 1: return launch_convrot<1, kOut>(w, scale, scale_type, out, rows, cols, s);
        case 2: return launch_convrot<2, kOut>(w, scale, scale_type, out, rows, cols, s);
        case 3: return launch_convrot<3, kOut>(w, scale, scale_type, out, rows, cols, s);
        case 4: return launch_convrot<4, kOut>(w, scale, scale_type, out, rows, cols, s);
        case 5: return launch_convrot<5, kOut>(w, scale, scale_type, out, rows, cols, s);
        case 6: return launch_convrot<6, kOut>(w, scale, scale_type, out, rows, cols, s);
        case 7: return launch_convrot<7, kOut>(w, scale, scale_type, out, rows, cols, s);
        default: return launch_convrot<8, kOut>(w, scale, scale_type, out, rows, cols, s);
    }
}

// ---------------------------------------------------------------------- svdq.nvfp4

// One run of 16 columns of row i a thread (cols % 16 == 0): the nvfp4 value, · c_i, · p_j,
// then `+ up[i, r] · down[r, j]` for r = 0 .. R−1, each product rounded before its add
// (internal/decode_schemes.py:464-489).
template <int kOut>
__global__ __launch_bounds__(256) void svdq_decode_kernel(SvdqDecode a) {
    const int64_t runs = a.rows * a.cols / 16;
    const int64_t run = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (run >= runs) return;
    const int64_t i = run / (a.cols / 16), j0 = (run % (a.cols / 16)) * 16;
    const uint8_t* packed = a.weight + run * 8;
    const float g = a.scale_2[0];
    TableDecode grid{};
    grid.grid = kGridBlocks;
    grid.block = 16;
    grid.tiled = a.tiled;
    grid.cols = a.cols;
    const float s = e4m3_value(a.scale[grid_index(grid, i, j0)]);
    const float c = a.channel ? num_at(a.channel, a.channel_type, i) : 1.0f;
    float v[16];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const uint32_t byte = packed[k];
        const uint32_t first = a.high_first ? byte >> 4 : byte & 15u;
        const uint32_t second = a.high_first ? byte & 15u : byte >> 4;
        v[2 * k] = table_law(a.divide ? kSecondDivide : kSecondMultiply, e2m1_value(first), s, g);
        v[2 * k + 1] = table_law(a.divide ? kSecondDivide : kSecondMultiply, e2m1_value(second), s, g);
    }
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        if (a.channel) v[k] = v[k] * c;
        v[k] = v[k] * num_at(a.smooth, a.smooth_type, j0 + k);
    }
    for (int r = 0; r < a.rank; ++r) {
        const float u = num_at(a.up, a.up_type, i * a.rank + r);
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const float prod = u * num_at(a.down, a.down_type, static_cast<int64_t>(r) * a.cols + j0 + k);
            v[k] = v[k] + prod;
        }
    }
#pragma unroll
    for (int k = 0; k < 16; ++k) store_one<kOut>(a.out, run * 16 + k, v[k]);
}

}  // namespace

hipError_t decode_table(const TableDecode& a, int code, int out_type, int matrices, hipStream_t s) {
    switch (code) {
        case kCodeI8: return table_out<kCodeI8>(a, out_type, matrices, s);
        case kCodeE4m3: return table_out<kCodeE4m3>(a, out_type, matrices, s);
        case kCodeE5m2: return table_out<kCodeE5m2>(a, out_type, matrices, s);
        default: return table_out<kCodeE2m1>(a, out_type, matrices, s);
    }
}

hipError_t decode_convrot(const int8_t* w, const void* scale, int scale_type, void* out, int out_type,
                          int64_t rows, int64_t cols, int digits, hipStream_t s) {
    switch (out_type) {
        case kNumF32: return convrot_digits<kNumF32>(w, scale, scale_type, out, rows, cols, digits, s);
        case kNumBf16: return convrot_digits<kNumBf16>(w, scale, scale_type, out, rows, cols, digits, s);
        default: return convrot_digits<kNumF16>(w, scale, scale_type, out, rows, cols, digits, s);
    }
}

hipError_t decode_svdq(const SvdqDecode& a, int out_type, hipStream_t s) {
    const int64_t blocks = (a.rows * a.cols / 16 + 255) / 256;
    switch (out_type) {
        case kNumF32:
            hipLaunchKernelGGL(svdq_decode_kernel<kNumF32>, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, s, a);
            break;
        case kNumBf16:
            hipLaunchKernelGGL(svdq_decode_kernel<kNumBf16>, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, s, a);
            break;
        default:
            hipLaunchKernelGGL(svdq_decode_kernel<kNumF16>, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, s, a);
    }
    return hipGetLastError();
}

}  // namespace cozyq
