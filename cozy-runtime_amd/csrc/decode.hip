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

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Two floats → two bf16 in one word, first in the low half: v_cvt_pk_bf16_f32, round to
// nearest even (NaN stays NaN).
__device__ __forceinline__ uint32_t bf16_pair(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
}

template <bool kStream>
__device__ __forceinline__ void put16(u32x4* dst, u32x4 v) {
    if constexpr (kStream) __builtin_nontemporal_store(v, dst);
    else *dst = v;
}

// 16 outputs from element `idx` on, as 16-byte stores; `kStream` marks them non-temporal (a
// decoded weight is written once), which pays where a wave's stores fill whole lines together
// and costs where each lane writes a line of its own.
template <int kOut, bool kStream = true>
__device__ __forceinline__ void store16(void* out, int64_t idx, const float (&v)[16]) {
    if constexpr (kOut == kNumF32) {
        u32x4* dst = reinterpret_cast<u32x4*>(static_cast<float*>(out) + idx);
#pragma unroll
        for (int k = 0; k < 4; ++k)
            put16<kStream>(dst + k, u32x4{bits_of(v[4 * k]), bits_of(v[4 * k + 1]), bits_of(v[4 * k + 2]),
                                          bits_of(v[4 * k + 3])});
    } else {
        uint32_t w[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            if constexpr (kOut == kNumBf16) w[k] = bf16_pair(v[2 * k], v[2 * k + 1]);
            else w[k] = narrow<true>(v[2 * k]) | (static_cast<uint32_t>(narrow<true>(v[2 * k + 1])) << 16);
        }
        u32x4* dst = reinterpret_cast<u32x4*>(static_cast<uint16_t*>(out) + idx);
        put16<kStream>(dst, u32x4{w[0], w[1], w[2], w[3]});
        put16<kStream>(dst + 1, u32x4{w[4], w[5], w[6], w[7]});
    }
}

// The values of 16 one-byte codes held in four words, first code in the low byte: E4M3 and E5M2
// through gfx950's v_cvt_pk_f32_fp8 / v_cvt_pk_f32_bf8 (OCP formats, exact, NaN and infinity
// kept), int8 by sign extension.
template <int kCode>
__device__ __forceinline__ void values16(const uint32_t (&w)[4], float (&v)[16]) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        if constexpr (kCode == kCodeI8) {
#pragma unroll
            for (int b = 0; b < 4; ++b) v[4 * q + b] = static_cast<float>(static_cast<int8_t>(w[q] >> (8 * b)));
        } else {
            f32x2 lo, hi;
            if constexpr (kCode == kCodeE4m3) {
                lo = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w[q]), false);
                hi = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w[q]), true);
            } else {
                lo = __builtin_amdgcn_cvt_pk_f32_bf8(static_cast<int>(w[q]), false);
                hi = __builtin_amdgcn_cvt_pk_f32_bf8(static_cast<int>(w[q]), true);
            }
            v[4 * q] = lo.x;
            v[4 * q + 1] = lo.y;
            v[4 * q + 2] = hi.x;
            v[4 * q + 3] = hi.y;
        }
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

// A wave's 64 runs of 16 outputs leave through LDS: each lane writes its run (2 or 4 16-byte
// chunks), then store k of the wave writes chunks [64k, 64k + 64) — 1 KB of whole lines — as
// non-temporal stores. Chunks of runs at or past `runs` are not stored.
template <int kOut>
__device__ __forceinline__ void store_runs(void* out, int64_t wave_run, int64_t runs, const float (&v)[16],
                                           u32x4* lds, int lane) {
    constexpr int kChunks = kOut == kNumF32 ? 4 : 2;
    u32x4 c[kChunks];
    if constexpr (kOut == kNumF32) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
            c[q] = u32x4{bits_of(v[4 * q]), bits_of(v[4 * q + 1]), bits_of(v[4 * q + 2]), bits_of(v[4 * q + 3])};
    } else {
        uint32_t w[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            if constexpr (kOut == kNumBf16) w[k] = bf16_pair(v[2 * k], v[2 * k + 1]);
            else w[k] = narrow<true>(v[2 * k]) | (static_cast<uint32_t>(narrow<true>(v[2 * k + 1])) << 16);
        }
        c[0] = u32x4{w[0], w[1], w[2], w[3]};
        c[1] = u32x4{w[4], w[5], w[6], w[7]};
    }
#pragma unroll
    for (int q = 0; q < kChunks; ++q) lds[lane * kChunks + (q ^ (lane & (kChunks - 1)))] = c[q];
    __builtin_amdgcn_wave_barrier();
    u32x4* base = reinterpret_cast<u32x4*>(static_cast<uint8_t*>(out) + wave_run * 16 * (kOut == kNumF32 ? 4 : 2));
#pragma unroll
    for (int k = 0; k < kChunks; ++k) {
        const int chunk = 64 * k + lane, owner = chunk / kChunks, q = chunk % kChunks;
        const u32x4 word = lds[owner * kChunks + (q ^ (owner & (kChunks - 1)))];
        if (wave_run + owner < runs) __builtin_nontemporal_store(word, base + chunk);
    }
}

// Runs of 16 elements: rows are whole runs (cols % 16 == 0), the parts 16-byte aligned (8 for
// packed E2M1) and the block size, if any, a multiple of 16, so a run has one block scale.
template <int kCode, int kOut>
__global__ __launch_bounds__(256) void table_run_kernel(TableDecode a) {
    const int64_t e = blockIdx.y;
    const int64_t runs = a.rows * a.cols / 16;
    const int64_t run = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    __shared__ u32x4 stage[4 * 64 * (kOut == kNumF32 ? 4 : 2)];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t wave_run = static_cast<int64_t>(blockIdx.x) * 256 + 64 * wave;
    if (wave_run >= runs) return;  // whole waves only: the stores below exchange within a wave
    const bool live = run < runs;
    const int64_t at = live ? run : wave_run;  // idle lanes decode the wave's first run, unstored
    const int64_t i = at / (a.cols / 16), j0 = (at % (a.cols / 16)) * 16;
    const uint8_t* weight = a.weight + e * a.weight_stride;
    const void* scale = static_cast<const uint8_t*>(a.scale) + e * a.scale_stride * a.scale_size;
    const float g = a.second ? a.scale_2[e * a.scale_2_step] : 1.0f;
    float v[16];
    if constexpr (kCode == kCodeE2m1) {
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        const u32x2 raw = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(weight + at * 8));
        // v_cvt_scalef32_pk_f32_fp4 at scale 1: a byte's low nibble to .x, its high one to .y.
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int word = static_cast<int>(k < 4 ? raw.x : raw.y);
            f32x2 pair;
            switch (k & 3) {
                case 0: pair = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(word, 1.0f, 0); break;
                case 1: pair = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(word, 1.0f, 1); break;
                case 2: pair = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(word, 1.0f, 2); break;
                default: pair = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(word, 1.0f, 3);
            }
            v[2 * k] = a.high_first ? pair.y : pair.x;
            v[2 * k + 1] = a.high_first ? pair.x : pair.y;
        }
    } else {
        const u32x4 raw = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(weight + at * 16));
        const uint32_t w4[4] = {raw.x, raw.y, raw.z, raw.w};
        values16<kCode>(w4, v);
    }
    if (a.grid == kGridCol) {
#pragma unroll
        for (int k = 0; k < 16; ++k) v[k] = table_law(a.second, v[k], num_at(scale, a.scale_type, j0 + k), g);
    } else {
        const float s = num_at(scale, a.scale_type, grid_index(a, i, j0));
#pragma unroll
        for (int k = 0; k < 16; ++k) v[k] = table_law(a.second, v[k], s, g);
    }
    if (a.post_mode == kPostOne) {
        const float p = num_at(a.post, a.post_type, 0);
#pragma unroll
        for (int k = 0; k < 16; ++k) v[k] = v[k] * p;
    } else if (a.post_mode == kPostColumn) {
#pragma unroll
        for (int k = 0; k < 16; ++k) v[k] = v[k] * num_at(a.post, a.post_type, j0 + k);
    }
    void* out = static_cast<uint8_t*>(a.out) + e * a.out_stride * (kOut == kNumF32 ? 4 : 2);
    store_runs<kOut>(out, wave_run, runs, v, stage + wave * 64 * (kOut == kNumF32 ? 4 : 2), lane);
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

// A plain DPP move. (Asked with bound_ctrl set, the backend folds the move into the consuming
// v_add_u32_dpp / v_subrev_u32_dpp; that form produced wrong sums on gfx950 in this kernel, so
// the moves stay separate.)
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

    constexpr float kInv = 1.0f / static_cast<float>(1 << kDigits);  // 1/√(4^k), exact
    constexpr int kGroup = 1 << (2 * kDigits);
    float s = active ? num_at(scale, scale_type, base / cols) : 0.0f;
    float f[64];
#pragma unroll
    for (int r = 0; r < 64; ++r) {
        if constexpr (kGroup < 64) {  // groups of 4 or 16 may start a new row inside the lane
            if (active && r % kGroup == 0 && r > 0) s = num_at(scale, scale_type, (base + r) / cols);
        }
        f[r] = (static_cast<float>(v[r]) * s) * kInv;
    }
    if constexpr (kOut == kNumF32 || kDigits > 6) {
        if (!active) return;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            float run[16];
#pragma unroll
            for (int b = 0; b < 16; ++b) run[b] = f[16 * k + b];
            store16<kOut, false>(out, base + 16 * k, run);
        }
    } else {
        // 16-bit outputs leave through LDS: each lane writes its 128 bytes, then store k of the
        // wave writes bytes [1024k, 1024k + 1024) of the wave's 8 KB, whole lines at once, so the
        // stores can stream. 16-byte chunks are XOR-swizzled by lane to spread LDS banks.
        __shared__ u32x4 stage[4 * 64 * 8];
        u32x4* mine = stage + wave * 512;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            uint32_t w[4];
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const float lo = f[8 * c + 2 * b], hi = f[8 * c + 2 * b + 1];
                if constexpr (kOut == kNumBf16) w[b] = bf16_pair(lo, hi);
                else w[b] = narrow<true>(lo) | (static_cast<uint32_t>(narrow<true>(hi)) << 16);
            }
            mine[lane * 8 + (c ^ (lane & 7))] = u32x4{w[0], w[1], w[2], w[3]};
        }
        __builtin_amdgcn_wave_barrier();
        const int64_t wave_base = block_base + 4096 * wave;  // first element of the wave
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int owner = 8 * k + lane / 8, chunk = lane % 8;  // lane `owner`'s chunk
            const u32x4 word = mine[owner * 8 + (chunk ^ (owner & 7))];
            const int64_t first = wave_base + 512 * k + 8 * lane;
            if (first < total)
                __builtin_nontemporal_store(word, reinterpret_cast<u32x4*>(static_cast<uint16_t*>(out) + first));
        }
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

// A workgroup takes 32 rows × 256 columns, a thread 2 rows × 16 columns (cols % 16 == 0): the
// nvfp4 value, · c_i, · p_j, then `+ up[i, r] · down[r, j]` for r = 0 .. R−1, each product
// rounded before its add (internal/decode_schemes.py:464-489). The factors pass through LDS as
// float32, 16 ranks at a time: down [16][256] (a run's four 16-byte pieces 256 bytes apart, so
// the 16 runs of a row read distinct banks) and up transposed [16][32]. Every global read is a
// bounded buffer load (past the end reads 0) issued without a branch; what rows or columns past
// the matrix read is never stored.
constexpr int kSvdqRows = 32, kSvdqCols = 256, kSvdqRanks = 16, kSvdqRowsPer = 2;

// N elements of a float32 / bf16 / f16 part at element offsets `off`, each clamped into the
// part's `n` elements, issued back to back.
template <int N>
__device__ __forceinline__ void load_nums(const void* base, int type, int64_t n, const int64_t (&off)[N],
                                          float (&out)[N]) {
    if (type == kNumF32) {
        const float* f = static_cast<const float*>(base);
#pragma unroll
        for (int k = 0; k < N; ++k) out[k] = f[off[k] < n ? off[k] : n - 1];
    } else {
        const uint16_t* h = static_cast<const uint16_t*>(base);
        uint16_t x[N];
#pragma unroll
        for (int k = 0; k < N; ++k) x[k] = h[off[k] < n ? off[k] : n - 1];
#pragma unroll
        for (int k = 0; k < N; ++k) out[k] = type == kNumBf16 ? widen<false>(x[k]) : widen<true>(x[k]);
    }
}


template <int kOut>
__global__ __launch_bounds__(256) void svdq_decode_kernel(SvdqDecode a) {
    __shared__ float down_lds[kSvdqRanks][kSvdqCols];
    __shared__ float up_lds[kSvdqRanks][kSvdqRows];
    const int t = threadIdx.x, run = t % 16, group = t / 16;
    const int64_t row0 = static_cast<int64_t>(blockIdx.y) * kSvdqRows;
    const int64_t col0 = static_cast<int64_t>(blockIdx.x) * kSvdqCols;
    const int64_t j0 = col0 + 16 * run;
    const float g = a.scale_2[0];
    const int second = a.divide ? kSecondDivide : kSecondMultiply;
    TableDecode grid{};
    grid.grid = kGridBlocks;
    grid.block = 16;
    grid.tiled = a.tiled;
    grid.cols = a.cols;
    // Rows and columns past the matrix read the last row's and column's parts: never stored.
    const int64_t jc = j0 < a.cols ? j0 : a.cols - 16;
    float p[16];
    {
        int64_t off[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) off[k] = jc + k;
        load_nums<16>(a.smooth, a.smooth_type, a.cols, off, p);
    }
    float v[kSvdqRowsPer][16];
#pragma unroll
    for (int m = 0; m < kSvdqRowsPer; ++m) {
        const int64_t r = row0 + kSvdqRowsPer * group + m;
        const int64_t i = r < a.rows ? r : a.rows - 1;
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        const u32x2 raw = *reinterpret_cast<const u32x2*>(a.weight + (i * a.cols + jc) / 2);
        const float s = e4m3_value(a.scale[grid_index(grid, i, jc)]);
        const float c = a.channel ? num_at(a.channel, a.channel_type, i) : 1.0f;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t byte = ((k < 4 ? raw.x : raw.y) >> (8 * (k & 3))) & 0xffu;
            const uint32_t first = a.high_first ? byte >> 4 : byte & 15u;
            const uint32_t next = a.high_first ? byte & 15u : byte >> 4;
            v[m][2 * k] = table_law(second, e2m1_value(first), s, g);
            v[m][2 * k + 1] = table_law(second, e2m1_value(next), s, g);
        }
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            if (a.channel) v[m][k] = v[m][k] * c;
            v[m][k] = v[m][k] * p[k];
        }
    }

    const int pos = 64 * ((t % 16) / 4) + 4 * (t / 16) + t % 4;  // column t's slot in down_lds
    constexpr int kUpPer = kSvdqRanks * kSvdqRows / 256;  // up entries a thread stages
    for (int r0 = 0; r0 < a.rank; r0 += kSvdqRanks) {
        const int chunk = a.rank - r0 < kSvdqRanks ? a.rank - r0 : kSvdqRanks;
        float x[kSvdqRanks], y[kUpPer];
        {
            int64_t off[kSvdqRanks];
#pragma unroll
            for (int rr = 0; rr < kSvdqRanks; ++rr) off[rr] = (r0 + rr) * a.cols + col0 + t;
            load_nums<kSvdqRanks>(a.down, a.down_type, a.rank * a.cols, off, x);
            int64_t uoff[kUpPer];
#pragma unroll
            for (int q = 0; q < kUpPer; ++q) {
                const int e = t + 256 * q;
                uoff[q] = (row0 + e / kSvdqRanks) * a.rank + r0 + e % kSvdqRanks;
            }
            load_nums<kUpPer>(a.up, a.up_type, a.rows * a.rank, uoff, y);
        }
        __syncthreads();  // the previous chunk's reads are done
#pragma unroll
        for (int rr = 0; rr < kSvdqRanks; ++rr) down_lds[rr][pos] = x[rr];
#pragma unroll
        for (int q = 0; q < kUpPer; ++q) {
            const int e = t + 256 * q;
            up_lds[e % kSvdqRanks][e / kSvdqRanks] = y[q];
        }
        __syncthreads();
        for (int rr = 0; rr < chunk; ++rr) {
            const float2 u = *reinterpret_cast<const float2*>(&up_lds[rr][kSvdqRowsPer * group]);
            float d[16];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float4 z = *reinterpret_cast<const float4*>(&down_lds[rr][64 * k + 4 * run]);
                d[4 * k] = z.x;
                d[4 * k + 1] = z.y;
                d[4 * k + 2] = z.z;
                d[4 * k + 3] = z.w;
            }
            const float um[kSvdqRowsPer] = {u.x, u.y};
#pragma unroll
            for (int m = 0; m < kSvdqRowsPer; ++m) {
#pragma unroll
                for (int k = 0; k < 16; ++k) {
                    const float prod = um[m] * d[k];
                    v[m][k] = v[m][k] + prod;
                }
            }
        }
    }

    const bool cols_in = j0 < a.cols;
#pragma unroll
    for (int m = 0; m < kSvdqRowsPer; ++m) {
        const int64_t i = row0 + kSvdqRowsPer * group + m;
        if (cols_in && i < a.rows) store16<kOut, false>(a.out, i * a.cols + j0, v[m]);
    }
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
    const dim3 grid(static_cast<uint32_t>((a.cols + kSvdqCols - 1) / kSvdqCols),
                    static_cast<uint32_t>((a.rows + kSvdqRows - 1) / kSvdqRows));
    if (grid.y > 65535) return hipErrorInvalidValue;
    switch (out_type) {
        case kNumF32: hipLaunchKernelGGL(svdq_decode_kernel<kNumF32>, grid, dim3(256), 0, s, a); break;
        case kNumBf16: hipLaunchKernelGGL(svdq_decode_kernel<kNumBf16>, grid, dim3(256), 0, s, a); break;
        default: hipLaunchKernelGGL(svdq_decode_kernel<kNumF16>, grid, dim3(256), 0, s, a);
    }
    return hipGetLastError();
}

}  // namespace cozyq
