// Per-token int8 of rows of at most kRowMaxK elements, one wave per row: the block-Hadamard
// rotation (256, 128 or none) and the row's quantization with no workgroup barrier.
//
// A lane loads 16-byte pieces l, l + 64, ... of the row (branch-free buffer loads; pieces past
// the row read as zeros), so a row's loads are eight instructions of whole lines a lane and a
// wave can hold the next row's loads in flight while it rotates the current one. The rotation
// runs through the wave's own LDS slice in passes of 2048 elements with the stage order and
// float32 association of the CPU law (internal/encoding/formats.py:657-671, the phases of
// rotate.h), so the codes and scales are bit-exact to it; the row maximum is a wave reduction.
#pragma once

#include <type_traits>

#include "common.h"
#include "rotate.h"

namespace cozyq {

constexpr int kRowMaxK = 4096;                 // longest row one wave quantizes
constexpr int kRowLoads = kRowMaxK / 512;      // 16-byte pieces a lane loads per row
constexpr int kRowPass = 2048;                 // elements a wave rotates through LDS per pass

template <int kRot>
struct PassLayout {
    static constexpr int kRuns = kRot / 16;              // 16-runs per group
    static constexpr int kGroupStride = kRuns * 20 + 16;  // padded as rotate.h's Layout
    static constexpr int kGroups = kRowPass / kRot;
    static constexpr int kFloats = kGroups * kGroupStride;
    __device__ static int at(int g, int hi, int lo) { return g * kGroupStride + hi * 20 + lo; }
};

// LDS floats one wave needs for rotation kRot (0: none).
template <int kRot>
constexpr int row_lds_floats() {
    if constexpr (kRot == 0) return 0;
    else return PassLayout<kRot>::kFloats;
}
template <int kRot>
constexpr int kRowLdsFloats = row_lds_floats<kRot>();

// Every LDS access the wave issued before has completed, and the compiler moves none across.
__device__ __forceinline__ void wave_lds_sync() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_view(const uint16_t* row, int K) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(row), 0, 2 * K, 0x00020000);
}

// The row's loads (row_view of a row of K 16-bit values).
__device__ __forceinline__ void row_loads(__amdgpu_buffer_rsrc_t view, int lane, uint4 (&raw)[kRowLoads]) {
#pragma unroll
    for (int i = 0; i < kRowLoads; ++i)
        raw[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(view, 16 * (lane + 64 * i), 0, 0));
}

template <bool kHalf>
__device__ __forceinline__ void unpack8(const uint4& raw, float* v) {
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[2 * i] = widen<kHalf>(static_cast<uint16_t>(w[i] & 0xffffu));
        v[2 * i + 1] = widen<kHalf>(static_cast<uint16_t>(w[i] >> 16));
    }
}

// Four codes of q8 packed little-endian.
template <bool kFast>
__device__ __forceinline__ uint32_t q8x4(const float* v, float scale, float rs) {
    uint32_t word = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j)
        word |= static_cast<uint32_t>(static_cast<uint8_t>(q8<kFast>(v[j], scale, rs))) << (8 * j);
    return word;
}

// One row (K <= kRowMaxK, K % max(kRot, 16) == 0) held in `raw` by row_loads, rotated by H_kRot
// (256: H4^⊗4 then ·1/16; 128: H2⊗H4^⊗3 unnormalized, 1/√128 folded into the scale; 0: none),
// quantized per row into `qr` and its scale into `*scale_out` (lane 0). `lds` is the wave's
// slice of kRowLdsFloats<kRot> floats.
template <bool kHalf, int kRot>
__device__ __forceinline__ void quantize_row_wave(const uint4 (&raw)[kRowLoads], int K, int lane,
                                                  float* lds, int8_t* qr, float* scale_out) {
    if constexpr (kRot == 0) {
        float v[kRowLoads][8];
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < kRowLoads; ++i) {
            unpack8<kHalf>(raw[i], v[i]);
#pragma unroll
            for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[i][j]));
        }
        amax = wave_max(amax);
        const float scale = fmaxf(amax / 127.0f, kScaleFloor);
        if (lane == 0) *scale_out = scale;
        const float rs = 1.0f / scale;
        auto emit = [&](auto fast) {
            constexpr bool kFast = decltype(fast)::value;
#pragma unroll
            for (int i = 0; i < kRowLoads; ++i) {
                const int e = 8 * (lane + 64 * i);
                if (e < K)
                    *reinterpret_cast<uint2*>(qr + e) =
                        make_uint2(q8x4<kFast>(v[i], scale, rs), q8x4<kFast>(v[i] + 4, scale, rs));
            }
        };
        if (scale < __builtin_huge_valf()) emit(std::true_type{}); else emit(std::false_type{});
    } else {
        using L = PassLayout<kRot>;
        constexpr int kPasses = kRowMaxK / kRowPass;
        constexpr int kPiecesPerPass = kRowPass / 8 / 64;  // 16-byte pieces a lane per pass
        constexpr int kRunsPerLane = kRowPass / 16 / 64;   // 16-runs a lane per pass
        float w[kPasses][kRunsPerLane][16];
        float amax = 0.0f;
#pragma unroll
        for (int p = 0; p < kPasses; ++p) {
            const int base = p * kRowPass;
            if (base >= K) break;
            const int width = min(kRowPass, K - base);
            const int groups = width / kRot;
            // Phase 1: the pass's pieces into LDS as floats.
#pragma unroll
            for (int i = 0; i < kPiecesPerPass; ++i) {
                const int e = 8 * (lane + 64 * i);  // within the pass
                if (e < width) {
                    float v[8];
                    unpack8<kHalf>(raw[p * kPiecesPerPass + i], v);
                    const int g = e / kRot, within = e % kRot;
                    float* dst = lds + L::at(g, within / 16, within % 16);
                    *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
                    *reinterpret_cast<float4*>(dst + 4) = make_float4(v[4], v[5], v[6], v[7]);
                }
            }
            wave_lds_sync();
            // Phase 2: the outer stages, a lane holding column t of a group's runs; the lane's
            // tasks unrolled so their LDS reads are in flight together.
            constexpr int kTasks = kRowPass / kRot * 16 / 64;
#pragma unroll
            for (int u = 0; u < kTasks; ++u) {
                const int task = lane + 64 * u;
                if (task >= groups * 16) break;
                const int g = task / 16, t = task % 16;
                float v[L::kRuns];
#pragma unroll
                for (int hi = 0; hi < L::kRuns; ++hi) v[hi] = lds[L::at(g, hi, t)];
                if constexpr (kRot == 256) {
#pragma unroll
                    for (int d2 = 0; d2 < 4; ++d2) h4(v[d2], v[4 + d2], v[8 + d2], v[12 + d2]);
#pragma unroll
                    for (int d1 = 0; d1 < 4; ++d1) h4(v[4 * d1], v[4 * d1 + 1], v[4 * d1 + 2], v[4 * d1 + 3]);
                } else {
#pragma unroll
                    for (int d2 = 0; d2 < 4; ++d2) {
                        const float a = v[d2], b = v[4 + d2];
                        v[d2] = a + b;
                        v[4 + d2] = a - b;
                    }
#pragma unroll
                    for (int d1 = 0; d1 < 2; ++d1) h4(v[4 * d1], v[4 * d1 + 1], v[4 * d1 + 2], v[4 * d1 + 3]);
                }
#pragma unroll
                for (int hi = 0; hi < L::kRuns; ++hi) lds[L::at(g, hi, t)] = v[hi];
            }
            wave_lds_sync();
            // Phase 3: the inner stages on contiguous 16-runs r = lane + 64·s.
#pragma unroll
            for (int s = 0; s < kRunsPerLane; ++s) {
                const int r = lane + 64 * s;
                float* o = w[p][s];
                if (r < groups * L::kRuns) {
                    const float* src = lds + L::at(r / L::kRuns, r % L::kRuns, 0);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float4 f = *reinterpret_cast<const float4*>(src + 4 * i);
                        o[4 * i] = f.x; o[4 * i + 1] = f.y; o[4 * i + 2] = f.z; o[4 * i + 3] = f.w;
                    }
#pragma unroll
                    for (int d4 = 0; d4 < 4; ++d4) h4(o[d4], o[4 + d4], o[8 + d4], o[12 + d4]);
#pragma unroll
                    for (int d3 = 0; d3 < 4; ++d3) h4(o[4 * d3], o[4 * d3 + 1], o[4 * d3 + 2], o[4 * d3 + 3]);
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        if constexpr (kRot == 256) o[i] = o[i] * 0.0625f;  // .mul_(1.0 / 16), exact
                        amax = fmaxf(amax, fabsf(o[i]));
                    }
                }
            }
            wave_lds_sync();  // the next pass (or row) writes the slice again
        }
        amax = wave_max(amax);
        const float scale = fmaxf(amax / 127.0f, kScaleFloor);
        if (lane == 0) *scale_out = kRot == 128 ? scale * 0.08838834764831845f : scale;
        const float rs = 1.0f / scale;
        auto emit = [&](auto fast) {
            constexpr bool kFast = decltype(fast)::value;
#pragma unroll
            for (int p = 0; p < kPasses; ++p)
#pragma unroll
                for (int s = 0; s < kRunsPerLane; ++s) {
                    const int at = p * kRowPass + 16 * (lane + 64 * s);
                    if (at < K)
                        *reinterpret_cast<uint4*>(qr + at) =
                            make_uint4(q8x4<kFast>(w[p][s], scale, rs), q8x4<kFast>(w[p][s] + 4, scale, rs),
                                       q8x4<kFast>(w[p][s] + 8, scale, rs), q8x4<kFast>(w[p][s] + 12, scale, rs));
                }
        };
        if (scale < __builtin_huge_valf()) emit(std::true_type{}); else emit(std::false_type{});
    }
}

}  // namespace cozyq
