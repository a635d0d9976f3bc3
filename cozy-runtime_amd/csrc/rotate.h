// The block-Hadamard rotation's LDS phases, shared by the rotate+quantize pass (quantize.hip)
// and the fused int8 decode GEMV (gemv.hip): the stage order and float32 association of the
// reference's law (internal/encoding/formats.py:657-671), so the rotated values, and hence the
// int8 codes, are bit-exact to the CPU law.
#pragma once

#include "common.h"

namespace cozyq {

// The rotated kernel stages 4096 elements of a row through LDS at a time: 16 groups of 256 or
// 32 of 128, one phase-3 task (16 contiguous outputs) per thread per chunk.
constexpr int kChunk = 4096;

// LDS position of element `lo` (0..15) of 16-run `hi` of group `g`: runs padded to 20 floats and
// groups by 16 more, so both the strided (phase 2) and the contiguous (phase 3) reads of a wave
// fall on distinct banks.
template <int kRot>
struct Layout {
    static constexpr int kRuns = kRot / 16;             // 16-runs per group
    static constexpr int kGroupStride = kRuns * 20 + 16;
    static constexpr int kGroups = kChunk / kRot;       // groups per chunk
    static constexpr int kFloats = kGroups * kGroupStride;
    __device__ static int at(int g, int hi, int lo) { return g * kGroupStride + hi * 20 + lo; }
};

__device__ __forceinline__ void h4(float& a, float& b, float& c, float& d) {
    // formats.py:670: (a+b+c-d, a+b-c+d, a-b+c+d, b+c+d-a), each left to right.
    const float o0 = a + b + c - d;
    const float o1 = a + b - c + d;
    const float o2 = a - b + c + d;
    const float o3 = b + c + d - a;
    a = o0; b = o1; c = o2; d = o3;
}

// Phases 2 and 3 of one chunk of `width` elements (a multiple of kRot) that phase 1 has written
// into `lds` (Layout<kRot>): a barrier, the outer two stages (thread = one column of a group's
// runs), a barrier, then the inner two stages on the thread's contiguous 16-run (group
// tid / runs, run tid % runs) into `w`, scaled by 1/16 for kRot = 256, and its |max| into
// `amax`. Threads past the chunk's groups leave `w` untouched. The caller barriers before
// writing `lds` again.
template <int kRot, int kThreads>
__device__ __forceinline__ void rotate_lds_chunk(float* lds, int width, int tid, float (&w)[16],
                                                 float& amax) {
    using L = Layout<kRot>;
    __syncthreads();
    // Phase 2: the outer two stages; thread holds one column `t` of a group's runs.
    const int groups = width / kRot;
    for (int task = tid; task < groups * 16; task += kThreads) {
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
    __syncthreads();
    // Phase 3: the inner two stages on one contiguous 16-run per thread.
    const int g = tid / L::kRuns, hi = tid % L::kRuns;
    if (g < groups) {
        const float* src = lds + L::at(g, hi, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 f = *reinterpret_cast<const float4*>(src + 4 * i);
            w[4 * i] = f.x; w[4 * i + 1] = f.y; w[4 * i + 2] = f.z; w[4 * i + 3] = f.w;
        }
#pragma unroll
        for (int d4 = 0; d4 < 4; ++d4) h4(w[d4], w[4 + d4], w[8 + d4], w[12 + d4]);
#pragma unroll
        for (int d3 = 0; d3 < 4; ++d3) h4(w[4 * d3], w[4 * d3 + 1], w[4 * d3 + 2], w[4 * d3 + 3]);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            if constexpr (kRot == 256) w[i] = w[i] * 0.0625f;  // .mul_(1.0 / 16), exact
            amax = fmaxf(amax, fabsf(w[i]));
        }
    }
}

// torch.round(v / s).clamp_(-127, 127): the correctly rounded quotient, half to even, clamp.
// `rs` = RN(1/s) for a finite s takes the quotient on div_rn; an infinite s (a row holding an
// infinity) divides.
template <bool kFast>
__device__ __forceinline__ int8_t q8(float v, float scale, float rs) {
    float r = __builtin_rintf(kFast ? div_rn(v, scale, rs) : v / scale);
    r = fminf(fmaxf(r, -127.0f), 127.0f);
    return static_cast<int8_t>(static_cast<int>(r));
}

}  // namespace cozyq
