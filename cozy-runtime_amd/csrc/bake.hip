// The LoRA bake on gfx950 (reference: `fused`, internal/lora_bake.py:775-815, and its Triton
// kernels :901-1053): a stored weight takes `up @ down` in place and is rounded back onto its
// own form — bf16 stochastically (16 noise bits added under the kept ones), f16 / f32 to
// nearest, fp8.rowwise E4M3 stochastically on the kept row scale, int8.convrot by a stochastic
// floor on the kept row scale (`down` rotated first, `rotate_factor_kernel`), canonical nvfp4 by
// stochastic E2M1 on its block grid (a block's E4M3 scale refitted only when its baked maximum
// outgrows 7/6 of it).
//
// Element (row, col)'s noise is Triton's Philox4x32-10 draw at counter row·cols + col (mod 2^32)
// under the seed, so a bake writes the bytes the reference's fused bake does for the same delta.
// The delta is one float32 FMA chain per element over ranks 0, 1, ... from +0.
//
// A workgroup of 256 lanes takes a 64-row × 128-column tile: lane (rg = tid/16, cg = tid%16)
// owns rows 4rg .. 4rg+3 and columns 4cg .. 4cg+3 and 64+4cg .. 64+4cg+3 (each 16-lane row of
// a wave reads 256 contiguous bytes of LDS per rank). `up` (transposed) and `down` are staged
// through LDS 32 ranks at a time. The hot part is the VALU: rank FMAs plus one Philox (ten
// rounds, two 32x32→64-bit multiplies each) per element, against a few bytes of HBM.
#include "common.h"
#include "kernels.h"

namespace cozyq {
namespace {

constexpr int kTileRows = 64, kTileCols = 128, kRankChunk = 32, kBakeThreads = 256;

// Philox4x32-10 (Salmon et al., SC'11) at counter (offset, 0, 0, 0) under key (k0, k1): the
// first output word, Triton's `tl.randint`.
__device__ __forceinline__ uint32_t philox_word(uint32_t offset, uint32_t k0, uint32_t k1) {
    uint32_t c0 = offset, c1 = 0, c2 = 0, c3 = 0;
#pragma unroll
    for (int round = 0; round < 10; ++round) {
        const uint64_t pb = static_cast<uint64_t>(0xCD9E8D57u) * c2;
        const uint64_t pa = static_cast<uint64_t>(0xD2511F53u) * c0;
        c0 = static_cast<uint32_t>(pb >> 32) ^ c1 ^ k0;
        c2 = static_cast<uint32_t>(pa >> 32) ^ c3 ^ k1;
        c1 = static_cast<uint32_t>(pb);
        c3 = static_cast<uint32_t>(pa);
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    return c0;
}

// Triton's `tl.rand` from a draw: the int32 view folded to non-negative (x < 0 → −x − 1),
// converted and scaled by the largest float32 that keeps (2^31 − 1)·scale under 1.
__device__ __forceinline__ float uniform(uint32_t word) {
    const int32_t x = static_cast<int32_t>(word);
    return static_cast<float>(x < 0 ? ~x : x) * 0x1.fffffep-32f;
}

// E4M3 byte → float32 with the reserved codes saturating to ±448.
__device__ __forceinline__ float e4m3_sat(uint32_t code) {
    const uint32_t field = (code >> 3) & 15u, mantissa = code & 7u;
    float magnitude = field == 0 ? static_cast<float>(mantissa) * 0.001953125f
                                 : static_cast<float>(mantissa + 8u) * float_of((field + 117u) << 23);
    if ((code & 127u) == 127u) magnitude = 448.0f;
    return code > 127u ? -magnitude : magnitude;
}

// float32 payload → E4M3 byte, saturating at 448: twenty noise bits added under the three kept
// mantissa bits and the rest truncated; below 2^-6 the value is lifted by 2^-6 into the binade
// whose step (2^-9) is the subnormal one, and lowered back by the code offset.
__device__ __forceinline__ uint32_t e4m3_stochastic(float payload, uint32_t noise) {
    const float magnitude = __builtin_fminf(__builtin_fabsf(payload), 448.0f);
    const bool small = magnitude < 0.015625f;
    const float lifted = small ? magnitude + 0.015625f : magnitude;
    const int kept = static_cast<int>((bits_of(lifted) + (noise >> 12)) >> 20);
    const int code = kept - (small ? 968 : 960);
    return static_cast<uint32_t>(payload < 0.0f ? (code | 128) : code);
}

// The least E4M3 code (0..126) whose value holds need ≥ 0: the float32 bits rounded up to three
// mantissa bits, or below 2^-6 a count of 2^-9 steps.
__device__ __forceinline__ uint32_t e4m3_at_least(float need) {
    const uint32_t bits = (bits_of(need) + 0xFFFFFu) & 0xFFF00000u;
    const int normal = ((static_cast<int>(bits >> 23) - 120) << 3) | static_cast<int>((bits >> 20) & 7u);
    const int code = need < 0.015625f ? static_cast<int>(__builtin_ceilf(__builtin_fmaxf(need * 512.0f, 0.0f)))
                                      : normal;
    return static_cast<uint32_t>(code < 0 ? 0 : (code > 126 ? 126 : code));
}

__device__ __forceinline__ float e2m1_of(uint32_t code) {
    const float index = static_cast<float>(code & 7u);
    const float magnitude = index < 4.0f ? index * 0.5f : (index < 6.0f ? index - 2.0f : (index < 7.0f ? 4.0f : 6.0f));
    return code >= 8u ? -magnitude : magnitude;
}

// |payload| (block units, saturating at 6) → E2M1 magnitude code, the upper neighbour when the
// draw is under the fraction of the step covered. The step is 0.5, 1 or 2, so dividing by it is
// multiplying by 2, 1 or 0.5: exact, and the same float32 results as the division.
__device__ __forceinline__ uint32_t e2m1_stochastic(float payload, float draw) {
    const float magnitude = __builtin_fminf(__builtin_fabsf(payload), 6.0f);
    const bool fine = magnitude < 2.0f, mid = magnitude < 4.0f;
    const float step = fine ? 0.5f : (mid ? 1.0f : 2.0f);
    const float per_step = fine ? 2.0f : (mid ? 1.0f : 0.5f);
    const float low = __builtin_fminf(__builtin_floorf(magnitude * per_step) * step, 6.0f);
    const float index = low < 2.0f ? low * 2.0f : (low < 4.0f ? low + 2.0f : (low < 6.0f ? 6.0f : 7.0f));
    return static_cast<uint32_t>(index + (draw < (magnitude - low) * per_step ? 1.0f : 0.0f));
}

template <int kCtrl>
__device__ __forceinline__ float dpp_f32(float v) {
    return float_of(static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(bits_of(v)), kCtrl, 0xf, 0xf, false)));
}

// The column of a lane's element j (0..7) within its tile.
__device__ __forceinline__ int tile_col(int cg, int j) { return (j < 4 ? 4 * cg : 64 + 4 * cg) + (j & 3); }

// acc[i][j] = Σ_r up[row_i, r] · down[r, col_j], one FMA chain in rank order from +0. Rows past
// `rows` and columns past `cols` stage zeros. Every lane of the workgroup calls it.
__device__ __forceinline__ void tile_delta(float (&acc)[4][8], const float* __restrict__ up,
                                           const float* __restrict__ down, int rows, int cols, int rank,
                                           int row0, int col0, float (*up_lds)[kTileRows],
                                           float (*down_lds)[kTileCols]) {
    const int tid = threadIdx.x, rg = tid >> 4, cg = tid & 15;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = 0.0f;
    for (int r0 = 0; r0 < rank; r0 += kRankChunk) {
        __syncthreads();  // the previous chunk is consumed
        for (int e = tid; e < kRankChunk * kTileRows; e += kBakeThreads) {
            const int k = e % kRankChunk, r = e / kRankChunk;
            const int row = row0 + r, rk = r0 + k;
            up_lds[k][r] = row < rows && rk < rank ? up[static_cast<int64_t>(row) * rank + rk] : 0.0f;
        }
        for (int e = tid; e < kRankChunk * kTileCols; e += kBakeThreads) {
            const int c = e % kTileCols, k = e / kTileCols;
            const int col = col0 + c, rk = r0 + k;
            down_lds[k][c] = col < cols && rk < rank ? down[static_cast<int64_t>(rk) * cols + col] : 0.0f;
        }
        __syncthreads();
        const int n = rank - r0 < kRankChunk ? rank - r0 : kRankChunk;
        for (int k = 0; k < n; ++k) {
            const f32x4 u = *reinterpret_cast<const f32x4*>(&up_lds[k][4 * rg]);
            const f32x4 d0 = *reinterpret_cast<const f32x4*>(&down_lds[k][4 * cg]);
            const f32x4 d1 = *reinterpret_cast<const f32x4*>(&down_lds[k][64 + 4 * cg]);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    acc[i][j] = __builtin_fmaf(u[i], d0[j], acc[i][j]);
                    acc[i][4 + j] = __builtin_fmaf(u[i], d1[j], acc[i][4 + j]);
                }
        }
    }
}

// Stored element types by form.
template <int kForm> struct Stored;
template <> struct Stored<kBakeBf16> { using T = uint16_t; };
template <> struct Stored<kBakeF16> { using T = uint16_t; };
template <> struct Stored<kBakeF32> { using T = float; };
template <> struct Stored<kBakeRowwise> { using T = uint8_t; };
template <> struct Stored<kBakeInt8> { using T = int8_t; };

// The nearest E4M3 byte of a payload, saturating at 448, ties to the even code; the sign bit is
// set for a negative payload only (so −0 stores +0), as the reference's nearest encoder does.
__device__ __forceinline__ uint32_t e4m3_nearest(float payload) {
    const uint32_t code = e4m3_rn(__builtin_fminf(__builtin_fabsf(payload), 448.0f));
    return payload < 0.0f ? (code | 128u) : code;
}

// |payload| (block units, saturating at 6) → the nearest E2M1 magnitude code, ties to the even
// code.
__device__ __forceinline__ uint32_t e2m1_nearest(float payload) {
    const float magnitude = __builtin_fminf(__builtin_fabsf(payload), 6.0f);
    const bool fine = magnitude < 2.0f, mid = magnitude < 4.0f;
    const float step = fine ? 0.5f : (mid ? 1.0f : 2.0f);
    const float per_step = fine ? 2.0f : (mid ? 1.0f : 0.5f);
    const float low = __builtin_fminf(__builtin_floorf(magnitude * per_step) * step, 6.0f);
    const float index = low < 2.0f ? low * 2.0f : (low < 4.0f ? low + 2.0f : (low < 6.0f ? 6.0f : 7.0f));
    const float fraction = (magnitude - low) * per_step;
    const uint32_t base = static_cast<uint32_t>(index);
    return base + ((fraction > 0.5f || (fraction == 0.5f && (base & 1u))) ? 1u : 0u);
}

// What a bake takes beyond the fused law (the reference's eager bake and `gain_rows`): a float32
// gain per row for plain and nvfp4 rows, dense float32 rows added to the delta (a LoKr's), and
// the flags kBakeNearest (round to nearest instead of stochastically) and kBakeNoDelta (the
// rows times their gain alone, no delta added).
struct Extra {
    const float* gain;
    const float* more;
    bool nearest, no_delta;
    const float* rescale;  // ROWWISE: each row's new scale (`refit` / `regrid`), or null to keep
    // nvfp4 `refit`: every block's scale refitted to peak·need_inv on the new second level
    bool refit;
    float level, need_inv;
};

// One element of a `_bake_kernel` form: the stored value (its bits), the delta, the row's unit
// (ROWWISE, INT8) or gain (plain, with kExtra), and the element's Philox counter → the new stored
// value. Without kExtra this is the fused law exactly; with it, plain rows are
// round(round(v·gain) + delta) and every form can round to nearest.
template <int kForm, bool kExtra>
__device__ __forceinline__ typename Stored<kForm>::T bake_one(typename Stored<kForm>::T v, float d, float unit,
                                                               float fresh, const Extra& x, uint32_t at, uint32_t k0,
                                                               uint32_t k1) {
    if constexpr (kForm == kBakeBf16 || kForm == kBakeF16 || kForm == kBakeF32) {
        float value;
        if constexpr (kForm == kBakeBf16) value = float_of(static_cast<uint32_t>(v) << 16);
        else if constexpr (kForm == kBakeF16) value = widen<true>(v);
        else value = v;
        if constexpr (kExtra) {
            value = value * unit;  // the row's gain (1 without one: exact)
            if (!x.no_delta) value = value + d;
        } else {
            value = value + d;
        }
        if constexpr (kForm == kBakeBf16) {
            if (kExtra && x.nearest) return bf16_rn(value);
            const uint32_t noise = philox_word(at, k0, k1);
            return static_cast<uint16_t>((bits_of(value) + (noise >> 16)) >> 16);
        } else if constexpr (kForm == kBakeF16) {
            return narrow<true>(value);
        } else {
            return value;
        }
    } else if constexpr (kForm == kBakeRowwise) {
        float payload;
        if (kExtra && x.rescale) {
            // `bake_rowwise` on a new grid (internal/lora_bake.py:340-352): the decoded row plus
            // the delta, over the row's new scale.
            payload = (e4m3_sat(v) * unit + d) / fresh;
        } else {
            payload = kExtra && x.no_delta ? e4m3_sat(v) : e4m3_sat(v) + d / unit;
        }
        if (kExtra && x.nearest) return static_cast<uint8_t>(e4m3_nearest(payload));
        return static_cast<uint8_t>(e4m3_stochastic(payload, philox_word(at, k0, k1)));
    } else {
        const float payload = kExtra && x.no_delta ? static_cast<float>(v) : static_cast<float>(v) + d / unit;
        const float stored = kExtra && x.nearest ? __builtin_rintf(payload)
                                                 : __builtin_floorf(payload + uniform(philox_word(at, k0, k1)));
        return static_cast<int8_t>(__builtin_fminf(__builtin_fmaxf(stored, -127.0f), 127.0f));
    }
}

// The delta of element (row, col) with the dense extra rows added (kExtra and `more` set).
template <bool kExtra>
__device__ __forceinline__ float with_more(float d, const Extra& x, int64_t at) {
    if constexpr (kExtra) {
        if (x.more) return d + x.more[at];
    }
    return d;
}

// kVec: cols % 4 == 0 and `data` aligned to four elements, so each lane's four-column group
// moves as one load and one store.
template <int kForm, bool kVec, bool kExtra>
__global__ __launch_bounds__(kBakeThreads) void bake_kernel(typename Stored<kForm>::T* __restrict__ data,
                                                            const float* __restrict__ scale,
                                                            const float* __restrict__ up,
                                                            const float* __restrict__ down, Extra x, int rows,
                                                            int cols, int rank, uint32_t seed) {
    using T = typename Stored<kForm>::T;
    __shared__ float up_lds[kRankChunk][kTileRows];
    __shared__ float down_lds[kRankChunk][kTileCols];
    const int row0 = blockIdx.y * kTileRows, col0 = blockIdx.x * kTileCols;
    float acc[4][8];
    tile_delta(acc, up, down, rows, cols, rank, row0, col0, up_lds, down_lds);
    const int rg = threadIdx.x >> 4, cg = threadIdx.x & 15;
    const uint32_t k1 = (seed >> 31) ? 0xFFFFFFFFu : 0u;  // the int32 seed sign-extended
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = row0 + 4 * rg + i;
        if (row >= rows) break;
        float unit = 1.0f, fresh = 1.0f;
        if constexpr (kForm == kBakeRowwise || kForm == kBakeInt8) unit = scale[row];
        else if (kExtra && x.gain) unit = x.gain[row];
        if constexpr (kForm == kBakeRowwise) {
            if (kExtra && x.rescale) fresh = x.rescale[row];
        }
        const int64_t line0 = static_cast<int64_t>(row) * cols;
        T* line = data + line0;
        const uint32_t line_at = static_cast<uint32_t>(static_cast<uint64_t>(row) * static_cast<uint64_t>(cols));
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int col = col0 + tile_col(cg, 4 * h);
            if (col >= cols) continue;
            if constexpr (kVec) {
                struct alignas(4 * sizeof(T)) Four { T v[4]; };
                Four four = *reinterpret_cast<const Four*>(line + col);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    four.v[e] = bake_one<kForm, kExtra>(four.v[e], with_more<kExtra>(acc[i][4 * h + e], x, line0 + col + e),
                                                        unit, fresh, x, line_at + col + e, seed, k1);
                *reinterpret_cast<Four*>(line + col) = four;
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (col + e < cols)
                        line[col + e] = bake_one<kForm, kExtra>(
                            line[col + e], with_more<kExtra>(acc[i][4 * h + e], x, line0 + col + e), unit, fresh,
                            x, line_at + col + e, seed, k1);
            }
        }
    }
}

// `bake_rowwise` with error feedback (internal/lora_bake.py:163-197 `encode_e4m3`, `feedback`):
// each row's payloads `(e4m3·scale + delta) / new` round to nearest, each element's rounding
// error carried into the next element of its 32-column run (a run's sum kept without a draw).
// The tile's payloads go through LDS, one lane walks each (row, run) in column order, and the
// codes come back through LDS to the lanes that own them. `fresh` is each row's scale after the
// bake (the kept one, or `refit` / `regrid`'s).
constexpr int kFeedbackRun = 32;

__global__ __launch_bounds__(kBakeThreads) void bake_feedback_kernel(uint8_t* __restrict__ data,
                                                                     const float* __restrict__ scale,
                                                                     const float* __restrict__ fresh,
                                                                     const float* __restrict__ up,
                                                                     const float* __restrict__ down,
                                                                     const float* __restrict__ more, int rows,
                                                                     int cols, int rank) {
    __shared__ float up_lds[kRankChunk][kTileRows];
    __shared__ float down_lds[kRankChunk][kTileCols];
    __shared__ float stage[kTileRows][kTileCols + 1];
    const int row0 = blockIdx.y * kTileRows, col0 = blockIdx.x * kTileCols;
    float acc[4][8];
    tile_delta(acc, up, down, rows, cols, rank, row0, col0, up_lds, down_lds);
    const int rg = threadIdx.x >> 4, cg = threadIdx.x & 15;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int rl = 4 * rg + i, row = row0 + rl;
        const float unit = row < rows ? scale[row] : 1.0f, now = row < rows ? fresh[row] : 1.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int cl = tile_col(cg, j), col = col0 + cl;
            float payload = 0.0f;  // columns past the end pad the run with zeros
            if (row < rows && col < cols) {
                const int64_t at = static_cast<int64_t>(row) * cols + col;
                const float d = more != nullptr ? acc[i][j] + more[at] : acc[i][j];
                payload = (e4m3_sat(data[at]) * unit + d) / now;
            }
            stage[rl][cl] = payload;
        }
    }
    __syncthreads();
    {
        const int rl = threadIdx.x >> 2, run = threadIdx.x & 3;  // 64 rows x 4 runs
        float carry = 0.0f;
        for (int k = 0; k < kFeedbackRun; ++k) {
            const int cl = run * kFeedbackRun + k;
            const float want = stage[rl][cl] + carry;
            const uint32_t code = e4m3_nearest(want);
            const float kept = e4m3_sat(code & 127u);
            carry = want - (code >= 128u ? -kept : kept);
            stage[rl][cl] = float_of(code);
        }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int rl = 4 * rg + i, row = row0 + rl;
        if (row >= rows) continue;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int cl = tile_col(cg, j), col = col0 + cl;
            if (col < cols) data[static_cast<int64_t>(row) * cols + col] = static_cast<uint8_t>(bits_of(stage[rl][cl]));
        }
    }
}

// `_bake_nvfp4_kernel`: codes [rows, cols/2] (element 2k in the low nibble), E4M3 block bytes
// [rows, cols/16], the float32 second level at `second`; cols % 16 == 0. A 16-column block is
// the four lanes cg = 4q .. 4q+3 of one half-row, so its maximum is a DPP quad reduction; every
// lane reaches it (rows or blocks past the end bake zeros and store nothing). Without kExtra the
// target is fma(e2m1, scale·level, delta), the fused law; with it, the eager law's separate
// roundings round(round(round(e2m1·(scale·level))·gain) + delta) (`bake_nvfp4`,
// internal/lora_bake.py:458-525), no delta under kBakeNoDelta, and nearest E2M1 on request.
template <bool kExtra>
__global__ __launch_bounds__(kBakeThreads) void bake_nvfp4_kernel(uint8_t* __restrict__ data, uint8_t* __restrict__ blocks,
                                                                  const float* __restrict__ second,
                                                                  const float* __restrict__ up,
                                                                  const float* __restrict__ down, Extra x, int rows,
                                                                  int cols, int rank, uint32_t seed) {
    __shared__ float up_lds[kRankChunk][kTileRows];
    __shared__ float down_lds[kRankChunk][kTileCols];
    const int row0 = blockIdx.y * kTileRows, col0 = blockIdx.x * kTileCols;
    float acc[4][8];
    tile_delta(acc, up, down, rows, cols, rank, row0, col0, up_lds, down_lds);
    const int rg = threadIdx.x >> 4, cg = threadIdx.x & 15;
    const uint32_t k1 = (seed >> 31) ? 0xFFFFFFFFu : 0u;
    const float level = second[0];
    const int width = cols / 2, count = cols / 16;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = row0 + 4 * rg + i;
        const float gain = kExtra && x.gain && row < rows ? x.gain[row] : 1.0f;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int col = col0 + tile_col(cg, 4 * h);
            const bool live = row < rows && col < cols;
            const int64_t pair = static_cast<int64_t>(row) * width + col / 2;
            const int64_t which = static_cast<int64_t>(row) * count + col / 16;
            const uint32_t codes = live ? (static_cast<uint32_t>(data[pair]) | (static_cast<uint32_t>(data[pair + 1]) << 8)) : 0u;
            const uint32_t kept = live ? static_cast<uint32_t>(blocks[which]) : 0u;
            const float scaled = e4m3_sat(kept) * level;
            float target[4];
            float peak = 0.0f;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float value = e2m1_of((codes >> (4 * e)) & 15u);
                if constexpr (kExtra) {
                    const float base = (value * scaled) * gain;
                    const float d = live ? with_more<true>(acc[i][4 * h + e], x, static_cast<int64_t>(row) * cols + col + e)
                                         : acc[i][4 * h + e];
                    target[e] = x.no_delta ? base : base + d;
                } else {
                    target[e] = __builtin_fmaf(value, scaled, acc[i][4 * h + e]);
                }
                peak = __builtin_fmaxf(peak, __builtin_fabsf(target[e]));
            }
            peak = __builtin_fmaxf(peak, dpp_f32<0xB1>(peak));  // quad_perm [1,0,3,2]
            peak = __builtin_fmaxf(peak, dpp_f32<0x4E>(peak));  // quad_perm [2,3,0,1]
            uint32_t block;
            float unit;
            if (kExtra && x.refit) {
                block = e4m3_at_least(peak * x.need_inv);
                unit = e4m3_sat(block) * x.level;
            } else {
                // The fused kernel divides by 6·level; the eager bake divides by a Python float,
                // which torch runs on the GPU as a multiply by the float32 reciprocal.
                const float need = kExtra ? peak * (1.0f / (6.0f * level)) : peak / (6.0f * level);
                const bool grown = need * 6.0f > e4m3_sat(kept) * 7.0f;
                block = grown ? e4m3_at_least(need) : kept;
                unit = e4m3_sat(block) * level;
            }
            const float den = unit > 0.0f ? unit : 1.0f;
            const uint32_t at = static_cast<uint32_t>(static_cast<uint64_t>(row) * static_cast<uint64_t>(cols) + col);
            uint32_t out = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t stored = (codes >> (4 * e)) & 15u;
                const float payload = kExtra && x.refit && unit == 0.0f ? 0.0f : target[e] / den;
                uint32_t nibble;
                if (kExtra && x.nearest) nibble = e2m1_nearest(payload);
                else nibble = e2m1_stochastic(payload, uniform(philox_word(at + e, seed, k1)));
                const bool negative = target[e] == 0.0f ? stored >= 8u : target[e] < 0.0f;
                out |= (nibble | (negative ? 8u : 0u)) << (4 * e);
            }
            if (live) {
                data[pair] = static_cast<uint8_t>(out);
                data[pair + 1] = static_cast<uint8_t>(out >> 8);
                if ((cg & 3) == 0) blocks[which] = static_cast<uint8_t>(block);
            }
        }
    }
}

// `norms` (internal/lora_bake.py:653-689): each row's L2 norm of the decoded stored weight plus
// `up @ down`, float32 out [rows]. One workgroup per 64 rows walks every 128-column tile in
// order, so a row's float64 sum of squares is the same on every call. kForm: a `_bake_kernel`
// form, or kBakeNvfp4 (codes at `data`, block bytes at `blocks`, level at `second`).

template <int kForm, bool kMax>
__global__ __launch_bounds__(kBakeThreads) void bake_norms_kernel(const void* __restrict__ data,
                                                                  const float* __restrict__ scale,
                                                                  const uint8_t* __restrict__ blocks,
                                                                  const float* __restrict__ second,
                                                                  const float* __restrict__ up,
                                                                  const float* __restrict__ down,
                                                                  const float* __restrict__ gain,
                                                                  const float* __restrict__ more, int rows, int cols,
                                                                  int rank, float* __restrict__ out) {
    __shared__ float up_lds[kRankChunk][kTileRows];
    __shared__ float down_lds[kRankChunk][kTileCols];
    const int row0 = blockIdx.x * kTileRows;
    const int rg = threadIdx.x >> 4, cg = threadIdx.x & 15;
    double sums[4] = {0.0, 0.0, 0.0, 0.0};
    for (int col0 = 0; col0 < cols; col0 += kTileCols) {
        float acc[4][8];
        tile_delta(acc, up, down, rows, cols, rank, row0, col0, up_lds, down_lds);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = row0 + 4 * rg + i;
            if (row >= rows) continue;
            float unit = 1.0f;
            if constexpr (kForm == kBakeRowwise || kForm == kBakeInt8) unit = scale[row];
            const float g = gain != nullptr ? gain[row] : 1.0f;
            const int64_t line0 = static_cast<int64_t>(row) * cols;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int col = col0 + tile_col(cg, j);
                if (col >= cols) continue;
                const int64_t at = line0 + col;
                float value;
                if constexpr (kForm == kBakeBf16) value = widen<false>(static_cast<const uint16_t*>(data)[at]);
                else if constexpr (kForm == kBakeF16) value = widen<true>(static_cast<const uint16_t*>(data)[at]);
                else if constexpr (kForm == kBakeF32) value = static_cast<const float*>(data)[at];
                else if constexpr (kForm == kBakeRowwise) value = e4m3_sat(static_cast<const uint8_t*>(data)[at]) * unit;
                else if constexpr (kForm == kBakeInt8) value = static_cast<float>(static_cast<const int8_t*>(data)[at]) * unit;
                else {
                    const uint32_t byte = static_cast<const uint8_t*>(data)[at >> 1];
                    const uint32_t code = (col & 1) ? (byte >> 4) : (byte & 15u);
                    value = e2m1_of(code) * (e4m3_sat(blocks[static_cast<int64_t>(row) * (cols / 16) + col / 16]) * second[0]);
                }
                // The eager target: the decoded row times its gain, plus the delta and the dense
                // rows, each step rounded on its own.
                if (gain != nullptr) value = value * g;
                const float d = more != nullptr ? acc[i][j] + more[at] : acc[i][j];
                const double t = static_cast<double>(value + d);
                if constexpr (kMax) sums[i] = __builtin_fmax(sums[i], __builtin_fabs(t));
                else sums[i] += t * t;
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        double v = sums[i];
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) {  // the 16 lanes of a row group
            const double other = __shfl_xor(v, off);
            v = kMax ? __builtin_fmax(v, other) : v + other;
        }
        const int row = row0 + 4 * rg + i;
        if (cg == 0 && row < rows) out[row] = static_cast<float>(kMax ? v : __builtin_sqrt(v));
    }
}

// A bake's accounting (`Stats`, `_account`, internal/lora_bake.py:249-268): from the weight before
// and after the bake and the same delta, per workgroup of 64 rows over every column tile in
// order, float64 sums of |target|², |delta|², |stored − target|², (stored − base)·delta, the
// saturated count, and the rank-space energies |delta @ downᵀ|², |(stored − target) @ downᵀ|²
// (the projections accumulated per row and rank in LDS in tile order). target = base + delta,
// both decoded as the eager reference decodes; `partial` receives kStatTerms doubles a workgroup.
constexpr int kStatTerms = 7, kStatRanks = 128;

struct StatsArgs {
    const void* before;
    const void* after;
    const float* scale_before;
    const float* scale_after;
    const uint8_t* blocks_before;
    const uint8_t* blocks_after;
    const float* second;
    const float* second_after;  // kBakeNvfp4: the level `after` decodes at (`refit` sets a new one)
    const float* gain;
    const float* more;
};

template <int kForm>
__device__ __forceinline__ float stat_value(const void* data, const float* scale, const uint8_t* blocks, float level,
                                            int64_t at, int row, int col, int cols) {
    if constexpr (kForm == kBakeBf16) return widen<false>(static_cast<const uint16_t*>(data)[at]);
    else if constexpr (kForm == kBakeF16) return widen<true>(static_cast<const uint16_t*>(data)[at]);
    else if constexpr (kForm == kBakeF32) return static_cast<const float*>(data)[at];
    else if constexpr (kForm == kBakeRowwise) return e4m3_sat(static_cast<const uint8_t*>(data)[at]) * scale[row];
    else if constexpr (kForm == kBakeInt8) return static_cast<float>(static_cast<const int8_t*>(data)[at]) * scale[row];
    else {
        const uint32_t byte = static_cast<const uint8_t*>(data)[at >> 1];
        const uint32_t code = (col & 1) ? (byte >> 4) : (byte & 15u);
        return e2m1_of(code) * (e4m3_sat(blocks[static_cast<int64_t>(row) * (cols / 16) + col / 16]) * level);
    }
}

template <int kForm>
__global__ __launch_bounds__(kBakeThreads) void bake_stats_kernel(StatsArgs a, const float* __restrict__ up,
                                                                  const float* __restrict__ down, int rows, int cols,
                                                                  int rank, double* __restrict__ partial) {
    __shared__ float up_lds[kRankChunk][kTileRows];
    __shared__ float down_lds[kRankChunk][kTileCols];
    __shared__ float proj[2][kTileRows][kStatRanks];  // delta and error projections, per row and rank
    __shared__ double red[kBakeThreads / 64][kStatTerms];
    const int row0 = blockIdx.x * kTileRows;
    const int tid = threadIdx.x, rg = tid >> 4, cg = tid & 15;
    const float level = kForm == kBakeNvfp4 ? a.second[0] : 1.0f;
    const float level_after = kForm == kBakeNvfp4 ? a.second_after[0] : 1.0f;
    double sum[5] = {0.0, 0.0, 0.0, 0.0, 0.0};  // target², delta², error², kept, saturated
    double effect = 0.0, effect_error = 0.0;
    // The rank-space projections are taken kStatRanks ranks at a time (LDS holds one slice per
    // row); each slice walks the columns again with the whole delta, and the element sums are
    // taken on the first walk only.
    for (int p0 = 0; p0 == 0 || p0 < rank; p0 += kStatRanks) {
        const int p1 = min(rank, p0 + kStatRanks);
        for (int e = tid; e < 2 * kTileRows * kStatRanks; e += kBakeThreads) (&proj[0][0][0])[e] = 0.0f;
        for (int col0 = 0; col0 < cols; col0 += kTileCols) {
            float acc[4][8];
            tile_delta(acc, up, down, rows, cols, rank, row0, col0, up_lds, down_lds);  // syncs before reuse
            float dv[4][8], ev[4][8];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = row0 + 4 * rg + i;
                const float gain = (kForm <= kBakeF32 || kForm == kBakeNvfp4) && a.gain && row < rows ? a.gain[row] : 1.0f;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int col = col0 + tile_col(cg, j);
                    dv[i][j] = 0.0f;
                    ev[i][j] = 0.0f;
                    if (row >= rows || col >= cols) continue;
                    const int64_t at = static_cast<int64_t>(row) * cols + col;
                    float base = stat_value<kForm>(a.before, a.scale_before, a.blocks_before, level, at, row, col, cols);
                    if constexpr (kForm <= kBakeF32 || kForm == kBakeNvfp4) base = base * gain;
                    const float d = a.more ? acc[i][j] + a.more[at] : acc[i][j];
                    const float target = base + d;
                    const float stored = stat_value<kForm>(a.after, a.scale_after, a.blocks_after, level_after, at, row, col, cols);
                    const float err = stored - target;
                    dv[i][j] = d;
                    ev[i][j] = err;
                    if (p0 != 0) continue;
                    sum[0] += static_cast<double>(target) * target;
                    sum[1] += static_cast<double>(d) * d;
                    sum[2] += static_cast<double>(err) * err;
                    sum[3] += static_cast<double>(stored - base) * static_cast<double>(d);
                    if constexpr (kForm == kBakeRowwise) {
                        sum[4] += __builtin_fabsf(target / a.scale_after[row]) > 464.0f ? 1.0 : 0.0;
                    } else if constexpr (kForm == kBakeInt8) {
                        const float code = static_cast<float>(static_cast<const int8_t*>(a.before)[at]);
                        sum[4] += __builtin_fabsf(code + d / a.scale_before[row]) > 127.5f ? 1.0 : 0.0;
                    } else if constexpr (kForm == kBakeNvfp4) {
                        const float unit = e4m3_sat(a.blocks_after[static_cast<int64_t>(row) * (cols / 16) + col / 16]) * level_after;
                        sum[4] += unit > 0.0f && __builtin_fabsf(target / unit) > 6.0f ? 1.0 : 0.0;
                    }
                }
            }
            // The slice's projections onto down's rows: each lane's 8 columns, then the 16 lanes
            // of a row group.
            for (int r = p0; r < p1; ++r) {
                float dcol[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int col = col0 + tile_col(cg, j);
                    dcol[j] = col < cols ? down[static_cast<int64_t>(r) * cols + col] : 0.0f;
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float pd = 0.0f, pe = 0.0f;
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        pd = __builtin_fmaf(dv[i][j], dcol[j], pd);
                        pe = __builtin_fmaf(ev[i][j], dcol[j], pe);
                    }
#pragma unroll
                    for (int off = 1; off < 16; off <<= 1) {
                        pd += __shfl_xor(pd, off);
                        pe += __shfl_xor(pe, off);
                    }
                    if (cg == 0) {
                        proj[0][4 * rg + i][r - p0] += pd;
                        proj[1][4 * rg + i][r - p0] += pe;
                    }
                }
            }
        }
        __syncthreads();
        for (int e = tid; e < kTileRows * kStatRanks; e += kBakeThreads) {
            const double pd = (&proj[0][0][0])[e], pe = (&proj[1][0][0])[e];
            effect += pd * pd;
            effect_error += pe * pe;
        }
        __syncthreads();  // the next slice clears the projections
    }
    double terms[kStatTerms] = {sum[0], sum[1], sum[2], sum[3], sum[4], effect, effect_error};
    const int wave = tid >> 6, lane = tid & 63;
#pragma unroll
    for (int t = 0; t < kStatTerms; ++t) {
        double v = terms[t];
        for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
        if (lane == 0) red[wave][t] = v;
    }
    __syncthreads();
    if (tid < kStatTerms) {
        double v = 0.0;
        for (int w = 0; w < kBakeThreads / 64; ++w) v += red[w][tid];
        partial[static_cast<int64_t>(blockIdx.x) * kStatTerms + tid] = v;
    }
}

// `rotate_factor`: each 256 columns of `down` times the regular Hadamard H4⊗H4⊗H4⊗H4, one
// 4-point stage per digit, outer digit (stride 64) first, each output evaluated left to right as
// (a+b+c−d, a+b−c+d, a−b+c+d, b+c+d−a), then 1/16. Four 256-groups per workgroup.
__global__ __launch_bounds__(256) void rotate_factor_kernel(const float* __restrict__ down, float* __restrict__ out,
                                                            int64_t groups) {
    __shared__ float lds[4][256];
    const int q = threadIdx.x >> 6, t = threadIdx.x & 63;
    const int64_t group = static_cast<int64_t>(blockIdx.x) * 4 + q;
    const bool live = group < groups;
    float* x = lds[q];
#pragma unroll
    for (int k = 0; k < 4; ++k) x[t + 64 * k] = live ? down[group * 256 + t + 64 * k] : 0.0f;
    __syncthreads();
#pragma unroll
    for (int stride = 64; stride >= 1; stride /= 4) {
        const int base = (t / stride) * 4 * stride + t % stride;
        const float a = x[base], b = x[base + stride], c = x[base + 2 * stride], d = x[base + 3 * stride];
        x[base] = ((a + b) + c) - d;
        x[base + stride] = ((a + b) - c) + d;
        x[base + 2 * stride] = ((a - b) + c) + d;
        x[base + 3 * stride] = ((b + c) + d) - a;
        __syncthreads();
    }
    if (live)
#pragma unroll
        for (int k = 0; k < 4; ++k) out[group * 256 + t + 64 * k] = x[t + 64 * k] * 0.0625f;
}

template <int kForm>
hipError_t launch_bake(void* data, const float* scale, const float* up, const float* down, const BakeOptions& o,
                       int rows, int cols, int rank, uint32_t seed, hipStream_t s) {
    using T = typename Stored<kForm>::T;
    const dim3 grid((cols + kTileCols - 1) / kTileCols, (rows + kTileRows - 1) / kTileRows), block(kBakeThreads);
    T* d = static_cast<T*>(data);
    const bool vec = cols % 4 == 0 && reinterpret_cast<uintptr_t>(data) % (4 * sizeof(T)) == 0;
    const Extra x{o.gain, o.more, (o.flags & kBakeNearest) != 0, (o.flags & kBakeNoDelta) != 0, o.rescale};
    const bool extra = o.gain || o.more || o.flags || o.rescale;
#define COZYQ_BAKE(V, E) hipLaunchKernelGGL((bake_kernel<kForm, V, E>), grid, block, 0, s, d, scale, up, down, x, rows, cols, rank, seed)
    if (vec) {
        if (extra) COZYQ_BAKE(true, true); else COZYQ_BAKE(true, false);
    } else {
        if (extra) COZYQ_BAKE(false, true); else COZYQ_BAKE(false, false);
    }
#undef COZYQ_BAKE
    return hipGetLastError();
}

template <int kForm>
hipError_t launch_norms(const void* data, const float* scale, const uint8_t* blocks, const float* second,
                        const float* up, const float* down, const float* gain, const float* more, int rows, int cols,
                        int rank, float* out, bool amax, hipStream_t s) {
    const dim3 grid((rows + kTileRows - 1) / kTileRows), block(kBakeThreads);
    if (amax)
        hipLaunchKernelGGL((bake_norms_kernel<kForm, true>), grid, block, 0, s, data, scale, blocks, second, up, down,
                           gain, more, rows, cols, rank, out);
    else
        hipLaunchKernelGGL((bake_norms_kernel<kForm, false>), grid, block, 0, s, data, scale, blocks, second, up, down,
                           gain, more, rows, cols, rank, out);
    return hipGetLastError();
}

}  // namespace

hipError_t bake(int form, void* data, const float* scale, const float* up, const float* down, const BakeOptions& o,
                int rows, int cols, int rank, uint32_t seed, hipStream_t s) {
    switch (form) {
        case kBakeBf16: return launch_bake<kBakeBf16>(data, scale, up, down, o, rows, cols, rank, seed, s);
        case kBakeF16: return launch_bake<kBakeF16>(data, scale, up, down, o, rows, cols, rank, seed, s);
        case kBakeF32: return launch_bake<kBakeF32>(data, scale, up, down, o, rows, cols, rank, seed, s);
        case kBakeRowwise: return launch_bake<kBakeRowwise>(data, scale, up, down, o, rows, cols, rank, seed, s);
        case kBakeInt8: return launch_bake<kBakeInt8>(data, scale, up, down, o, rows, cols, rank, seed, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t bake_nvfp4(uint8_t* data, uint8_t* blocks, const float* second, const float* up, const float* down,
                      const BakeOptions& o, int rows, int cols, int rank, uint32_t seed, hipStream_t s) {
    const dim3 grid((cols + kTileCols - 1) / kTileCols, (rows + kTileRows - 1) / kTileRows), block(kBakeThreads);
    Extra x{o.gain, o.more, (o.flags & kBakeNearest) != 0, (o.flags & kBakeNoDelta) != 0, nullptr, false, 0.0f, 0.0f};
    if (o.refit) {
        // The reference's float64 second level, stored as float32; a block's need is its peak
        // over 6·second as torch divides by a Python scalar: times the float32 reciprocal.
        x.refit = true;
        x.level = static_cast<float>(o.level);
        x.need_inv = 1.0f / static_cast<float>(6.0 * o.level);
    }
    if (o.gain || o.more || o.flags || o.refit)
        hipLaunchKernelGGL((bake_nvfp4_kernel<true>), grid, block, 0, s, data, blocks, second, up, down, x, rows, cols, rank, seed);
    else
        hipLaunchKernelGGL((bake_nvfp4_kernel<false>), grid, block, 0, s, data, blocks, second, up, down, x, rows, cols, rank, seed);
    return hipGetLastError();
}

hipError_t bake_norms(int form, const void* data, const float* scale, const uint8_t* blocks, const float* second,
                      const float* up, const float* down, const float* gain, const float* more, int rows, int cols,
                      int rank, float* out, bool amax, hipStream_t s) {
#define COZYQ_NORMS(F) \
    case F: return launch_norms<F>(data, scale, blocks, second, up, down, gain, more, rows, cols, rank, out, amax, s);
    switch (form) {
        COZYQ_NORMS(kBakeBf16)
        COZYQ_NORMS(kBakeF16)
        COZYQ_NORMS(kBakeF32)
        COZYQ_NORMS(kBakeRowwise)
        COZYQ_NORMS(kBakeInt8)
        COZYQ_NORMS(kBakeNvfp4)
        default: return hipErrorInvalidValue;
    }
#undef COZYQ_NORMS
}

hipError_t bake_feedback(uint8_t* data, const float* scale, const float* fresh, const float* up, const float* down,
                         const float* more, int rows, int cols, int rank, hipStream_t s) {
    const dim3 grid((cols + kTileCols - 1) / kTileCols, (rows + kTileRows - 1) / kTileRows), block(kBakeThreads);
    hipLaunchKernelGGL(bake_feedback_kernel, grid, block, 0, s, data, scale, fresh, up, down, more, rows, cols, rank);
    return hipGetLastError();
}

hipError_t bake_stats(int form, const BakeStats& st, const float* up, const float* down, int rows, int cols, int rank,
                      double* partial, hipStream_t s) {
    const StatsArgs a{st.before, st.after, st.scale_before, st.scale_after, st.blocks_before, st.blocks_after,
                      st.second, st.second_after != nullptr ? st.second_after : st.second, st.gain, st.more};
    const dim3 grid((rows + kTileRows - 1) / kTileRows), block(kBakeThreads);
#define COZYQ_STATS(F) \
    case F: hipLaunchKernelGGL((bake_stats_kernel<F>), grid, block, 0, s, a, up, down, rows, cols, rank, partial); break;
    switch (form) {
        COZYQ_STATS(kBakeBf16)
        COZYQ_STATS(kBakeF16)
        COZYQ_STATS(kBakeF32)
        COZYQ_STATS(kBakeRowwise)
        COZYQ_STATS(kBakeInt8)
        COZYQ_STATS(kBakeNvfp4)
        default: return hipErrorInvalidValue;
    }
#undef COZYQ_STATS
    return hipGetLastError();
}

hipError_t rotate_factor(const float* down, float* out, int64_t groups, hipStream_t s) {
    const dim3 grid(static_cast<unsigned>((groups + 3) / 4)), block(256);
    hipLaunchKernelGGL(rotate_factor_kernel, grid, block, 0, s, down, out, groups);
    return hipGetLastError();
}

}  // namespace cozyq
