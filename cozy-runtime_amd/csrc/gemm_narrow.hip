// The int8 and fp8 rowwise GEMMs on narrow tiles (configs 1..4), with the epilogues of the
// 256x256 kernel: int8 on v_mfma_i32_16x16x64_i8 (exact int32; the CPU law's (acc·xs)·ws, cast,
// then + bias in the output dtype, internal/int8_linear.py:445-448 and :276), fp8 on
// v_mfma_f32_16x16x128_f8f6f4 ((acc·xs)·ws + bias in float32, one cast). They serve grids the
// 256x256 tile would leave under-filled: few rows, where tiles of kTM x kTN spread the weight
// stream over hundreds of workgroups (at M = 256 the 58.7 MB fp8 weight is 7.3 us of HBM against
// 6 us of MFMA), and any shape with fewer than 160 256x256 tiles.
//
// A workgroup of 4 waves (2 x 2) owns a kTM x kTN tile; K advances 128 bytes a step. The int8
// and fp8 forms (deep_kernel) bring both operands by LDS-DMA into a ring of K steps; the w4a8
// form (narrow_kernel) unpacks its codes in registers into a double-buffered stage. Every global
// read is a buffer load bounded by the matrix (rows past M or N and bytes past K read as zeros),
// so no launch shape can read outside the operands. MFMA A is the W tile, B the X tile: each
// lane's four results are four consecutive output columns of one row.
#include <type_traits>

#include "common.h"
#include "kernels.h"

namespace cozyq {
namespace {

constexpr int kStep = 128;    // K bytes a stage
constexpr int kThreads = 256;
constexpr uint32_t kOutOfRange = 0x80000000u;  // a buffer offset past num_records reads zeros

// Physical 16-byte chunk of logical chunk c (0..7) in a 128-byte LDS row r: the 16 rows one
// fragment read touches at a chunk fall on 16 distinct 4-bank groups.
__device__ __forceinline__ int swz(int r, int c) { return c ^ ((r >> 1) & 7); }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_from(const uint8_t* base, int row0, int rows,
                                                          int K) {
    const int64_t span = static_cast<int64_t>(rows - row0) * K;
    const uint32_t bytes = span > 0x7fffffff ? 0x7fffffffu : static_cast<uint32_t>(span);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base + static_cast<int64_t>(row0) * K),
                                             0, bytes, 0x00020000);
}

// w4a8.convrot weights (internal/prebuilt.py:437-492): 4-bit codes [N, K/2] (even k in the low
// nibble), one E4M3 group scale per 16 codes [N, K/16], and a codebook of 16 float32 levels (or
// the uniform grid q − 8). A code's int8 level is clamp(rne(level · group scale), ±127), a NaN
// product 0 — one float32 multiply, so a 256 x 16 table T[scale byte][code] holds every level.
struct W4 {
    const uint8_t* group_scale;
    const float* codebook;  // null: the uniform grid
};

// The 16 levels of a codebook (null: the uniform grid q − 8).
__device__ __forceinline__ void w4_levels(const float* codebook, float (&book)[16]) {
#pragma unroll
    for (int c = 0; c < 16; ++c) book[c] = codebook != nullptr ? codebook[c] : static_cast<float>(c - 8);
}

// T[b][c] for b = the calling thread's index (256 threads), as 16 bytes at table + 16·b.
__device__ __forceinline__ void w4_table_row(const float (&book)[16], uint32_t* table, int b) {
    const float e = e4m3_value(static_cast<uint32_t>(b));
    uint32_t words[4] = {0, 0, 0, 0};
#pragma unroll
    for (int c = 0; c < 16; ++c) {
        const float level = book[c];
        float r = __builtin_rintf(level * e);  // torch.round: half to even
        r = __builtin_isnan(r) ? 0.0f : fminf(fmaxf(r, -127.0f), 127.0f);
        words[c / 4] |= static_cast<uint32_t>(static_cast<uint8_t>(static_cast<int>(r))) << (8 * (c % 4));
    }
    *reinterpret_cast<uint4*>(table + 4 * b) = make_uint4(words[0], words[1], words[2], words[3]);
}

__device__ __forceinline__ void w4_table_row(const float* codebook, uint32_t* table, int b) {
    float book[16];
    w4_levels(codebook, book);
    w4_table_row(book, table, b);
}

// 16 codes (8 bytes, k order) of one group with scale byte b -> their 16 int8 levels (k order),
// by byte selects from the group's table row: codes 0..7 from its low 8 bytes, 8..15 from its
// high 8, chosen per byte by the code's bit 3.
__device__ __forceinline__ uint4 w4_unpack16(uint32_t c01, uint32_t c23, const uint32_t* table,
                                             uint32_t b) {
    const uint4 t = *reinterpret_cast<const uint4*>(table + 4 * b);
    auto four = [&](uint32_t spread) {  // four codes, one a byte
        const uint32_t sel = spread & 0x07070707u;
        const uint32_t lo = __builtin_amdgcn_perm(t.y, t.x, sel);  // levels of codes 0..7
        const uint32_t hi = __builtin_amdgcn_perm(t.w, t.z, sel);  // levels of codes 8..15
        const uint32_t m = ((spread >> 3) & 0x01010101u) * 0xffu;
        return (hi & m) | (lo & ~m);
    };
    uint32_t out[4];
#pragma unroll
    for (int d = 0; d < 2; ++d) {
        const uint32_t x = d ? c23 : c01;
        const uint32_t lo = x & 0x0f0f0f0fu, hi = (x >> 4) & 0x0f0f0f0fu;
        // byte i holds k = 2i (low nibble) and 2i + 1 (high): interleave into k order.
        out[2 * d] = four(__builtin_amdgcn_perm(hi, lo, 0x05010400u));
        out[2 * d + 1] = four(__builtin_amdgcn_perm(hi, lo, 0x07030602u));
    }
    return make_uint4(out[0], out[1], out[2], out[3]);
}

// kW4: W is w4a8.convrot codes (with `w4`), unpacked to int8 levels in registers on the way
// into LDS; the rest is the int8 path (kInt8 must be true).
template <bool kInt8, int kTM, int kTN, bool kOutHalf, bool kBias, int kEpi, bool kW4 = false>
__global__ __launch_bounds__(kThreads) void narrow_kernel(
    const uint8_t* __restrict__ X, const uint8_t* __restrict__ W, const float* __restrict__ xs,
    const float* __restrict__ ws, const uint16_t* __restrict__ bias, uint16_t* __restrict__ out,
    int64_t ldo, int M, int N, int K, int tiles_m, W4 w4) {
    static_assert(kTM % 32 == 0 && kTN % 32 == 0 && kTM <= 128 && kTN <= 128, "tile");
    static_assert(!kW4 || kInt8, "w4a8 runs the int8 path");
    constexpr int kXLoads = kTM * 8 / kThreads;   // 16-byte chunks a thread stages a step
    constexpr int kWLoads = kTN * 8 / kThreads;
    constexpr int kBI = kTN / 32, kBJ = kTM / 32;  // 16x16 blocks of a wave: n by m
    __shared__ __attribute__((aligned(16))) uint8_t lx[2][kTM * kStep];
    __shared__ __attribute__((aligned(16))) uint8_t lw[2][kTN * kStep];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    // M-tiles fastest: the workgroups in flight together share their weight tiles in L2.
    // Workgroup b runs on XCD b % 8: the M-tiles of one N-tile go to the same XCD (b, b + 8, ...),
    // so the ones after the first find that weight panel in its L2.
    const int tiles_n = gridDim.x / tiles_m;
    const bool xcd = tiles_m > 1 && tiles_n % 8 == 0;
    const int tm = xcd ? (blockIdx.x >> 3) % tiles_m : blockIdx.x % tiles_m;
    const int tn = xcd ? ((blockIdx.x >> 3) / tiles_m) * 8 + (blockIdx.x & 7) : blockIdx.x / tiles_m;
    const int m0 = __builtin_amdgcn_readfirstlane(tm * kTM);
    const int n0 = __builtin_amdgcn_readfirstlane(tn * kTN);
    const __amdgpu_buffer_rsrc_t xr = rows_from(X, m0, M, K);
    // kW4: W rows are K/2 code bytes, and the group scales K/16 bytes a row.
    const __amdgpu_buffer_rsrc_t wr = rows_from(W, n0, N, kW4 ? K / 2 : K);
    const __amdgpu_buffer_rsrc_t gr = rows_from(kW4 ? w4.group_scale : W, n0, N, kW4 ? K / 16 : K);
    const int nk = (K + kStep - 1) / kStep;
    __shared__ __attribute__((aligned(16))) uint32_t table[kW4 ? 256 * 4 : 4];
    if constexpr (kW4) {
        w4_table_row(w4.codebook, table, threadIdx.x);
        __syncthreads();
    }

    // Chunk tid + 256·i: row (tid + 256·i) / 8 of the tile, 16-byte column tid % 8.
    const int col = tid & 7;
    uint4 sx[kXLoads], sw[kWLoads];
    uint32_t sg[kWLoads];  // kW4: the chunk's group scale byte (its 16 codes in sw[i].x, .y)
    auto load = [&](int ks) {
        const int kb = ks * kStep + col * 16;
#pragma unroll
        for (int i = 0; i < kXLoads; ++i) {
            const int r = (tid >> 3) + 32 * i;
            const uint32_t off = kb < K ? static_cast<uint32_t>(r * K + kb) : kOutOfRange;
            sx[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
        }
#pragma unroll
        for (int i = 0; i < kWLoads; ++i) {
            const int r = (tid >> 3) + 32 * i;
            if constexpr (kW4) {
                // The chunk's 16 codes (8 bytes) and its group scale: zeros past K level to 0.
                const uint32_t off = kb < K ? static_cast<uint32_t>(r * (K / 2) + kb / 2) : kOutOfRange;
                const uint32_t goff = kb < K ? static_cast<uint32_t>(r * (K / 16) + kb / 16) : kOutOfRange;
                const auto c = __builtin_amdgcn_raw_buffer_load_b64(wr, off, 0, 0);
                sw[i] = make_uint4(c[0], c[1], 0, 0);
                sg[i] = __builtin_amdgcn_raw_buffer_load_b8(gr, goff, 0, 0);
            } else {
                const uint32_t off = kb < K ? static_cast<uint32_t>(r * K + kb) : kOutOfRange;
                sw[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wr, off, 0, 0));
            }
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int i = 0; i < kXLoads; ++i) {
            const int r = (tid >> 3) + 32 * i;
            *reinterpret_cast<uint4*>(&lx[buf][r * kStep + swz(r, col) * 16]) = sx[i];
        }
#pragma unroll
        for (int i = 0; i < kWLoads; ++i) {
            const int r = (tid >> 3) + 32 * i;
            uint4 v = sw[i];
            if constexpr (kW4) v = w4_unpack16(sw[i].x, sw[i].y, table, sg[i] & 0xffu);
            *reinterpret_cast<uint4*>(&lw[buf][r * kStep + swz(r, col) * 16]) = v;
        }
    };

    typedef std::conditional_t<kInt8, i32x4, f32x4> Acc;
    Acc acc[kBI][kBJ];
#pragma unroll
    for (int i = 0; i < kBI; ++i)
#pragma unroll
        for (int j = 0; j < kBJ; ++j) acc[i][j] = Acc{0, 0, 0, 0};

    load(0);
    store(0);
    if (nk > 1) load(1);
    __syncthreads();

    const int fr = lane & 15, fq = lane >> 4;
    for (int ks = 0; ks < nk; ++ks) {
        const int cur = ks & 1;
        if constexpr (kInt8) {
            // 16x16x64: lane group fq supplies 16-byte chunk fq of each 64-byte K half h.
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                i32x4 a[kBI], b[kBJ];
#pragma unroll
                for (int i = 0; i < kBI; ++i) {
                    const int r = wn * (kTN / 2) + i * 16 + fr;
                    a[i] = *reinterpret_cast<const i32x4*>(&lw[cur][r * kStep + swz(r, 4 * h + fq) * 16]);
                }
#pragma unroll
                for (int j = 0; j < kBJ; ++j) {
                    const int r = wm * (kTM / 2) + j * 16 + fr;
                    b[j] = *reinterpret_cast<const i32x4*>(&lx[cur][r * kStep + swz(r, 4 * h + fq) * 16]);
                }
#pragma unroll
                for (int i = 0; i < kBI; ++i)
#pragma unroll
                    for (int j = 0; j < kBJ; ++j) acc[i][j] = mfma_i8(a[i], b[j], acc[i][j]);
            }
        } else {
        // Lane group fq reads chunks fq and fq + 4 (the f8f6f4 K layout, `common.h`).
        i32x8 a[kBI], b[kBJ];
#pragma unroll
        for (int i = 0; i < kBI; ++i) {
            const int r = wn * (kTN / 2) + i * 16 + fr;
            const uint8_t* row = &lw[cur][r * kStep];
            const i32x4 lo = *reinterpret_cast<const i32x4*>(row + swz(r, fq) * 16);
            const i32x4 hi = *reinterpret_cast<const i32x4*>(row + swz(r, fq + 4) * 16);
            a[i] = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
#pragma unroll
        for (int j = 0; j < kBJ; ++j) {
            const int r = wm * (kTM / 2) + j * 16 + fr;
            const uint8_t* row = &lx[cur][r * kStep];
            const i32x4 lo = *reinterpret_cast<const i32x4*>(row + swz(r, fq) * 16);
            const i32x4 hi = *reinterpret_cast<const i32x4*>(row + swz(r, fq + 4) * 16);
            b[j] = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
#pragma unroll
        for (int i = 0; i < kBI; ++i)
#pragma unroll
            for (int j = 0; j < kBJ; ++j) acc[i][j] = mfma_f8(a[i], b[j], acc[i][j]);
        }
        if (ks + 1 < nk) {
            store(cur ^ 1);
            if (ks + 2 < nk) load(ks + 2);
        }
        __syncthreads();
    }

    // Epilogue: the lane's four consecutive columns of one row, an 8-byte store.
#pragma unroll
    for (int j = 0; j < kBJ; ++j) {
        const int m = m0 + wm * (kTM / 2) + j * 16 + fr;
        if (m >= M) continue;
        const float xsm = xs[m];
#pragma unroll
        for (int i = 0; i < kBI; ++i) {
            const int n = n0 + wn * (kTN / 2) + i * 16 + 4 * fq;
            if (n >= N) continue;  // N % 8 == 0: n..n+3 are all in
            uint16_t o[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if constexpr (kInt8) {
                    // Each step rounded on its own, no fused multiply-add.
                    const float v = __fmul_rn(__fmul_rn(static_cast<float>(acc[i][j][r]), xsm), ws[n + r]);
                    o[r] = narrow<kOutHalf>(v);
                    if constexpr (kBias) o[r] = narrow<kOutHalf>(__fadd_rn(widen<kOutHalf>(o[r]), widen<kOutHalf>(bias[n + r])));
                } else {
                    float v = __fmul_rn(__fmul_rn(acc[i][j][r], xsm), ws[n + r]);
                    if constexpr (kBias) v = __fadd_rn(v, widen<kOutHalf>(bias[n + r]));
                    o[r] = narrow<kOutHalf>(v);
                }
                if constexpr (kEpi == 1) o[r] = narrow<kOutHalf>(gelu_tanh(widen<kOutHalf>(o[r])));
            }
            *reinterpret_cast<uint2*>(out + static_cast<int64_t>(m) * ldo + n) =
                make_uint2(o[0] | (static_cast<uint32_t>(o[1]) << 16), o[2] | (static_cast<uint32_t>(o[3]) << 16));
        }
    }
}

// The deep form of configs 1..4 (int8 and fp8 rowwise, not w4a8): the same tile, MFMA order and
// epilogue as narrow_kernel, with the operands brought by LDS-DMA into a ring of kStages K steps
// in LDS instead of through registers, so kStages - 1 steps of loads are in flight (one in
// narrow_kernel): at few rows each workgroup streams its weight rows at the latency of a step,
// and that depth is what fills HBM. Per step a wave issues kTM/32 + kTN/32 loads of 1 KiB (8 rows
// of 128 bytes, lane l at row l/8, physical chunk l%8 holding logical chunk swz(row, l%8)).

// One operand's loads of a K step: load j fills rows (4j + wave)·8 .. + 8 of the operand's half.
template <int kLoads>
__device__ __forceinline__ void deep_issue(__amdgpu_buffer_rsrc_t rsrc, uint8_t* half, const int (&rowoff)[kLoads],
                                           const int (&chunk)[kLoads], int k0, int K, int wave) {
#pragma unroll
    for (int j = 0; j < kLoads; ++j) {
        const uint32_t off = (k0 + chunk[j] < K) ? static_cast<uint32_t>(rowoff[j] + k0) : kOutOfRange;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (LdsPtr*)(half + (4 * j + wave) * 1024), 16, off, 0, 0, 0);
    }
}

template <bool kInt8, int kTM, int kTN, int kStages, bool kOutHalf, bool kBias, int kEpi>
__global__ __launch_bounds__(kThreads) void deep_kernel(
    const uint8_t* __restrict__ X, const uint8_t* __restrict__ W, const float* __restrict__ xs,
    const float* __restrict__ ws, const uint16_t* __restrict__ bias, uint16_t* __restrict__ out,
    int64_t ldo, int M, int N, int K, int tiles_m) {
    static_assert(kTM % 32 == 0 && kTN % 32 == 0 && kTM <= 128 && kTN <= 128 && kStages >= 2, "tile");
    constexpr int kLX = kTM / 32, kLW = kTN / 32;  // a wave's loads a step
    constexpr int kStageBytes = (kTM + kTN) * kStep;
    constexpr int kBI = kTN / 32, kBJ = kTM / 32;  // 16x16 blocks of a wave: n by m
    static_assert((kStages - 2) * (kLX + kLW) < 64, "vmcnt range");
    __shared__ __attribute__((aligned(1024))) uint8_t lds[kStages * kStageBytes];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    // Workgroup b runs on XCD b % 8: the M-tiles of one N-tile go to the same XCD (b, b + 8, ...),
    // so the ones after the first find that weight panel in its L2.
    const int tiles_n = gridDim.x / tiles_m;
    const bool xcd = tiles_m > 1 && tiles_n % 8 == 0;
    const int tm = xcd ? (blockIdx.x >> 3) % tiles_m : blockIdx.x % tiles_m;
    const int tn = xcd ? ((blockIdx.x >> 3) / tiles_m) * 8 + (blockIdx.x & 7) : blockIdx.x / tiles_m;
    const int m0 = __builtin_amdgcn_readfirstlane(tm * kTM);
    const int n0 = __builtin_amdgcn_readfirstlane(tn * kTN);
    const __amdgpu_buffer_rsrc_t xr = rows_from(X, m0, M, K);
    const __amdgpu_buffer_rsrc_t wr = rows_from(W, n0, N, K);
    const int nk = (K + kStep - 1) / kStep;

    int xoff[kLX], xchunk[kLX], woff[kLW], wchunk[kLW];
#pragma unroll
    for (int j = 0; j < kLX; ++j) {
        const int r = (4 * j + wave) * 8 + (lane >> 3);
        xchunk[j] = 16 * swz(r, lane & 7);
        xoff[j] = r * K + xchunk[j];
    }
#pragma unroll
    for (int j = 0; j < kLW; ++j) {
        const int r = (4 * j + wave) * 8 + (lane >> 3);
        wchunk[j] = 16 * swz(r, lane & 7);
        woff[j] = r * K + wchunk[j];
    }
    // Every step's loads are issued, past the last too (zeros into a slot nothing reads), so a
    // wave's count of loads in flight is the same at every wait.
    auto issue = [&](int ks) {
        uint8_t* base = lds + (ks % kStages) * kStageBytes;
        deep_issue<kLX>(xr, base, xoff, xchunk, ks * kStep, K, wave);
        deep_issue<kLW>(wr, base + kTM * kStep, woff, wchunk, ks * kStep, K, wave);
    };

    typedef std::conditional_t<kInt8, i32x4, f32x4> Acc;
    Acc acc[kBI][kBJ];
#pragma unroll
    for (int i = 0; i < kBI; ++i)
#pragma unroll
        for (int j = 0; j < kBJ; ++j) acc[i][j] = Acc{0, 0, 0, 0};

#pragma unroll
    for (int ks = 0; ks < kStages - 1; ++ks) issue(ks);

    const int fr = lane & 15, fq = lane >> 4;
    for (int ks = 0; ks < nk; ++ks) {
        // Step ks landed (this wave's share; the barrier makes every wave's visible) and every
        // wave is done with step ks - 1, whose slot takes step ks + kStages - 1.
        fence();
        wait_vmcnt<(kStages - 2) * (kLX + kLW)>();
        __builtin_amdgcn_s_barrier();
        fence();
        issue(ks + kStages - 1);
        const uint8_t* lx = lds + (ks % kStages) * kStageBytes;
        const uint8_t* lw = lx + kTM * kStep;
        if constexpr (kInt8) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                i32x4 a[kBI], b[kBJ];
#pragma unroll
                for (int i = 0; i < kBI; ++i) {
                    const int r = wn * (kTN / 2) + i * 16 + fr;
                    a[i] = *reinterpret_cast<const i32x4*>(&lw[r * kStep + swz(r, 4 * h + fq) * 16]);
                }
#pragma unroll
                for (int j = 0; j < kBJ; ++j) {
                    const int r = wm * (kTM / 2) + j * 16 + fr;
                    b[j] = *reinterpret_cast<const i32x4*>(&lx[r * kStep + swz(r, 4 * h + fq) * 16]);
                }
#pragma unroll
                for (int i = 0; i < kBI; ++i)
#pragma unroll
                    for (int j = 0; j < kBJ; ++j) acc[i][j] = mfma_i8(a[i], b[j], acc[i][j]);
            }
        } else {
            i32x8 a[kBI], b[kBJ];
#pragma unroll
            for (int i = 0; i < kBI; ++i) {
                const int r = wn * (kTN / 2) + i * 16 + fr;
                const uint8_t* row = &lw[r * kStep];
                const i32x4 lo = *reinterpret_cast<const i32x4*>(row + swz(r, fq) * 16);
                const i32x4 hi = *reinterpret_cast<const i32x4*>(row + swz(r, fq + 4) * 16);
                a[i] = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            }
#pragma unroll
            for (int j = 0; j < kBJ; ++j) {
                const int r = wm * (kTM / 2) + j * 16 + fr;
                const uint8_t* row = &lx[r * kStep];
                const i32x4 lo = *reinterpret_cast<const i32x4*>(row + swz(r, fq) * 16);
                const i32x4 hi = *reinterpret_cast<const i32x4*>(row + swz(r, fq + 4) * 16);
                b[j] = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            }
#pragma unroll
            for (int i = 0; i < kBI; ++i)
#pragma unroll
                for (int j = 0; j < kBJ; ++j) acc[i][j] = mfma_f8(a[i], b[j], acc[i][j]);
        }
    }
    wait_vmcnt<0>();  // the zero-filling loads past the last step land before the wave ends

    // Epilogue: narrow_kernel's.
#pragma unroll
    for (int j = 0; j < kBJ; ++j) {
        const int m = m0 + wm * (kTM / 2) + j * 16 + fr;
        if (m >= M) continue;
        const float xsm = xs[m];
#pragma unroll
        for (int i = 0; i < kBI; ++i) {
            const int n = n0 + wn * (kTN / 2) + i * 16 + 4 * fq;
            if (n >= N) continue;  // N % 8 == 0: n..n+3 are all in
            uint16_t o[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if constexpr (kInt8) {
                    const float v = __fmul_rn(__fmul_rn(static_cast<float>(acc[i][j][r]), xsm), ws[n + r]);
                    o[r] = narrow<kOutHalf>(v);
                    if constexpr (kBias) o[r] = narrow<kOutHalf>(__fadd_rn(widen<kOutHalf>(o[r]), widen<kOutHalf>(bias[n + r])));
                } else {
                    float v = __fmul_rn(__fmul_rn(acc[i][j][r], xsm), ws[n + r]);
                    if constexpr (kBias) v = __fadd_rn(v, widen<kOutHalf>(bias[n + r]));
                    o[r] = narrow<kOutHalf>(v);
                }
                if constexpr (kEpi == 1) o[r] = narrow<kOutHalf>(gelu_tanh(widen<kOutHalf>(o[r])));
            }
            *reinterpret_cast<uint2*>(out + static_cast<int64_t>(m) * ldo + n) =
                make_uint2(o[0] | (static_cast<uint32_t>(o[1]) << 16), o[2] | (static_cast<uint32_t>(o[3]) << 16));
        }
    }
}

// The ring depth of each deep tile: as many K steps as 64 KiB of LDS hold (two workgroups a
// CU), 2 to 8: 32x64 5, 64x64 4, 128x64 and 128x128 2. Measured at few rows with the weight
// streamed from HBM, 96 and 128 KiB rings (8 and 12 steps for 32x64) were no faster.
constexpr int kDeepLds = 65536;
template <int kTM, int kTN>
constexpr int deep_stages() {
    constexpr int fit = kDeepLds / ((kTM + kTN) * kStep);
    return fit < 2 ? 2 : fit > 8 ? 8 : fit;
}

template <bool kInt8, int kTM, int kTN, bool kOutHalf, bool kBias, int kEpi, bool kW4>
hipError_t launch(const uint8_t* q, const float* xs, const uint8_t* w, const float* ws,
                  const void* bias, void* out, int64_t ldo, int M, int N, int K, W4 w4,
                  hipStream_t s) {
    const int tiles_m = (M + kTM - 1) / kTM, tiles_n = (N + kTN - 1) / kTN;
    if constexpr (kW4) {
        narrow_kernel<kInt8, kTM, kTN, kOutHalf, kBias, kEpi, kW4><<<tiles_m * tiles_n, kThreads, 0, s>>>(
            q, w, xs, ws, static_cast<const uint16_t*>(bias), static_cast<uint16_t*>(out), ldo, M, N,
            K, tiles_m, w4);
    } else {
        deep_kernel<kInt8, kTM, kTN, deep_stages<kTM, kTN>(), kOutHalf, kBias, kEpi><<<tiles_m * tiles_n, kThreads, 0, s>>>(
            q, w, xs, ws, static_cast<const uint16_t*>(bias), static_cast<uint16_t*>(out), ldo, M, N,
            K, tiles_m);
    }
    return hipGetLastError();
}

template <bool kInt8, int kTM, int kTN, bool kW4 = false>
hipError_t shaped(const uint8_t* q, const float* xs, const uint8_t* w, const float* ws,
                  const void* bias, void* out, int64_t ldo, bool out_half, int M, int N, int K,
                  int epilogue, hipStream_t s, W4 w4 = W4{nullptr, nullptr}) {
    const bool b = bias != nullptr;
#define COZYQ_CASE(H, B, E) \
    if (out_half == H && b == B && epilogue == E) return launch<kInt8, kTM, kTN, H, B, E, kW4>(q, xs, w, ws, bias, out, ldo, M, N, K, w4, s);
    COZYQ_CASE(false, false, 0)
    COZYQ_CASE(false, true, 0)
    COZYQ_CASE(true, false, 0)
    COZYQ_CASE(true, true, 0)
    COZYQ_CASE(false, false, 1)
    COZYQ_CASE(false, true, 1)
    COZYQ_CASE(true, false, 1)
    COZYQ_CASE(true, true, 1)
#undef COZYQ_CASE
    return hipErrorInvalidValue;
}

// Tile configs 1..4 (config 0 is the 256x256 kernel of gemm.hip): 128x128, 128x64, 64x64,
// 32x64 (rows x columns). Every config computes each output with the same MFMA sequence over K
// and the same epilogue.
template <bool kInt8, bool kW4 = false>
hipError_t narrow(const uint8_t* q, const float* xs, const uint8_t* w, const float* ws,
                  const void* bias, void* out, int64_t ldo, bool out_half, int M, int N, int K,
                  int epilogue, int config, hipStream_t s, W4 w4 = W4{nullptr, nullptr}) {
    switch (config) {
        case 1: return shaped<kInt8, 128, 128, kW4>(q, xs, w, ws, bias, out, ldo, out_half, M, N, K, epilogue, s, w4);
        case 2: return shaped<kInt8, 128, 64, kW4>(q, xs, w, ws, bias, out, ldo, out_half, M, N, K, epilogue, s, w4);
        case 3: return shaped<kInt8, 64, 64, kW4>(q, xs, w, ws, bias, out, ldo, out_half, M, N, K, epilogue, s, w4);
        case 4: return shaped<kInt8, 32, 64, kW4>(q, xs, w, ws, bias, out, ldo, out_half, M, N, K, epilogue, s, w4);
        default: return hipErrorNotSupported;
    }
}

// The unpack law over a whole weight (internal/prebuilt.py:471-492): one thread a group of 16.
__global__ __launch_bounds__(kThreads) void w4a8_unpack_kernel(const uint8_t* __restrict__ codes,
                                                               const uint8_t* __restrict__ gs,
                                                               const float* __restrict__ codebook,
                                                               int8_t* __restrict__ out, int64_t groups,
                                                               int K) {
    __shared__ __attribute__((aligned(16))) uint32_t table[256 * 4];
    w4_table_row(codebook, table, threadIdx.x);
    __syncthreads();
    const int64_t g = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (g >= groups) return;
    const int64_t per_row = K / 16;
    const int64_t row = g / per_row, grp = g % per_row;
    const uint2 c = *reinterpret_cast<const uint2*>(codes + row * (K / 2) + grp * 8);
    const uint4 v = w4_unpack16(c.x, c.y, table, gs[row * per_row + grp]);
    *reinterpret_cast<uint4*>(out + row * K + grp * 16) = v;
}

// The w4a8.convrot GEMV for 1..2 quantized rows (more take the row-tile kernel below, faster from
// 3 rows): the int8 decode GEMV's structure on 4-bit codes.
// Each wave streams kW4Rows whole weight rows as contiguous 1 KiB code loads (lane l at byte
// 16·l of a span: 32 codes, columns 2048·j + 32·l .., two groups, whose scale bytes are the row's
// bytes 128·j + 2·l and + 1), non-temporal; the codes unpack to int8 levels through the
// workgroup's 256 x 16 level table (w4_unpack16); the quantized activation rows sit in LDS. The
// dot products are the trace of v_mfma_i32_16x16x64_i8 (lane l supplies A row l%16 and B column
// l%16, k-block l/16: the same 16 columns of the weight row and of the activation), exact int32,
// and the epilogue is the int8 law's, so every output equals the tiled GEMM's bit for bit.
constexpr int kW4Waves = 4;
constexpr int kW4Rows = 4;       // weight rows a wave
constexpr int kW4Batch = 2;      // 1 KiB code spans of each row in flight
constexpr int kW4MaxK = 8192;    // activation rows a thread stages: K ≤ this
constexpr int kW4Policy = 3;     // sc0 nt: each code byte is read once per call
constexpr int kW4RowsMax = 16;   // rows the row-tile form takes (one MFMA's B columns)
// 17..32 rows: the row-tile form with two 16-row activation blocks, for K ≤ 4096 (its
// activation registers) and M·K ≤ 98304. Graph replays over weights past the MALL, µs narrow
// tile / row tile, bit-equal: K=3072 N=12288 M=17 19.6 / 15.3, M=24 19.7 / 16.2, M=32 19.7 /
// 17.7; K=4096 N=14336 M=20 25.1 / 22.5, M=32 25.1 / 26.2 (past the area rule); K=3072 N=3072
// M=32 19.0 / 8.5.
constexpr int kW4Rows2Max = 32;
constexpr int kW4Rows2MaxK = 4096;
constexpr int64_t kW4Rows2Area = 98304;
constexpr int kW4GemvRows = 2;   // rows the GEMV form takes
constexpr uint32_t kFarW4 = 0x7fff0000u;  // a buffer offset past every resource here (reads 0)

template <bool kOutHalf, bool kBias, int kM>
__global__ __launch_bounds__(64 * kW4Waves) void w4a8_decode_kernel(
    const int8_t* __restrict__ q, const float* __restrict__ xs, const uint8_t* __restrict__ codes, W4 w4,
    const float* __restrict__ ws, const uint16_t* __restrict__ bias, uint16_t* __restrict__ out, int N, int K) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];  // the level table, then kM code rows
    constexpr int kThreadsW4 = 64 * kW4Waves;
    constexpr int kPieces = kW4MaxK / 16 / kThreadsW4;
    static_assert(kThreadsW4 == 256, "one level-table row a thread");
    uint32_t* const table = reinterpret_cast<uint32_t*>(smem);
    int8_t* const xq = reinterpret_cast<int8_t*>(smem + 256 * 16);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int spans = (K + 2047) / 2048, stride = spans * 2048;
    const int nw = blockIdx.x * (kW4Waves * kW4Rows) + wave * kW4Rows;  // the wave's first row

    // 1. The activation rows' 16-byte pieces first (loads complete in issue order).
    const __amdgpu_buffer_rsrc_t qr = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(q), 0, kM * K, 0x00020000);
    uint4 xv[kM][kPieces];
#pragma unroll
    for (int m = 0; m < kM; ++m)
#pragma unroll
        for (int p = 0; p < kPieces; ++p) {
            const int b = 16 * (tid + kThreadsW4 * p);
            xv[m][p] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                qr, b < K ? m * K + b : 0x7ffffff0, 0, 0));
        }
    // The epilogue's operands (the rows' scales, the weight rows' scales, the bias) come with the
    // activation, ahead of the code stream (common.h `row_epilogue`).
    const RowEpilogue<kW4Rows, kBias> epi = row_epilogue<kW4Rows, kBias>(ws, bias, nw, N);
    float xsv[kM];
    {
        const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(xs), 0, 4 * kM, 0x00020000);
#pragma unroll
        for (int m = 0; m < kM; ++m) xsv[m] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(sr, 4 * m, 0, 0));
    }
    asm volatile("" ::: "memory");

    // 2. The code stream and each lane's two group-scale bytes.
    const int64_t rows_bytes = static_cast<int64_t>(N) * (K / 2);
    const __amdgpu_buffer_rsrc_t cr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(codes), 0, rows_bytes > 0x7fffffff ? 0x7fffffff : static_cast<int>(rows_bytes), 0x00020000);
    const __amdgpu_buffer_rsrc_t gr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(w4.group_scale), 0, static_cast<int>(static_cast<int64_t>(N) * (K / 16)), 0x00020000);
    uint4 wv[kW4Rows][kW4Batch];
    uint32_t gv[kW4Rows][kW4Batch];
    auto issue = [&](int first) {
#pragma unroll
        for (int i = 0; i < kW4Rows; ++i)
#pragma unroll
            for (int b = 0; b < kW4Batch; ++b) {
                const int row = nw + i, col = 2048 * (first + b) + 32 * lane;
                const bool live = row < N && col < K;
                wv[i][b] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                    cr, live ? row * (K / 2) + col / 2 : 0x7ffffff0, 0, kW4Policy));
                gv[i][b] = __builtin_amdgcn_raw_buffer_load_b16(gr, live ? row * (K / 16) + col / 16 : 0x7ffffff0, 0, 0);
            }
    };
    issue(0);

    // 3. The level table (row tid) and the activation codes into LDS, zeros past K.
    w4_table_row(w4.codebook, table, tid);
#pragma unroll
    for (int m = 0; m < kM; ++m)
#pragma unroll
        for (int p = 0; p < kPieces; ++p) {
            const int b = 16 * (tid + kThreadsW4 * p);
            if (b < stride) *reinterpret_cast<uint4*>(xq + m * stride + b) = xv[m][p];
        }
    __syncthreads();

    // 4. Products: the trace accumulates over the spans.
    i32x4 acc[kW4Rows][kM];
#pragma unroll
    for (int i = 0; i < kW4Rows; ++i)
#pragma unroll
        for (int m = 0; m < kM; ++m) acc[i][m] = i32x4{0, 0, 0, 0};
    for (int first = 0; first < spans; first += kW4Batch) {
        if (first != 0) issue(first);
#pragma unroll
        for (int b = 0; b < kW4Batch; ++b) {
            if (first + b >= spans) break;
            i32x4 xb[kM][2];
#pragma unroll
            for (int m = 0; m < kM; ++m)
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    xb[m][h] = *reinterpret_cast<const i32x4*>(xq + m * stride + 2048 * (first + b) + 32 * lane + 16 * h);
#pragma unroll
            for (int i = 0; i < kW4Rows; ++i) {
                const uint4 c = wv[i][b];
                const i32x4 l0 = __builtin_bit_cast(i32x4, w4_unpack16(c.x, c.y, table, gv[i][b] & 0xffu));
                const i32x4 l1 = __builtin_bit_cast(i32x4, w4_unpack16(c.z, c.w, table, (gv[i][b] >> 8) & 0xffu));
#pragma unroll
                for (int m = 0; m < kM; ++m) {
                    acc[i][m] = mfma_i8(l0, xb[m][0], acc[i][m]);
                    acc[i][m] = mfma_i8(l1, xb[m][1], acc[i][m]);
                }
            }
        }
    }

    // 5. The trace: D[a][a] sits in lane a + 16·(a/4), register a % 4; the 64 lanes' sum.
    const int a = lane & 15;
    const bool diagonal = (lane >> 4) == (a >> 2);
    int dot[kW4Rows][kM];
#pragma unroll
    for (int i = 0; i < kW4Rows; ++i)
#pragma unroll
        for (int m = 0; m < kM; ++m) {
            const i32x4 d = acc[i][m];
            const int r = a & 3;
            int v = r == 0 ? d[0] : (r == 1 ? d[1] : (r == 2 ? d[2] : d[3]));
            v = diagonal ? v : 0;
            v = diagonal_sum(v);
            dot[i][m] = v;
        }
    if (lane != 0 || nw >= N) return;  // N % 8 == 0: a wave's four rows are all in or all out
#pragma unroll
    for (int m = 0; m < kM; ++m) {
        uint32_t o[2];
#pragma unroll
        for (int i = 0; i < kW4Rows; ++i) {
            // internal/int8_linear.py:445-448 then :276: (acc·xs)·ws, cast, + bias in the output dtype.
            const float v = __fmul_rn(__fmul_rn(static_cast<float>(dot[i][m]), xsv[m]), epi.ws[i]);
            uint32_t h = ::cozyq::narrow<kOutHalf>(v);  // (this file's `narrow` launcher hides it)
            if constexpr (kBias)
                h = ::cozyq::narrow<kOutHalf>(__fadd_rn(widen<kOutHalf>(static_cast<uint16_t>(h)), widen<kOutHalf>(epi.bias[i])));
            o[i / 2] = (i & 1) ? (o[i / 2] | (h << 16)) : h;
        }
        *reinterpret_cast<uint2*>(out + static_cast<int64_t>(m) * N + nw) = make_uint2(o[0], o[1]);
    }
}

// The w4a8.convrot linear for 3..32 quantized rows: one 16-row weight tile a workgroup, its K
// split over kW4RWaves waves, on the plain v_mfma_i32_16x16x64_i8 (A = 16 weight rows, B = the
// activation rows, zero past M; kCols blocks of 16 of them, each A unpacked once for all).
// Lane l (row r = l%16, part g = l/16) of a wave loads 16 contiguous code bytes of weight row r
// per 128-code step t (codes 128t + 32g .. + 32: two groups, whose two scale bytes are adjacent)
// and the same 32 activation elements of row r in two 16-byte pieces, so each of the step's two
// MFMAs meets A and B on the same 16 k's; the 4 lanes of a row read 64 contiguous bytes. Every
// load is issued before the level table is built; steps past a wave's share read zeros
// (activation zeros make them add nothing). The waves' int32 partials meet in LDS (exact, in any
// order), and the epilogue is the int8 law's, so the outputs equal every tile config's bit for
// bit.
constexpr int kW4RWaves = 4;

template <bool kOutHalf, bool kBias, int kSteps, int kCols>
__global__ __launch_bounds__(64 * kW4RWaves) void w4a8_rows_kernel(
    const int8_t* q, const float* xs, const uint8_t* codes, W4 w4, const float* ws,
    const uint16_t* bias, uint16_t* out, int M, int N, int K) {
    // (No pointer here is __restrict__: loads through restrict read-only arguments count as
    // invariant and may be sunk below later loads; these must stay in issue order.)
    __shared__ __attribute__((aligned(16))) uint32_t table[256 * 4];
    __shared__ i32x4 part[kW4RWaves][kCols][64];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane & 15, g = lane >> 4;
    const int n0 = blockIdx.x * 16;
    const int steps = K / 128;  // K % 256 == 0
    const int t0 = wave * steps / kW4RWaves, t1 = (wave + 1) * steps / kW4RWaves;

    // 0. The codebook's levels ahead of the streams: the table is built once they are issued,
    //    and a wait for a load issued after them would wait for every one of them (in order).
    float book[16];
    w4_levels(w4.codebook, book);
    asm volatile("" ::: "memory");

    // 1. The activation pieces: row 16c + r of each 16-row block c, elements 128t + 32g + 16h
    //    .. + 16 (zeros past M or the wave's steps).
    const __amdgpu_buffer_rsrc_t qr = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(q), 0, M * K, 0x00020000);
    i32x4 xb[kCols][kSteps][2];
#pragma unroll
    for (int c = 0; c < kCols; ++c)
#pragma unroll
        for (int j = 0; j < kSteps; ++j)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int t = t0 + j, row = 16 * c + r;
                const uint32_t off = t < t1 && row < M ? static_cast<uint32_t>(row * K + 128 * t + 32 * g + 16 * h) : kFarW4;
                xb[c][j][h] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(qr, off, 0, 0));
            }
    asm volatile("" ::: "memory");

    // 2. The codes (16 bytes a lane a step, non-temporal) and the group scales.
    const int64_t rows_bytes = static_cast<int64_t>(N - n0) * (K / 2);
    const __amdgpu_buffer_rsrc_t cr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(codes + static_cast<int64_t>(n0) * (K / 2)), 0,
        rows_bytes > 0x7fffffff ? 0x7fffffff : static_cast<int>(rows_bytes), 0x00020000);
    const __amdgpu_buffer_rsrc_t gr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(w4.group_scale + static_cast<int64_t>(n0) * (K / 16)), 0,
        static_cast<int>(static_cast<int64_t>(N - n0) * (K / 16)), 0x00020000);
    uint4 cv[kSteps];
#pragma unroll
    for (int j = 0; j < kSteps; ++j) {
        const int t = t0 + j;
        const bool live = t < t1 && n0 + r < N;
        cv[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
            cr, live ? static_cast<uint32_t>(r * (K / 2) + 64 * t + 16 * g) : kFarW4, 0, kW4Policy));
    }
    // The group scales: one 16-byte load brings row r's scale bytes of two steps (8 a step, the
    // four lane groups' pairs) where a 2-byte load a step brought a lane's own pair; the lane
    // shifts its pair out at the product. Bytes of a dead step are never used (its activation
    // reads zeros). Measured (graph replays, weights past the MALL): M = 16, K = 3072, N = 12288
    // 12.6 -> 11.8 us; M = 4 10.7 -> 10.0.
    constexpr int kPairs = (kSteps + 1) / 2;
    uint4 sv[kPairs];
#pragma unroll
    for (int u = 0; u < kPairs; ++u) {
        const int t = t0 + 2 * u;
        const bool live = t < t1 && n0 + r < N;
        sv[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
            gr, live ? static_cast<uint32_t>(r * (K / 16) + 8 * t) : kFarW4, 0, 0));
    }

    // 3. The level table (row tid); a bare barrier (a full one would also wait for the loads).
    w4_table_row(book, table, tid);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");

    // 4. Products over the wave's steps.
    i32x4 acc[kCols];
#pragma unroll
    for (int c = 0; c < kCols; ++c) acc[c] = i32x4{0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < kSteps; ++j) {
        const uint4 s4 = sv[j / 2];
        const uint32_t d = (j & 1) ? ((g >> 1) ? s4.w : s4.z) : ((g >> 1) ? s4.y : s4.x);
        const uint32_t sb = (d >> (16 * (g & 1))) & 0xffffu;
        const i32x4 l0 = __builtin_bit_cast(i32x4, w4_unpack16(cv[j].x, cv[j].y, table, sb & 0xffu));
        const i32x4 l1 = __builtin_bit_cast(i32x4, w4_unpack16(cv[j].z, cv[j].w, table, sb >> 8));
#pragma unroll
        for (int c = 0; c < kCols; ++c) {
            acc[c] = mfma_i8(l0, xb[c][j][0], acc[c]);
            acc[c] = mfma_i8(l1, xb[c][j][1], acc[c]);
        }
    }

    // 5. The waves' partials (lane l: activation row l%16, weight rows 4·(l/16) + 0..3), then
    //    (acc·xs)·ws, cast, + bias in the output dtype (internal/int8_linear.py:445-448, :276).
#pragma unroll
    for (int c = 0; c < kCols; ++c) part[wave][c][lane] = acc[c];
    __syncthreads();
    if (wave != 0) return;
    const int n = n0 + 4 * g;
    if (n >= N) return;  // N % 8 == 0: a lane's four rows are all in or all out
#pragma unroll
    for (int c = 0; c < kCols; ++c) {
#pragma unroll
        for (int w = 1; w < kW4RWaves; ++w) acc[c] += part[w][c][lane];
        const int row = 16 * c + r;
        if (row >= M) continue;
        uint32_t o[2];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float v = __fmul_rn(__fmul_rn(static_cast<float>(acc[c][i]), xs[row]), ws[n + i]);
            uint32_t h = ::cozyq::narrow<kOutHalf>(v);
            if constexpr (kBias)
                h = ::cozyq::narrow<kOutHalf>(__fadd_rn(widen<kOutHalf>(static_cast<uint16_t>(h)), widen<kOutHalf>(bias[n + i])));
            o[i / 2] = (i & 1) ? (o[i / 2] | (h << 16)) : h;
        }
        *reinterpret_cast<uint2*>(out + static_cast<int64_t>(row) * N + n) = make_uint2(o[0], o[1]);
    }
}

template <bool kOutHalf, bool kBias>
hipError_t launch_w4a8_rows(const int8_t* q, const float* xs, const uint8_t* codes, W4 w4, const float* ws,
                            const void* bias, void* out, int M, int N, int K, hipStream_t s) {
    const int blocks = (N + 15) / 16;
    const int per_wave = (K / 128 + kW4RWaves - 1) / kW4RWaves;
    const auto* b = static_cast<const uint16_t*>(bias);
    auto* o = static_cast<uint16_t*>(out);
    if (M > 16) {  // two 16-row activation blocks (the caller keeps K <= kW4Rows2MaxK)
        if (per_wave <= 4)
            w4a8_rows_kernel<kOutHalf, kBias, 4, 2><<<blocks, 64 * kW4RWaves, 0, s>>>(q, xs, codes, w4, ws, b, o, M, N, K);
        else
            w4a8_rows_kernel<kOutHalf, kBias, 8, 2><<<blocks, 64 * kW4RWaves, 0, s>>>(q, xs, codes, w4, ws, b, o, M, N, K);
    } else if (per_wave <= 4)
        w4a8_rows_kernel<kOutHalf, kBias, 4, 1><<<blocks, 64 * kW4RWaves, 0, s>>>(q, xs, codes, w4, ws, b, o, M, N, K);
    else if (per_wave <= 8)
        w4a8_rows_kernel<kOutHalf, kBias, 8, 1><<<blocks, 64 * kW4RWaves, 0, s>>>(q, xs, codes, w4, ws, b, o, M, N, K);
    else
        w4a8_rows_kernel<kOutHalf, kBias, 16, 1><<<blocks, 64 * kW4RWaves, 0, s>>>(q, xs, codes, w4, ws, b, o, M, N, K);
    return hipGetLastError();
}

// The int8 product for 5..32 quantized rows with K <= 4096 (cozyq_gemm's shape rule, no
// epilogue activation): w4a8_rows_kernel's tile on int8 weights. One 16-row weight tile a
// workgroup, K split over its waves; lane l (row r = l%16, part g = l/16) loads 32 contiguous
// weight bytes of row r per 128-byte step t (k = 128t + 32g .. + 32, two 16-byte pieces) and the
// same k's of each activation row, zeros past K, M or N. The waves' int32 partials meet in LDS
// and the epilogue is the int8 law's, so the outputs equal every tile config's bit for bit.
constexpr int kI8RowsMaxK = 4096;

template <bool kOutHalf, bool kBias, int kSteps, int kCols>
__global__ __launch_bounds__(64 * kW4RWaves) void int8_rows_kernel(
    const int8_t* q, const float* xs, const int8_t* w, const float* ws, const uint16_t* bias,
    uint16_t* out, int64_t ldo, int M, int N, int K) {
    // (Not __restrict__, as in w4a8_rows_kernel: the loads must stay in issue order.)
    __shared__ i32x4 part[kW4RWaves][kCols][64];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane & 15, g = lane >> 4;
    const int n0 = blockIdx.x * 16;
    const int steps = (K + 127) / 128;  // K % 16 == 0: a 16-byte piece is wholly in or past K
    const int t0 = wave * steps / kW4RWaves, t1 = (wave + 1) * steps / kW4RWaves;

    // 1. The activation pieces of each 16-row block c, then 2. the weight pieces (non-temporal).
    const __amdgpu_buffer_rsrc_t qr = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(q), 0, M * K, 0x00020000);
    i32x4 xb[kCols][kSteps][2];
#pragma unroll
    for (int c = 0; c < kCols; ++c)
#pragma unroll
        for (int j = 0; j < kSteps; ++j)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int t = t0 + j, row = 16 * c + r, k = 128 * t + 32 * g + 16 * h;
                const uint32_t off = t < t1 && row < M && k < K ? static_cast<uint32_t>(row * K + k) : kFarW4;
                xb[c][j][h] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(qr, off, 0, 0));
            }
    asm volatile("" ::: "memory");
    const int64_t rows_bytes = static_cast<int64_t>(N - n0) * K;
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t*>(w + static_cast<int64_t>(n0) * K), 0,
        rows_bytes > 0x7fffffff ? 0x7fffffff : static_cast<int>(rows_bytes), 0x00020000);
    i32x4 wv[kSteps][2];
#pragma unroll
    for (int j = 0; j < kSteps; ++j)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int t = t0 + j, k = 128 * t + 32 * g + 16 * h;
            const bool live = t < t1 && n0 + r < N && k < K;
            wv[j][h] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(
                wr, live ? static_cast<uint32_t>(r * K + k) : kFarW4, 0, kW4Policy));
        }

    // 3. Products over the wave's steps.
    i32x4 acc[kCols];
#pragma unroll
    for (int c = 0; c < kCols; ++c) acc[c] = i32x4{0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < kSteps; ++j)
#pragma unroll
        for (int c = 0; c < kCols; ++c) {
            acc[c] = mfma_i8(wv[j][0], xb[c][j][0], acc[c]);
            acc[c] = mfma_i8(wv[j][1], xb[c][j][1], acc[c]);
        }

    // 4. The waves' partials, then (acc·xs)·ws, cast, + bias in the output dtype
    //    (internal/int8_linear.py:445-448, :276).
#pragma unroll
    for (int c = 0; c < kCols; ++c) part[wave][c][lane] = acc[c];
    __syncthreads();
    if (wave != 0) return;
    const int n = n0 + 4 * g;
    if (n >= N) return;  // N % 8 == 0: a lane's four rows are all in or all out
#pragma unroll
    for (int c = 0; c < kCols; ++c) {
#pragma unroll
        for (int v = 1; v < kW4RWaves; ++v) acc[c] += part[v][c][lane];
        const int row = 16 * c + r;
        if (row >= M) continue;
        uint32_t o[2];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float v = __fmul_rn(__fmul_rn(static_cast<float>(acc[c][i]), xs[row]), ws[n + i]);
            uint32_t h = ::cozyq::narrow<kOutHalf>(v);
            if constexpr (kBias)
                h = ::cozyq::narrow<kOutHalf>(__fadd_rn(widen<kOutHalf>(static_cast<uint16_t>(h)), widen<kOutHalf>(bias[n + i])));
            o[i / 2] = (i & 1) ? (o[i / 2] | (h << 16)) : h;
        }
        *reinterpret_cast<uint2*>(out + static_cast<int64_t>(row) * ldo + n) = make_uint2(o[0], o[1]);
    }
}

template <bool kOutHalf, bool kBias>
hipError_t launch_int8_rows(const int8_t* q, const float* xs, const int8_t* w, const float* ws,
                            const void* bias, void* out, int64_t ldo, int M, int N, int K, hipStream_t s) {
    const int blocks = (N + 15) / 16;
    const int per_wave = ((K + 127) / 128 + kW4RWaves - 1) / kW4RWaves;
    const auto* b = static_cast<const uint16_t*>(bias);
    auto* o = static_cast<uint16_t*>(out);
    if (M > 16) {
        if (per_wave <= 4)
            int8_rows_kernel<kOutHalf, kBias, 4, 2><<<blocks, 64 * kW4RWaves, 0, s>>>(q, xs, w, ws, b, o, ldo, M, N, K);
        else
            int8_rows_kernel<kOutHalf, kBias, 8, 2><<<blocks, 64 * kW4RWaves, 0, s>>>(q, xs, w, ws, b, o, ldo, M, N, K);
    } else if (per_wave <= 4)
        int8_rows_kernel<kOutHalf, kBias, 4, 1><<<blocks, 64 * kW4RWaves, 0, s>>>(q, xs, w, ws, b, o, ldo, M, N, K);
    else
        int8_rows_kernel<kOutHalf, kBias, 8, 1><<<blocks, 64 * kW4RWaves, 0, s>>>(q, xs, w, ws, b, o, ldo, M, N, K);
    return hipGetLastError();
}

template <bool kOutHalf, bool kBias>
hipError_t launch_w4a8_decode(const int8_t* q, const float* xs, const uint8_t* codes, W4 w4, const float* ws,
                              const void* bias, void* out, int M, int N, int K, hipStream_t s) {
    const int blocks = (N + kW4Waves * kW4Rows - 1) / (kW4Waves * kW4Rows);
    const int64_t lds = 256 * 16 + static_cast<int64_t>(M) * ((K + 2047) / 2048) * 2048;
    const auto* b = static_cast<const uint16_t*>(bias);
    auto* o = static_cast<uint16_t*>(out);
    switch (M) {
        case 1: w4a8_decode_kernel<kOutHalf, kBias, 1><<<blocks, 64 * kW4Waves, lds, s>>>(q, xs, codes, w4, ws, b, o, N, K); break;
        default: w4a8_decode_kernel<kOutHalf, kBias, 2><<<blocks, 64 * kW4Waves, lds, s>>>(q, xs, codes, w4, ws, b, o, N, K); break;
    }
    return hipGetLastError();
}

}  // namespace

hipError_t gemm_w4a8_narrow(const int8_t* q, const float* xs, const uint8_t* codes,
                            const uint8_t* group_scale, const float* codebook, const float* ws,
                            const void* bias, void* out, bool out_half, int M, int N, int K,
                            int config, hipStream_t s) {
    // 1..2 rows by shape: the GEMV form; 3..16 (and 17..32 by the rule above) the row-tile
    // kernel (the same bits as every tile config). The GEMV form's MFMA chains grow with the rows, the row tile's do not (graph
    // replays over weights past the MALL, us GEMV / row tile: K=3072 N=12288 M=2 10.2 / 10.0,
    // M=3 13.7 / 10.1, M=4 15.7 / 10.3; K=4096 N=14336 M=1 11.2 / 13.3, M=2 12.7 / 13.2, M=3
    // 16.6 / 13.6; K=3072 N=3072 M=3 7.4 / 5.9).
    if (config < 0 && M <= kW4GemvRows && K <= kW4MaxK) {
        const W4 w4{group_scale, codebook};
        if (out_half)
            return bias ? launch_w4a8_decode<true, true>(q, xs, codes, w4, ws, bias, out, M, N, K, s)
                        : launch_w4a8_decode<true, false>(q, xs, codes, w4, ws, bias, out, M, N, K, s);
        return bias ? launch_w4a8_decode<false, true>(q, xs, codes, w4, ws, bias, out, M, N, K, s)
                    : launch_w4a8_decode<false, false>(q, xs, codes, w4, ws, bias, out, M, N, K, s);
    }
    const bool two = M <= kW4Rows2Max && K <= kW4Rows2MaxK && static_cast<int64_t>(M) * K <= kW4Rows2Area;
    if (config < 0 && ((M <= kW4RowsMax && K <= kW4MaxK) || two)) {
        const W4 w4{group_scale, codebook};
        if (out_half)
            return bias ? launch_w4a8_rows<true, true>(q, xs, codes, w4, ws, bias, out, M, N, K, s)
                        : launch_w4a8_rows<true, false>(q, xs, codes, w4, ws, bias, out, M, N, K, s);
        return bias ? launch_w4a8_rows<false, true>(q, xs, codes, w4, ws, bias, out, M, N, K, s)
                    : launch_w4a8_rows<false, false>(q, xs, codes, w4, ws, bias, out, M, N, K, s);
    }
    return narrow<true, true>(reinterpret_cast<const uint8_t*>(q), xs, codes, ws, bias, out, N,
                              out_half, M, N, K, 0, config < 0 ? narrow_config(M, N) : config, s,
                              W4{group_scale, codebook});
}

hipError_t int8_rows_gemm(const int8_t* q, const float* xs, const int8_t* w, const float* ws,
                          const void* bias, void* out, int64_t ldo, bool out_half, int M, int N,
                          int K, hipStream_t s) {
    if (M < 1 || M > 32 || K > kI8RowsMaxK || N % 8) return hipErrorNotSupported;
    if (out_half)
        return bias ? launch_int8_rows<true, true>(q, xs, w, ws, bias, out, ldo, M, N, K, s)
                    : launch_int8_rows<true, false>(q, xs, w, ws, bias, out, ldo, M, N, K, s);
    return bias ? launch_int8_rows<false, true>(q, xs, w, ws, bias, out, ldo, M, N, K, s)
                : launch_int8_rows<false, false>(q, xs, w, ws, bias, out, ldo, M, N, K, s);
}

hipError_t w4a8_unpack(const uint8_t* codes, const uint8_t* group_scale, const float* codebook,
                       int8_t* out, int N, int K, hipStream_t s) {
    const int64_t groups = static_cast<int64_t>(N) * (K / 16);
    if (groups == 0) return hipSuccess;
    w4a8_unpack_kernel<<<static_cast<unsigned>((groups + kThreads - 1) / kThreads), kThreads, 0, s>>>(
        codes, group_scale, codebook, out, groups, K);
    return hipGetLastError();
}

// The narrow tile for M x N (fitted on `bench.py --only tiles`, int8 and fp8). Few rows are
// bound by the weight stream, which every M-tile reads again: when N alone gives a 64-column tile
// 192 workgroups (~3/4 of the CUs), the tile that takes all M rows in one M-tile (up to 128)
// streams it once. Otherwise the largest tile whose grid reaches 288 workgroups (~1.1 a CU: two
// deep workgroups share a CU), else the smallest.
int narrow_config(int M, int N) {
    static constexpr int kTiles = 5;  // configs 1..4 have narrow tiles
    static constexpr int kRows[kTiles] = {0, 128, 128, 64, 32}, kCols[kTiles] = {0, 128, 64, 64, 64};
    if ((N + 63) / 64 >= 192) {
        if (M <= 32) return 4;
        if (M <= 64) return 3;
        if (M <= 128) return 2;
    }
    for (int c = 1; c < kTiles; ++c) {
        const int64_t groups = static_cast<int64_t>((M + kRows[c] - 1) / kRows[c]) * ((N + kCols[c] - 1) / kCols[c]);
        if (groups >= 288) return c;
    }
    return kTiles - 1;
}

hipError_t gemm_fp8_narrow(const uint8_t* q, const float* xs, const uint8_t* w, const float* ws,
                           const void* bias, void* out, int64_t ldo, bool out_half, int M, int N,
                           int K, int epilogue, int config, hipStream_t s) {
    return narrow<false>(q, xs, w, ws, bias, out, ldo, out_half, M, N, K, epilogue, config, s);
}

hipError_t gemm_int8_narrow(const int8_t* q, const float* xs, const int8_t* w, const float* ws,
                            const void* bias, void* out, int64_t ldo, bool out_half, int M, int N,
                            int K, int epilogue, int config, hipStream_t s) {
    return narrow<true>(reinterpret_cast<const uint8_t*>(q), xs, reinterpret_cast<const uint8_t*>(w),
                        ws, bias, out, ldo, out_half, M, N, K, epilogue, config, s);
}

}  // namespace cozyq
