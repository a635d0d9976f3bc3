// Launches of the 256x256- and 256x192-tile GEMMs (gemm_tile.h) for the int8, fp8 and MXFP8
// lanes, one tile a workgroup in launch_tile's order.
#include "gemm_tile.h"

namespace cozyq {
namespace {

template <int kKind, bool kOutHalf, bool kBias, int kEpi, int kTN = 256>
hipError_t launch(const void* q, const float* xs, const void* w, const float* ws,
                  const uint8_t* xe, const uint8_t* we, const void* bias, void* out,
                  int32_t* acc, int64_t ldo, int M, int N, int K, hipStream_t s) {
    const int tiles_m = (M + kTile - 1) / kTile, tiles_n = (N + kTN - 1) / kTN;
    if constexpr (kKind != kMx && kTN == 256 && kEpi != 2) {  // the 8-wave tile
        gemm8_kernel<kKind, kOutHalf, kBias, kEpi><<<tiles_m * tiles_n, kThreads8, 0, s>>>(
            static_cast<const uint8_t*>(q), static_cast<const uint8_t*>(w), xs, ws,
            static_cast<const uint16_t*>(bias), static_cast<uint16_t*>(out), ldo, M, N, K, tiles_m, tiles_n);
        return hipGetLastError();
    }
    gemm_kernel<kKind, kOutHalf, kBias, kEpi, kTN><<<tiles_m * tiles_n, kThreads, 0, s>>>(
        static_cast<const uint8_t*>(q), static_cast<const uint8_t*>(w), xs, ws, xe, we,
        static_cast<const uint16_t*>(bias), static_cast<uint16_t*>(out), acc, ldo, M, N, K,
        tiles_m, tiles_n);
    return hipGetLastError();
}

// Where a grid of 256x256 tiles ends in a partial round of at most half the CUs, the tiles of
// its full rounds are a block of whole columns (tiles_m x `head` tiles, a multiple of the CU
// count) and the rest of the columns go to a second launch of 256x128 tiles: one round of
// half-sized tiles in place of a round at most half full. 0 where the grid does not split so.
int tail_columns(int M, int N) {
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) return 0;
    const int64_t cus = cu_count(device);
    const int64_t tm = (M + kTile - 1) / kTile, tn = (N + kTile - 1) / kTile;
    const int64_t tiles = tm * tn, rounds = (tiles + cus - 1) / cus;
    const int64_t last = tiles - (rounds - 1) * cus;
    if (rounds < 2 || 2 * last > cus || ((rounds - 1) * cus) % tm != 0) return 0;
    const int64_t head = (rounds - 1) * cus / tm;  // 256-column tiles in the head launch
    if (head >= tn || tm * ((N - head * kTile + 127) / 128) > cus) return 0;
    return static_cast<int>(head * kTile);
}

template <int kKind>
hipError_t dispatch(const void* q, const float* xs, const void* w, const float* ws,
                    const uint8_t* xe, const uint8_t* we, const void* bias, void* out,
                    int64_t ldo, bool out_half, int M, int N, int K, int epilogue, bool wide,
                    hipStream_t s) {
    const bool b = bias != nullptr;
    const int head = wide ? 0 : tail_columns(M, N);
    // The tail's operands: W rows, their scales (MX: E8M0 rows of K/32 bytes), biases and output
    // columns from `head` on.
    const auto w8 = static_cast<const uint8_t*>(w);
    const void* tw = w8 + static_cast<int64_t>(head) * K;
    const float* tws = ws == nullptr ? nullptr : ws + head;
    const uint8_t* twe = we == nullptr ? nullptr : we + static_cast<int64_t>(head) * (K / 32);
    const void* tb = bias == nullptr ? nullptr : static_cast<const uint16_t*>(bias) + head;
    void* to = static_cast<uint16_t*>(out) + head;
#define COZYQ_CASE(H, B, E)                                                                     \
    if (out_half == H && b == B && epilogue == E) {                                             \
        if (wide) return launch<kKind, H, B, E, 192>(q, xs, w, ws, xe, we, bias, out, nullptr, ldo, M, N, K, s); \
        if (head == 0) return launch<kKind, H, B, E>(q, xs, w, ws, xe, we, bias, out, nullptr, ldo, M, N, K, s); \
        const hipError_t e_ = launch<kKind, H, B, E>(q, xs, w, ws, xe, we, bias, out, nullptr, ldo, M, head, K, s); \
        if (e_ != hipSuccess) return e_;                                                        \
        return launch<kKind, H, B, E, 128>(q, xs, tw, tws, xe, twe, tb, to, nullptr, ldo, M, N - head, K, s); \
    }
    COZYQ_CASE(false, false, 0)
    COZYQ_CASE(false, true, 0)
    COZYQ_CASE(true, false, 0)
    COZYQ_CASE(true, true, 0)
    if constexpr (kKind != kMx) {
        COZYQ_CASE(false, false, 1)
        COZYQ_CASE(false, true, 1)
        COZYQ_CASE(true, false, 1)
        COZYQ_CASE(true, true, 1)
    }
#undef COZYQ_CASE
    return hipErrorInvalidValue;
}

}  // namespace

// The large tiles run one workgroup a CU, so a grid costs its number of rounds over the 256 CUs,
// each round a tile's time. 256x192 tiles do 3/4 of a 256x256 tile's work at ~90% of its rate
// (more operand bytes per MFMA): they win where their rounds cost under 6/5 of the 256x256
// grid's (N = 3072 or 9216 at M = 4096: 256 or 768 tiles, one or three rounds, against 192 or
// 576, one or three rounds of bigger tiles; measured 12-16% faster).
bool wide_tile(int M, int N) {
    constexpr int64_t kCUs = 256;
    const int64_t tm = (M + 255) / 256;
    const int64_t r256 = (tm * ((N + 255) / 256) + kCUs - 1) / kCUs;
    const int64_t r192 = (tm * ((N + 191) / 192) + kCUs - 1) / kCUs;
    return 5 * r192 < 6 * r256;
}


// The shape rule, fitted on MI355X over 19 shapes x 5 configs for each of int8 and fp8 (M 128 to
// 16384, N 640 to 14336, K 1280 to 12288). A 256x256 tile takes ~13 ns per K byte whatever the
// grid, so a grid of fewer tiles than CUs costs a whole tile's time (40 us at K = 3072 for 12
// tiles or 192). From 160 tiles (5/8 of the 256 CUs) it still leads: 4096x3072x3072 at 192 tiles
// 49.9 us against 61.3 us for 128x128, 1024x14336x4096 at 224 tiles 65.6 against 100.4. Below,
// narrow tiles win by up to 2x (1024x3072x3072: 45.9 us against 21.3 us for 64x64). Among the
// large tiles, 256x192 (config 5) where it takes fewer rounds (wide_tile).
int gemm_config(bool fp8, int M, int N, int K) {
    (void)fp8; (void)K;
    const int64_t big = static_cast<int64_t>((M + 255) / 256) * ((N + 255) / 256);
    if (big >= 160) return wide_tile(M, N) ? 5 : 0;
    return narrow_config(M, N);
}

hipError_t gemm_int8(const int8_t* q, const float* xs, const int8_t* w, const float* ws,
                     const void* bias, void* out, int64_t ldo, bool out_half, int M, int N, int K,
                     int epilogue, int config, hipStream_t s) {
    // 1..4 rows by the shape rule: the GEMV on the quantized rows, where it applies.
    if (config < 0 && M <= 4 && epilogue == 0) {
        const hipError_t e = int8_codes_gemv(q, xs, w, ws, bias, out, ldo, out_half, M, N, K, s);
        if (e != hipErrorNotSupported) return e;
    }
    // 5..32 rows of a weight of at most 4096 outputs: the 16-row weight tile, whose N/16
    // workgroups fill the chip where the narrow tiles' N/64 do not (graph replays over weights past
    // the MALL, µs narrow / row tile, bit-equal: K=3072 N=3072 M=16 8.4 / 6.6, M=32 9.0 / 8.6;
    // K=1024 N=1032 M=16 4.9 / 3.1; K=2048 N=4096 M=32 7.1 / 6.1). Wider weights keep the narrow
    // tile (K=3072 N=12288 M=5 10.1 / 12.8, M=16 10.4 / 14.4).
    if (config < 0 && M >= 5 && M <= 32 && N <= 4096 && epilogue == 0) {
        const hipError_t e = int8_rows_gemm(q, xs, w, ws, bias, out, ldo, out_half, M, N, K, s);
        if (e != hipErrorNotSupported) return e;
    }
    if (config < 0) config = gemm_config(false, M, N, K);
    if (config > 0 && config < 5)
        return gemm_int8_narrow(q, xs, w, ws, bias, out, ldo, out_half, M, N, K, epilogue, config, s);
    return dispatch<kInt8>(q, xs, w, ws, nullptr, nullptr, bias, out, ldo, out_half, M, N, K,
                           epilogue, config == 5, s);
}

hipError_t gemm_int8_acc(const int8_t* q, const int8_t* w, int32_t* acc, int M, int N, int K,
                         hipStream_t s) {
    return launch<kInt8, false, false, 2>(q, nullptr, w, nullptr, nullptr, nullptr, nullptr,
                                          nullptr, acc, N, M, N, K, s);
}

hipError_t gemm_fp8(const uint8_t* q, const float* xs, const uint8_t* w, const float* ws,
                    const void* bias, void* out, int64_t ldo, bool out_half, int M, int N, int K,
                    int epilogue, int config, hipStream_t s) {
    if (config < 0) config = gemm_config(true, M, N, K);
    if (config > 0 && config < 5)
        return gemm_fp8_narrow(q, xs, w, ws, bias, out, ldo, out_half, M, N, K, epilogue, config, s);
    return dispatch<kFp8>(q, xs, w, ws, nullptr, nullptr, bias, out, ldo, out_half, M, N, K,
                          epilogue, config == 5, s);
}

hipError_t gemm_mx(const uint8_t* q, const uint8_t* qe, const uint8_t* w, const uint8_t* we,
                   const void* bias, void* out, int64_t ldo, bool out_half, int M, int N, int K,
                   hipStream_t s) {
    return dispatch<kMx>(q, nullptr, w, nullptr, qe, we, bias, out, ldo, out_half, M, N, K, 0,
                         wide_tile(M, N), s);
}

}  // namespace cozyq
