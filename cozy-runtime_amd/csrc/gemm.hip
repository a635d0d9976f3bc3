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
    gemm_kernel<kKind, kOutHalf, kBias, kEpi, kTN><<<tiles_m * tiles_n, kThreads, 0, s>>>(
        static_cast<const uint8_t*>(q), static_cast<const uint8_t*>(w), xs, ws, xe, we,
        static_cast<const uint16_t*>(bias), static_cast<uint16_t*>(out), acc, ldo, M, N, K,
        tiles_m, tiles_n);
    return hipGetLastError();
}

template <int kKind>
hipError_t dispatch(const void* q, const float* xs, const void* w, const float* ws,
                    const uint8_t* xe, const uint8_t* we, const void* bias, void* out,
                    int64_t ldo, bool out_half, int M, int N, int K, int epilogue, bool wide,
                    hipStream_t s) {
    const bool b = bias != nullptr;
#define COZYQ_CASE(H, B, E)                                                                     \
    if (out_half == H && b == B && epilogue == E)                                               \
        return wide ? launch<kKind, H, B, E, 192>(q, xs, w, ws, xe, we, bias, out, nullptr, ldo, M, N, K, s) \
                    : launch<kKind, H, B, E>(q, xs, w, ws, xe, we, bias, out, nullptr, ldo, M, N, K, s);
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
