// Test entry: one MFMA of each kind the kernels use, on operands given per lane, so a GPU test
// can confirm the lane layouts the GEMMs assume (which row/column/K slice a lane supplies, which
// outputs it receives, and which K block an E8M0 scale applies to) against a CPU product.
#include "common.h"
#include "kernels.h"

namespace cozyq {
namespace {

// a, b: 64 lanes x 32 bytes (i8 and bf16 kinds use the first 16); sa, sb: 64 bytes;
// d: 64 lanes x 16 words (int32 or float32; the 16x16 kinds fill the first 4).
__global__ void mfma_probe_kernel(int kind, const uint8_t* a, const uint8_t* b, const uint8_t* sa,
                                  const uint8_t* sb, uint32_t* d) {
    const int l = threadIdx.x;
    const i32x8 a8 = *reinterpret_cast<const i32x8*>(a + 32 * l);
    const i32x8 b8 = *reinterpret_cast<const i32x8*>(b + 32 * l);
    const i32x4 a4 = {a8[0], a8[1], a8[2], a8[3]};
    const i32x4 b4 = {b8[0], b8[1], b8[2], b8[3]};
    uint32_t r[16] = {};
    if (kind == 4) {
        typedef int32_t i32x16 __attribute__((ext_vector_type(16)));
        i32x16 z;
        for (int i = 0; i < 16; ++i) z[i] = 0;
        const i32x16 c = __builtin_amdgcn_mfma_i32_32x32x32_i8(a4, b4, z, 0, 0, 0);
        for (int i = 0; i < 16; ++i) r[i] = static_cast<uint32_t>(c[i]);
    } else if (kind == 5 || kind == 6) {
        f32x16 z;
        for (int i = 0; i < 16; ++i) z[i] = 0.0f;
        const f32x16 c = kind == 5 ? mfma_f8_32(a8, b8, z) : mfma_f8_32_scaled(a8, b8, z, sa[l], sb[l]);
        for (int i = 0; i < 16; ++i) r[i] = bits_of(c[i]);
    } else if (kind == 7) {
        f32x16 z;
        for (int i = 0; i < 16; ++i) z[i] = 0.0f;
        const int32_t a0 = a8[0], b0 = b8[0];
        const f32x16 c = __builtin_amdgcn_mfma_f32_32x32x2f32(__builtin_bit_cast(float, a0),
                                                              __builtin_bit_cast(float, b0), z, 0, 0, 0);
        for (int i = 0; i < 16; ++i) r[i] = bits_of(c[i]);
    } else if (kind == 8) {
        typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
        f32x16 z;
        for (int i = 0; i < 16; ++i) z[i] = 0.0f;
        const f32x16 c = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a4),
                                                                __builtin_bit_cast(f16x8_t, b4), z, 0, 0, 0);
        for (int i = 0; i < 16; ++i) r[i] = bits_of(c[i]);
    } else if (kind == 0) {
        const i32x4 c = mfma_i8(a4, b4, i32x4{0, 0, 0, 0});
        for (int i = 0; i < 4; ++i) r[i] = static_cast<uint32_t>(c[i]);
    } else if (kind == 1) {
        const f32x4 c = mfma_f8(a8, b8, f32x4{0, 0, 0, 0});
        for (int i = 0; i < 4; ++i) r[i] = bits_of(c[i]);
    } else if (kind == 2) {
        const f32x4 c = mfma_f8_scaled(a8, b8, f32x4{0, 0, 0, 0}, sa[l], sb[l]);
        for (int i = 0; i < 4; ++i) r[i] = bits_of(c[i]);
    } else {
        const bf16x8 ab = __builtin_bit_cast(bf16x8, a4);
        const bf16x8 bb = __builtin_bit_cast(bf16x8, b4);
        const f32x4 c = mfma_bf16(ab, bb, f32x4{0, 0, 0, 0});
        for (int i = 0; i < 4; ++i) r[i] = bits_of(c[i]);
    }
    for (int i = 0; i < 16; ++i) d[16 * l + i] = r[i];
}

// Two floats a thread through gfx950's v_cvt_pk_fp8_f32 (OCP E4M3, round to nearest even): the
// conversion the quantizers may use in place of the software encoder once it agrees bit for bit.
__global__ void e4m3_probe_kernel(const float* in, uint8_t* out, int64_t pairs) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= pairs) return;
    const int packed = __builtin_amdgcn_cvt_pk_fp8_f32(in[2 * i], in[2 * i + 1], 0, false);
    out[2 * i] = static_cast<uint8_t>(packed & 0xff);
    out[2 * i + 1] = static_cast<uint8_t>((packed >> 8) & 0xff);
}

// div_rn against the hardware's correctly rounded division, one pair a thread.
__global__ void div_probe_kernel(const float* x, const float* s, float* out, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    out[i] = div_rn(x[i], s[i], 1.0f / s[i]);
}

}  // namespace

hipError_t div_probe(const float* x, const float* s, float* out, int64_t n, hipStream_t st) {
    if (n == 0) return hipSuccess;
    div_probe_kernel<<<static_cast<unsigned>((n + 255) / 256), 256, 0, st>>>(x, s, out, n);
    return hipGetLastError();
}

hipError_t e4m3_probe(const float* in, uint8_t* out, int64_t n, hipStream_t s) {
    const int64_t pairs = n / 2;
    if (pairs == 0) return hipSuccess;
    e4m3_probe_kernel<<<static_cast<unsigned>((pairs + 255) / 256), 256, 0, s>>>(in, out, pairs);
    return hipGetLastError();
}

hipError_t mfma_probe(int kind, const void* a, const void* b, const void* sa, const void* sb,
                      void* d, hipStream_t s) {
    mfma_probe_kernel<<<1, 64, 0, s>>>(kind, static_cast<const uint8_t*>(a),
                                       static_cast<const uint8_t*>(b),
                                       static_cast<const uint8_t*>(sa),
                                       static_cast<const uint8_t*>(sb), static_cast<uint32_t*>(d));
    return hipGetLastError();
}

}  // namespace cozyq
