// Deterministic synthetic tensors generated on the device.
//
// Same generator as nnzap_amd/synth.py: element i of a standard-normal
// stream `seed` is Box-Muller on splitmix64 outputs 2i and 2i+1 (uniforms
// (u64 >> 11) * 2^-53), evaluated in double precision in the same operation
// order as the host generator, scaled, then rounded once to bf16 (RNE).
// Used to fill the 311M-element bf16 embedding table of the benchmark model
// in milliseconds instead of minutes on the host.
#include "common.h"

namespace {

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// RNE double -> bf16 on the bit pattern (normal float32 range), falling back
// to round-to-odd float then RNE for anything else (both a single rounding).
__device__ __forceinline__ uint16_t f64_to_bf16(double x) {
    const uint64_t b = (uint64_t)__double_as_longlong(x);
    const uint16_t sign = (uint16_t)((b >> 48) & 0x8000u);
    const uint64_t t = b & 0x7FFFFFFFFFFFFFFFull;
    const uint64_t r = t + ((1ull << 44) - 1) + ((t >> 45) & 1ull);
    const int64_t e = (int64_t)(r >> 52) - 896;
    if (e >= 1 && e <= 254) return sign | (uint16_t)(e << 7) | (uint16_t)((r >> 45) & 0x7F);
    float f = (float)x;
    uint32_t fb = __float_as_uint(f);
    const double back = (double)f;
    if (back != x) fb = ((fabs(back) > fabs(x)) ? fb - 1u : fb) | 1u;
    return f32_to_bf16_rne(__uint_as_float(fb));
}

__global__ void normal_bf16_kernel(uint16_t *out, uint64_t n, uint64_t seed, double scale) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const uint64_t g = 0x9E3779B97F4A7C15ull;
        const double u1 = (double)(mix64(seed + (2 * i + 1) * g) >> 11) * 0x1.0p-53;
        const double u2 = (double)(mix64(seed + (2 * i + 2) * g) >> 11) * 0x1.0p-53;
        const double r = sqrt(-2.0 * log1p(-u1));
        const double z = r * cos((2.0 * M_PI) * u2);
        out[i] = f64_to_bf16(scale * z);
    }
}

}  // namespace

extern "C" int nnz_synth_normal_bf16(nnz_ctx *ctx, void *out, uint64_t n, uint64_t seed,
                                     double scale) {
    NNZ_CHECK_CTX(ctx);
    NNZ_REQUIRE(ctx, out && n > 0, NNZ_EINVAL, "synth_normal_bf16: bad arguments");
    normal_bf16_kernel<<<4096, 256, 0, ctx->stream>>>((uint16_t *)out, n, seed, scale);
    NNZ_LAUNCHED(ctx);
    return NNZ_OK;
}
