// datagen.hip — synthetic benchmark inputs, generated in HBM.
//
// Not part of the primitives: bench.py and the GPU tests use it to build
// the seeded inputs of the benchmark configurations directly on the device
// (1 GiB inputs are not shipped or copied from the host).  The formulas are
// counter-based splitmix64 (Vigna, public domain):
//   w_i = mix64(seed + (i + 1) * 0x9E3779B97F4A7C15)
// so any element can be regenerated independently on the host.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <vector>

namespace {

constexpr uint64_t kGamma = 0x9E3779B97F4A7C15ull;

__host__ __device__ __forceinline__ uint64_t mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
__host__ __device__ __forceinline__ uint64_t word(uint64_t seed, uint64_t i)
{
    return mix64(seed + (i + 1) * kGamma);
}

enum Gen { kReduceI32, kU8U32, kNormalF32, kKeysU32, kKeysAnd3, kKeysU64Low16, kIotaU32 };

template <int G>
__global__ __launch_bounds__(256) void gen_kernel(void *out, uint64_t n, uint64_t s0, uint64_t s1,
                                                  uint64_t s2)
{
    const uint64_t stride = (uint64_t)gridDim.x * 256;
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) {
        if constexpr (G == kReduceI32) {
            const uint64_t hi = word(s0, i) >> 32;
            static_cast<int32_t *>(out)[i] = (int32_t)((hi * 2001ull) >> 32) - 1000;
        } else if constexpr (G == kU8U32) {
            static_cast<uint32_t *>(out)[i] = (uint32_t)(word(s0, i) >> 56);
        } else if constexpr (G == kNormalF32) {
            const double inv53 = 1.0 / 9007199254740992.0;
            const double u1 = (double)((word(s0, 2 * i) >> 11) + 1) * inv53;
            const double u2 = (double)(word(s0, 2 * i + 1) >> 11) * inv53;
            static_cast<float *>(out)[i] =
                (float)(sqrt(-2.0 * log(u1)) * cos(6.283185307179586476925286766559 * u2));
        } else if constexpr (G == kKeysU32) {
            static_cast<uint32_t *>(out)[i] = (uint32_t)word(s0, i);
        } else if constexpr (G == kKeysAnd3) {
            static_cast<uint32_t *>(out)[i] =
                (uint32_t)word(s0, i) & (uint32_t)word(s1, i) & (uint32_t)word(s2, i);
        } else if constexpr (G == kKeysU64Low16) {
            static_cast<uint64_t *>(out)[i] = word(s0, i) & 0xFFFFull;
        } else {
            static_cast<uint32_t *>(out)[i] = (uint32_t)i;
        }
    }
}

template <int G>
int launch(void *out, uint64_t n, uint64_t s0, uint64_t s1, uint64_t s2, void *stream)
{
    if (n == 0) return 0;
    if (!out) return -1;
    uint64_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipStream_t s = static_cast<hipStream_t>(stream);
    gen_kernel<G><<<(uint32_t)blocks, 256, 0, s>>>(out, n, s0, s1, s2);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

// Plain streaming copy: a kernel of known traffic (read 4n + write 4n bytes)
// against which hardware byte counters (FETCH_SIZE / WRITE_SIZE) are
// calibrated, and the read+write ceiling of the part.  One short-lived
// workgroup per 8 KiB (two non-temporal 16-byte vectors per thread) was the
// fastest of the copy shapes measured at 2^28 x uint32: 348 us (6.18 TB/s),
// against 357-366 us for 4 vectors per thread, 383-431 us for 8, and 418 us
// for a grid-stride loop of one vector per thread.
typedef uint32_t u32x4c __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(256) void copy_probe_kernel(const u32x4c *__restrict__ in, u32x4c *__restrict__ out,
                                                         uint64_t nvec)
{
    const uint64_t b = (uint64_t)blockIdx.x * 512 + threadIdx.x;
    u32x4c v0 = {0, 0, 0, 0}, v1 = {0, 0, 0, 0};
    if (b < nvec) v0 = __builtin_nontemporal_load(in + b);
    if (b + 256 < nvec) v1 = __builtin_nontemporal_load(in + b + 256);
    if (b < nvec) __builtin_nontemporal_store(v0, out + b);
    if (b + 256 < nvec) __builtin_nontemporal_store(v1, out + b + 256);
}

}  // namespace

extern "C" {

// n must be a multiple of 4 and both pointers 16-byte aligned.
int lcpp_copy_probe_u32(const void *in, void *out, uint64_t n, void *stream)
{
    if (n == 0) return 0;
    if (!in || !out || (n & 3) || ((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(out)) & 15))
        return -1;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const uint64_t blocks = (n / 4 + 511) / 512;
    if (blocks > 0x7FFFFFFFull) return -1;
    copy_probe_kernel<<<(uint32_t)blocks, 256, 0, s>>>(static_cast<const u32x4c *>(in), static_cast<u32x4c *>(out),
                                                       n / 4);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int lcpp_gen_reduce_i32(uint64_t seed, uint64_t n, void *out, void *stream)
{
    return launch<kReduceI32>(out, n, seed, 0, 0, stream);
}
int lcpp_gen_u8_u32(uint64_t seed, uint64_t n, void *out, void *stream)
{
    return launch<kU8U32>(out, n, seed, 0, 0, stream);
}
int lcpp_gen_normal_f32(uint64_t seed, uint64_t n, void *out, void *stream)
{
    return launch<kNormalF32>(out, n, seed, 0, 0, stream);
}
int lcpp_gen_keys_u32(uint64_t seed, uint64_t n, void *out, void *stream)
{
    return launch<kKeysU32>(out, n, seed, 0, 0, stream);
}
int lcpp_gen_keys_u32_and3(uint64_t sa, uint64_t sb, uint64_t sc, uint64_t n, void *out,
                           void *stream)
{
    return launch<kKeysAnd3>(out, n, sa, sb, sc, stream);
}
int lcpp_gen_keys_u64_low16(uint64_t seed, uint64_t n, void *out, void *stream)
{
    return launch<kKeysU64Low16>(out, n, seed, 0, 0, stream);
}
int lcpp_gen_iota_u32(uint64_t n, void *out, void *stream)
{
    return launch<kIotaU32>(out, n, 0, 0, 0, stream);
}

// CSR segments on the host: L_s = 0 with p = 0.05 (stream seed_empty), else
// geometric on {1,2,...} with mean 128/0.95 (stream seed_len); cumulative
// offsets rescaled so the total is exactly n_items.
int lcpp_gen_segments_host(uint64_t seed_empty, uint64_t seed_len, uint64_t n_items,
                           uint64_t n_segments, uint32_t *begin, uint32_t *end)
{
    if (n_segments == 0) return 0;
    if (n_items > 0xFFFFFFFFull || !begin || !end) return -1;
    const double inv53 = 1.0 / 9007199254740992.0;
    const double p = 0.95 / 128.0;
    const double log1mp = log1p(-p);
    std::vector<uint64_t> c(n_segments + 1);
    c[0] = 0;
    for (uint64_t s = 0; s < n_segments; ++s) {
        const double ue = (double)(word(seed_empty, s) >> 11) * inv53;
        uint64_t len = 0;
        if (ue >= 0.05) {
            const double ul = (double)((word(seed_len, s) >> 11) + 1) * inv53;
            len = 1 + (uint64_t)floor(log(ul) / log1mp);
        }
        c[s + 1] = c[s] + len;
    }
    const uint64_t total = c[n_segments];
    for (uint64_t s = 0; s <= n_segments; ++s) {
        const uint64_t off = total ? (uint64_t)(((unsigned __int128)c[s] * n_items) / total)
                                   : (s ? n_items : 0);
        if (s < n_segments) begin[s] = (uint32_t)off;
        if (s > 0) end[s - 1] = (uint32_t)off;
    }
    return 0;
}

}  // extern "C"
