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

#include "by_key.hpp"  // the wave64 primitives under test (common.hpp, wave_seg_scan)

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

enum Gen { kReduceI32, kU8U32, kNormalF32, kKeysU32, kKeysAnd3, kKeysU64Low16, kIotaU32, kKeysU64 };

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
        } else if constexpr (G == kKeysU64) {
            static_cast<uint64_t *>(out)[i] = word(s0, i);
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

// ---------------------------------------------------------------- test checkers
// Device restatements of the oracle's O(N) property checkers, for sort sizes
// whose host check would take minutes.  The GPU tests pin them against the
// host checkers (and planted mistakes) at small sizes.
//
// Sortedness and multiset hashes of a u32 array: out[0] += number of i with
// a[i] > a[i+1]; out[1] += sum of a[i]; out[2] += sum of mix64(a[i]) (both
// sums mod 2^64 are order-independent, so equal multisets give equal sums).
__global__ __launch_bounds__(256) void sorted_hash_kernel(const uint32_t *__restrict__ a, uint64_t n,
                                                          unsigned long long *out)
{
    uint64_t desc = 0, s1 = 0, s2 = 0;
    const uint64_t stride = (uint64_t)gridDim.x * 256;
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) {
        const uint32_t x = a[i];
        if (i + 1 < n && x > a[i + 1]) ++desc;
        s1 += x;
        s2 += mix64(x);
    }
    atomicAdd(&out[0], (unsigned long long)desc);
    atomicAdd(&out[1], (unsigned long long)s1);
    atomicAdd(&out[2], (unsigned long long)s2);
}

// Stable-pairs checker (values = input index): counts positions i where
// vals_out[i] >= n, keys_out[i] != keys_in[vals_out[i]], or (keys_out[i],
// vals_out[i]) is not strictly below (keys_out[i+1], vals_out[i+1]).  Zero
// bad positions <=> the output is the stable sort of the input: the pairs
// are distinct, so the n values < n form a permutation.
__global__ __launch_bounds__(256) void stable_pairs_kernel(const uint32_t *__restrict__ kin,
                                                           const uint32_t *__restrict__ kout,
                                                           const uint32_t *__restrict__ vout, uint64_t n,
                                                           unsigned long long *bad)
{
    uint64_t b = 0;
    const uint64_t stride = (uint64_t)gridDim.x * 256;
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) {
        const uint32_t v = vout[i], k = kout[i];
        if (v >= n || kin[v] != k) ++b;
        if (i + 1 < n) {
            const uint32_t k1 = kout[i + 1], v1 = vout[i + 1];
            if (k > k1 || (k == k1 && v >= v1)) ++b;
        }
    }
    atomicAdd(bad, (unsigned long long)b);
}

// Probe of the LDS ordering the sort's stable ranking relies on: in one
// returning LDS atomic add instruction, lanes that hit the same address get
// their old values in lane order.  Each wave repeatedly draws a digit per
// lane (pattern 0: uniform over 256; 1: digit 0 with probability 1/3, else
// uniform; 2: one digit for the whole wave; 3: two digits), adds 1 at its
// digit's counter and checks that every lane's result equals the counter's
// value before the instruction plus the number of lower lanes with the same
// digit.  Every LDS index is < 256 + 64 per wave; violations are counted.
__global__ __launch_bounds__(256) void lds_order_probe_kernel(uint64_t seed, uint32_t pattern, uint32_t rounds,
                                                              unsigned long long *violations)
{
    __shared__ uint32_t cnt[4][256];
    __shared__ uint32_t before[4][256];
    const uint32_t lane = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
    const uint32_t w = threadIdx.x / 64;
    for (uint32_t i = lane; i < 256; i += 64) cnt[w][i] = 0;
    __builtin_amdgcn_wave_barrier();
    uint64_t bad = 0;
    const uint64_t gid = (uint64_t)blockIdx.x * 4 + w;
    for (uint32_t r = 0; r < rounds; ++r) {
        const uint64_t h = word(seed, (gid * rounds + r) * 64 + lane);
        uint32_t d;
        if (pattern == 0) d = (uint32_t)h & 255u;
        else if (pattern == 1) d = ((h >> 32) % 3 == 0) ? 0u : ((uint32_t)h & 255u);
        else if (pattern == 2) d = (uint32_t)word(seed, gid * rounds + r) & 255u;
        else d = ((uint32_t)h & 1u) ? 17u : 200u;
        // counter values before this instruction
        for (uint32_t i = lane; i < 256; i += 64) before[w][i] = cnt[w][i];
        __builtin_amdgcn_wave_barrier();
        const uint32_t got = atomicAdd(&cnt[w][d], 1u);
        // lower lanes with the same digit, from one ballot per candidate
        uint32_t lower = 0;
        for (uint32_t j = 0; j < 64; ++j) {
            const uint32_t dj = (uint32_t)__builtin_amdgcn_readlane((int)d, (int)j);
            lower += (j < lane && dj == d) ? 1u : 0u;
        }
        if (got != before[w][d] + lower) ++bad;
        __builtin_amdgcn_wave_barrier();
    }
    if (bad) atomicAdd(violations, (unsigned long long)bad);
}

// ---------------------------------------------------------------- copy shapes
// Pure permutation copies of n uint32 (read 4n, write 4n bytes) in the access
// shapes of the primitives' kernels, so each kernel can be compared with what
// its own shape achieves as a copy.  Occupancy is pinned with unused dynamic
// LDS where the shape says so, to the workgroups per CU of the kernel it stands
// for (a copy needs fewer registers than the kernel and would otherwise run
// more workgroups per CU):
//   1      the exclusive scan's tile: one 256-thread workgroup per tile of 20
//          16-byte vectors per thread held in registers, non-temporal loads
//          and stores; 4 workgroups per CU (36 KiB LDS each).
//   2      as 1 with the copy's own occupancy.
//   3      a grid-stride loop of 16-byte vectors over 2048 workgroups.
//   4      the onesweep's tile: 512 threads x 32 wave-striped dword loads, then
//          32 dword stores, thread-striped over the tile; 3 workgroups per CU
//          (48 KiB LDS each).
//   5..8   the onesweep's tile (as 4) writing its keys as if sorted into 256
//          digit runs of 64 keys (256 B) each, every tile's run of digit d
//          following the previous tile's (positions d * n/256 + tile * 64 + ..):
//          5  runs line-aligned, XCD runs of 16 tiles (the sort's workgroup ->
//             tile map);
//          6  run boundaries inside cache lines (digit pairs 2k, 2k+1 split
//             their 128 slots at 64 +- a_k, mirrored by odd tiles, so runs stay
//             contiguous across tiles), XCD runs of 16;
//          7  as 6 with plain dispatch order (runs of 1);
//          8  line-aligned runs, but every store instruction straddles lines
//             whose other half comes from the neighbouring wave of the same tile.
// Shape 0 is copy_probe_kernel above.  n must be a multiple of 16384 and at
// least 65536 (shapes 4-8), or a multiple of 20480 (shapes 1, 2).
__device__ __forceinline__ uint32_t dg_xcd_tile(uint32_t b, uint32_t grid, uint32_t log_run)
{
    const uint32_t log_group = log_run + 3;
    const uint32_t g = b >> log_group;
    if ((g + 1) << log_group > grid) return b;
    const uint32_t r = b & ((1u << log_group) - 1);
    return (g << log_group) + ((r & 7) << log_run) + (r >> 3);
}

// `zero` is 0 at run time: every stored vector depends on all of the
// thread's loads, so the tile is held in registers before the first store
// (as in the scan, whose stores wait for the look-back).
template <int VECS>
__global__ __launch_bounds__(256) void shape_scan_tile(const u32x4c *__restrict__ in, u32x4c *__restrict__ out,
                                                       uint32_t zero)
{
    const uint64_t base = (uint64_t)blockIdx.x * 256 * VECS;
    u32x4c v[VECS];
#pragma unroll
    for (int k = 0; k < VECS; ++k) v[k] = __builtin_nontemporal_load(in + base + (uint64_t)k * 256 + threadIdx.x);
    u32x4c t = v[0];
#pragma unroll
    for (int k = 1; k < VECS; ++k) t ^= v[k];
    const uint32_t dep = (t.x ^ t.y ^ t.z ^ t.w) & zero;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < VECS; ++k) __builtin_nontemporal_store(v[k] + dep, out + base + (uint64_t)k * 256 + threadIdx.x);
}

__global__ __launch_bounds__(256) void shape_grid_stride(const u32x4c *__restrict__ in, u32x4c *__restrict__ out,
                                                         uint64_t nvec)
{
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < nvec; i += (uint64_t)gridDim.x * 256)
        __builtin_nontemporal_store(__builtin_nontemporal_load(in + i), out + i);
}

// Output position of sorted slot i of `tile` in shapes 4..8 (see above).
__device__ __forceinline__ uint32_t shape_pos(int shape, uint32_t tile, uint32_t i, uint32_t n)
{
    const uint32_t region = n >> 8;
    if (shape == 4) return tile * 16384u + i;
    if (shape == 5) return (i >> 6) * region + tile * 64u + (i & 63u);
    if (shape == 8) {
        const uint32_t i2 = (i + 16u) & 16383u;
        return (i2 >> 6) * region + tile * 64u + (i2 & 63u);
    }
    const uint32_t kk = i >> 7, r = i & 127u;
    const uint32_t a = (kk * 37u) % 29u + 1u;
    const bool odd = tile & 1u;
    const uint32_t split = odd ? 64u - a : 64u + a;
    const uint32_t d = r < split ? 2 * kk : 2 * kk + 1;
    const uint32_t within = r < split ? r : r - split;
    const uint32_t pre = tile * 64u + (odd ? ((d & 1u) ? 0u - a : a) : 0u);
    return d * region + pre + within;
}

__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(6, 6)))
void shape_onesweep_tile(const uint32_t *__restrict__ in, uint32_t *__restrict__ out, uint32_t n, int shape,
                         uint32_t log_run, uint32_t zero)
{
    const uint32_t tile = dg_xcd_tile(blockIdx.x, gridDim.x, log_run);
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t base = tile * 16384u;
    uint32_t k[32];
#pragma unroll
    for (int u = 0; u < 32; ++u) k[u] = __builtin_nontemporal_load(in + base + wave * 2048u + (uint32_t)u * 64u + lane);
    uint32_t t = 0;  // as in shape_scan_tile: the stores wait for every load
#pragma unroll
    for (int u = 0; u < 32; ++u) t ^= k[u];
    const uint32_t dep = t & zero;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        const uint32_t p = shape_pos(shape, tile, (uint32_t)j * 512u + tid, n);
        if (p < n) out[p] = k[j] + dep;
    }
}

// Known-answer kernel for the shared wave64 primitives the product kernels
// are built from (common.hpp, by_key.hpp), over int32 data: lane l of wave w
// holds element w * 64 + l; n is a multiple of 64, so every wave is either
// wholly in range or exits whole (the DPP and ballot steps see full waves).
//   0  out[w] = wave_allreduce(x, Sum)        (the wave's lane 0 writes)
//   1  out[i] = wave_inclusive_scan(x, Sum) - x (exclusive sum)
//   2  out[i] = wave_inclusive_scan(x, Sum)
//   3  out[i] = sum since the last lane <= i whose flag is set, or since
//      lane 0 (wave_seg_scan of (flag, x) pairs)
//   4  out[i] = mask_rank(ballot(flag != 0)): flagged lanes below lane i
//   5  out[i] = wave_inclusive_scan(x, Max)
//   6  out[w] = wave_allreduce(x, Min)
//   7  out[i] = wave_shr1(x, fill = -1): x of lane i - 1
// Sums wrap (two's complement), as the primitives' integer sums do.
__global__ __launch_bounds__(256) void wave_kat_kernel(const int32_t *__restrict__ in,
                                                       const int32_t *__restrict__ flags, int32_t *__restrict__ out,
                                                       uint32_t n, int kind)
{
    using namespace lcpp;
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= n) return;
    const int32_t x = in[i];
    const uint32_t lane = lane_id();
    switch (kind) {
    case 0: {
        const int32_t r = wave_allreduce(x, SumOp());
        if (lane == 0) out[i / kWave] = r;
        break;
    }
    case 1: out[i] = wave_inclusive_scan(x, SumOp()) - x; break;
    case 2: out[i] = wave_inclusive_scan(x, SumOp()); break;
    case 3: {
        bool f = flags[i] != 0;
        int32_t v = x;
        wave_seg_scan(f, v, SumOp());
        out[i] = v;
        break;
    }
    case 4: out[i] = (int32_t)mask_rank(ballot(flags[i] != 0)); break;
    case 5: out[i] = wave_inclusive_scan(x, MaxOp()); break;
    case 6: {
        const int32_t r = wave_allreduce(x, MinOp());
        if (lane == 0) out[i / kWave] = r;
        break;
    }
    default: out[i] = wave_shr1(x, -1); break;
    }
}

}  // namespace

extern "C" {

int lcpp_copy_probe_u32(const void *in, void *out, uint64_t n, void *stream);

// Copy of n uint32 in access shape `shape` (0..8, see the copy shapes above);
// 16-byte aligned pointers.  Shapes 0-3 copy in[i] to out[i]; 4-8 permute.  Returns -1 for a shape or size it does not take.
int lcpp_dg_copy_shape(const void *in, void *out, uint64_t n, int shape, void *stream)
{
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (!in || !out || ((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(out)) & 15)) return -1;
    if (n > 0xFFFFFFFFull) return -1;
    const auto *vi = static_cast<const u32x4c *>(in);
    auto *vo = static_cast<u32x4c *>(out);
    if (shape == 0) return lcpp_copy_probe_u32(in, out, n, stream);
    if (shape == 1 || shape == 2) {
        if (n % (256 * 20 * 4)) return -1;
        shape_scan_tile<20><<<(uint32_t)(n / (256 * 20 * 4)), 256, shape == 1 ? 36u << 10 : 0u, s>>>(vi, vo, 0u);
    } else if (shape == 3) {
        if (n % 4) return -1;
        shape_grid_stride<<<2048, 256, 0, s>>>(vi, vo, n / 4);
    } else if (shape >= 4 && shape <= 8) {
        if (n % 16384 || n < 65536) return -1;
        const uint32_t log_run = shape == 4 || shape == 7 ? 0u : 4u;
        shape_onesweep_tile<<<(uint32_t)(n / 16384), 512, 48u << 10, s>>>(static_cast<const uint32_t *>(in),
                                                                   static_cast<uint32_t *>(out), (uint32_t)n, shape,
                                                                   log_run, 0u);
    } else {
        return -1;
    }
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

// out[3] (device, zeroed by the caller): descents, sum, sum of mix64.
int lcpp_dg_sorted_hash_u32(const void *a, uint64_t n, void *out, void *stream)
{
    if (!out || (n && !a)) return -1;
    sorted_hash_kernel<<<2048, 256, 0, static_cast<hipStream_t>(stream)>>>(
        static_cast<const uint32_t *>(a), n, static_cast<unsigned long long *>(out));
    return hipGetLastError() == hipSuccess ? 0 : -4;
}
// *bad (device, zeroed by the caller) += bad positions of a stable u32/u32
// sort whose values were the input indices.
int lcpp_dg_check_stable_pairs_u32(const void *keys_in, const void *keys_out, const void *vals_out, uint64_t n,
                                   void *bad, void *stream)
{
    if (!bad || (n && (!keys_in || !keys_out || !vals_out))) return -1;
    stable_pairs_kernel<<<2048, 256, 0, static_cast<hipStream_t>(stream)>>>(
        static_cast<const uint32_t *>(keys_in), static_cast<const uint32_t *>(keys_out),
        static_cast<const uint32_t *>(vals_out), n, static_cast<unsigned long long *>(bad));
    return hipGetLastError() == hipSuccess ? 0 : -4;
}
// *violations (device, zeroed by the caller) += lanes whose atomic result
// broke lane order, over `waves` waves x `rounds` instructions.
int lcpp_dg_lds_order_probe(uint64_t seed, uint32_t pattern, uint32_t waves, uint32_t rounds, void *violations,
                            void *stream)
{
    if (!violations || pattern > 3 || waves == 0 || (waves & 3)) return -1;
    lds_order_probe_kernel<<<waves / 4, 256, 0, static_cast<hipStream_t>(stream)>>>(
        seed, pattern, rounds, static_cast<unsigned long long *>(violations));
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

// One of the wave64 known-answer cases above (kind 0..7) over n int32
// elements, n a multiple of 64; `flags` is read by kinds 3 and 4 only.
// out holds n / 64 elements for kinds 0 and 6, n otherwise.
int lcpp_dg_wave_kat(int kind, const void *in, const void *flags, void *out, uint64_t n, void *stream)
{
    if (kind < 0 || kind > 7 || !in || !out || n == 0 || (n % 64) || n > 0x7FFFFFFFull) return -1;
    if ((kind == 3 || kind == 4) && !flags) return -1;
    wave_kat_kernel<<<(uint32_t)((n + 255) / 256), 256, 0, static_cast<hipStream_t>(stream)>>>(
        static_cast<const int32_t *>(in), static_cast<const int32_t *>(flags), static_cast<int32_t *>(out),
        (uint32_t)n, kind);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

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
int lcpp_gen_keys_u64(uint64_t seed, uint64_t n, void *out, void *stream)
{
    return launch<kKeysU64>(out, n, seed, 0, 0, stream);
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
