// common.hpp — wave64 building blocks for the gfx950 (CDNA4) primitives.
//
// The reference builds everything on 32-lane warps (warp/details/*_shlf.h).
// Here a wavefront is 64 lanes: reductions and scans take log2(64) = 6
// steps, ballots are 64-bit masks and lane masks come from v_mbcnt.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <limits>
#include <type_traits>

#include "../../include/lcpp_amd.h"

namespace lcpp {

constexpr int kWave = 64;

// ---------------------------------------------------------------- lanes
__device__ __forceinline__ uint32_t lane_id()
{
    return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
}

// Orders one wave's LDS accesses around a hand-off between its lanes (a
// lane reads what another lane of the same wave wrote): the LDS serves a
// wave's instructions in issue order, so only the compiler must not move
// accesses across this point.
__device__ __forceinline__ void wave_lds_sync()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// popcount(mask & lanes_below_me): rank of this lane among the lanes of `mask`.
__device__ __forceinline__ uint32_t mask_rank(uint64_t mask)
{
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                     __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

__device__ __forceinline__ uint64_t ballot(bool p) { return __ballot(p); }

// Match-any over an 8-bit value: the lanes of the wave whose low 8 bits of v
// equal this lane's (one ballot per bit; common/utils.h:273-324, MatchAny<8>,
// does the same over 32 lanes).  Every lane of the wave must be active.
__device__ __forceinline__ uint64_t match_any8(uint32_t v)
{
    uint64_t peers = ~0ull;
#pragma unroll
    for (int b = 0; b < 8; ++b) {
        const bool bit = (v >> b) & 1u;
        const uint64_t ones = ballot(bit);
        peers &= bit ? ones : ~ones;
    }
    return peers;
}

// ---------------------------------------------------------------- ops
struct SumOp {
    template <class T>
    __device__ __forceinline__ T operator()(T a, T b) const
    {
        if constexpr (std::is_integral_v<T>) {
            using U = std::make_unsigned_t<T>;
            return (T)((U)a + (U)b);  // two's-complement wraparound
        } else {
            return a + b;
        }
    }
    template <class T>
    static constexpr T identity() { return T(0); }
};
struct MinOp {
    template <class T>
    __device__ __forceinline__ T operator()(T a, T b) const { return b < a ? b : a; }
    template <class T>
    static constexpr T identity() { return std::numeric_limits<T>::max(); }
};
struct MaxOp {
    template <class T>
    __device__ __forceinline__ T operator()(T a, T b) const { return a < b ? b : a; }
    template <class T>
    static constexpr T identity() { return std::numeric_limits<T>::lowest(); }
};

// ---------------------------------------------------------------- shuffles
template <class T>
__device__ __forceinline__ T shfl_xor(T x, int m)
{
    if constexpr (sizeof(T) == 4) {
        return __builtin_bit_cast(T, __shfl_xor(__builtin_bit_cast(int, x), m));
    } else {
        static_assert(sizeof(T) == 8, "4- or 8-byte types only");
        int2 v = __builtin_bit_cast(int2, x);
        v.x = __shfl_xor(v.x, m);
        v.y = __shfl_xor(v.y, m);
        return __builtin_bit_cast(T, v);
    }
}

template <class T>
__device__ __forceinline__ T shfl_up(T x, int d)
{
    if constexpr (sizeof(T) == 4) {
        return __builtin_bit_cast(T, __shfl_up(__builtin_bit_cast(int, x), d));
    } else {
        int2 v = __builtin_bit_cast(int2, x);
        v.x = __shfl_up(v.x, d);
        v.y = __shfl_up(v.y, d);
        return __builtin_bit_cast(T, v);
    }
}

template <class T>
__device__ __forceinline__ T read_lane(T x, int lane)
{
    if constexpr (sizeof(T) == 4) {
        return __builtin_bit_cast(T, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), lane));
    } else {
        int2 v = __builtin_bit_cast(int2, x);
        v.x = __builtin_amdgcn_readlane(v.x, lane);
        v.y = __builtin_amdgcn_readlane(v.y, lane);
        return __builtin_bit_cast(T, v);
    }
}

// DPP permutation of a 4- or 8-byte value inside each row of 16 lanes
// (a VALU operand modifier: no LDS round trip, unlike __shfl_xor, which
// lowers to ds_bpermute_b32).
constexpr int kDppQuadXor1 = 0xB1;       // quad_perm [1,0,3,2]: lane ^ 1
constexpr int kDppQuadXor2 = 0x4E;       // quad_perm [2,3,0,1]: lane ^ 2
constexpr int kDppRowShr = 0x110;        // + n: lane i <- lane i - n inside its row of 16
constexpr int kDppWaveShr1 = 0x138;      // lane i <- lane i - 1 across the wave
constexpr int kDppRowMirror = 0x140;     // lane i <-> 15 - i within each 16
constexpr int kDppRowHalfMirror = 0x141; // lane i <-> 7 - i within each 8
constexpr int kDppRowBcast15 = 0x142;    // row r + 1 <- lane 15 of row r
constexpr int kDppRowBcast31 = 0x143;    // rows 2 and 3 <- lane 31
// Lanes whose source is outside the pattern, or whose row is not in
// ROW_MASK, get `old`.
template <int CTRL, int ROW_MASK = 0xF, class T>
__device__ __forceinline__ T dpp_move(T x, T old)
{
    if constexpr (sizeof(T) == 4) {
        return __builtin_bit_cast(T, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old), __builtin_bit_cast(int, x),
                                                                 CTRL, ROW_MASK, 0xF, false));
    } else {
        static_assert(sizeof(T) == 8, "4- or 8-byte types only");
        int2 v = __builtin_bit_cast(int2, x), o = __builtin_bit_cast(int2, old);
        v.x = __builtin_amdgcn_update_dpp(o.x, v.x, CTRL, ROW_MASK, 0xF, false);
        v.y = __builtin_amdgcn_update_dpp(o.y, v.y, CTRL, ROW_MASK, 0xF, false);
        return __builtin_bit_cast(T, v);
    }
}
template <int CTRL, class T>
__device__ __forceinline__ T dpp_perm(T x)
{
    return dpp_move<CTRL>(x, T(0));
}

// Reduction over the 64 lanes whose result is wave-uniform: DPP steps make
// every lane of a row of 16 hold the row's fold (pairs: lane ^ 1, lane ^ 2,
// then the two quads of each 8, then the two 8s of each 16), and the four row
// folds are read out of lanes 0, 16, 32, 48.  `op` must be commutative and
// associative (the pairing differs from a butterfly).
template <class T, class Op>
__device__ __forceinline__ T wave_reduce_dpp(T x, Op op)
{
    x = op(x, dpp_perm<kDppQuadXor1>(x));
    x = op(x, dpp_perm<kDppQuadXor2>(x));
    x = op(x, dpp_perm<kDppRowHalfMirror>(x));
    x = op(x, dpp_perm<kDppRowMirror>(x));
    return op(op(read_lane(x, 0), read_lane(x, 16)), op(read_lane(x, 32), read_lane(x, 48)));
}

// All-reduce over the 64 lanes; every lane gets the result (wave_reduce_dpp:
// the same pairing as a lane ^ 1, ^ 2, ... butterfly, so float sums are
// bit-identical to one).  `op` must be commutative and associative.
template <class T, class Op>
__device__ __forceinline__ T wave_allreduce(T x, Op op)
{
    return wave_reduce_dpp(x, op);
}

// Inclusive scan over the 64 lanes (lane order) with DPP: Kogge-Stone
// inside each row of 16 (row_shr 1, 2, 4, 8), then row 0's total into row 1
// and row 2's into row 3 (row_bcast15), then the first half's total into
// rows 2 and 3 (row_bcast31).  Lanes with no source take Op's identity.
// 6 VALU steps (the DPP folds into the op's instruction for 4-byte types);
// the __shfl_up form took 6 ds_bpermute round trips (64-bit scans: 757 us
// with it against 744 us, both at 2^27).
template <class T, class Op>
__device__ __forceinline__ T wave_inclusive_scan(T x, Op op)
{
    const T id = Op::template identity<T>();
    x = op(dpp_move<kDppRowShr + 1>(x, id), x);
    x = op(dpp_move<kDppRowShr + 2>(x, id), x);
    x = op(dpp_move<kDppRowShr + 4>(x, id), x);
    x = op(dpp_move<kDppRowShr + 8>(x, id), x);
    x = op(dpp_move<kDppRowBcast15, 0xA>(x, id), x);
    x = op(dpp_move<kDppRowBcast31, 0xC>(x, id), x);
    return x;
}

// x of lane - 1 (lane 0: `fill`), a DPP wave shift.
template <class T>
__device__ __forceinline__ T wave_shr1(T x, T fill)
{
    return dpp_move<kDppWaveShr1>(x, fill);
}

// ---------------------------------------------------------------- atomics
// Device-coherent (agent scope) accesses: the 8 XCDs of an MI355X have
// private L2s, so cross-workgroup publication must bypass them.
template <class T>
__device__ __forceinline__ T ld_relaxed(const T *p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <class T>
__device__ __forceinline__ T ld_acquire(const T *p)
{
    return __hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT);
}
template <class T>
__device__ __forceinline__ void st_relaxed(T *p, T v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <class T>
__device__ __forceinline__ void st_release(T *p, T v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ticket(uint32_t *ctr)
{
    return __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------- 16-byte vectors
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Streaming (non-temporal) 16-byte load/store: data touched once.
__device__ __forceinline__ u32x4 ld16_nt(const void *p)
{
    return __builtin_nontemporal_load(static_cast<const u32x4 *>(p));
}
__device__ __forceinline__ void st16_nt(void *p, u32x4 v)
{
    __builtin_nontemporal_store(v, static_cast<u32x4 *>(p));
}

// Split a 16-byte vector into 4 or 2 elements of T and back.  The vector
// components are copied into scalars first: clang folds
// __builtin_bit_cast(T, v.y) on an ext_vector component to component 0.
template <class T>
__device__ __forceinline__ void unpack16(u32x4 v, T (&out)[16 / sizeof(T)])
{
    const uint32_t a = v.x, b = v.y, c = v.z, d = v.w;
    if constexpr (sizeof(T) == 4) {
        out[0] = __builtin_bit_cast(T, a);
        out[1] = __builtin_bit_cast(T, b);
        out[2] = __builtin_bit_cast(T, c);
        out[3] = __builtin_bit_cast(T, d);
    } else {
        static_assert(sizeof(T) == 8, "4- or 8-byte types only");
        const uint64_t lo = ((uint64_t)b << 32) | a;
        const uint64_t hi = ((uint64_t)d << 32) | c;
        out[0] = __builtin_bit_cast(T, lo);
        out[1] = __builtin_bit_cast(T, hi);
    }
}
template <class T>
__device__ __forceinline__ u32x4 pack16(const T (&in)[16 / sizeof(T)])
{
    u32x4 v;
    if constexpr (sizeof(T) == 4) {
        const uint32_t a = __builtin_bit_cast(uint32_t, in[0]);
        const uint32_t b = __builtin_bit_cast(uint32_t, in[1]);
        const uint32_t c = __builtin_bit_cast(uint32_t, in[2]);
        const uint32_t d = __builtin_bit_cast(uint32_t, in[3]);
        v.x = a;
        v.y = b;
        v.z = c;
        v.w = d;
    } else {
        const uint64_t lo = __builtin_bit_cast(uint64_t, in[0]);
        const uint64_t hi = __builtin_bit_cast(uint64_t, in[1]);
        v.x = (uint32_t)lo;
        v.y = (uint32_t)(lo >> 32);
        v.z = (uint32_t)hi;
        v.w = (uint32_t)(hi >> 32);
    }
    return v;
}

// ---------------------------------------------------------------- raw buffers
// A raw buffer resource (stride 0) over [p, p + bytes): loads past `bytes`
// return 0 and stores past it are dropped by the address unit, so a ragged
// last tile needs no per-element guards.  Word 3 = 0x00020000 selects 32-bit
// data format, the gfx9-family raw-buffer encoding.  Offsets are 32-bit, so
// one resource covers < 2 GiB.
constexpr int kRawBufferWord3 = 0x00020000;
// Cache-policy operand of the buffer builtins on gfx94x/gfx950: bit 1 = nt
// (streaming, no reuse expected); bit 4 = sc1 (device scope: the load is
// served coherently across the XCDs' L2s, as an agent-scope atomic load).
constexpr int kPolicyNT = 2;
constexpr int kPolicySc1 = 16;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *p, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, (int)bytes, kRawBufferWord3);
}
__device__ __forceinline__ u32x4 buf_ld16_nt(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff)
{
    return __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, kPolicyNT);
}
__device__ __forceinline__ void buf_st16_nt(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, u32x4 v)
{
    __builtin_amdgcn_raw_buffer_store_b128(v, r, (int)voff, (int)soff, kPolicyNT);
}
// One 4- or 8-byte element (0 when out of range).
template <class T>
__device__ __forceinline__ T buf_ld_elem(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff)
{
    if constexpr (sizeof(T) == 4) {
        return __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 0));
    } else {
        static_assert(sizeof(T) == 8, "4- or 8-byte types only");
        const auto w = __builtin_amdgcn_raw_buffer_load_b64(r, (int)voff, (int)soff, 0);
        const uint32_t lo = w[0], hi = w[1];
        return __builtin_bit_cast(T, ((uint64_t)hi << 32) | lo);
    }
}
// The same with the streaming (nt) policy.
template <class T>
__device__ __forceinline__ T buf_ld_elem_nt(__amdgpu_buffer_rsrc_t r, uint32_t voff)
{
    if constexpr (sizeof(T) == 4) {
        return __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, 0, kPolicyNT));
    } else {
        static_assert(sizeof(T) == 8, "4- or 8-byte types only");
        const auto w = __builtin_amdgcn_raw_buffer_load_b64(r, (int)voff, 0, kPolicyNT);
        const uint32_t lo = w[0], hi = w[1];
        return __builtin_bit_cast(T, ((uint64_t)hi << 32) | lo);
    }
}
template <class T>
__device__ __forceinline__ void buf_st_elem(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, T v)
{
    if constexpr (sizeof(T) == 4) {
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, (int)voff, (int)soff, 0);
    } else {
        typedef uint32_t u32x2v __attribute__((vector_size(8)));
        const uint64_t b = __builtin_bit_cast(uint64_t, v);
        u32x2v w;
        w[0] = (uint32_t)b;
        w[1] = (uint32_t)(b >> 32);
        __builtin_amdgcn_raw_buffer_store_b64(w, r, (int)voff, (int)soff, 0);
    }
}

// ---------------------------------------------------------------- waits and the status word
// Upper bound on the polls of one look-back wait (~0.5 s of s_sleep-paced
// polling).  A wait that exceeds it gives up, so a kernel always drains even
// if a predecessor's word were never published; the give-up is recorded in
// the call's status word (below), so the result is reported as wrong instead
// of a hung GPU.
constexpr uint32_t kSpinLimit = 1u << 20;

// Every primitive that uses temp storage keeps a status header in its first
// 256 bytes; the first 32-bit word is zeroed by the call's first kernel and
// collects LCPP_DEVICE_STATUS_* bits (lcpp_amd.h), read back by
// lcpp_temp_status().  The rest of the temp layout starts after the header.
constexpr uint64_t kStatusBytes = 256;

// What a kernel that waits on other workgroups needs besides its data:
// where a wait that gives up reports, how long a wait lasts, and a test hook
// (a tile that never publishes, so the waits behind it give up on purpose:
// the kernels still drain normally, every access stays in bounds).
struct WaitCtl {
    uint32_t *status;     // status word (zeroed earlier in the same call)
    uint32_t spin_limit;  // re-polls before a wait gives up (>= 1)
    uint32_t withhold;    // tile that does not publish its look-back words (~0u: none)
};
__device__ __forceinline__ void report_timeout(const WaitCtl &c)
{
    __hip_atomic_fetch_or(c.status, (uint32_t)LCPP_DEVICE_STATUS_LOOKBACK_TIMEOUT, __ATOMIC_RELAXED,
                          __HIP_MEMORY_SCOPE_AGENT);
}
// Host: the WaitCtl of a call whose status word is `status` (the test hooks
// set by lcpp_test_set_lookback_fault apply).
WaitCtl wait_ctl(uint32_t *status);

// ---------------------------------------------------------------- misc

// (no a + b - 1 that would wrap for sizes near 2^64)
__host__ __device__ constexpr uint64_t ceil_div(uint64_t a, uint64_t b) { return a / b + (a % b != 0); }
__host__ __device__ constexpr uint64_t align_up(uint64_t a, uint64_t b) { return ceil_div(a, b) * b; }

// Host-side launch bookkeeping (profile.cpp): brackets a launch with HIP
// events when instrumentation is enabled.
struct LaunchScope {
    LaunchScope(const char *name, hipStream_t s);
    ~LaunchScope();
    void *rec;
};

// Host cache of per-device launch facts (CU count, occupancy, function
// attributes): one slot per device ordinal, filled by the first call on that
// device.  Racing first calls compute the same value, so relaxed atomics
// suffice and concurrent callers never see a torn or foreign-device value.
// `compute` runs with the device current and returns a non-zero value.
constexpr int kMaxDevices = 64;
struct DeviceCache {
    std::atomic<int> v[kMaxDevices];
};
template <class F>
int device_cached(DeviceCache &c, F compute)
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return compute();
    int x = c.v[dev].load(std::memory_order_relaxed);
    if (x == 0) {
        x = compute();
        c.v[dev].store(x, std::memory_order_relaxed);
    }
    return x;
}

// Compute units of the current device (256 on MI355X; 256 if the query fails).
inline int device_cus()
{
    static DeviceCache cache;
    return device_cached(cache, [] {
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus > 0)
            return cus;
        return 256;
    });
}

}  // namespace lcpp

#define LCPP_LAUNCH(NAME, STREAM, ...)                       \
    do {                                                      \
        ::lcpp::LaunchScope lcpp_scope_(NAME, STREAM);        \
        __VA_ARGS__;                                          \
    } while (0)

#define LCPP_CHECK_LAUNCH()                                   \
    do {                                                      \
        if (hipGetLastError() != hipSuccess) return LCPP_ERR_HIP; \
    } while (0)
