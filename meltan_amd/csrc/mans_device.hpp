// Device-side building blocks shared by the scan kernels (gfx950, wave64).
//
// All HIP sources are compiled with -ffp-contract=off: a multiply and an add
// written separately stay two correctly rounded operations, which is what
// the reference's scalar dots.c loop (dots.c:40-47) executes on x86-64.
// Fast paths that may fuse say so with an explicit fmaf().
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mans {

constexpr uint32_t kEmptyId = 0xFFFFFFFFu;
constexpr uint64_t kEmptySlot = ~0ull;
constexpr int kMetricCosine = 0;
constexpr int kMetricL2 = 1;
constexpr int kMetricIP = 2;
constexpr float kFltMax = 3.402823466e+38f;

typedef float f4v __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));  // 32x32 MFMA accumulator
typedef int i4v __attribute__((ext_vector_type(4)));
typedef int i16v __attribute__((ext_vector_type(16)));    // 32x32 i8 MFMA accumulator

// 128-bit streaming load (the corpus is read once per query batch).
__device__ __forceinline__ f4v load_stream(const float* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const f4v*>(p));
}

// Intra-wave barrier for LDS traffic between lanes of one wave.
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Order-preserving map float -> uint32 (-0 is folded onto +0 first, so the
// packed order agrees with float comparison).
__device__ __forceinline__ uint32_t ordered_bits(float x) {
    x = x + 0.0f;
    uint32_t u = __float_as_uint(x);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float from_ordered_bits(uint32_t o) {
    uint32_t u = (o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o;
    return __uint_as_float(u);
}

// (key, id) packed so that unsigned comparison is (key asc, id asc).
__device__ __forceinline__ uint64_t pack_slot(float key, uint32_t id) {
    return ((uint64_t)ordered_bits(key) << 32) | (uint64_t)id;
}
__device__ __forceinline__ float slot_key(uint64_t s) { return from_ordered_bits((uint32_t)(s >> 32)); }
__device__ __forceinline__ uint32_t slot_id(uint64_t s) { return (uint32_t)s; }

// Host distance formulas (ParallelFlatScan.swift:237-257, BoundedExactScan.swift:346-363,
// IVFFlatSearch.swift:294-311), evaluated with the same correctly rounded
// operations in the same order.
__device__ __forceinline__ float host_distance(float dot, float qn, float vn, int metric) {
    if (metric == kMetricIP) return -dot;
    if (metric == kMetricL2) {
        float d = qn - 2.0f * dot + vn;
        return d > 0.0f ? d : 0.0f;
    }
    float denom = sqrtf(qn * vn);
    return denom < 1e-10f ? 1.0f : 1.0f - dot / denom;
}

// Sequential dot in the order of dots.c:40-47.
// (Unrolled so the loads are issued ahead; the additions stay in order.)
__device__ __forceinline__ float exact_dot(const float* __restrict__ a, const float* __restrict__ b,
                                           int dim) {
    float acc = 0.0f;
#pragma unroll 8
    for (int d = 0; d < dim; ++d) acc = acc + a[d] * b[d];
    return acc;
}

// Sum over the 16 lanes of a DPP row; every lane of the row gets the total.
__device__ __forceinline__ float row16_sum(float v) {
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false));  // row_ror:8
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xF, 0xF, false));  // row_ror:4
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));   // quad_perm 2,3,0,1
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));   // quad_perm 1,0,3,2
    return v;
}

__device__ __forceinline__ uint64_t lanemask_lt() {
    uint32_t lane = __lane_id();
    return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

// Ascending bitonic sort of `size` (power of two) packed slots in LDS by one
// wave, through LDS (any size).
__device__ __forceinline__ void wave_bitonic_sort_lds(uint64_t* buf, int size) {
    const int lane = __lane_id();
    for (int k2 = 2; k2 <= size; k2 <<= 1) {
        for (int j = k2 >> 1; j > 0; j >>= 1) {
            for (int i = lane; i < size; i += 64) {
                int ixj = i ^ j;
                if (ixj > i) {
                    uint64_t a = buf[i], b = buf[ixj];
                    bool up = (i & k2) == 0;
                    if ((a > b) == up) {
                        buf[i] = b;
                        buf[ixj] = a;
                    }
                }
            }
            wave_sync();
        }
    }
}

// x from lane (lane ^ j), j a power of two below 64: DPP for j = 1, 2, 8
// (quad permutes, and a rotate by 8 within a 16-lane row), ds_swizzle
// (xor mode, within 32 lanes) for 4 and 16, a permute for 32.
__device__ __forceinline__ uint32_t lane_xor32(uint32_t x, int j) {
    switch (j) {
    case 1: return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0xB1, 0xF, 0xF, false);
    case 2: return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x4E, 0xF, 0xF, false);
    case 4: return (uint32_t)__builtin_amdgcn_ds_swizzle((int)x, 0x1F | (4 << 10));
    case 8: return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x128, 0xF, 0xF, false);
    case 16: return (uint32_t)__builtin_amdgcn_ds_swizzle((int)x, 0x1F | (16 << 10));
    default: return (uint32_t)__shfl_xor((int)x, j);
    }
}

__device__ __forceinline__ uint64_t lane_xor64(uint64_t x, int j) {
    uint32_t lo = lane_xor32((uint32_t)x, j);
    uint32_t hi = lane_xor32((uint32_t)(x >> 32), j);
    return ((uint64_t)hi << 32) | lo;
}

// Ascending bitonic sort of 64 * E values held in registers, element
// i = lane + 64 e in v[e].  Exchanges across lanes use lane_xor64; those
// within a lane are plain compares.
template <int E>
__device__ __forceinline__ void wave_sort_regs(uint64_t (&v)[E]) {
    const int lane = __lane_id();
    constexpr int N = 64 * E;
#pragma unroll
    for (int k2 = 2; k2 <= N; k2 <<= 1) {
#pragma unroll
        for (int j = k2 >> 1; j > 0; j >>= 1) {
            if (j >= 64) {
                const int je = j / 64;
#pragma unroll
                for (int e = 0; e < E; ++e) {
                    const int pe = e ^ je;
                    if (pe > e) {
                        const bool up = ((lane + 64 * e) & k2) == 0;
                        uint64_t a = v[e], b = v[pe];
                        bool sw = (a > b) == up;
                        v[e] = sw ? b : a;
                        v[pe] = sw ? a : b;
                    }
                }
            } else {
#pragma unroll
                for (int e = 0; e < E; ++e) {
                    uint64_t b = lane_xor64(v[e], j);
                    const bool up = ((lane + 64 * e) & k2) == 0;
                    const bool lower = (lane & j) == 0;
                    uint64_t mn = v[e] < b ? v[e] : b;
                    uint64_t mx = v[e] < b ? b : v[e];
                    v[e] = (lower == up) ? mn : mx;
                }
            }
        }
    }
}

__device__ __forceinline__ uint64_t shfl64(uint64_t x, int src) {
    uint32_t lo = (uint32_t)__shfl((int)(uint32_t)x, src);
    uint32_t hi = (uint32_t)__shfl((int)(uint32_t)(x >> 32), src);
    return ((uint64_t)hi << 32) | lo;
}

// Bitonic merge (half-cleaners J, J/2, ..., 1) of one slot per lane:
// every aligned run of 2J lanes holding a bitonic sequence ends up ascending.
template <int J>
__device__ __forceinline__ uint64_t wave_bitonic_merge(uint64_t v) {
    const int lane = __lane_id();
#pragma unroll
    for (int j = J; j > 0; j >>= 1) {
        uint64_t b = lane_xor64(v, j);
        const bool lower = (lane & j) == 0;
        uint64_t mn = v < b ? v : b;
        uint64_t mx = v < b ? b : v;
        v = lower ? mn : mx;
    }
    return v;
}

// The kc (32 or 64) smallest slots of four ascending lists of kc slots
// (lists[w * stride + i], padded with kEmptySlot), ascending in lanes
// [0, kc) of the calling wave.  For sorted A and B, min(A[i], B[kc-1-i])
// is a bitonic sequence holding the kc smallest of both lists.
__device__ __forceinline__ uint64_t wave_top_of_four(const uint64_t* lists, int stride, int kc) {
    const int lane = __lane_id();
    if (kc == 64) {
        uint64_t a = lists[lane], b = lists[stride + 63 - lane];
        uint64_t c = lists[2 * stride + lane], d = lists[3 * stride + 63 - lane];
        uint64_t x = wave_bitonic_merge<32>(a < b ? a : b);
        uint64_t y = wave_bitonic_merge<32>(c < d ? c : d);
        uint64_t yr = shfl64(y, 63 - lane);
        return wave_bitonic_merge<32>(x < yr ? x : yr);
    }
    // kc == 32: lists 0 and 1 merge in lanes 0-31, lists 2 and 3 in 32-63.
    const int h = lane & 31;
    const int off = lane >= 32 ? 2 * stride : 0;
    uint64_t a = lists[off + h], b = lists[off + stride + 31 - h];
    uint64_t x = wave_bitonic_merge<16>(a < b ? a : b);
    uint64_t xr = shfl64(x, lane ^ 63);  // lane i < 32 gets lane 63 - i
    return wave_bitonic_merge<16>(x < xr ? x : xr);
}

template <int E>
__device__ __forceinline__ void wave_sort_lds_via_regs(uint64_t* buf) {
    const int lane = __lane_id();
    uint64_t v[E];
#pragma unroll
    for (int e = 0; e < E; ++e) v[e] = buf[lane + 64 * e];
    wave_sort_regs<E>(v);
#pragma unroll
    for (int e = 0; e < E; ++e) buf[lane + 64 * e] = v[e];
}

// Ascending bitonic sort of `size` (power of two) packed slots in LDS by one wave.
// Sizes up to 256 (up to MAXREG) are sorted in registers.
template <int MAXREG = 512>
__device__ __forceinline__ void wave_bitonic_sort(uint64_t* buf, int size) {
    if (size >= 64 && size <= MAXREG && (size & (size - 1)) == 0) {
        if (size == 64) wave_sort_lds_via_regs<1>(buf);
        else if (MAXREG >= 128 && size == 128) wave_sort_lds_via_regs<MAXREG >= 128 ? 2 : 1>(buf);
        else if (MAXREG >= 256 && size == 256) wave_sort_lds_via_regs<MAXREG >= 256 ? 4 : 1>(buf);
        else if (MAXREG >= 512) wave_sort_lds_via_regs<MAXREG >= 512 ? 8 : 1>(buf);
        wave_sync();
        return;
    }
    wave_bitonic_sort_lds(buf, size);
}

// Ascending bitonic sort of `size` (power of two) slots in LDS by the whole block.
__device__ __forceinline__ void block_bitonic_sort(uint64_t* buf, int size) {
    const int tid = threadIdx.x, nt = blockDim.x;
    for (int k2 = 2; k2 <= size; k2 <<= 1) {
        for (int j = k2 >> 1; j > 0; j >>= 1) {
            for (int i = tid; i < size; i += nt) {
                int ixj = i ^ j;
                if (ixj > i) {
                    uint64_t a = buf[i], b = buf[ixj];
                    bool up = (i & k2) == 0;
                    if ((a > b) == up) {
                        buf[i] = b;
                        buf[ixj] = a;
                    }
                }
            }
            __syncthreads();
        }
    }
}

// Wave-private top-`kc` selector over a stream of (key, id) offers.
// Offers with key <= threshold are appended to an LDS buffer of `cap` slots
// (cap a power of two, cap >= kc + 64); when the buffer cannot take another
// full wave of offers it is sorted and cut back to kc, and the threshold
// becomes the kc-th key.  Every slot dropped has key >= the final kc-th key
// of the stream, which is what the lower-bound proofs downstream rely on.
// CAP > 0: the capacity is fixed at CAP (only the sorts of CAP and 64 slots
// are compiled in).
template <int CAP = 0>
struct WaveTopKT {
    uint64_t* buf;
    int cap;
    int kc;
    int count;
    float thresh;

    __device__ __forceinline__ void sort_first(int size) {
        if constexpr (CAP > 0) {
            if (size == 64) wave_sort_lds_via_regs<1>(buf);
            else wave_bitonic_sort<CAP>(buf, CAP);
            wave_sync();
        } else {
            wave_bitonic_sort(buf, size);
        }
    }

    __device__ __forceinline__ void init(uint64_t* b, int capacity, int keep) {
        buf = b;
        cap = CAP > 0 ? CAP : capacity;
        kc = keep;
        count = 0;
        thresh = __int_as_float(0x7F800000);  // +inf
    }

    __device__ __forceinline__ void compact() {
        const int lane = __lane_id();
        for (int i = count + lane; i < cap; i += 64) buf[i] = kEmptySlot;
        wave_sync();
        sort_first(cap);
        if (count >= kc) {
            count = kc;
            thresh = slot_key(buf[kc - 1]);
        }
    }

    __device__ __forceinline__ void offer(bool valid, float key, uint32_t id) {
        bool pass = valid && key <= thresh;
        uint64_t mask = __ballot(pass);
        if (mask == 0) return;
        if (pass) {
            int pos = count + __popcll(mask & lanemask_lt());
            buf[pos] = pack_slot(key, id);
        }
        count += __popcll(mask);
        if (count > cap - 64) {
            wave_sync();
            compact();
        }
    }

    // Offers `n` packed slots from LDS (another wave's finished list).
    __device__ __forceinline__ void offer_slots(const uint64_t* src, int n) {
        const int lane = __lane_id();
        for (int base = 0; base < n; base += 64) {
            int i = base + lane;
            uint64_t s = i < n ? src[i] : kEmptySlot;
            bool v = s != kEmptySlot;
            offer(v, v ? slot_key(s) : 0.0f, slot_id(s));
        }
    }

    // Sorts the buffer; slots [0, min(count, kc)) hold the result, the rest
    // of [0, cap) is padded with kEmptySlot.  (At most 64 slots in use: only
    // the first 64 are sorted.)
    __device__ __forceinline__ void finish() {
        wave_sync();
        const int lane = __lane_id();
        for (int i = count + lane; i < cap; i += 64) buf[i] = kEmptySlot;
        wave_sync();
        sort_first(count <= 64 ? 64 : cap);
        if (count > kc) count = kc;
        if (count == kc) thresh = slot_key(buf[kc - 1]);
        for (int i = count + lane; i < cap; i += 64) buf[i] = kEmptySlot;
        wave_sync();
    }
};

using WaveTopK = WaveTopKT<0>;

}  // namespace mans
