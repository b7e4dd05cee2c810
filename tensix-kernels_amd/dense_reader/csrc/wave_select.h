// wave_select.h: selecting the largest 64-bit keys across a wavefront (gfx950, 64 lanes), shared by the top-k merge
// and the LM-head pick. A wavefront's list is sorted over its lanes, the largest in lane 0; a batch of 64 keys (one a
// lane) is sorted by a bitonic network over the lanes and merged in: the larger of list[i] and batch[63 - i] is a
// bitonic sequence holding the best 64 of both, which six more steps sort. Keys are distinct where a caller needs one
// answer whatever the order of the work (a key carries its candidate's index below its value).
#ifndef DR_WAVE_SELECT_H
#define DR_WAVE_SELECT_H

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wsel {

__device__ __forceinline__ unsigned long long xor_lane(unsigned long long v, int m) {
    const uint32_t lo = __shfl_xor((uint32_t)v, m), hi = __shfl_xor((uint32_t)(v >> 32), m);
    return ((unsigned long long)hi << 32) | lo;
}

__device__ __forceinline__ unsigned long long from_lane(unsigned long long v, int src) {
    const uint32_t lo = __shfl((uint32_t)v, src), hi = __shfl((uint32_t)(v >> 32), src);
    return ((unsigned long long)hi << 32) | lo;
}

// sort the wavefront's 64 values, largest in lane 0
__device__ __forceinline__ unsigned long long wave_sort(unsigned long long v, int lane) {
#pragma unroll
    for (int size = 2; size <= 64; size <<= 1) {
#pragma unroll
        for (int j = size >> 1; j > 0; j >>= 1) {
            const unsigned long long p = xor_lane(v, j);
            // blocks of `size` alternate descending / ascending (the last, 64, descending); the lower lane of a pair
            // in a descending block keeps the larger value
            const bool desc = (lane & size) == 0 || size == 64;
            const bool lower = (lane & j) == 0;
            v = (lower == desc) ? (p > v ? p : v) : (p < v ? p : v);
        }
    }
    return v;
}

// list and batch sorted (largest in lane 0): the best 64 of both, sorted
__device__ __forceinline__ unsigned long long wave_merge(unsigned long long list, unsigned long long batch,
                                                         int lane) {
    const unsigned long long r = from_lane(batch, 63 - lane);
    unsigned long long v = list > r ? list : r;
#pragma unroll
    for (int j = 32; j > 0; j >>= 1) {
        const unsigned long long p = xor_lane(v, j);
        v = (lane & j) == 0 ? (p > v ? p : v) : (p < v ? p : v);
    }
    return v;
}

__device__ __forceinline__ unsigned long long lane_value(unsigned long long v, int src) {
    const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)v, src);
    const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(v >> 32), src);
    return ((unsigned long long)hi << 32) | lo;
}

// A wavefront's running best: list (sorted over the lanes), thr its k_out-th value (only larger candidates can
// enter), and up to 64 entrants waiting in pend (LDS) to be sorted and merged in at once.
struct WaveBest {
    unsigned long long list = 0ull, thr = 0ull;
    int count = 0;

    __device__ __forceinline__ void flush(unsigned long long* pend, int kout, int lane) {
        if (count == 0) return;
        __builtin_amdgcn_wave_barrier();
        const unsigned long long v = lane < count ? pend[lane] : 0ull;
        list = wave_merge(list, wave_sort(v, lane), lane);
        thr = lane_value(list, kout - 1);
        count = 0;
        __builtin_amdgcn_wave_barrier();
    }

    // one candidate a lane (0: none)
    __device__ __forceinline__ void add(unsigned long long v, unsigned long long* pend, int kout, int lane) {
        unsigned long long m = __ballot(v > thr);
        if (m == 0ull) return;
        if (count + __popcll(m) > 64) {
            flush(pend, kout, lane);
            m = __ballot(v > thr);
            if (m == 0ull) return;
        }
        if (v > thr) pend[count + __popcll(m & ((1ull << lane) - 1ull))] = v;
        count += __popcll(m);
    }
};

}  // namespace wsel

#endif
