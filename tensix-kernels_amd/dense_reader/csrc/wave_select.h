// wave_select.h: selecting the largest 64-bit keys across a wavefront (gfx950, 64 lanes), and the best candidates of
// a row of top-k records over several workgroups; shared by the top-k merge and the LM-head pick. A wavefront's list is sorted over its lanes, the largest in lane 0; a batch of 64 keys (one a
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

// ---- the best candidates of one row of top-k records, over several workgroups ----------------------------------------
//
// Records [n_records][2 * rows * k] uint32 (keys, then ids; dr_topk's layout). Slot c of row r is record c / k, slot
// c % k. A caller's Comp maps (key, id, c) to a 64-bit key (0: not a candidate); select_row keeps each row's best 64.
// The row's slots are cut into slices of cs, one workgroup (SEL_T threads) each; each wavefront keeps its best,
// wavefront 0 merges the workgroup's, and with more than one slice the workgroups meet in the workspace: each writes
// its list (device-scope atomic stores: the L2s of the XCDs are not coherent with each other, and an agent-scope fence
// would write back or invalidate a whole L2), waits for its stores, counts itself on the row's counter, and the last
// one merges every slice's list and resets the counter. select_row returns true in the workgroup that holds the row's
// final list (in wavefront 0's lanes, the largest in lane 0) and the count of the row's candidates.

constexpr int SEL_T = 256;                   // threads a workgroup
constexpr int SEL_W = SEL_T / 64;            // wavefronts
constexpr int SEL_SLICES = 64;               // workgroups a row at most

struct SelArgs {
    const uint32_t* rec;
    int nrec, rows, k, keep, slices, cs;
    unsigned long long* wlist;  // [rows][slices][64] (slices > 1)
    uint32_t* counters;         // [rows] arrivals, then [rows] candidate counts (slices > 1)
};

struct SelShared {
    unsigned long long lists[SEL_W][64];
    unsigned long long pend[SEL_W][64];
    int cnt[SEL_W];
    int last;
};

template <class Comp>
__device__ __forceinline__ bool select_row(const SelArgs& A, int r, int sl, Comp comp, SelShared& sh,
                                           unsigned long long& list, int& count) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const size_t rlen = 2 * (size_t)A.rows * A.k;
    const long long total = (long long)A.nrec * A.k;
    const long long c0 = (long long)sl * A.cs, c1 = min(c0 + (long long)A.cs, total);

    // this wavefront's batches of the slice: 64 slots each, four batches' loads in flight at a time
    WaveBest best;
    int n = 0;
    const int nb = (int)((c1 - c0 + 63) / 64);
    for (int b0 = wave; b0 < nb; b0 += 4 * SEL_W) {
        unsigned long long v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const long long c = c0 + (long long)(b0 + u * SEL_W) * 64 + lane;
            const long long cc = c < c1 ? c : c0;  // (in bounds; masked below)
            const long long ri = cc / A.k;
            const int j = (int)(cc - ri * A.k);
            const uint32_t* kp = A.rec + (size_t)ri * rlen + (size_t)r * A.k + j;
            const uint32_t key = kp[0], id = kp[(size_t)A.rows * A.k];
            v[u] = c < c1 ? comp(key, id, (uint32_t)cc) : 0ull;
            n += v[u] != 0ull;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) best.add(v[u], sh.pend[wave], A.keep, lane);
    }
    best.flush(sh.pend[wave], A.keep, lane);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) n += __shfl_xor(n, o);
    sh.lists[wave][lane] = best.list;
    if (lane == 0) sh.cnt[wave] = n;
    __syncthreads();
    list = best.list;
    count = 0;
#pragma unroll
    for (int w = 0; w < SEL_W; ++w) count += sh.cnt[w];
    if (wave == 0) {
#pragma unroll
        for (int w = 1; w < SEL_W; ++w) list = wave_merge(list, sh.lists[w][lane], lane);
    }
    if (A.slices == 1) return true;

    // meet the row's other workgroups in the workspace; the last one merges every slice's list
    if (wave == 0) {
        __hip_atomic_store(A.wlist + ((size_t)r * A.slices + sl) * 64 + lane, list, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        if (lane == 0)
            __hip_atomic_fetch_add(A.counters + A.rows + r, (uint32_t)count, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0);  // this wavefront's stores and count have reached the point of coherence
    }
    __syncthreads();
    if (threadIdx.x == 0)
        sh.last = __hip_atomic_fetch_add(A.counters + r, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                  (uint32_t)(A.slices - 1);
    __syncthreads();
    if (!sh.last) return false;
    // every list of this wavefront's share loaded at once (slices <= SEL_SLICES), each merged in (sorted already)
    constexpr int Q = SEL_SLICES / SEL_W;
    unsigned long long lv[Q];
#pragma unroll
    for (int i = 0; i < Q; ++i) {
        const int q = min(wave + i * SEL_W, A.slices - 1);
        lv[i] = __hip_atomic_load(A.wlist + ((size_t)r * A.slices + q) * 64 + lane, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
    }
    unsigned long long mine = 0ull;
#pragma unroll
    for (int i = 0; i < Q; ++i)
        if (wave + i * SEL_W < A.slices) mine = wave_merge(mine, lv[i], lane);  // (uniform)
    sh.lists[wave][lane] = mine;
    if (threadIdx.x == 0)
        sh.cnt[0] = (int)__hip_atomic_load(A.counters + A.rows + r, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    count = sh.cnt[0];
    if (wave == 0) {
        list = mine;
#pragma unroll
        for (int w = 1; w < SEL_W; ++w) list = wave_merge(list, sh.lists[w][lane], lane);
        if (lane == 0) {
            __hip_atomic_store(A.counters + r, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(A.counters + A.rows + r, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    return true;
}

// the host's plan: slices of about 1024 slots (four batches of 64 a wavefront), at most SEL_SLICES a row
inline void select_plan(int n_records, int k, int* slices, int* cs) {
    const long long total = (long long)n_records * k;
    long long sl = (total + 1023) / 1024;
    sl = sl < 1 ? 1 : (sl > SEL_SLICES ? SEL_SLICES : sl);
    long long c = (total + sl - 1) / sl;
    c = (c + 63) / 64 * 64;
    *slices = (int)((total + c - 1) / c);
    *cs = (int)c;
}

// the workspace: the rows' arrival counters and candidate counts (a 256-byte aligned block), then the slice lists
inline int64_t select_counter_bytes(int rows) { return ((int64_t)rows * 8 + 255) / 256 * 256; }

inline int64_t select_workspace_bytes(int n_records, int rows, int k) {
    int slices, cs;
    select_plan(n_records, k, &slices, &cs);
    if (slices == 1) return 0;
    return select_counter_bytes(rows) + (int64_t)rows * slices * 64 * 8;
}

}  // namespace wsel

#endif
