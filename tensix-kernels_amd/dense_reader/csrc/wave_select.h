// wave_select.h: selecting the largest 64-bit keys across a wavefront (gfx950, 64 lanes), and the best candidates of
// a row of top-k records over several workgroups; shared by the top-k merge and the LM-head pick. A wavefront's list
// is sorted decreasing over its lanes, the largest in lane 0; a batch of 64 keys (one a lane) is sorted increasing by
// a bitonic network over the lanes and merged in: the larger of list[i] and batch[i] is a bitonic sequence holding the
// best 64 of both, which six more steps sort. Every exchange between lanes is a DPP or permlane move, not an LDS
// permute. Keys are distinct where a caller needs one answer whatever the order of the work (a key carries its
// candidate's index below its value).
#ifndef DR_WAVE_SELECT_H
#define DR_WAVE_SELECT_H

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wsel {

// ---- exchanges between lane l and lane l ^ J, with no LDS round trip ---------------------------------------------------
//
// xpair<J>(v, a, b) leaves {a, b} = {v of this lane, v of lane l ^ J}, in either order: DPP moves for J <= 8
// (quad_perm for 1 and 2; row_shl:4 into banks 0 and 2 and row_shr:4 into banks 1 and 3 for 4; row_ror:8 for 8) and
// gfx950's v_permlane16_swap / v_permlane32_swap for 16 and 32, which swap rows (halves) between two registers in one
// VALU op. A compare-exchange or a sum needs the pair only, not which of the two is this lane's.

template <int J>
__device__ __forceinline__ uint32_t dpp_xor(uint32_t v) {
    static_assert(J == 1 || J == 2 || J == 4 || J == 8, "DPP moves cover the distances 1, 2, 4 and 8");
    if constexpr (J == 1) {
        return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xf, 0xf, false);  // quad_perm [1,0,3,2]
    } else if constexpr (J == 2) {
        return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xf, 0xf, false);  // quad_perm [2,3,0,1]
    } else if constexpr (J == 4) {
        const int t = __builtin_amdgcn_mov_dpp((int)v, 0x104, 0xf, 0x5, false);            // row_shl:4, lanes 0-3, 8-11
        return (uint32_t)__builtin_amdgcn_update_dpp(t, (int)v, 0x114, 0xf, 0xa, false);  // row_shr:4, lanes 4-7, 12-15
    } else {
        return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x128, 0xf, 0xf, false);  // row_ror:8
    }
}

template <int J>
__device__ __forceinline__ void xpair32(uint32_t v, uint32_t& a, uint32_t& b) {
    if constexpr (J == 16) {
        const auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        a = p[0];
        b = p[1];
    } else if constexpr (J == 32) {
        const auto p = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        a = p[0];
        b = p[1];
    } else {
        a = v;
        b = dpp_xor<J>(v);
    }
}

template <int J>
__device__ __forceinline__ void xpair(unsigned long long v, unsigned long long& a, unsigned long long& b) {
    uint32_t al, bl, ah, bh;
    xpair32<J>((uint32_t)v, al, bl);
    xpair32<J>((uint32_t)(v >> 32), ah, bh);
    a = ((unsigned long long)ah << 32) | al;
    b = ((unsigned long long)bh << 32) | bl;
}

// one compare-exchange at distance J: the lane keeps the larger of its value and lane l ^ J's where `larger`, else
// the smaller
template <int J>
__device__ __forceinline__ unsigned long long cmpx(unsigned long long v, bool larger) {
    unsigned long long a, b;
    xpair<J>(v, a, b);
    return ((b > a) == larger) ? b : a;
}

// v plus lane l ^ J's v: both lanes of a pair add the same two values, so they hold the same bits after, as after a
// shuffle butterfly's step at that distance
template <int J>
__device__ __forceinline__ float add_xor(float v) {
    uint32_t a, b;
    xpair32<J>(__float_as_uint(v), a, b);
    return __uint_as_float(a) + __uint_as_float(b);
}

// the sum of v over the wavefront, on every lane: a butterfly at distances 32, 16, ..., 1. Both lanes of a pair add
// the same two values, so every lane ends with the same bits, in the order a shuffle butterfly would give.
__device__ __forceinline__ float wave_sum_xor(float v) {
    uint32_t a, b;
    xpair32<32>(__float_as_uint(v), a, b);
    v = __uint_as_float(a) + __uint_as_float(b);
    xpair32<16>(__float_as_uint(v), a, b);
    v = __uint_as_float(a) + __uint_as_float(b);
    v += __uint_as_float(dpp_xor<8>(__float_as_uint(v)));
    v += __uint_as_float(dpp_xor<4>(__float_as_uint(v)));
    v += __uint_as_float(dpp_xor<2>(__float_as_uint(v)));
    v += __uint_as_float(dpp_xor<1>(__float_as_uint(v)));
    return v;
}

// the sum of v over the wavefront, on every lane
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
    uint32_t a, b;
    xpair32<32>(v, a, b);
    v = a + b;
    xpair32<16>(v, a, b);
    v = a + b;
    v += dpp_xor<8>(v);
    v += dpp_xor<4>(v);
    v += dpp_xor<2>(v);
    return v + dpp_xor<1>(v);
}

// the steps of one bitonic stage: blocks of SIZE lanes alternate increasing and decreasing (the last, 64, increasing);
// in an increasing block the lower lane of a pair keeps the smaller value
template <int SIZE, int J>
__device__ __forceinline__ unsigned long long sort_steps(unsigned long long v, int lane) {
    const bool up = (lane & SIZE) == 0, lower = (lane & J) == 0;
    v = cmpx<J>(v, lower != up);
    if constexpr (J > 1)
        return sort_steps<SIZE, J / 2>(v, lane);
    else
        return v;
}

template <int SIZE>
__device__ __forceinline__ unsigned long long sort_stages(unsigned long long v, int lane) {
    v = sort_steps<SIZE, SIZE / 2>(v, lane);
    if constexpr (SIZE < 64)
        return sort_stages<SIZE * 2>(v, lane);
    else
        return v;
}

// sort the wavefront's 64 values in increasing order over the lanes (the largest in lane 63)
__device__ __forceinline__ unsigned long long wave_sort_up(unsigned long long v, int lane) {
    return sort_stages<2>(v, lane);
}

template <int J>
__device__ __forceinline__ unsigned long long merge_steps(unsigned long long v, int lane) {
    v = cmpx<J>(v, (lane & J) == 0);
    if constexpr (J > 1)
        return merge_steps<J / 2>(v, lane);
    else
        return v;
}

// list sorted decreasing over the lanes, up sorted increasing: the best 64 of both, decreasing. The larger of list[i]
// and up[i] (list's i-th largest against up's (63 - i)-th largest) is a bitonic sequence holding the best 64, which
// six half-cleaner steps sort.
__device__ __forceinline__ unsigned long long wave_merge(unsigned long long list, unsigned long long up, int lane) {
    return merge_steps<32>(list > up ? list : up, lane);
}

// ---- lists of at most 32 (a caller keeping 32 or fewer): two lists a register -----------------------------------------
//
// A pair register holds one list decreasing in lanes 0-31 and another increasing in lanes 32-63: together a bitonic
// sequence of 64. merge32<UP> leaves the best 32 of the two decreasing in lanes 0-31 (UP false) or increasing in lanes
// 32-63 (UP true), in six steps: the half-cleaner at 32 moves the larger half there, five more sort it.
template <bool UP>
__device__ __forceinline__ unsigned long long merge32(unsigned long long v, int lane) {
    v = cmpx<32>(v, ((lane & 32) == 0) != UP);
    v = cmpx<16>(v, ((lane & 16) == 0) != UP);
    v = cmpx<8>(v, ((lane & 8) == 0) != UP);
    v = cmpx<4>(v, ((lane & 4) == 0) != UP);
    v = cmpx<2>(v, ((lane & 2) == 0) != UP);
    return cmpx<1>(v, ((lane & 1) == 0) != UP);
}

// the best 32 of the lists in P (two a register; `used` of the N registers hold any, the rest none; uniform),
// decreasing in lanes 0-31: a tree of merge32 whose merges on one level are independent of each other (one merge's
// result in lanes 0-31 and the next one's in lanes 32-63 make the next level's pair register)
template <int N>
__device__ __forceinline__ unsigned long long tree32(unsigned long long (&P)[N], int used, int lane) {
#pragma unroll
    for (int w = N; w > 1; w >>= 1) {
        if (used > 1) {
#pragma unroll
            for (int p = 0; p < w / 2; ++p) {
                unsigned long long lo = 0ull, hi = 0ull;
                if (2 * p < used) lo = merge32<false>(P[2 * p], lane);
                if (2 * p + 1 < used) hi = merge32<true>(P[2 * p + 1], lane);
                P[p] = lane < 32 ? lo : hi;
            }
            used = (used + 1) / 2;
        }
    }
    return merge32<false>(P[0], lane);
}

// a pair register from two lists stored decreasing (64 apart or wherever a and b point): a's first 32 in lanes 0-31,
// b's first 32 reversed in lanes 32-63
__device__ __forceinline__ unsigned long long pair_of(const unsigned long long* a, const unsigned long long* b,
                                                      int lane) {
    return lane < 32 ? a[lane] : b[63 - lane];
}

// the largest v over the wavefront, on every lane
__device__ __forceinline__ unsigned long long wave_max(unsigned long long v) {
    unsigned long long a, b;
    xpair<32>(v, a, b);
    v = a > b ? a : b;
    xpair<16>(v, a, b);
    v = a > b ? a : b;
    xpair<8>(v, a, b);
    v = a > b ? a : b;
    xpair<4>(v, a, b);
    v = a > b ? a : b;
    xpair<2>(v, a, b);
    v = a > b ? a : b;
    xpair<1>(v, a, b);
    return a > b ? a : b;
}

__device__ __forceinline__ unsigned long long lane_value(unsigned long long v, int src) {
    const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)v, src);
    const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(v >> 32), src);
    return ((unsigned long long)hi << 32) | lo;
}

// the largest t with at least k lanes holding m >= t (k <= 64; 0 when no larger t has k): the k-th largest m over the
// wavefront, found bit by bit from the top with one ballot a bit
__device__ __forceinline__ uint32_t wave_kth_largest(uint32_t m, int k) {
    uint32_t t = 0u;
#pragma unroll
    for (int b = 31; b >= 0; --b) {
        const uint32_t c = t | (1u << b);
        if ((int)__popcll(__ballot(m >= c)) >= k) t = c;
    }
    return t;
}

// A wavefront's running best: list (sorted decreasing over the lanes; NARROW, k_out <= 32: over lanes 0-31 only), thr
// its k_out-th value or the floor, whichever is larger (only larger candidates can enter), and up to 64 entrants
// waiting in pend (LDS) to be sorted and merged in at once.
template <bool NARROW>
struct WaveBest {
    unsigned long long list = 0ull, thr = 0ull, floor = 0ull;
    int count = 0;

    // v: this lane's candidates of the first load round (U a lane, 0: none). The k_out-th largest of the lanes'
    // largest high words, t, has k_out lanes holding a candidate at or above t << 32, so a candidate below it is
    // beaten by k_out others and cannot be among the best k_out: most candidates stay out of the sorts from the start.
    template <int U>
    __device__ __forceinline__ void raise_floor(const unsigned long long (&v)[U], int kout) {
        uint32_t m = 0u;
#pragma unroll
        for (int u = 0; u < U; ++u) m = max(m, (uint32_t)(v[u] >> 32));
        const uint32_t t = wave_kth_largest(m, kout);
        if (t != 0u) {
            floor = ((unsigned long long)t << 32) - 1ull;  // (entry: v > thr)
            thr = thr > floor ? thr : floor;
        }
    }

    __device__ __forceinline__ void flush(unsigned long long* pend, int kout, int lane) {
        if (count == 0) return;
        __builtin_amdgcn_wave_barrier();
        const unsigned long long v = lane < count ? pend[lane] : 0ull;
        const unsigned long long up = wave_sort_up(v, lane);
        if constexpr (NARROW)
            list = merge32<false>(lane < 32 ? list : up, lane);  // (up's best 32 are increasing in lanes 32-63)
        else
            list = wave_merge(list, up, lane);
        thr = lane_value(list, kout - 1);
        thr = thr > floor ? thr : floor;
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
// c % k. A caller's Comp maps (key, id, c) to a 64-bit key (0: not a candidate); select_row keeps each row's best 64
// (NARROW: 32).
// The row's slots are cut into slices of cs, one workgroup (SEL_T threads) each; each wavefront keeps its best,
// wavefront 0 merges the workgroup's, and with more than one slice the workgroups meet in the workspace: each writes
// its list (device-scope atomic stores: the L2s of the XCDs are not coherent with each other, and an agent-scope fence
// would write back or invalidate a whole L2), waits for its stores, counts itself on the row's counter, and the last
// one merges every slice's list and resets the counter. select_row returns true in the workgroup that holds the row's
// final list (in wavefront 0's lanes, the largest in lane 0) and the count of the row's candidates.

#ifndef DR_SEL_T
#define DR_SEL_T 256
#endif
constexpr int SEL_T = DR_SEL_T;              // threads a workgroup
constexpr int SEL_W = SEL_T / 64;            // wavefronts
constexpr int SEL_SLICES = 64;               // workgroups a row at most

struct SelArgs {
    const uint32_t* rec;
    int nrec, rows, k, keep, slices, cs;
    unsigned long long* wlist;  // [rows][slices][64] (slices > 1)
    uint32_t* counters;         // [rows], SEL_CSTRIDE apart: workgroups of the row arrived (slices > 1)
    uint32_t* counts;           // [rows][slices]: each slice's candidate count (slices > 1)
};

// a row's arrival counter has a 256-byte line of its own (the rows' atomics do not queue behind each other), in a
// region of fixed size at the workspace's start: the lists and counts of a launch of any shape lie after it, so a
// workspace shared by launches of any shape never finds an earlier launch's lists where a counter should be zero
constexpr int SEL_CSTRIDE = 64;
constexpr int SEL_MAXROWS = 32;  // the rows of a record (dr_topk's limit)
constexpr int64_t SEL_COUNTER_BYTES = (int64_t)SEL_MAXROWS * SEL_CSTRIDE * 4;

struct SelShared {
    unsigned long long lists[SEL_W][64];
    unsigned long long pend[SEL_W][64];
    int cnt[SEL_W];
    int last;
};

// the best of the workgroup's wavefront lists in sh.lists (after a barrier), in wavefront 0
template <bool NARROW>
__device__ __forceinline__ unsigned long long merge_waves(const SelShared& sh, int lane) {
    if constexpr (NARROW) {
        unsigned long long P[SEL_W / 2];
#pragma unroll
        for (int i = 0; i < SEL_W / 2; ++i) P[i] = pair_of(sh.lists[2 * i], sh.lists[2 * i + 1], lane);
        return tree32(P, SEL_W / 2, lane);
    } else {
        unsigned long long list = sh.lists[0][lane];
#pragma unroll
        for (int w = 1; w < SEL_W; ++w) list = wave_merge(list, sh.lists[w][63 - lane], lane);  // (read increasing)
        return list;
    }
}

// NARROW: the caller keeps at most 32 (A.keep <= 32), so every list needs its best 32 only
template <bool NARROW, class Comp>
__device__ __forceinline__ bool select_row(const SelArgs& A, int r, int sl, Comp comp, SelShared& sh,
                                           unsigned long long& list, int& count) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;  // (wave: uniform)
    const size_t rlen = 2 * (size_t)A.rows * A.k;
    const long long total = (long long)A.nrec * A.k;
    const long long c0 = (long long)sl * A.cs, c1 = min(c0 + (long long)A.cs, total);

    // this wavefront's batches of the slice: 64 slots each, four batches' loads in flight at a time (every address,
    // then every load, then the keys: no branch between the loads). Slot c is record c / k, place c % k, in 32-bit
    // arithmetic where the slots fit.
    WaveBest<NARROW> best;
    int n = 0;
    const int nb = (int)((c1 - c0 + 63) / 64);
    auto batches = [&](auto index) {
        using I = decltype(index);
        for (int b0 = wave; b0 < nb; b0 += 4 * SEL_W) {
            long long c[4];
            const uint32_t* kp[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                c[u] = c0 + (long long)(b0 + u * SEL_W) * 64 + lane;
                const I cc = (I)(c[u] < c1 ? c[u] : c0);  // (in bounds; masked below)
                const I ri = cc / (I)A.k, j = cc - ri * (I)A.k;
                kp[u] = A.rec + (size_t)ri * rlen + (size_t)r * A.k + (size_t)j;
            }
            uint32_t key[4], id[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                key[u] = kp[u][0];
                id[u] = kp[u][(size_t)A.rows * A.k];
            }
            unsigned long long v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                v[u] = c[u] < c1 ? comp(key[u], id[u], (uint32_t)c[u]) : 0ull;
                n += __popcll(__ballot(v[u] != 0ull));  // (the wavefront's count, uniform)
            }
            if (b0 == wave) best.raise_floor(v, A.keep);  // (the first round)
#pragma unroll
            for (int u = 0; u < 4; ++u) best.add(v[u], sh.pend[wave], A.keep, lane);
        }
    };
    if (c1 <= 0xFFFFFFFFll)
        batches(uint32_t{});
    else
        batches((unsigned long long){});
    best.flush(sh.pend[wave], A.keep, lane);
    sh.lists[wave][lane] = best.list;
    if (lane == 0) sh.cnt[wave] = n;
    __syncthreads();
    list = best.list;
    count = 0;
#pragma unroll
    for (int w = 0; w < SEL_W; ++w) count += sh.cnt[w];
    if (wave == 0) list = merge_waves<NARROW>(sh, lane);
    if (A.slices == 1) return true;

    // meet the row's other workgroups in the workspace; the last one merges every slice's list
    if (wave == 0) {
        if (!NARROW || lane < 32)
            __hip_atomic_store(A.wlist + ((size_t)r * A.slices + sl) * 64 + lane, list, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        if (lane == 0)
            __hip_atomic_store(A.counts + (size_t)r * A.slices + sl, (uint32_t)count, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0);  // this wavefront's stores have reached the point of coherence
    }
    __syncthreads();
    if (threadIdx.x == 0)
        sh.last = __hip_atomic_fetch_add(A.counters + (size_t)r * SEL_CSTRIDE, 1u, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)(A.slices - 1);
    __syncthreads();
    if (!sh.last) return false;
    // every list of this wavefront's share (wave, wave + SEL_W, ...; slices <= SEL_SLICES) and the slices' counts (one
    // a lane of wavefront 0), loaded at once
    constexpr int Q = SEL_SLICES / SEL_W;
    const unsigned long long* wl = A.wlist + (size_t)r * A.slices * 64;
    unsigned long long mine = 0ull;
    uint32_t rc = 0u;
    if (wave == 0 && lane < A.slices)
        rc = __hip_atomic_load(A.counts + (size_t)r * A.slices + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if constexpr (NARROW) {
        // two lists a pair register: list 2i's best 32 in lanes 0-31, list 2i + 1's reversed in lanes 32-63
        unsigned long long P[Q / 2];
#pragma unroll
        for (int i = 0; i < Q / 2; ++i) {
            const int q = wave + (2 * i + (lane >> 5)) * SEL_W;
            P[i] = q < A.slices ? __hip_atomic_load(wl + (size_t)q * 64 + (lane < 32 ? lane : 63 - lane),
                                                    __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                : 0ull;
        }
        const int nq = (A.slices - wave + SEL_W - 1) / SEL_W;
        mine = tree32(P, (nq + 1) / 2, lane);
    } else {
        unsigned long long lv[Q];
#pragma unroll
        for (int i = 0; i < Q; ++i) {
            const int q = min(wave + i * SEL_W, A.slices - 1);
            lv[i] = __hip_atomic_load(wl + (size_t)q * 64 + (63 - lane), __ATOMIC_RELAXED,  // (read increasing)
                                      __HIP_MEMORY_SCOPE_AGENT);
        }
#pragma unroll
        for (int i = 0; i < Q; ++i)
            if (wave + i * SEL_W < A.slices) mine = wave_merge(mine, lv[i], lane);  // (uniform)
    }
    sh.lists[wave][lane] = mine;
    if (wave == 0) {
        rc = wave_sum_u32(rc);
        if (lane == 0) sh.cnt[0] = (int)rc;
    }
    __syncthreads();
    count = sh.cnt[0];
    if (wave == 0) {
        list = merge_waves<NARROW>(sh, lane);
        if (lane == 0) __hip_atomic_store(A.counters + (size_t)r * SEL_CSTRIDE, 0u, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
    }
    return true;
}

// slots a workgroup takes (about; four batches of 64 a wavefront at 1024)
#ifndef DR_SEL_SLOTS
#define DR_SEL_SLOTS 1024
#endif

// the host's plan: slices of about DR_SEL_SLOTS slots, at most SEL_SLICES a row
inline void select_plan(int n_records, int k, int* slices, int* cs) {
    const long long total = (long long)n_records * k;
    long long sl = (total + DR_SEL_SLOTS - 1) / DR_SEL_SLOTS;
    sl = sl < 1 ? 1 : (sl > SEL_SLICES ? SEL_SLICES : sl);
    long long c = (total + sl - 1) / sl;
    c = (c + 63) / 64 * 64;
    *slices = (int)((total + c - 1) / c);
    *cs = (int)c;
}

// the workspace: SEL_MAXROWS arrival counters (256 bytes each), the slice lists, the slices' counts (rows <=
// SEL_MAXROWS)
inline int64_t select_workspace_bytes(int n_records, int rows, int k) {
    int slices, cs;
    select_plan(n_records, k, &slices, &cs);
    if (slices == 1) return 0;
    return SEL_COUNTER_BYTES + (int64_t)rows * slices * 64 * 8 + (int64_t)rows * slices * 4;
}

// A's workspace pointers in a caller's workspace of at least select_workspace_bytes (A.slices planned); false when it
// is missing or short
inline bool select_bind(SelArgs& A, void* workspace, int64_t workspace_bytes) {
    const int64_t need = select_workspace_bytes(A.nrec, A.rows, A.k);
    if (need == 0) return true;
    if (workspace == nullptr || workspace_bytes < need) return false;
    uint8_t* w = reinterpret_cast<uint8_t*>(workspace);
    A.counters = reinterpret_cast<uint32_t*>(w);
    A.wlist = reinterpret_cast<unsigned long long*>(w + SEL_COUNTER_BYTES);
    A.counts = reinterpret_cast<uint32_t*>(w + SEL_COUNTER_BYTES + (int64_t)A.rows * A.slices * 64 * 8);
    return true;
}

}  // namespace wsel

#endif
