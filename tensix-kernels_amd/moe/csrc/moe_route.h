// moe_route.h: the MoE router's top k and routing weights for one row of logits, one wavefront (gfx950). Used by the
// router kernel (moe_route.hip, dr_moe_route) and by the gate/up expert gather when it routes its own token
// (dense_reader.hip, dr_moe_route_gate_up), so both give the same ids and weights bit for bit.
//
// Up to 1024 experts, up to 16 a lane in registers. The keys are made once: sigmoid(logit) + bias in double precision,
// or the logits themselves as floats. DeepSeek-V3's group-limited routing
// optionally keeps only the best groups (scored through LDS). Then k rounds each take the best untaken key across the
// wavefront (a butterfly over the lanes' own bests, the lower id first among equal keys), with no barrier. The weights
// come last, one lane a pick: the softmax over the picked logits (float), or the picks' sigmoids (over their sum when
// normalized; double), times the scale, rounded to bf16 once.
// This replaces moe/kernels/moe_route.cpp's fixed-point arithmetic on one RISC-V core (moe/moe8.py:1139-1253).

#ifndef DR_MOE_ROUTE_H
#define DR_MOE_ROUTE_H

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>

#include "moe.h"

namespace moe_route {

constexpr int MAXE = 1024;
constexpr int MAXK = 16;

struct RouteArgs {
    const float* logits;
    int rows, ld_logits, experts, k, kind;
    const float* bias;
    void* ids;
    int ids32, ld_ids;
    uint16_t* w;
    int ld_w;
    uint16_t* shared;
    int ld_shared;
    double scale;
    int norm, n_group, topk_group;
    long long slot;
};

// the LDS a row's routing uses (group scores)
struct RouteLds {
    double key[MAXE];
    double gscore[32];
};

__device__ __forceinline__ double sigmoid_d(double x) { return 1.0 / (1.0 + exp(-x)); }

// float -> bf16 bits, round to nearest even (a NaN: the quiet NaN)
__device__ __forceinline__ uint16_t bf16_bits(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// (ka, ia) comes before (kb, ib): the larger key, the lower id among equal keys (below, for float and double keys)

__device__ __forceinline__ void put_id(const RouteArgs& A, int r, int j, long long id) {
    const size_t i = (size_t)r * A.ld_ids + j;
    if (A.ids32)
        reinterpret_cast<uint32_t*>(A.ids)[i] = (uint32_t)id;
    else
        reinterpret_cast<uint16_t*>(A.ids)[i] = (uint16_t)id;
}

// a candidate (key, id); id == none: no expert. Keys are doubles where they are sigmoid(logit) + bias, else the
// logits themselves, which floats order exactly (and in half the lane moves)
template <typename K>
struct Cand {
    K k;
    int i;
};

template <typename K>
__device__ __forceinline__ bool before(K ka, int ia, K kb, int ib) {
    return ka > kb || (ka == kb && ia < ib);
}

template <typename K>
__device__ __forceinline__ Cand<K> pick_of(Cand<K> a, Cand<K> b, int none) {
    return (b.i != none && (a.i == none || before(b.k, b.i, a.k, a.i))) ? b : a;
}

// the candidate of the lane DPP control CTRL names (rows outside ROWS, or no such lane: no expert)
template <int CTRL, int ROWS>
__device__ __forceinline__ Cand<double> dpp_cand(Cand<double> c, int none) {
    const long long bits = __double_as_longlong(c.k);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)bits, CTRL, ROWS, 0xf, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(bits >> 32), CTRL, ROWS, 0xf, false);
    const int id = __builtin_amdgcn_update_dpp(none, c.i, CTRL, ROWS, 0xf, false);
    return Cand<double>{__longlong_as_double(((long long)hi << 32) | (unsigned)lo), id};
}
template <int CTRL, int ROWS>
__device__ __forceinline__ Cand<float> dpp_cand(Cand<float> c, int none) {
    const int kb = __builtin_amdgcn_update_dpp(0, __float_as_int(c.k), CTRL, ROWS, 0xf, false);
    const int id = __builtin_amdgcn_update_dpp(none, c.i, CTRL, ROWS, 0xf, false);
    return Cand<float>{__int_as_float(kb), id};
}

__device__ __forceinline__ double lane_key(double v, int lane) {
    const long long bits = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_readlane((int)bits, lane);
    const int hi = __builtin_amdgcn_readlane((int)(bits >> 32), lane);
    return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}
__device__ __forceinline__ float lane_key(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// the wavefront's best candidate, on every lane: row_shr 1, 2, 4, 8 carry each row's best to its lane 15,
// row_bcast 15 and 31 carry those to lane 63, which every lane then reads (VALU moves, no LDS round trips)
template <typename K>
__device__ __forceinline__ Cand<K> wave_best(Cand<K> c, int none) {
    c = pick_of(c, dpp_cand<0x111, 0xf>(c, none), none);  // row_shr:1
    c = pick_of(c, dpp_cand<0x112, 0xf>(c, none), none);  // row_shr:2
    c = pick_of(c, dpp_cand<0x114, 0xf>(c, none), none);  // row_shr:4
    c = pick_of(c, dpp_cand<0x118, 0xf>(c, none), none);  // row_shr:8
    c = pick_of(c, dpp_cand<0x142, 0xa>(c, none), none);  // row_bcast:15 into rows 1 and 3
    c = pick_of(c, dpp_cand<0x143, 0xc>(c, none), none);  // row_bcast:31 into rows 2 and 3
    return Cand<K>{lane_key(c.k, 63), __builtin_amdgcn_readlane(c.i, 63)};
}

// v of the lane DPP control CTRL names (0 where there is none)
template <int CTRL, int ROWS>
__device__ __forceinline__ double dpp_double(double v) {
    const long long bits = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)bits, CTRL, ROWS, 0xf, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(bits >> 32), CTRL, ROWS, 0xf, false);
    return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}

__device__ __forceinline__ double lane_double(double v, int lane) {
    const long long bits = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_readlane((int)bits, lane);
    const int hi = __builtin_amdgcn_readlane((int)(bits >> 32), lane);
    return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}

template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_float(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROWS, 0xf, false));
}
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_float<0x111, 0xf>(v);
    v += dpp_float<0x112, 0xf>(v);
    v += dpp_float<0x114, 0xf>(v);
    v += dpp_float<0x118, 0xf>(v);
    v += dpp_float<0x142, 0xa>(v);
    v += dpp_float<0x143, 0xc>(v);
    return lane_key(v, 63);
}

// the sum of v over the wavefront, on every lane, in a fixed order (the steps of wave_best)
__device__ __forceinline__ double wave_sum(double v) {
    v += dpp_double<0x111, 0xf>(v);
    v += dpp_double<0x112, 0xf>(v);
    v += dpp_double<0x114, 0xf>(v);
    v += dpp_double<0x118, 0xf>(v);
    v += dpp_double<0x142, 0xa>(v);
    v += dpp_double<0x143, 0xc>(v);
    return lane_double(v, 63);
}

// the wavefront's LDS writes done and seen by all its lanes (the routing runs in one wavefront, which may be one of
// several in its workgroup: no workgroup barrier)
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

// Row r's routing, by one wavefront (lane l), PER experts a lane (e = l + 64 i, PER >= ceil(E / 64)): lane j < k gets
// pick j's expert id (mine) and its weight's bf16 bits (wbits), slots in decreasing order of the pick's key. Each
// round's winner brings its logit along from its lane, so no logit is read twice. K: the key type, double for
// sigmoid(logit) + bias, float for the logits themselves (the same order: float to double is exact).
template <int PER, typename K>
__device__ __forceinline__ void route_row_k(const RouteArgs& A, int r, int l, RouteLds& L, int& mine, uint16_t& wbits) {
    const float* lg = A.logits + (size_t)r * A.ld_logits;
    const int E = A.experts;
    const bool sig = A.kind == 1 && A.bias != nullptr;
    K key[PER];
    float xs[PER];
    uint32_t taken = 0u;  // bit i: expert l + 64 i is picked (or absent)
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int e = l + 64 * i;
        K kv = -INFINITY;
        xs[i] = 0.f;
        if (e < E) {
            xs[i] = lg[e];
            kv = sig ? (K)(sigmoid_d((double)xs[i]) + (double)A.bias[e]) : (K)xs[i];
            kv = kv != kv ? (K)-INFINITY : kv;  // (a NaN key is never preferred)
        } else {
            taken |= 1u << i;
        }
        key[i] = kv;
    }
    if (A.n_group > 0) {
        // a group's score: the sum of its two largest keys; the topk_group best groups stay (through LDS: a group's
        // experts lie across the lanes)
#pragma unroll
        for (int i = 0; i < PER; ++i)
            if (l + 64 * i < E) L.key[l + 64 * i] = (double)key[i];
        wave_lds_sync();
        const int ng = A.n_group, gs = E / ng;
        if (l < ng) {
            double b1 = -INFINITY, b2 = -INFINITY;
            for (int j = 0; j < gs; ++j) {
                const double v = L.key[l * gs + j];
                if (v > b1) {
                    b2 = b1;
                    b1 = v;
                } else if (v > b2) {
                    b2 = v;
                }
            }
            L.gscore[l] = b1 + b2;
        }
        wave_lds_sync();
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int e = l + 64 * i;
            if (e >= E) continue;
            const int gi = e / gs;
            int rank = 0;
            for (int j = 0; j < ng; ++j) rank += before(L.gscore[j], j, L.gscore[gi], gi);
            if (rank >= A.topk_group) key[i] = -INFINITY;
        }
    }
    // k rounds: each lane's best untaken expert (and its logit), then the wavefront's best (wave_best: every lane gets
    // the same winner, whose own lane holds it as its best); the winner's lane marks it taken; lane j keeps pick j
    mine = 0;
    float mx = 0.f;  // (lane j: pick j's logit)
    for (int j = 0; j < A.k; ++j) {
        Cand<K> c{(K)-INFINITY, E};  // (no expert yet: any untaken one comes before it)
        float cx = 0.f;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int e = l + 64 * i;
            if (!((taken >> i) & 1u)) {
                const Cand<K> n = pick_of(c, Cand<K>{key[i], e}, E);
                cx = n.i == e ? xs[i] : cx;
                c = n;
            }
        }
        const int bi = wave_best(c, E).i;
        const float bx = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cx), bi & 63));
        if (l == (bi & 63)) taken |= 1u << (bi >> 6);
        if (l == j) {
            mine = bi;
            mx = bx;
        }
    }
    // the weights, lane j for pick j: the softmax over the picked logits (less the largest, pick 0's), in float (within
    // a bf16 ulp of the exact weight, which is all the bf16 result keeps), or the sigmoids (over their sum when
    // normalized) in double; the sums over the k lanes by a butterfly
    const bool has = l < A.k;
    if (A.kind == 0) {
        const float m = lane_key(mx, 0);
        float v = has ? expf(mx - m) : 0.f;
        v /= wave_sum(v);
        wbits = bf16_bits((float)((double)v * A.scale));
    } else {
        const double lx = has ? (double)mx : 0.0;
        double v = has ? sigmoid_d(lx) : 0.0;
        if (A.norm) v /= wave_sum(v);
        wbits = bf16_bits((float)(v * A.scale));
    }
}

template <int PER>
__device__ __forceinline__ void route_row_n(const RouteArgs& A, int r, int l, RouteLds& L, int& mine, uint16_t& wbits) {
    if (A.kind == 1 && A.bias != nullptr)
        route_row_k<PER, double>(A, r, l, L, mine, wbits);
    else
        route_row_k<PER, float>(A, r, l, L, mine, wbits);
}

// The same routing for up to 64 experts keyed by their logits (softmax, or sigmoid without a bias), no groups, k <= E:
// by rank instead of k rounds. Lane e holds expert e's key; every lane reads all E keys from LDS and counts those
// that come before its own (the larger key, the lower id among equal keys): that count is its slot, and the experts
// whose slot is below k are the picks. One more pass through LDS brings pick j to lane j. No chain of lane moves: the
// k rounds' butterflies take ≈ 1.5 µs at one wavefront, this ≈ 0.3. The picks, their order and the weights (computed
// as route_row_k does, from the same values in the same order) are the same bit for bit.
__device__ __forceinline__ void route_row_rank(const RouteArgs& A, int r, int l, RouteLds& L, int& mine,
                                               uint16_t& wbits) {
    const float* lg = A.logits + (size_t)r * A.ld_logits;
    const int E = A.experts;
    float* key = reinterpret_cast<float*>(L.key);  // [64] the keys, then the picks' logits [MAXK] and ids [MAXK]
    float* px = key + 64;
    int* pid = reinterpret_cast<int*>(key + 64 + MAXK);
    const float x = l < E ? lg[l] : 0.f;
    const float kv = x != x ? -INFINITY : x;  // (a NaN key is never preferred)
    if (l < E) key[l] = kv;
    wave_lds_sync();
    int rank = 0;
    if (l < E) {
        for (int i = 0; i < E; ++i) rank += before(key[i], i, kv, l);
        if (rank < A.k) {
            px[rank] = x;
            pid[rank] = l;
        }
    }
    wave_lds_sync();
    const bool has = l < A.k;
    mine = has ? pid[l] : 0;
    const float mx = has ? px[l] : 0.f;
    if (A.kind == 0) {
        const float m = lane_key(mx, 0);
        float v = has ? expf(mx - m) : 0.f;
        v /= wave_sum(v);
        wbits = bf16_bits((float)((double)v * A.scale));
    } else {
        const double lx = has ? (double)mx : 0.0;
        double v = has ? sigmoid_d(lx) : 0.0;
        if (A.norm) v /= wave_sum(v);
        wbits = bf16_bits((float)(v * A.scale));
    }
}

// route_row_n with the fewest experts a lane that hold E (1, 4 or 16; at most MAXPER, E <= 64 MAXPER: a caller
// whose registers matter compiles only the small cases)
template <int MAXPER = MAXE / 64>
__device__ __forceinline__ void route_row(const RouteArgs& A, int r, int l, RouteLds& L, int& mine, uint16_t& wbits) {
    if (A.experts <= 64 && A.n_group == 0 && A.k <= A.experts && !(A.kind == 1 && A.bias != nullptr))
        route_row_rank(A, r, l, L, mine, wbits);
    else if (MAXPER == 1 || A.experts <= 64)
        route_row_n<1>(A, r, l, L, mine, wbits);
    else if (MAXPER == 4 || A.experts <= 256)
        route_row_n<(MAXPER < 4 ? MAXPER : 4)>(A, r, l, L, mine, wbits);
    else
        route_row_n<MAXPER>(A, r, l, L, mine, wbits);
}

// row r's outputs: the k picks and weights (lane j < k), the slot column, the shared gate
__device__ __forceinline__ void route_store(const RouteArgs& A, int r, int l, int mine, uint16_t wbits) {
    if (l < A.k) {
        put_id(A, r, l, mine);
        A.w[(size_t)r * A.ld_w + l] = wbits;
    }
    if (l == 0 && A.slot >= 0) {
        put_id(A, r, A.k, A.slot);
        A.w[(size_t)r * A.ld_w + A.k] = 0x3F80u;  // 1.0
    }
    if (l == 0 && A.shared != nullptr)
        A.shared[(size_t)r * A.ld_shared] = bf16_bits((float)sigmoid_d(A.logits[(size_t)r * A.ld_logits + A.experts]));
}

// R's arguments checked as dr_moe_route takes them, and as a RouteArgs (DR_OK, else DR_EINVAL; moe_route.hip)
__attribute__((visibility("hidden"))) int route_args(const dr_route* R, RouteArgs& A);

}  // namespace moe_route

#endif
