// moe_route.hip: the MoE router's top k and routing weights on MI355X (gfx950), behind dr_moe_route (include/moe.h).
//
// One wavefront a row of logits (up to 32 rows, up to 1024 experts, 16 a lane in registers). The keys (the logit, or
// sigmoid(logit) + bias) are made once in double precision. DeepSeek-V3's group-limited routing optionally keeps only
// the best groups (scored through LDS). Then k rounds each take the best untaken key across the wavefront (a butterfly
// over the lanes' own bests, the lower id first among equal keys), with no barrier. The weights come last, one lane a
// pick, in double, rounded to bf16 once: the softmax over the picked logits, or the picks' sigmoids (over their sum
// when normalized), times the scale. This replaces
// moe/kernels/moe_route.cpp's fixed-point arithmetic on one RISC-V core (moe/moe8.py:1139-1253).

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>

#include "moe.h"

namespace {

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

__device__ __forceinline__ double sigmoid_d(double x) { return 1.0 / (1.0 + exp(-x)); }

// float -> bf16 bits, round to nearest even (a NaN: the quiet NaN)
__device__ __forceinline__ uint16_t bf16_bits(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// (ka, ia) comes before (kb, ib): the larger key, the lower id among equal keys
__device__ __forceinline__ bool before(double ka, int ia, double kb, int ib) {
    return ka > kb || (ka == kb && ia < ib);
}

__device__ __forceinline__ void put_id(const RouteArgs& A, int r, int j, long long id) {
    const size_t i = (size_t)r * A.ld_ids + j;
    if (A.ids32)
        reinterpret_cast<uint32_t*>(A.ids)[i] = (uint32_t)id;
    else
        reinterpret_cast<uint16_t*>(A.ids)[i] = (uint16_t)id;
}

// a candidate (key, id); id == none: no expert
struct Cand {
    double k;
    int i;
};

__device__ __forceinline__ Cand pick_of(Cand a, Cand b, int none) {
    return (b.i != none && (a.i == none || before(b.k, b.i, a.k, a.i))) ? b : a;
}

// the candidate of the lane DPP control CTRL names (rows outside ROWS, or no such lane: no expert)
template <int CTRL, int ROWS>
__device__ __forceinline__ Cand dpp_cand(Cand c, int none) {
    const long long bits = __double_as_longlong(c.k);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)bits, CTRL, ROWS, 0xf, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(bits >> 32), CTRL, ROWS, 0xf, false);
    const int id = __builtin_amdgcn_update_dpp(none, c.i, CTRL, ROWS, 0xf, false);
    return Cand{__longlong_as_double(((long long)hi << 32) | (unsigned)lo), id};
}

// the wavefront's best candidate, on every lane: row_shr 1, 2, 4, 8 carry each row's best to its lane 15,
// row_bcast 15 and 31 carry those to lane 63, which every lane then reads (VALU moves, no LDS round trips)
__device__ __forceinline__ Cand wave_best(Cand c, int none) {
    c = pick_of(c, dpp_cand<0x111, 0xf>(c, none), none);  // row_shr:1
    c = pick_of(c, dpp_cand<0x112, 0xf>(c, none), none);  // row_shr:2
    c = pick_of(c, dpp_cand<0x114, 0xf>(c, none), none);  // row_shr:4
    c = pick_of(c, dpp_cand<0x118, 0xf>(c, none), none);  // row_shr:8
    c = pick_of(c, dpp_cand<0x142, 0xa>(c, none), none);  // row_bcast:15 into rows 1 and 3
    c = pick_of(c, dpp_cand<0x143, 0xc>(c, none), none);  // row_bcast:31 into rows 2 and 3
    const long long bits = __double_as_longlong(c.k);
    const int lo = __builtin_amdgcn_readlane((int)bits, 63);
    const int hi = __builtin_amdgcn_readlane((int)(bits >> 32), 63);
    return Cand{__longlong_as_double(((long long)hi << 32) | (unsigned)lo), __builtin_amdgcn_readlane(c.i, 63)};
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

__global__ __launch_bounds__(64) void dr_route_k(const RouteArgs A) {
    constexpr int PER = MAXE / 64;  // experts a lane: e = lane + 64 i
    __shared__ double key_lds[MAXE];
    __shared__ double gscore[32];
    const int r = blockIdx.x, l = threadIdx.x;
    const float* lg = A.logits + (size_t)r * A.ld_logits;
    const int E = A.experts;
    const bool sig = A.kind == 1 && A.bias != nullptr;
    double key[PER];
    uint32_t taken = 0u;  // bit i: expert lane + 64 i is picked (or absent)
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int e = l + 64 * i;
        double kv = -INFINITY;
        if (e < E) {
            const double x = lg[e];
            kv = sig ? sigmoid_d(x) + (double)A.bias[e] : x;
            kv = kv != kv ? -INFINITY : kv;  // (a NaN key is never preferred)
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
            if (l + 64 * i < E) key_lds[l + 64 * i] = key[i];
        __syncthreads();
        const int ng = A.n_group, gs = E / ng;
        if (l < ng) {
            double b1 = -INFINITY, b2 = -INFINITY;
            for (int j = 0; j < gs; ++j) {
                const double v = key_lds[l * gs + j];
                if (v > b1) {
                    b2 = b1;
                    b1 = v;
                } else if (v > b2) {
                    b2 = v;
                }
            }
            gscore[l] = b1 + b2;
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int e = l + 64 * i;
            if (e >= E) continue;
            const int gi = e / gs;
            int rank = 0;
            for (int j = 0; j < ng; ++j) rank += before(gscore[j], j, gscore[gi], gi);
            if (rank >= A.topk_group) key[i] = -INFINITY;
        }
    }
    // k rounds: each lane's best untaken expert, then the wavefront's best (wave_best: every lane gets the same
    // winner); the winner's lane marks it taken; lane j keeps pick j
    int mine = 0;
    for (int j = 0; j < A.k; ++j) {
        Cand c{-INFINITY, E};  // (no expert yet: any untaken one comes before it)
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int e = l + 64 * i;
            if (!((taken >> i) & 1u)) c = pick_of(c, Cand{key[i], e}, E);
        }
        const int bi = wave_best(c, E).i;
        if (l == (bi & 63)) taken |= 1u << (bi >> 6);
        if (l == j) mine = bi;
    }
    // the weights, lane j for pick j: the softmax over the picked logits (less the largest, pick 0's), or the sigmoids
    // (over their sum when normalized); the sums over the k lanes by a butterfly
    const bool has = l < A.k;
    const double lx = has ? (double)lg[mine] : 0.0;
    double v;
    if (A.kind == 0) {
        const double m = lane_double(lx, 0);
        v = has ? exp(lx - m) : 0.0;
        v /= wave_sum(v);
    } else {
        v = has ? sigmoid_d(lx) : 0.0;
        if (A.norm) v /= wave_sum(v);
    }
    if (has) {
        put_id(A, r, l, mine);
        A.w[(size_t)r * A.ld_w + l] = bf16_bits((float)(v * A.scale));
    }
    if (l == 0 && A.slot >= 0) {
        put_id(A, r, A.k, A.slot);
        A.w[(size_t)r * A.ld_w + A.k] = 0x3F80u;  // 1.0
    }
    if (l == 0 && A.shared != nullptr) A.shared[(size_t)r * A.ld_shared] = bf16_bits((float)sigmoid_d(lg[E]));
}

}  // namespace

extern "C" int dr_moe_route(const dr_route* R) {
    if (R == nullptr || R->logits == nullptr || R->ids == nullptr || R->w == nullptr) return DR_EINVAL;
    const int kk = R->k + (R->slot >= 0 ? 1 : 0);
    if (R->rows < 1 || R->rows > 32 || R->experts < 1 || R->experts > MAXE || R->experts % 32 || R->k < 1 ||
        R->k > MAXK || R->k > R->experts || kk > MAXK || R->ld_ids < kk || R->ld_w < kk || (R->kind != 0 && R->kind != 1) ||
        R->ld_logits < R->experts + (R->shared != nullptr ? 1 : 0) || !(R->scale > 0.0))
        return DR_EINVAL;
    if (R->slot >= (R->ids32 ? (1LL << 32) : (1LL << 16))) return DR_EINVAL;
    if (R->n_group > 0) {
        const int ng = R->n_group, tg = R->topk_group;
        if (R->kind != 1 || R->bias == nullptr || ng > 32 || R->experts % ng || R->experts / ng < 2 || tg < 1 || tg > ng ||
            tg * (R->experts / ng) < R->k)
            return DR_EINVAL;
    }
    RouteArgs A{R->logits, R->rows, R->ld_logits, R->experts, R->k, R->kind, R->bias, R->ids, R->ids32 != 0,
                R->ld_ids, reinterpret_cast<uint16_t*>(R->w), R->ld_w, reinterpret_cast<uint16_t*>(R->shared),
                R->ld_shared, R->scale, R->norm != 0, R->n_group > 0 ? R->n_group : 0, R->topk_group, R->slot};
    hipLaunchKernelGGL(dr_route_k, dim3(R->rows), dim3(64), 0, reinterpret_cast<hipStream_t>(R->stream), A);
    return hipGetLastError() == hipSuccess ? DR_OK : DR_EHIP;
}
