// moe_route.hip: the MoE router's top k and routing weights on MI355X (gfx950), behind dr_moe_route (include/moe.h).
//
// One wavefront a row of logits (up to 32 rows, up to 1024 experts). The keys (the logit, or sigmoid(logit) + bias)
// are made once in double precision into LDS. DeepSeek-V3's group-limited routing optionally keeps only the best
// groups. Then k rounds each take the best untaken key across the wavefront (a butterfly over the lanes' own bests,
// the lower id first among equal keys). The weights come last, in double, rounded to bf16 once: the softmax over the
// picked logits, or the picks' sigmoids (over their sum when normalized), times the scale. This replaces
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

__global__ __launch_bounds__(64) void dr_route_k(const RouteArgs A) {
    __shared__ double key[MAXE];
    __shared__ uint32_t taken[MAXE / 32];
    __shared__ double gscore[32];
    __shared__ int pick[MAXK];
    const int r = blockIdx.x, l = threadIdx.x;
    const float* lg = A.logits + (size_t)r * A.ld_logits;
    const int E = A.experts;
    for (int e = l; e < E; e += 64) {
        const double x = lg[e];
        double kv = (A.kind == 1 && A.bias != nullptr) ? sigmoid_d(x) + (double)A.bias[e] : x;
        key[e] = kv != kv ? -INFINITY : kv;  // (a NaN key is never preferred)
    }
    for (int i = l; i < MAXE / 32; i += 64) taken[i] = 0u;
    __syncthreads();
    if (A.n_group > 0) {
        // a group's score: the sum of its two largest keys; the topk_group best groups stay
        const int ng = A.n_group, gs = E / ng;
        if (l < ng) {
            double b1 = -INFINITY, b2 = -INFINITY;
            for (int j = 0; j < gs; ++j) {
                const double v = key[l * gs + j];
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
        bool drop = false;
        if (l < ng) {
            int rank = 0;
            for (int j = 0; j < ng; ++j) rank += before(gscore[j], j, gscore[l], l);
            drop = rank >= A.topk_group;
        }
        __syncthreads();
        if (drop)
            for (int j = 0; j < gs; ++j) key[l * gs + j] = -INFINITY;
        __syncthreads();
    }
    for (int j = 0; j < A.k; ++j) {
        double bk = -INFINITY;
        int bi = E;  // (no expert yet: any untaken one comes before it)
        for (int e = l; e < E; e += 64) {
            if ((taken[e >> 5] >> (e & 31)) & 1u) continue;
            if (bi == E || before(key[e], e, bk, bi)) {
                bk = key[e];
                bi = e;
            }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const double ok = __shfl_xor(bk, o);
            const int oi = __shfl_xor(bi, o);
            if (oi != E && (bi == E || before(ok, oi, bk, bi))) {
                bk = ok;
                bi = oi;
            }
        }
        if (l == 0) {
            pick[j] = bi;
            taken[bi >> 5] |= 1u << (bi & 31);
        }
        __syncthreads();
    }
    if (l != 0) return;
    double v[MAXK];
    double sum = 0.0;
    if (A.kind == 0) {
        const double m = lg[pick[0]];  // (the largest logit: the first pick)
        for (int j = 0; j < A.k; ++j) {
            v[j] = exp((double)lg[pick[j]] - m);
            sum += v[j];
        }
        for (int j = 0; j < A.k; ++j) v[j] /= sum;
    } else {
        for (int j = 0; j < A.k; ++j) {
            v[j] = sigmoid_d(lg[pick[j]]);
            sum += v[j];
        }
        if (A.norm)
            for (int j = 0; j < A.k; ++j) v[j] /= sum;
    }
    for (int j = 0; j < A.k; ++j) {
        put_id(A, r, j, pick[j]);
        A.w[(size_t)r * A.ld_w + j] = bf16_bits((float)(v[j] * A.scale));
    }
    if (A.slot >= 0) {
        put_id(A, r, A.k, A.slot);
        A.w[(size_t)r * A.ld_w + A.k] = 0x3F80u;  // 1.0
    }
    if (A.shared != nullptr) A.shared[(size_t)r * A.ld_shared] = bf16_bits((float)sigmoid_d(lg[E]));
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
