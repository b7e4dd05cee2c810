// moe_route.hip: the MoE router's top k and routing weights on MI355X (gfx950), behind dr_moe_route (include/moe.h):
// one wavefront a row of logits (up to 32 rows), the routing of moe_route.h (moe/moe8.py:1139-1253).

#include <hip/hip_runtime.h>

#include "moe.h"
#include "moe_route.h"

namespace {

using namespace moe_route;

__global__ __launch_bounds__(64) void dr_route_k(const RouteArgs A) {
    __shared__ RouteLds L;
    const int r = blockIdx.x, l = threadIdx.x;
    int mine;
    uint16_t wbits;
    route_row(A, r, l, L, mine, wbits);
    route_store(A, r, l, mine, wbits);
}

}  // namespace

namespace moe_route {

int route_args(const dr_route* R, RouteArgs& A) {
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
    A = RouteArgs{R->logits, R->rows, R->ld_logits, R->experts, R->k, R->kind, R->bias, R->ids, R->ids32 != 0,
                  R->ld_ids, reinterpret_cast<uint16_t*>(R->w), R->ld_w, reinterpret_cast<uint16_t*>(R->shared),
                  R->ld_shared, R->scale, R->norm != 0, R->n_group > 0 ? R->n_group : 0, R->topk_group, R->slot};
    return DR_OK;
}

}  // namespace moe_route

extern "C" int dr_moe_route(const dr_route* R) {
    moe_route::RouteArgs A;
    const int st = moe_route::route_args(R, A);
    if (st != DR_OK) return st;
    hipLaunchKernelGGL(dr_route_k, dim3(R->rows), dim3(64), 0, reinterpret_cast<hipStream_t>(R->stream), A);
    return hipGetLastError() == hipSuccess ? DR_OK : DR_EHIP;
}
