// head_pick.hip: the LM head's pick for MI355X (gfx950), behind the C ABI of include/lm_head.h.
//
// Input: the top-k records an LM head's dense_reader matmuls wrote (one record per 32-column tile of the vocabulary;
// in each, rows x k bf16 keys, then their ids). A row's slots are selected over several workgroups (wave_select.h's
// select_row; the workgroup that ends with the row's list finishes it):
//   dr_pick_k          the best `top` valid slots by key (a 64-bit key per slot: the 16-bit key above the slot's
//                      index complemented, so the earlier slot wins a tie and every key is distinct); then each
//                      candidate's exact logit, x[r] . head[id] in float32 (one wavefront a candidate, a fixed sum
//                      order), rounded to bf16 if asked; then the pick: the lowest id among the largest logits, a NaN
//                      counting as the largest.
//   dr_pick_records_k  the slot of the largest key rank (no rescore), through a token map.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dense_reader.h"
#include "lm_head.h"
#include "wave_select.h"

// no multiply-add contraction beyond the explicit FMAs: one rounding order in every instantiation
#pragma clang fp contract(off)

namespace {

using namespace wsel;

constexpr int MAXTOP = 32;

// a float's bits as an unsigned key in torch's order: NaN above everything, -0 equal to +0
// (lm_head_topk/kernels/head_pick_writer.cpp:16-24)
__device__ __forceinline__ uint32_t order32(uint32_t b) {
    if ((b & 0x7FFFFFFFu) == 0) b = 0;
    if ((b & 0x7F800000u) == 0x7F800000u && (b & 0x007FFFFFu) != 0) return 0xFFFFFFFFu;
    return (b >> 31) ? ~b : (b | 0x80000000u);
}

// a record key's rank (key != 0): a NaN's above every key, -0's (0x7FFF) equal to +0's (0x8000)
// (lm_head_topk/kernels/head_pick_records.cpp:25-32)
__device__ __forceinline__ uint32_t rank16(uint32_t kk) {
    const uint32_t mag = (kk >= 0x8000u ? kk : ~kk) & 0x7FFFu;
    if ((mag & 0x7F80u) == 0x7F80u && (mag & 0x007Fu) != 0) return 0x10000u;
    return kk == 0x7FFFu ? 0x8000u : kk;
}

// float32 to bf16 bits, to nearest even (a NaN stays a NaN)
__device__ __forceinline__ uint32_t bf16_bits(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu) != 0) return (u >> 16) | 0x40u;
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// the records of one row: slot c is record c / k, slot c % k
__device__ __forceinline__ uint32_t slot_id(const SelArgs& A, int r, uint32_t c) {
    const uint32_t p = c / (uint32_t)A.k, s = c - p * (uint32_t)A.k;
    return A.rec[(size_t)p * 2 * A.rows * A.k + (size_t)A.rows * A.k + (size_t)r * A.k + s];
}

// PACK (slots and vocab below 2^24): a key carries its slot's id in its low 24 bits (the 16-bit key, then the slot's
// index complemented in 24 bits, then the id), so the candidates' ids need no second read of the records
template <bool PACK>
__global__ __launch_bounds__(SEL_T) void dr_pick_k(SelArgs A, uint32_t vocab, int round_bf16,
                                                   const uint16_t* __restrict__ x, int ldx, int dim,
                                                   const uint16_t* __restrict__ head, long long ld_head,
                                                   uint32_t* __restrict__ out, uint32_t* __restrict__ ids_out) {
    __shared__ SelShared sh;
    __shared__ uint32_t cid[MAXTOP];
    __shared__ float logit[MAXTOP];
    __shared__ int s_n;
    const int r = blockIdx.x % A.rows, sl = blockIdx.x / A.rows;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;

    // 1. the best `top` valid slots by key, the earlier slot first among equals
    unsigned long long list;
    int count;
    const bool mine = select_row<true>(
        A, r, sl,
        [vocab](uint32_t key, uint32_t id, uint32_t c) -> unsigned long long {
            key &= 0xFFFFu;
            if (key == 0u || id >= vocab) return 0ull;
            if constexpr (PACK)
                return ((unsigned long long)key << 48) | ((unsigned long long)(0xFFFFFFu - c) << 24) | id;
            else
                return ((unsigned long long)key << 32) | (unsigned long long)(0xFFFFFFFFu - c);
        },
        sh, list, count);
    if (!mine) return;
    if (wave == 0) {
        const bool have = lane < A.keep && list != 0ull;
        const int n = __popcll(__ballot(have));
        uint32_t id = 0xFFFFFFFFu;
        if (have) id = PACK ? (uint32_t)(list & 0xFFFFFFu) : slot_id(A, r, 0xFFFFFFFFu - (uint32_t)(list & 0xFFFFFFFFu));
        if (lane < MAXTOP) cid[lane] = id;
        if (lane == 0) s_n = n;
    }
    __syncthreads();
    const int n = s_n;

    // 2. the candidates' logits: x[r] . head[id], one wavefront a candidate, float32 in a fixed order (lane l sums
    // d = 8 l + 512 i + j, i then j ascending; then the lanes, a butterfly). A wavefront takes RG candidates at once
    // (j, j + SEL_W, ...) and issues every load of a span of DSPAN values for all of them before the first is used.
    constexpr int DSPAN = 8 * 512, RG = MAXTOP / SEL_W < 4 ? MAXTOP / SEL_W : 4;
    const uint16_t* xr = x + (size_t)r * ldx;
    for (int j0 = wave; j0 < n; j0 += RG * SEL_W) {
        const uint16_t* hr[RG];
#pragma unroll
        for (int t = 0; t < RG; ++t)  // (past n: candidate j0's row again, its sum not kept)
            hr[t] = head + (size_t)cid[j0 + t * SEL_W < n ? j0 + t * SEL_W : j0] * (size_t)ld_head;
        float acc[RG];
#pragma unroll
        for (int t = 0; t < RG; ++t) acc[t] = 0.f;
        for (int s0 = 0; s0 < dim; s0 += DSPAN) {
            uint4 xv[8], hv[RG][8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int d0 = min(s0 + i * 512 + lane * 8, dim - 8);  // (in bounds; past dim masked below)
                xv[i] = *reinterpret_cast<const uint4*>(xr + d0);
#pragma unroll
                for (int t = 0; t < RG; ++t) hv[t][i] = *reinterpret_cast<const uint4*>(hr[t] + d0);
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const bool past = s0 + i * 512 + lane * 8 >= dim;
                if (past) xv[i] = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
                for (int t = 0; t < RG; ++t) {
                    const uint4 h = past ? make_uint4(0u, 0u, 0u, 0u) : hv[t][i];
                    float a = acc[t];
                    a = __builtin_fmaf(bf16_lo(xv[i].x), bf16_lo(h.x), a);
                    a = __builtin_fmaf(bf16_hi(xv[i].x), bf16_hi(h.x), a);
                    a = __builtin_fmaf(bf16_lo(xv[i].y), bf16_lo(h.y), a);
                    a = __builtin_fmaf(bf16_hi(xv[i].y), bf16_hi(h.y), a);
                    a = __builtin_fmaf(bf16_lo(xv[i].z), bf16_lo(h.z), a);
                    a = __builtin_fmaf(bf16_hi(xv[i].z), bf16_hi(h.z), a);
                    a = __builtin_fmaf(bf16_lo(xv[i].w), bf16_lo(h.w), a);
                    a = __builtin_fmaf(bf16_hi(xv[i].w), bf16_hi(h.w), a);
                    acc[t] = a;
                }
            }
        }
#pragma unroll
        for (int t = 0; t < RG; ++t) {
            const float sum = wave_sum_xor(acc[t]);
            const int j = j0 + t * SEL_W;
            if (lane == 0 && j < n) logit[j] = round_bf16 ? __uint_as_float(bf16_bits(sum) << 16) : sum;
        }
    }
    __syncthreads();

    // 3. the pick: the lowest id among the largest logits (lm_head_topk/lmhead.py:40-46), by a wavefront maximum of
    // the candidates' (logit rank, id complemented)
    if (wave == 0) {
        unsigned long long cand = 0ull;  // (every candidate's is above 0: its rank is)
        if (lane < n)
            cand = ((unsigned long long)order32(__float_as_uint(logit[lane])) << 32) | (0xFFFFFFFFu - cid[lane]);
        const unsigned long long best = wave_max(cand);
        uint32_t* o = out + (size_t)r * 32;
        if (lane == 0) {
            const uint32_t tok = best != 0ull ? 0xFFFFFFFFu - (uint32_t)best : 0u;
            o[0] = tok;
            o[1] = n > 0 ? cid[0] : 0xFFFFFFFFu;
            o[2] = (uint32_t)n;
            if (ids_out != nullptr && r == 0) ids_out[0] = tok;
        } else if (lane >= 3 && lane < 32) {
            o[lane] = 0u;
        }
    }
}

__global__ __launch_bounds__(SEL_T) void dr_pick_records_k(SelArgs A, uint32_t vocab,
                                                           const uint32_t* __restrict__ tmap,
                                                           uint32_t* __restrict__ out, uint32_t* __restrict__ ids_out) {
    __shared__ SelShared sh;
    const int r = blockIdx.x % A.rows, sl = blockIdx.x / A.rows;
    unsigned long long list;
    int count;
    const bool mine = select_row<true>(
        A, r, sl,
        [vocab](uint32_t key, uint32_t id, uint32_t c) -> unsigned long long {
            key &= 0xFFFFu;
            if (key == 0u || id >= vocab) return 0ull;
            return ((unsigned long long)rank16(key) << 32) | (unsigned long long)(0xFFFFFFFFu - c);
        },
        sh, list, count);
    if (!mine || threadIdx.x != 0) return;
    uint32_t* o = out + (size_t)r * 32;
    uint32_t tok = 0u, id = 0xFFFFFFFFu;
    if (list != 0ull) {
        id = slot_id(A, r, 0xFFFFFFFFu - (uint32_t)(list & 0xFFFFFFFFu));
        tok = tmap != nullptr ? tmap[id] : id;
    }
    o[0] = tok;
    o[1] = id;
    o[2] = (uint32_t)count;
    for (int w = 3; w < 32; ++w) o[w] = 0u;
    if (ids_out != nullptr && r == 0) ids_out[0] = tok;
}

inline hipStream_t S(void* s) { return reinterpret_cast<hipStream_t>(s); }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

extern "C" {

namespace {

int plan_select(SelArgs& A, const void* records, int n_records, int rows, int k, int keep, void* workspace,
                int64_t workspace_bytes) {
    A = SelArgs{reinterpret_cast<const uint32_t*>(records), n_records, rows, k, keep, 1, 0, nullptr, nullptr, nullptr};
    select_plan(n_records, k, &A.slices, &A.cs);
    return select_bind(A, workspace, workspace_bytes) ? DR_OK : DR_EINVAL;
}

}  // namespace

int dr_head_pick(const void* records, int n_records, int rows, int k, int top, int round_bf16, const void* x, int ldx,
                 int dim, const void* head, int64_t ld_head, int64_t vocab, void* out, void* ids_out, void* workspace,
                 int64_t workspace_bytes, void* stream) {
    if (records == nullptr || x == nullptr || head == nullptr || out == nullptr || n_records < 1 || rows < 1 ||
        rows > 32 || k < 1 || top < 1 || top > MAXTOP || dim < 8 || dim % 8 != 0 || ldx < dim || ldx % 8 != 0 ||
        ld_head < dim || ld_head % 8 != 0 || vocab < 1 || vocab > (int64_t)0xFFFFFFFFu || !aligned16(x) ||
        !aligned16(head))
        return DR_EINVAL;
    if ((int64_t)n_records * k >= ((int64_t)1 << 32)) return DR_ERANGE;
    SelArgs A;
    const int st = plan_select(A, records, n_records, rows, k, top, workspace, workspace_bytes);
    if (st != DR_OK) return st;
    const bool pack = (int64_t)n_records * k <= ((int64_t)1 << 24) && vocab <= ((int64_t)1 << 24);
    hipLaunchKernelGGL(pack ? dr_pick_k<true> : dr_pick_k<false>, dim3(rows * A.slices), dim3(SEL_T), 0, S(stream), A,
                       (uint32_t)vocab, round_bf16, reinterpret_cast<const uint16_t*>(x), ldx, dim,
                       reinterpret_cast<const uint16_t*>(head), (long long)ld_head, reinterpret_cast<uint32_t*>(out),
                       reinterpret_cast<uint32_t*>(ids_out));
    return hipGetLastError() == hipSuccess ? DR_OK : DR_EHIP;
}

int dr_head_pick_records(const void* records, int n_records, int rows, int k, int64_t vocab, const void* token_map,
                         void* out, void* ids_out, void* workspace, int64_t workspace_bytes, void* stream) {
    if (records == nullptr || out == nullptr || n_records < 1 || rows < 1 || rows > 32 || k < 1 || vocab < 1 ||
        vocab > (int64_t)0xFFFFFFFFu)
        return DR_EINVAL;
    if ((int64_t)n_records * k >= ((int64_t)1 << 32)) return DR_ERANGE;
    SelArgs A;
    const int st = plan_select(A, records, n_records, rows, k, 1, workspace, workspace_bytes);
    if (st != DR_OK) return st;
    hipLaunchKernelGGL(dr_pick_records_k, dim3(rows * A.slices), dim3(SEL_T), 0, S(stream), A, (uint32_t)vocab,
                       reinterpret_cast<const uint32_t*>(token_map), reinterpret_cast<uint32_t*>(out),
                       reinterpret_cast<uint32_t*>(ids_out));
    return hipGetLastError() == hipSuccess ? DR_OK : DR_EHIP;
}

}  // extern "C"
