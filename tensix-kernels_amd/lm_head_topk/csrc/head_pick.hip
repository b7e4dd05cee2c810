// head_pick.hip: the LM head's pick for MI355X (gfx950), behind the C ABI of include/lm_head.h.
//
// Input: the top-k records an LM head's dense_reader matmuls wrote (one record per 32-column tile of the vocabulary;
// in each, rows x k bf16 keys, then their ids). One workgroup takes one row:
//   dr_pick_k          the best `top` valid slots by key (a 64-bit key per slot: the 16-bit key above the slot's
//                      index complemented, so the earlier slot wins a tie and every key is distinct), selected with
//                      the wavefront lists of wave_select.h; then each candidate's exact logit, x[r] . head[id] in
//                      float32 (one wavefront a candidate, a fixed sum order), rounded to bf16 if asked; then the pick:
//                      the lowest id among the largest logits, a NaN counting as the largest.
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

constexpr int PICK_T = 256;          // threads a workgroup (four wavefronts)
constexpr int PICK_W = PICK_T / 64;  // wavefronts
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
struct RowSlots {
    const uint32_t* rec;
    size_t rlen;
    int rows, k, r;
    __device__ __forceinline__ void get(int c, uint32_t& key, uint32_t& id) const {
        const int p = c / k, s = c - p * k;
        const uint32_t* w = rec + (size_t)p * rlen;
        key = w[(size_t)r * k + s] & 0xFFFFu;
        id = w[(size_t)rows * k + (size_t)r * k + s];
    }
};

__global__ __launch_bounds__(PICK_T) void dr_pick_k(const uint32_t* __restrict__ rec, int nrec, int rows, int k,
                                                    int top, int round_bf16, const uint16_t* __restrict__ x, int ldx,
                                                    int dim, const uint16_t* __restrict__ head, long long ld_head,
                                                    uint32_t vocab, uint32_t* __restrict__ out,
                                                    uint32_t* __restrict__ ids_out) {
    __shared__ unsigned long long lists[PICK_W][64];
    __shared__ unsigned long long pend[PICK_W][64];
    __shared__ uint32_t cid[MAXTOP];
    __shared__ float logit[MAXTOP];
    __shared__ int s_n;
    const int r = blockIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const RowSlots R{rec, 2 * (size_t)rows * k, rows, k, r};
    const int total = nrec * k;

    // 1. the best `top` valid slots by key, the earlier slot first among equals
    WaveBest best;
    for (int base = wave * 64; base < total; base += PICK_T) {
        const int c = base + lane;
        unsigned long long v = 0ull;
        if (c < total) {
            uint32_t key, id;
            R.get(c, key, id);
            if (key != 0u && id < vocab)
                v = ((unsigned long long)key << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)c);
        }
        best.add(v, pend[wave], top, lane);
    }
    best.flush(pend[wave], top, lane);
    lists[wave][lane] = best.list;
    __syncthreads();
    if (wave == 0) {
        unsigned long long list = best.list;
#pragma unroll
        for (int w = 1; w < PICK_W; ++w) list = wave_merge(list, lists[w][lane], lane);
        const bool have = lane < top && list != 0ull;
        const int n = __popcll(__ballot(have));
        if (lane < MAXTOP) {
            uint32_t id = 0xFFFFFFFFu;
            if (have) {
                uint32_t key;
                R.get((int)(0xFFFFFFFFu - (uint32_t)(list & 0xFFFFFFFFu)), key, id);
            }
            cid[lane] = id;
        }
        if (lane == 0) s_n = n;
    }
    __syncthreads();
    const int n = s_n;

    // 2. the candidates' logits: x[r] . head[id], one wavefront a candidate, float32 in a fixed order
    const uint16_t* xr = x + (size_t)r * ldx;
    for (int j = wave; j < n; j += PICK_W) {
        const uint16_t* hr = head + (size_t)cid[j] * (size_t)ld_head;
        float acc = 0.f;
        for (int d0 = lane * 8; d0 < dim; d0 += 512) {
            const uint4 xv = *reinterpret_cast<const uint4*>(xr + d0);
            const uint4 hv = *reinterpret_cast<const uint4*>(hr + d0);
            acc = __builtin_fmaf(bf16_lo(xv.x), bf16_lo(hv.x), acc);
            acc = __builtin_fmaf(bf16_hi(xv.x), bf16_hi(hv.x), acc);
            acc = __builtin_fmaf(bf16_lo(xv.y), bf16_lo(hv.y), acc);
            acc = __builtin_fmaf(bf16_hi(xv.y), bf16_hi(hv.y), acc);
            acc = __builtin_fmaf(bf16_lo(xv.z), bf16_lo(hv.z), acc);
            acc = __builtin_fmaf(bf16_hi(xv.z), bf16_hi(hv.z), acc);
            acc = __builtin_fmaf(bf16_lo(xv.w), bf16_lo(hv.w), acc);
            acc = __builtin_fmaf(bf16_hi(xv.w), bf16_hi(hv.w), acc);
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
        if (lane == 0) logit[j] = round_bf16 ? __uint_as_float(bf16_bits(acc) << 16) : acc;
    }
    __syncthreads();

    // 3. the pick: the lowest id among the largest logits (lm_head_topk/lmhead.py:40-46)
    if (threadIdx.x == 0) {
        uint32_t tok = 0, best_key = 0;
        bool any = false;
        for (int j = 0; j < n; ++j) {
            const uint32_t kk = order32(__float_as_uint(logit[j]));
            const uint32_t id = cid[j];
            if (!any || kk > best_key || (kk == best_key && id < tok)) {
                best_key = kk;
                tok = id;
                any = true;
            }
        }
        uint32_t* o = out + (size_t)r * 32;
        o[0] = any ? tok : 0u;
        o[1] = n > 0 ? cid[0] : 0xFFFFFFFFu;
        o[2] = (uint32_t)n;
        for (int w = 3; w < 32; ++w) o[w] = 0u;
        if (ids_out != nullptr && r == 0) ids_out[0] = o[0];
    }
}

__global__ __launch_bounds__(PICK_T) void dr_pick_records_k(const uint32_t* __restrict__ rec, int nrec, int rows,
                                                            int k, uint32_t vocab, const uint32_t* __restrict__ tmap,
                                                            uint32_t* __restrict__ out, uint32_t* __restrict__ ids_out) {
    __shared__ unsigned long long s_best[PICK_W];
    __shared__ int s_cnt[PICK_W];
    const int r = blockIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const RowSlots R{rec, 2 * (size_t)rows * k, rows, k, r};
    const int total = nrec * k;
    unsigned long long b = 0ull;
    int cnt = 0;
    for (int c = threadIdx.x; c < total; c += PICK_T) {
        uint32_t key, id;
        R.get(c, key, id);
        if (key == 0u || id >= vocab) continue;
        ++cnt;
        const unsigned long long v =
            ((unsigned long long)rank16(key) << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)c);
        b = v > b ? v : b;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const unsigned long long p = xor_lane(b, o);
        b = p > b ? p : b;
        cnt += __shfl_xor(cnt, o);
    }
    if (lane == 0) {
        s_best[wave] = b;
        s_cnt[wave] = cnt;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long v = 0ull;
        int n = 0;
        for (int w = 0; w < PICK_W; ++w) {
            v = s_best[w] > v ? s_best[w] : v;
            n += s_cnt[w];
        }
        uint32_t* o = out + (size_t)r * 32;
        uint32_t tok = 0u, id = 0xFFFFFFFFu;
        if (n > 0) {
            uint32_t key;
            R.get((int)(0xFFFFFFFFu - (uint32_t)(v & 0xFFFFFFFFu)), key, id);
            tok = tmap != nullptr ? tmap[id] : id;
        }
        o[0] = tok;
        o[1] = id;
        o[2] = (uint32_t)n;
        for (int w = 3; w < 32; ++w) o[w] = 0u;
        if (ids_out != nullptr && r == 0) ids_out[0] = tok;
    }
}

inline hipStream_t S(void* s) { return reinterpret_cast<hipStream_t>(s); }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

extern "C" {

int dr_head_pick(const void* records, int n_records, int rows, int k, int top, int round_bf16, const void* x, int ldx,
                 int dim, const void* head, int64_t ld_head, int64_t vocab, void* out, void* ids_out, void* stream) {
    if (records == nullptr || x == nullptr || head == nullptr || out == nullptr || n_records < 1 || rows < 1 ||
        rows > 32 || k < 1 || top < 1 || top > MAXTOP || dim < 8 || dim % 8 != 0 || ldx < dim || ldx % 8 != 0 ||
        ld_head < dim || ld_head % 8 != 0 || vocab < 1 || vocab > (int64_t)0xFFFFFFFFu || !aligned16(x) ||
        !aligned16(head))
        return DR_EINVAL;
    if ((int64_t)n_records * k >= ((int64_t)1 << 31)) return DR_ERANGE;
    hipLaunchKernelGGL(dr_pick_k, dim3(rows), dim3(PICK_T), 0, S(stream), reinterpret_cast<const uint32_t*>(records),
                       n_records, rows, k, top, round_bf16, reinterpret_cast<const uint16_t*>(x), ldx, dim,
                       reinterpret_cast<const uint16_t*>(head), (long long)ld_head, (uint32_t)vocab,
                       reinterpret_cast<uint32_t*>(out), reinterpret_cast<uint32_t*>(ids_out));
    return hipGetLastError() == hipSuccess ? DR_OK : DR_EHIP;
}

int dr_head_pick_records(const void* records, int n_records, int rows, int k, int64_t vocab, const void* token_map,
                         void* out, void* ids_out, void* stream) {
    if (records == nullptr || out == nullptr || n_records < 1 || rows < 1 || rows > 32 || k < 1 || vocab < 1 ||
        vocab > (int64_t)0xFFFFFFFFu)
        return DR_EINVAL;
    if ((int64_t)n_records * k >= ((int64_t)1 << 31)) return DR_ERANGE;
    hipLaunchKernelGGL(dr_pick_records_k, dim3(rows), dim3(PICK_T), 0, S(stream),
                       reinterpret_cast<const uint32_t*>(records), n_records, rows, k, (uint32_t)vocab,
                       reinterpret_cast<const uint32_t*>(token_map), reinterpret_cast<uint32_t*>(out),
                       reinterpret_cast<uint32_t*>(ids_out));
    return hipGetLastError() == hipSuccess ? DR_OK : DR_EHIP;
}

}  // extern "C"
