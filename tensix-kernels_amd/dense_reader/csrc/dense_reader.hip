// dense_reader.hip: the dense_reader decode matmul for MI355X (gfx950), behind the C ABI of include/dense_reader.h.
//
// HBM layout of a packed weight [K, N] (K = in, N = out). N is cut into panels of 16 columns, the reference's
// block-float face rows (16 output columns at one k share one exponent, dense_writer.cpp:186-188, moe/moe8.py:
// 122-138). A panel is a run of k-blocks; one k-block is 1 KiB of codes, read by one wavefront with one 16-byte load a
// lane: lane l = 16 kq + c holds column c of the panel, at the kq-th quarter of the k-block's values:
//   bfp8  (64 k a block):  16 k of column c, one int8 m (two's complement, |m| <= 127) a byte, k in byte order;
//   bfp4  (128 k a block): 32 k of column c; dword d holds k 8d .. 8d+7, byte j the nibbles (k 8d+j low, 8d+4+j
//                          high), each u = m + 8 (offset binary, m in -7 .. 7);
//   bf16  (32 k a block):  8 k of column c, the bf16 values.
// The exponents sit apart: one byte per (panel, k), in k order (panel p at exps + p * k_pad). K is padded to 128 and
// N to 32 (or what the caller asks); padding holds zeros (m = 0).
//
// The matmul (dr_gemv) gives each 32-column output tile one workgroup of `chunks` wavefronts; wavefront w sums the
// tile's panels over one K chunk, and the chunks' partial sums are added in chunk order. The split depends on K only,
// so every weight of one K sees the same sums in the same order: a block list equals one call per block bit for bit,
// and repeated calls are bit-identical. Decode stays in registers: the block-float exponent of (k, panel) is folded
// into x once per (k, panel) -- x * 2^(E - bias) is exact -- and broadcast across the 16 lanes of a row with DPP
// row_newbcast, so each weight value costs one convert and one FMA (bfp8), or, for bfp4, half a byte permute and half
// a bf16 dot2 against bf16 values 136 + m whose 136 * sum(x') is subtracted once.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dense_reader.h"

namespace {

constexpr int KALIGN = 128;  // K padding: a multiple of every format's k-block
constexpr int MAXCH = 16;    // chunks (wavefronts) per output tile at most
constexpr int TILE = 32;

__host__ __device__ constexpr int kblk(int fmt) { return fmt == DR_BFP8 ? 64 : (fmt == DR_BFP4 ? 128 : 32); }

typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;

__device__ __forceinline__ float bf16_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// fp32 -> bf16 bits, round to nearest even; a NaN becomes the quiet NaN 0x7FC0
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

template <int I>
__device__ __forceinline__ float row_bcast(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x150 + I, 0xF, 0xF, false));
}
template <int I>
__device__ __forceinline__ uint32_t row_bcast_u(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x150 + I, 0xF, 0xF, false);
}

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
}

struct SegDev {
    const uint8_t* codes;
    const uint8_t* exps;
    const uint8_t* codes_up;
    const uint8_t* exps_up;
    const void* scale;
    const void* scale_up;
    int fmt, n, n_pad, glu, scale_f32, col0;
    int n_out, tiles, tile_begin;
};

struct Args {
    const uint16_t* x;
    int m, k, k_pad, ldx;
    void* y;
    int ldy, y_f32;
    const uint16_t* res;
    int ldr, res_mode;
    int act;
    int nseg;
    SegDev seg[4];
    uint32_t* rec;
    int tk_k, tk_rows, slot0, n_valid, write_y, tk_fp32, row0;
    long long base;
    int chunks, kch;
};

// ---- the K loop of one wavefront: partial sums of PW panels x MR rows over k-blocks [b0, b1) ----------------------

// bfp8: lane (kq, c) accumulates column c over k = 64 b + 16 kq + i; lane (kq, i) makes x' for that k
template <int MR, int PW>
__device__ __forceinline__ void loop_bfp8(const Args& a, const uint8_t* const* cb, const uint8_t* const* eb, int b0,
                                          int b1, int lane, float (&acc)[PW][MR]) {
    for (int b = b0; b < b1; b += 2) {
        const bool two = b + 1 < b1;
        uint4 c[2][PW];
        int e[2][PW];
        float xv[2][MR];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int bb = (u == 0 || two) ? b + u : b;
#pragma unroll
            for (int q = 0; q < PW; ++q) {
                c[u][q] = *reinterpret_cast<const uint4*>(cb[q] + (size_t)bb * 1024 + lane * 16);
                e[u][q] = eb[q][bb * 64 + lane];
            }
            const int kx = bb * 64 + lane;
#pragma unroll
            for (int m = 0; m < MR; ++m) xv[u][m] = (kx < a.k && m < a.m) ? bf16_to_f32(a.x[(size_t)m * a.ldx + kx]) : 0.f;
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            if (u == 1 && !two) break;
            float xs[PW][MR];
#pragma unroll
            for (int q = 0; q < PW; ++q)
#pragma unroll
                for (int m = 0; m < MR; ++m) xs[q][m] = __builtin_ldexpf(xv[u][m], e[u][q] - 133);
            uint32_t w[PW][4];
#pragma unroll
            for (int q = 0; q < PW; ++q) {
                w[q][0] = c[u][q].x;
                w[q][1] = c[u][q].y;
                w[q][2] = c[u][q].z;
                w[q][3] = c[u][q].w;
            }
#define DR_STEP8(I)                                                                          \
    {                                                                                        \
        _Pragma("unroll") for (int q = 0; q < PW; ++q) {                                     \
            const float f = (float)(int)(signed char)(w[q][(I) / 4] >> (8 * ((I) % 4)));     \
            _Pragma("unroll") for (int m = 0; m < MR; ++m) acc[q][m] =                       \
                __builtin_fmaf(row_bcast<(I)>(xs[q][m]), f, acc[q][m]);                      \
        }                                                                                    \
    }
            DR_STEP8(0) DR_STEP8(1) DR_STEP8(2) DR_STEP8(3) DR_STEP8(4) DR_STEP8(5) DR_STEP8(6) DR_STEP8(7)
            DR_STEP8(8) DR_STEP8(9) DR_STEP8(10) DR_STEP8(11) DR_STEP8(12) DR_STEP8(13) DR_STEP8(14) DR_STEP8(15)
#undef DR_STEP8
        }
    }
}

// bfp4: lane (kq, c) accumulates column c over k = 128 b + 32 kq + j (j < 32); lane (kq, i) makes the bf16 pair x'
// for k = 128 b + 32 kq + 2i, +1. Weight values enter as bf16 136 + m (0x4300 | u), so acc = sum x' (136 + m) and
// sx (per lane, the x' it made) gives the 136 * sum x' to take off.
template <int MR, int PW>
__device__ __forceinline__ void loop_bfp4(const Args& a, const uint8_t* const* cb, const uint8_t* const* eb, int b0,
                                          int b1, int lane, float (&acc)[PW][MR], float (&sx)[PW][MR]) {
    constexpr uint32_t MAGIC = 0x43434343u;
    const int kq = lane >> 4, i = lane & 15;
    for (int b = b0; b < b1; b += 2) {
        const bool two = b + 1 < b1;
        uint4 c[2][PW];
        uint32_t e[2][PW];
        uint32_t xp[2][MR];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int bb = (u == 0 || two) ? b + u : b;
            const int k0 = bb * 128 + kq * 32 + 2 * i;
#pragma unroll
            for (int q = 0; q < PW; ++q) {
                c[u][q] = *reinterpret_cast<const uint4*>(cb[q] + (size_t)bb * 1024 + lane * 16);
                e[u][q] = *reinterpret_cast<const uint16_t*>(eb[q] + k0);
            }
#pragma unroll
            for (int m = 0; m < MR; ++m)
                xp[u][m] = (k0 < a.k && m < a.m) ? *reinterpret_cast<const uint32_t*>(a.x + (size_t)m * a.ldx + k0) : 0u;
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            if (u == 1 && !two) break;
            uint32_t xs[PW][MR];
#pragma unroll
            for (int q = 0; q < PW; ++q)
#pragma unroll
                for (int m = 0; m < MR; ++m) {
                    const float f0 = __builtin_ldexpf(bf16_to_f32(xp[u][m] & 0xFFFFu), (int)(e[u][q] & 0xFFu) - 129);
                    const float f1 = __builtin_ldexpf(bf16_to_f32(xp[u][m] >> 16), (int)(e[u][q] >> 8) - 129);
                    // exact: x has 8 significant bits, the power of two keeps them (a denormal result may lose
                    // some; sx then takes the same truncated values the dot products see)
                    const uint32_t p = (__float_as_uint(f0) >> 16) | (__float_as_uint(f1) & 0xFFFF0000u);
                    xs[q][m] = p;
                    sx[q][m] += bf16_to_f32(p & 0xFFFFu) + bf16_to_f32(p >> 16);
                }
#define DR_STEP4(D)                                                                                    \
    {                                                                                                  \
        _Pragma("unroll") for (int q = 0; q < PW; ++q) {                                               \
            const uint32_t w = (D) == 0 ? c[u][q].x : (D) == 1 ? c[u][q].y : (D) == 2 ? c[u][q].z : c[u][q].w; \
            const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;                          \
            const uint32_t a0 = __builtin_amdgcn_perm(MAGIC, lo, 0x04010400u);                         \
            const uint32_t a1 = __builtin_amdgcn_perm(MAGIC, lo, 0x04030402u);                         \
            const uint32_t a2 = __builtin_amdgcn_perm(MAGIC, hi, 0x04010400u);                         \
            const uint32_t a3 = __builtin_amdgcn_perm(MAGIC, hi, 0x04030402u);                         \
            _Pragma("unroll") for (int m = 0; m < MR; ++m) {                                           \
                acc[q][m] = dot2(a0, row_bcast_u<4 * (D) + 0>(xs[q][m]), acc[q][m]);                   \
                acc[q][m] = dot2(a1, row_bcast_u<4 * (D) + 1>(xs[q][m]), acc[q][m]);                   \
                acc[q][m] = dot2(a2, row_bcast_u<4 * (D) + 2>(xs[q][m]), acc[q][m]);                   \
                acc[q][m] = dot2(a3, row_bcast_u<4 * (D) + 3>(xs[q][m]), acc[q][m]);                   \
            }                                                                                          \
        }                                                                                              \
    }
            DR_STEP4(0) DR_STEP4(1) DR_STEP4(2) DR_STEP4(3)
#undef DR_STEP4
        }
    }
}

// bf16: lane (kq, c) accumulates column c over k = 32 b + 8 kq + j; x pairs are read as they are (the 16 lanes of a
// row read the same 16 bytes)
template <int MR, int PW>
__device__ __forceinline__ void loop_bf16(const Args& a, const uint8_t* const* cb, int b0, int b1, int lane,
                                          float (&acc)[PW][MR]) {
    const int kq = lane >> 4;
    for (int b = b0; b < b1; b += 2) {
        const bool two = b + 1 < b1;
        uint4 c[2][PW];
        uint4 xq[2][MR];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int bb = (u == 0 || two) ? b + u : b;
#pragma unroll
            for (int q = 0; q < PW; ++q) c[u][q] = *reinterpret_cast<const uint4*>(cb[q] + (size_t)bb * 1024 + lane * 16);
            const int k0 = bb * 32 + kq * 8;
#pragma unroll
            for (int m = 0; m < MR; ++m)
                xq[u][m] = (k0 < a.k && m < a.m) ? *reinterpret_cast<const uint4*>(a.x + (size_t)m * a.ldx + k0)
                                                 : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            if (u == 1 && !two) break;
#pragma unroll
            for (int q = 0; q < PW; ++q)
#pragma unroll
                for (int m = 0; m < MR; ++m) {
                    float s = acc[q][m];
                    s = dot2(c[u][q].x, xq[u][m].x, s);
                    s = dot2(c[u][q].y, xq[u][m].y, s);
                    s = dot2(c[u][q].z, xq[u][m].z, s);
                    s = dot2(c[u][q].w, xq[u][m].w, s);
                    acc[q][m] = s;
                }
        }
    }
}

__device__ __forceinline__ float load_scale(const void* s, int f32, int col) {
    if (s == nullptr) return 1.f;
    return f32 ? reinterpret_cast<const float*>(s)[col] : bf16_to_f32(reinterpret_cast<const uint16_t*>(s)[col]);
}

__device__ __forceinline__ float act_glu(float g, int act) {
    // silu(g) = g * sigmoid(g); gelu_tanh(g) = g * sigmoid(1.5957691216 g + 0.0713548162 g^3) (dense_ops.h:46-59)
    const float z = act == 1 ? g * (1.5957691216f + 0.0713548162f * (g * g)) : g;
    return g / (1.f + __expf(-z));
}

// the reference's top-k key of a bf16 (dense_writer.cpp:215): a monotonic uint16, 0 below everything
__device__ __forceinline__ uint32_t key_bf16(uint32_t b) { return b ^ (0x8000u | (0x7FFFu & (0u - (b >> 15)))); }
__device__ __forceinline__ uint32_t key_f32(float f) {
    const uint32_t u = __float_as_uint(f);
    return u ^ ((u >> 31) ? 0xFFFFFFFFu : 0x80000000u);
}

template <int MR, int PW>
__global__ __launch_bounds__(1024) void dr_gemv(const Args a) {
    __shared__ float part[MAXCH][PW][MR][16];
    __shared__ float tval[MR][TILE];
    __shared__ uint32_t tkey[MR][TILE];

    const int g = blockIdx.x;
    int s = 0;
#pragma unroll
    for (int j = 1; j < 4; ++j)
        if (j < a.nseg && g >= a.seg[j].tile_begin) s = j;
    const SegDev& sg = a.seg[s];
    const int t = g - sg.tile_begin;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int fmt = sg.fmt;
    const int nkb = a.k_pad / kblk(fmt);
    const size_t pstride = (size_t)nkb * 1024;

    const uint8_t* cb[PW];
    const uint8_t* eb[PW];
#pragma unroll
    for (int q = 0; q < PW; ++q) {
        int p;
        const uint8_t* cbase = sg.codes;
        const uint8_t* ebase = sg.exps;
        if (PW == 2) {
            p = 2 * t + q;
        } else if (sg.glu == 1) {
            p = 4 * t + q;  // interleave_glu: gate tile 2t, up tile 2t + 1
        } else {
            p = 2 * t + (q & 1);
            if (q >= 2) {
                cbase = sg.codes_up;
                ebase = sg.exps_up;
            }
        }
        cb[q] = cbase + (size_t)p * pstride;
        eb[q] = ebase + (size_t)p * a.k_pad;
    }

    float acc[PW][MR], corr[PW][MR];
#pragma unroll
    for (int q = 0; q < PW; ++q)
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[q][m] = corr[q][m] = 0.f;

    const int kb = kblk(fmt);
    const int k0 = wave * a.kch, k1 = min(k0 + a.kch, a.k_pad);
    const int b0 = k0 / kb, b1 = k1 / kb;
    if (fmt == DR_BFP8) {
        loop_bfp8<MR, PW>(a, cb, eb, b0, b1, lane, acc);
    } else if (fmt == DR_BFP4) {
        float sx[PW][MR];
#pragma unroll
        for (int q = 0; q < PW; ++q)
#pragma unroll
            for (int m = 0; m < MR; ++m) sx[q][m] = 0.f;
        loop_bfp4<MR, PW>(a, cb, eb, b0, b1, lane, acc, sx);
        // the wavefront's 136 * sum x' (every lane made distinct x'), taken off every column
#pragma unroll
        for (int q = 0; q < PW; ++q)
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                float v = sx[q][m];
#pragma unroll
                for (int o = 1; o < 64; o <<= 1) v += __shfl_xor(v, o);
                corr[q][m] = 136.f * v;
            }
    } else {
        loop_bf16<MR, PW>(a, cb, b0, b1, lane, acc);
    }

    // the wavefront's column sums: the four quarter-rows of each column, in a fixed order
#pragma unroll
    for (int q = 0; q < PW; ++q)
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            float v = acc[q][m];
            v += __shfl_xor(v, 16);
            v += __shfl_xor(v, 32);
            if (lane < 16) part[wave][q][m][lane] = v - corr[q][m];
        }
    __syncthreads();

    // the epilogue: thread (m, col) of the 32-column output tile
    const int tid = threadIdx.x;
    const int mrows = min(a.m, MR);
    const bool topk = a.rec != nullptr;
    for (int e = tid; e < TILE * MR; e += blockDim.x) {
        const int m = e / TILE, col = e % TILE;
        const int oc = t * TILE + col;  // output column of this segment
        const bool valid = m < mrows && oc < sg.n_out;
        float v = 0.f;
        const int cq = col >> 4, cc = col & 15;
        if (PW == 4) {
            float gsum = 0.f, usum = 0.f;
            for (int w = 0; w < a.chunks; ++w) {
                gsum += part[w][cq][m][cc];
                usum += part[w][2 + cq][m][cc];
            }
            float sgv = 1.f, suv = 1.f;
            if (valid) {
                if (sg.glu == 1) {
                    sgv = load_scale(sg.scale, sg.scale_f32, 2 * t * TILE + col);
                    suv = load_scale(sg.scale, sg.scale_f32, 2 * t * TILE + TILE + col);
                } else {
                    sgv = load_scale(sg.scale, sg.scale_f32, oc);
                    suv = load_scale(sg.scale_up, sg.scale_f32, oc);
                }
            }
            v = act_glu(gsum * sgv, a.act) * (usum * suv);
        } else {
            const size_t ycol = (size_t)sg.col0 + oc;
            if (valid && a.res != nullptr && a.res_mode == 2) v = bf16_to_f32(a.res[(size_t)m * a.ldr + ycol]);
            for (int w = 0; w < a.chunks; ++w) v += part[w][cq][m][cc];
            if (valid) {
                v *= load_scale(sg.scale, sg.scale_f32, oc);
                if (a.res != nullptr && a.res_mode == 1) v += bf16_to_f32(a.res[(size_t)m * a.ldr + ycol]);
            }
        }
        float out = v;
        uint32_t ob = 0;
        if (!a.y_f32) {
            ob = f32_to_bf16(v);
            out = bf16_to_f32(ob);
        }
        if (valid && (!topk || a.write_y)) {
            const size_t idx = (size_t)m * a.ldy + sg.col0 + oc;
            if (a.y_f32)
                reinterpret_cast<float*>(a.y)[idx] = v;
            else
                reinterpret_cast<uint16_t*>(a.y)[idx] = (uint16_t)ob;
        }
        if (topk) {
            const bool in = valid && oc < a.n_valid;
            tval[m][col] = a.tk_fp32 ? v : out;
            tkey[m][col] = !in ? 0u : (a.tk_fp32 ? key_f32(v) : key_bf16(ob));
            if (a.tk_fp32 && !in) tkey[m][col] = 0u;
        }
    }
    if (!topk) return;
    __syncthreads();
    // one wavefront ranks each row's 32 keys: the best k, highest first, ties to the lower column
    if (wave == 0) {
        const int K = a.tk_k, R = a.tk_rows;
        const size_t rlen = 2 * (size_t)R * K;
        uint32_t* rec = a.rec + (size_t)(a.slot0 + t) * rlen;
        for (int m = 0; m < mrows; ++m) {
            const int r = a.row0 + m;
            if (r >= R) break;
            const int c = lane & 31;
            const uint32_t key = tkey[m][c];
            int rank = 0, nval = 0;
            for (int j = 0; j < TILE; ++j) {
                const uint32_t kj = tkey[m][j];
                nval += kj != 0u;
                rank += (kj > key) || (kj == key && j < c);
            }
            if (lane < 32 && key != 0u && rank < K) {
                const float val = tval[m][c];
                rec[(size_t)r * K + rank] = a.tk_fp32 ? __float_as_uint(val) : key;
                rec[(size_t)R * K + (size_t)r * K + rank] = (uint32_t)(a.base + (long long)t * TILE + c);
            }
            if (lane >= nval && lane < K) {
                rec[(size_t)r * K + lane] = a.tk_fp32 ? 0xFF800000u : 0u;
                rec[(size_t)R * K + (size_t)r * K + lane] = 0xFFFFFFFFu;
            }
        }
    }
}

// ---- packing ---------------------------------------------------------------------------------------------------------

// one face row (16 columns at one k) to block-float: the shared exponent is the largest biased fp32 exponent; each
// value's 24-bit mantissa (hidden bit set) is shifted down by its exponent's distance from it (to 0 past 31), rounded
// to MB bits, ties to even (bits shifted out first are not sticky), at most 2^MB - 1; a zero or denormal value is 0;
// the sign stays only on a non-zero magnitude (moe/moe8.py:117-154, the bfloat4_b case, MB 3; bfloat8_b is MB 7)
template <int MB>
__device__ __forceinline__ uint32_t bfp_face_row(const float (&v)[16], int (&sm)[16]) {
    uint32_t shared = 0;
#pragma unroll
    for (int c = 0; c < 16; ++c) shared = max(shared, (__float_as_uint(v[c]) >> 23) & 0xFFu);
    constexpr int SHIFT = 24 - MB;
#pragma unroll
    for (int c = 0; c < 16; ++c) {
        const uint32_t bits = __float_as_uint(v[c]);
        const uint32_t ex = (bits >> 23) & 0xFFu;
        const uint32_t man = (bits & 0x7FFFFFu) | 0x800000u;
        const uint32_t diff = shared - ex;
        uint32_t m = diff > 31 ? 0u : (man >> diff);
        const uint32_t rnd = m & ((1u << SHIFT) - 1u);
        m >>= SHIFT;
        const uint32_t tie = 1u << (SHIFT - 1);
        m += (rnd > tie) || (rnd == tie && (m & 1u));
        m = min(m, (1u << MB) - 1u);
        if (ex == 0) m = 0;
        const int sgn = (m != 0) && (bits >> 31);
        sm[c] = sgn ? -(int)m : (int)m;
    }
    return shared;
}

__device__ __forceinline__ uint32_t bf16_rne_bits(float f) { return f32_to_bf16(f); }

template <int FMT>
__global__ __launch_bounds__(256) void dr_pack_k(const float* __restrict__ w, long long ld_w, int n, int k,
                                                 const float* __restrict__ cdiv, uint8_t* __restrict__ codes,
                                                 uint8_t* __restrict__ exps, int n_pad, int k_pad) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const int kgroups = k_pad / 8;
    const long long total = (long long)(n_pad / 16) * kgroups;
    if (idx >= total) return;
    const int p = (int)(idx / kgroups), kg = (int)(idx % kgroups);
    const int nkb = k_pad / kblk(FMT);
    const int kk0 = kg * 8;
    float v[8][16];
#pragma unroll
    for (int c = 0; c < 16; ++c) {
        const int col = p * 16 + c;
        const float d = (cdiv != nullptr && col < n) ? cdiv[col] : 1.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int kk = kk0 + i;
            float x = (col < n && kk < k) ? w[(long long)col * ld_w + kk] : 0.f;
            if (cdiv != nullptr && col < n) x = x / d;
            v[i][c] = x;
        }
    }
    uint8_t* pbase = codes + (size_t)p * nkb * 1024;
    if (FMT == DR_BF16) {
        const int b = kk0 / 32, kq = (kk0 % 32) / 8;
#pragma unroll
        for (int c = 0; c < 16; ++c) {
            uint32_t h[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) h[i] = bf16_rne_bits(v[i][c]);
            const uint4 o = make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16));
            *reinterpret_cast<uint4*>(pbase + (size_t)b * 1024 + (kq * 16 + c) * 16) = o;
        }
        return;
    }
    int sm[8][16];
    uint32_t ex[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) ex[i] = bfp_face_row<FMT == DR_BFP8 ? 7 : 3>(v[i], sm[i]);
    *reinterpret_cast<uint2*>(exps + (size_t)p * k_pad + kk0) =
        make_uint2(ex[0] | (ex[1] << 8) | (ex[2] << 16) | (ex[3] << 24), ex[4] | (ex[5] << 8) | (ex[6] << 16) | (ex[7] << 24));
    if (FMT == DR_BFP8) {
        const int b = kk0 / 64, kq = (kk0 % 64) / 16, off = kk0 % 16;
#pragma unroll
        for (int c = 0; c < 16; ++c) {
            uint32_t lo = 0, hi = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                lo |= ((uint32_t)sm[i][c] & 0xFFu) << (8 * i);
                hi |= ((uint32_t)sm[4 + i][c] & 0xFFu) << (8 * i);
            }
            *reinterpret_cast<uint2*>(pbase + (size_t)b * 1024 + (kq * 16 + c) * 16 + off) = make_uint2(lo, hi);
        }
    } else {
        const int b = kk0 / 128, kq = (kk0 % 128) / 32, d = (kk0 % 32) / 8;
#pragma unroll
        for (int c = 0; c < 16; ++c) {
            uint32_t word = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t ulo = (uint32_t)(sm[j][c] + 8), uhi = (uint32_t)(sm[4 + j][c] + 8);
                word |= (ulo | (uhi << 4)) << (8 * j);
            }
            *reinterpret_cast<uint32_t*>(pbase + (size_t)b * 1024 + (kq * 16 + c) * 16 + d * 4) = word;
        }
    }
}

template <int FMT>
__global__ __launch_bounds__(256) void dr_unpack_k(const uint8_t* __restrict__ codes, const uint8_t* __restrict__ exps,
                                                   int n, int k, int k_pad, float* __restrict__ out, long long ld_out) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long long)n * k) return;
    const int kk = (int)(idx / n), col = (int)(idx % n);
    const int p = col / 16, c = col % 16;
    const int nkb = k_pad / kblk(FMT);
    const uint8_t* pbase = codes + (size_t)p * nkb * 1024;
    float val;
    if (FMT == DR_BF16) {
        const int b = kk / 32, kq = (kk % 32) / 8, i = kk % 8;
        const uint16_t h = *reinterpret_cast<const uint16_t*>(pbase + (size_t)b * 1024 + (kq * 16 + c) * 16 + 2 * i);
        val = bf16_to_f32(h);
    } else {
        const int e = exps[(size_t)p * k_pad + kk];
        int m;
        if (FMT == DR_BFP8) {
            const int b = kk / 64, kq = (kk % 64) / 16, i = kk % 16;
            m = (int)(signed char)pbase[(size_t)b * 1024 + (kq * 16 + c) * 16 + i];
            val = __builtin_ldexpf((float)m, e - 133);
        } else {
            const int b = kk / 128, kq = (kk % 128) / 32, d = (kk % 32) / 8, j = kk % 8;
            const uint8_t byte = pbase[(size_t)b * 1024 + (kq * 16 + c) * 16 + d * 4 + (j & 3)];
            m = (int)((j < 4 ? byte : (byte >> 4)) & 15) - 8;
            val = __builtin_ldexpf((float)m, e - 129);
        }
    }
    out[(long long)kk * ld_out + col] = val;
}

// ---- top-k merge -----------------------------------------------------------------------------------------------------

constexpr int MERGE_T = 128;
constexpr int MERGE_MAXK = 64;

__global__ __launch_bounds__(MERGE_T) void dr_merge_k(const uint32_t* __restrict__ rec, int nrec, int rows, int k,
                                                      int fp32, int kout, float* __restrict__ vals,
                                                      int32_t* __restrict__ ids) {
    extern __shared__ unsigned long long lst[];  // [MERGE_T][kout]
    __shared__ unsigned long long best[MERGE_T];
    __shared__ int who[MERGE_T];
    const int r = blockIdx.x, tid = threadIdx.x;
    unsigned long long* mine = lst + (size_t)tid * kout;
    for (int j = 0; j < kout; ++j) mine[j] = 0ull;
    const size_t rlen = 2 * (size_t)rows * k;
    const long long total = (long long)nrec * k;
    for (long long cidx = tid; cidx < total; cidx += MERGE_T) {
        const long long ri = cidx / k;
        const int j = (int)(cidx % k);
        const uint32_t key = rec[ri * rlen + (size_t)r * k + j];
        const uint32_t id = rec[ri * rlen + (size_t)rows * k + (size_t)r * k + j];
        unsigned long long comp;
        if (id == 0xFFFFFFFFu || (!fp32 && key == 0u)) {
            comp = 0ull;
        } else {
            const uint32_t ok = fp32 ? key_f32(__uint_as_float(key)) : key;
            comp = ((unsigned long long)ok << 32) | (unsigned long long)(0xFFFFFFFFu - id);
        }
        if (comp <= mine[kout - 1]) continue;
        int pos = kout - 1;
        while (pos > 0 && mine[pos - 1] < comp) {
            mine[pos] = mine[pos - 1];
            --pos;
        }
        mine[pos] = comp;
    }
    int head = 0;
    for (int o = 0; o < kout; ++o) {
        best[tid] = head < kout ? mine[head] : 0ull;
        who[tid] = tid;
        __syncthreads();
        for (int st = MERGE_T / 2; st > 0; st >>= 1) {
            if (tid < st) {
                const unsigned long long a = best[tid], b = best[tid + st];
                if (b > a || (b == a && who[tid + st] < who[tid])) {
                    best[tid] = b;
                    who[tid] = who[tid + st];
                }
            }
            __syncthreads();
        }
        const unsigned long long w = best[0];
        const int wt = who[0];
        if (tid == 0) {
            if (w == 0ull) {
                vals[(size_t)r * kout + o] = -__builtin_huge_valf();
                ids[(size_t)r * kout + o] = -1;
            } else {
                const uint32_t ok = (uint32_t)(w >> 32);
                const uint32_t id = 0xFFFFFFFFu - (uint32_t)(w & 0xFFFFFFFFu);
                float val;
                if (fp32) {
                    val = __uint_as_float((ok >> 31) ? (ok ^ 0x80000000u) : ~ok);
                } else {
                    const uint32_t bits = ok >= 0x8000u ? (ok & 0x7FFFu) : (~ok & 0xFFFFu);
                    val = __uint_as_float(bits << 16);
                }
                vals[(size_t)r * kout + o] = val;
                ids[(size_t)r * kout + o] = (int32_t)id;
            }
        }
        __syncthreads();
        if (tid == wt && w != 0ull) ++head;
        __syncthreads();
    }
}

inline hipStream_t S(void* s) { return reinterpret_cast<hipStream_t>(s); }

int hip_status(hipError_t e) { return e == hipSuccess ? DR_OK : DR_EHIP; }

void plan(int k, int* chunks, int* kch) {
    const int k_pad = (k + KALIGN - 1) / KALIGN * KALIGN;
    int c = (k_pad + 255) / 256;
    if (c > MAXCH) c = MAXCH;
    int ch = (k_pad + c - 1) / c;
    ch = (ch + KALIGN - 1) / KALIGN * KALIGN;
    *kch = ch;
    *chunks = (k_pad + ch - 1) / ch;
}

int rows_per_pass(int m) { return m <= 1 ? 1 : m <= 2 ? 2 : m <= 4 ? 4 : 8; }

template <int MR>
hipError_t launch_mr(const Args& a, int pw, int grid, hipStream_t st) {
    if (pw == 2)
        hipLaunchKernelGGL((dr_gemv<MR, 2>), dim3(grid), dim3(64 * a.chunks), 0, st, a);
    else
        hipLaunchKernelGGL((dr_gemv<MR, 4>), dim3(grid), dim3(64 * a.chunks), 0, st, a);
    return hipGetLastError();
}

}  // namespace

extern "C" {

int64_t dr_codes_bytes(int fmt, int k_pad, int n_pad) {
    const int64_t v = (int64_t)k_pad * n_pad;
    return fmt == DR_BFP8 ? v : fmt == DR_BFP4 ? v / 2 : 2 * v;
}

int64_t dr_exps_bytes(int fmt, int k_pad, int n_pad) { return fmt == DR_BF16 ? 0 : (int64_t)k_pad * n_pad / 16; }

int dr_pack(const float* w, int64_t ld_w, int n, int k, int fmt, const float* col_div, void* codes, void* exps,
            int n_pad, int k_pad, void* stream) {
    if (w == nullptr || codes == nullptr || n <= 0 || k <= 0 || n_pad < n || n_pad % 32 || k_pad < k ||
        k_pad % KALIGN || ld_w < k || (fmt != DR_BF16 && exps == nullptr) || fmt < 0 || fmt > 2)
        return DR_EINVAL;
    const long long total = (long long)(n_pad / 16) * (k_pad / 8);
    const int grid = (int)((total + 255) / 256);
    auto* c8 = reinterpret_cast<uint8_t*>(codes);
    auto* e8 = reinterpret_cast<uint8_t*>(exps);
    if (fmt == DR_BFP8)
        hipLaunchKernelGGL(dr_pack_k<DR_BFP8>, dim3(grid), dim3(256), 0, S(stream), w, (long long)ld_w, n, k, col_div, c8, e8, n_pad, k_pad);
    else if (fmt == DR_BFP4)
        hipLaunchKernelGGL(dr_pack_k<DR_BFP4>, dim3(grid), dim3(256), 0, S(stream), w, (long long)ld_w, n, k, col_div, c8, e8, n_pad, k_pad);
    else
        hipLaunchKernelGGL(dr_pack_k<DR_BF16>, dim3(grid), dim3(256), 0, S(stream), w, (long long)ld_w, n, k, col_div, c8, e8, n_pad, k_pad);
    return hip_status(hipGetLastError());
}

int dr_unpack(const void* codes, const void* exps, int fmt, int n, int k, int n_pad, int k_pad, float* out,
              int64_t ld_out, void* stream) {
    if (codes == nullptr || out == nullptr || n <= 0 || k <= 0 || n > n_pad || k > k_pad || k_pad % KALIGN ||
        n_pad % 32 || ld_out < n || (fmt != DR_BF16 && exps == nullptr) || fmt < 0 || fmt > 2)
        return DR_EINVAL;
    const long long total = (long long)n * k;
    const int grid = (int)((total + 255) / 256);
    auto* c8 = reinterpret_cast<const uint8_t*>(codes);
    auto* e8 = reinterpret_cast<const uint8_t*>(exps);
    if (fmt == DR_BFP8)
        hipLaunchKernelGGL(dr_unpack_k<DR_BFP8>, dim3(grid), dim3(256), 0, S(stream), c8, e8, n, k, k_pad, out, (long long)ld_out);
    else if (fmt == DR_BFP4)
        hipLaunchKernelGGL(dr_unpack_k<DR_BFP4>, dim3(grid), dim3(256), 0, S(stream), c8, e8, n, k, k_pad, out, (long long)ld_out);
    else
        hipLaunchKernelGGL(dr_unpack_k<DR_BF16>, dim3(grid), dim3(256), 0, S(stream), c8, e8, n, k, k_pad, out, (long long)ld_out);
    return hip_status(hipGetLastError());
}

int dr_plan(int k, int m, int32_t* chunks, int32_t* kch, int32_t* rpp) {
    if (k <= 0 || m <= 0) return DR_EINVAL;
    int c, ch;
    plan(k, &c, &ch);
    if (chunks) *chunks = c;
    if (kch) *kch = ch;
    if (rpp) *rpp = rows_per_pass(m);
    return DR_OK;
}

int dr_matmul(const dr_launch* L) {
    if (L == nullptr || L->x == nullptr || L->y == nullptr || L->m <= 0 || L->k <= 0 || L->k % 32 ||
        L->ldx < L->k || L->nseg < 1 || L->nseg > 4)
        return DR_EINVAL;
    Args a{};
    a.x = reinterpret_cast<const uint16_t*>(L->x);
    a.m = L->m;
    a.k = L->k;
    a.k_pad = (L->k + KALIGN - 1) / KALIGN * KALIGN;
    a.ldx = L->ldx;
    a.y = L->y;
    a.ldy = L->ldy;
    a.y_f32 = L->y_f32 != 0;
    a.res = reinterpret_cast<const uint16_t*>(L->residual);
    a.ldr = L->ldr;
    a.res_mode = L->residual ? (L->residual_mode == 2 ? 2 : 1) : 0;
    a.act = L->act;
    if (a.act != 0 && a.act != 1) return DR_EINVAL;
    a.nseg = L->nseg;
    const int pw = L->seg[0].glu ? 4 : 2;
    int tiles = 0;
    for (int i = 0; i < L->nseg; ++i) {
        const dr_segment& s = L->seg[i];
        SegDev& d = a.seg[i];
        if (s.fmt < 0 || s.fmt > 2 || s.n <= 0 || s.n_pad < s.n || s.n_pad % 32 || s.col0 < 0 || s.col0 % 32 ||
            s.codes == nullptr || (s.fmt != DR_BF16 && s.exps == nullptr) || s.glu < 0 || s.glu > 2 ||
            (s.glu ? 4 : 2) != pw)
            return DR_EINVAL;
        if (s.glu == 1 && s.n % 64) return DR_EINVAL;
        if (s.glu == 2 && (s.codes_up == nullptr || (s.fmt != DR_BF16 && s.exps_up == nullptr))) return DR_EINVAL;
        d.codes = reinterpret_cast<const uint8_t*>(s.codes);
        d.exps = reinterpret_cast<const uint8_t*>(s.exps);
        d.codes_up = reinterpret_cast<const uint8_t*>(s.codes_up);
        d.exps_up = reinterpret_cast<const uint8_t*>(s.exps_up);
        d.scale = s.scale;
        d.scale_up = s.scale_up;
        d.fmt = s.fmt;
        d.n = s.n;
        d.n_pad = s.n_pad;
        d.glu = s.glu;
        d.scale_f32 = s.scale_f32 != 0;
        d.col0 = s.col0;
        d.n_out = s.glu == 1 ? s.n / 2 : s.n;
        d.tiles = (d.n_out + TILE - 1) / TILE;
        d.tile_begin = tiles;
        tiles += d.tiles;
        if ((int64_t)s.col0 + d.n_out > L->ldy) return DR_EINVAL;
    }
    if (a.res != nullptr && (L->ldr < a.seg[0].col0 + a.seg[0].n_out || L->nseg != 1 || pw != 2)) return DR_EINVAL;
    const dr_topk& T = L->topk;
    a.rec = reinterpret_cast<uint32_t*>(T.records);
    if (a.rec != nullptr) {
        if (T.k < 1 || T.k > 32 || T.rows < 1 || T.rows > 32 || T.rows > L->m || T.slot0 < 0 || L->nseg != 1 ||
            pw != 2 || T.slot0 + tiles > T.records_cap || T.n_valid < 0)
            return DR_EINVAL;
        a.tk_k = T.k;
        a.tk_rows = T.rows;
        a.slot0 = T.slot0;
        a.n_valid = T.n_valid;
        a.base = T.base;
        a.write_y = T.write_y != 0;
        a.tk_fp32 = T.fp32 != 0;
    }
    plan(L->k, &a.chunks, &a.kch);
    const int mr = rows_per_pass(L->m);
    hipStream_t st = S(L->stream);
    const size_t ysz = a.y_f32 ? 4 : 2;
    for (int r0 = 0; r0 < L->m; r0 += mr) {
        Args p = a;
        p.m = L->m - r0 < mr ? L->m - r0 : mr;
        p.x = a.x + (size_t)r0 * a.ldx;
        p.y = reinterpret_cast<uint8_t*>(L->y) + (size_t)r0 * a.ldy * ysz;
        if (a.res) p.res = a.res + (size_t)r0 * a.ldr;
        p.row0 = r0;
        if (a.rec != nullptr && r0 >= a.tk_rows && !a.write_y) continue;
        hipError_t e;
        switch (mr) {
            case 1: e = launch_mr<1>(p, pw, tiles, st); break;
            case 2: e = launch_mr<2>(p, pw, tiles, st); break;
            case 4: e = launch_mr<4>(p, pw, tiles, st); break;
            default: e = launch_mr<8>(p, pw, tiles, st); break;
        }
        if (e != hipSuccess) return DR_EHIP;
    }
    return DR_OK;
}

int dr_topk_merge(const void* records, int n_records, int rows, int k, int fp32, int k_out, float* vals,
                  int32_t* ids, void* stream) {
    if (records == nullptr || vals == nullptr || ids == nullptr || n_records < 1 || rows < 1 || k < 1 || k_out < 1 ||
        k_out > MERGE_MAXK)
        return DR_EINVAL;
    const size_t lds = (size_t)MERGE_T * k_out * sizeof(unsigned long long);
    hipLaunchKernelGGL(dr_merge_k, dim3(rows), dim3(MERGE_T), lds, S(stream),
                       reinterpret_cast<const uint32_t*>(records), n_records, rows, k, fp32, k_out, vals, ids);
    return hip_status(hipGetLastError());
}

const char* dr_status_string(int s) {
    switch (s) {
        case DR_OK: return "ok";
        case DR_EINVAL: return "dense_reader: an argument outside what the op takes";
        case DR_EHIP: return "dense_reader: HIP runtime error";
        case DR_ERANGE: return "dense_reader: a size beyond a limit";
        default: return "dense_reader: unknown status";
    }
}

int dr_version(void) { return 1; }

}  // extern "C"
