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
// The exponents sit apart, one byte per (panel, k), panel p at exps + p * k_pad, in groups of 256 k: byte 4 l + j of
// group g is the one lane l needs for the j-th of its four block-float k of that group (bfp8: k = 256 g + 64 j + l;
// bfp4: the pair k = 256 g + 128 (j >> 1) + 32 kq + 2 i + (j & 1), l = 16 kq + i), so a lane reads one dword of
// exponents per 256 k. K is padded to 256 and N to 32 (or what the caller asks); padding holds zeros (m = 0).
//
// The matmul (dr_gemv) gives each 32-column output tile one workgroup. K is cut into chunks of 256 or 512 values (by
// K and the kernel); a wavefront sums the tile's panels over one chunk at a time, with every load of the chunk in
// flight at once, and the chunks' partial sums are added in chunk order. The split depends on K and the kernel only,
// so every weight of one K sees the same sums in the same order: a block list equals one call per block bit for bit,
// and repeated calls are bit-identical. Decode stays in registers: the block-float exponent of (k, panel) is folded
// into x once per (k, panel) -- x * 2^(E - bias) is exact -- and broadcast across the 16 lanes of a row with DPP
// row_newbcast, so each weight value costs one convert and one FMA (bfp8), or, for bfp4, half a byte permute and half
// a bf16 dot2 against bf16 values 136 + m whose 136 * sum(x') is subtracted once.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <stdint.h>

#include "dense_reader.h"
#include "moe.h"
#include "../../moe/csrc/moe_route.h"
#include "wave_select.h"

// No contraction of a multiply and an add into an FMA unless the code asks for one: the compiler would otherwise
// decide per kernel instantiation, and a weight would round differently in a block list than alone.
#pragma clang fp contract(off)

namespace {

constexpr int KALIGN = 256;  // K padding: one exponent group; a multiple of every format's k-block
constexpr int MAXW = 8;      // wavefronts a workgroup at most (512 threads: up to 256 VGPRs a lane)
// The expert-gathered GEMV's down modes: up to 16 wavefronts (1024 threads; those kernels stay under 128 VGPRs). A
// CU's bytes follow the chunks it has in flight: the gpt-oss down (180 workgroups of 24 chunks) 8.0 -> 6.9 us with 16
// wavefronts of one or two chunks against 8 of three (12 of two: 7.5 us).
constexpr int MAXW_DOWN = 16;
constexpr int TILE = 32;

// output columns of a workgroup's tile: 16 (one panel) for a narrow launch (PW = 1), else 32
template <int PW>
__host__ __device__ constexpr int tile_w() {
    return PW == 1 ? 16 : TILE;
}

__host__ __device__ constexpr int kblk(int fmt) {
    return fmt == DR_BFP8 ? 64 : (fmt == DR_BFP4 || fmt == DR_INT4 || fmt == DR_BFP4_KB) ? 128 : 32;
}

// DR_BFP4_KB: the byte of a panel's exponents that holds column c's exponent for k (one a 16-k group): per 128-k block
// 128 bytes, lane (kq, c) of the block's wavefront load at 2 (16 kq + c), its two groups (k 32 kq + 0..15, + 16..31)
__host__ __device__ constexpr int exp_off_kb(int k, int c) {
    return (k >> 7) * 128 + (((k & 127) >> 5) * 16 + c) * 2 + ((k & 31) >> 4);
}

// the byte of a panel's exponents that holds k (see the layout above)
__host__ __device__ constexpr int exp_off(int fmt, int k) {
    const int g = k >> 8, r = k & 255;
    if (fmt == DR_BFP8) return g * 256 + 4 * (r & 63) + (r >> 6);
    const int jb = r >> 7, r2 = r & 127, kq = r2 >> 5, i = (r2 & 31) >> 1, h = r2 & 1;
    return g * 256 + 4 * (16 * kq + i) + 2 * jb + h;
}

typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;

__device__ __forceinline__ float bf16_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// fp32 -> bf16 bits, round to nearest even; a NaN becomes the quiet NaN 0x7FC0
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
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
    const uint16_t* gscale;  // DR_INT4: the group scales [panel][k-block][4][16] bf16
    int fmt, n, n_pad, glu, scale_f32, col0;
    int n_out, tiles, tile_begin;
    unsigned pstride;  // bytes of codes a panel
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
    int tk_group;            // tiles a record (> 1: each tile's record is staged in tstage, dr_group_k ranks groups)
    uint32_t* tstage;        // [tiles][2 * rows * k] (tk_group > 1): each tile's record
    uint32_t* rec_out;       // where tile t's record goes: rec_out + t * 2 * rows * k (the host's choice of the record
                             // slots or the staging: the kernel reads one pointer)
    long long base;
    int chunks, kch, waves;
    int splits, cps, tiles;  // split K: splits workgroups a tile, cps chunks each; tiles of the launch
    uint32_t* counters;      // [tiles] (splits > 1): workgroups of the tile done, reset to 0 by the last
    float* wpart;            // [tiles][splits][PW * ROWS * 16] (splits > 1): each workgroup's column sums
    int pairs;               // > 0: 32-row launch of tile pairs (dr_mfma_pairs), this many workgroups
    int pair_begin[4];       // each segment's first workgroup
    int pair_tiles[4];       // each segment's tiles a workgroup (2, or 1 for bf16)
};

// the expert-gathered launches' arguments (DR_MOE_*): the workgroup's expert (gate/up modes) or each chunk's (down
// modes), read from ids. A struct of their own: the dense kernels keep Args as it is (a larger argument block moved
// the compiler's register choices in the dense K loop).
struct MoeArgs : Args {
    const void* ids;
    int ids32, ld_ids, slots, id_rows, experts;
    const uint16_t* rw;  // routing weights [id_rows][ld_rw] bf16
    int ld_rw;
    int en, tpe;         // gate/up modes: an expert's output columns, its 32-column tiles
    int ek, ekp;         // down modes: an expert's rows (x's block width) and the rows packed (a multiple of 256)
    long long cstride, estride;  // bytes from one expert's codes / exponents to the next
    const uint16_t* bias;        // gate/up modes: [experts][2][en] bf16 (gate, up) or null
    int routed;                  // DR_MOE_GATE_UP: every workgroup routes row 0 of route.logits itself (its ids and w
    moe_route::RouteArgs route;  // are route's outputs, which workgroup 0 writes)
};

// the in-launch routing's experts a lane at most (E <= 256): the router's larger cases would raise the gather kernel's
// registers for every launch
constexpr int ROUTE_MAXPER = 4;

// ---- the K loop of one wavefront: partial sums of PW panels x MR rows over [k0, k1) ------------------------------
//
// k0 and k1 are multiples of 256 (one exponent group: 4 bfp8 blocks, 2 bfp4 blocks, 8 bf16 blocks). Each group's
// loads (PW 16-byte code loads a block, one exponent dword a panel, the x values) are all issued before any of them
// is used and none sits under a branch, so a wavefront has a whole group in flight at once.

// acc += broadcast(s from lane I of this row of 16) * f, one VOP2 with DPP. The VALU write of s must be 2 wait states
// before the DPP read of it: the first use of a fresh s carries an s_nop 1 (NOP = true).
template <int I, bool NOP>
__device__ __forceinline__ void fmac_bcast(float& acc, float s, float f) {
    if constexpr (NOP)
        asm volatile("s_nop 1\n\tv_fmac_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf"
                     : "+v"(acc) : "v"(s), "v"(f), "i"(I));
    else
        asm volatile("v_fmac_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf"
                     : "+v"(acc) : "v"(s), "v"(f), "i"(I));
}

// acc += dot(broadcast(bf16 pair p from lane J of this row of 16), bf16 pair a), one VOP2 with DPP (same hazard rule
// for p). A DOT's result must be 3 wait states before any other VALU instruction reads it (another v_dot2c reading it
// as its accumulator needs none); the compiler sees no DOT in inline asm, so the last dot2c into an accumulator before
// other code reads it carries an s_nop 2 (LAST = true).
template <int J, bool NOP, bool LAST = false>
__device__ __forceinline__ void dot2_bcast(float& acc, uint32_t p, uint32_t a) {
    if constexpr (NOP && LAST)
        asm volatile("s_nop 1\n\tv_dot2c_f32_bf16_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf\n\ts_nop 2"
                     : "+v"(acc) : "v"(p), "v"(a), "i"(J));
    else if constexpr (NOP)
        asm volatile("s_nop 1\n\tv_dot2c_f32_bf16_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf"
                     : "+v"(acc) : "v"(p), "v"(a), "i"(J));
    else if constexpr (LAST)
        asm volatile("v_dot2c_f32_bf16_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf\n\ts_nop 2"
                     : "+v"(acc) : "v"(p), "v"(a), "i"(J));
    else
        asm volatile("v_dot2c_f32_bf16_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf"
                     : "+v"(acc) : "v"(p), "v"(a), "i"(J));
}

// After the last v_dot2c of a run of bfp4_step: every accumulator passes through an empty volatile asm. Volatile asm
// statements keep their order, so no instruction that reads an accumulator can be scheduled before the last dot2c
// and its s_nop 2 (the other accumulators' last dot2c lie at least four dot2c further back); without it the compiler
// may hoist a reader of one accumulator between the dot2c of the others, inside the DOT result's wait states.
template <int PW, int MR>
__device__ __forceinline__ void dot_fence(float (&acc)[PW][MR]) {
#pragma unroll
    for (int q = 0; q < PW; ++q)
#pragma unroll
        for (int m = 0; m < MR; ++m) asm volatile("" : "+v"(acc[q][m]));
}

// a value the compiler cannot see through: masks made with it keep a load unconditional (a known-zero mask lets the
// compiler put the load under a branch, and a load under a branch waits for every load before it)
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
}

// A wave-uniform value made here, in SGPRs: a kernel argument the compiler would otherwise load where it is first
// used (a block list's segment fields, indexed at run time, were three dependent scalar loads at the end of each
// tile-pair workgroup; loaded before the K loop they wait behind nothing).
template <typename T>
__device__ __forceinline__ T pin(T v) {
    asm volatile("" : "+s"(v));
    return v;
}

// the bf16 bits of x[m][k], 0 for a row m or column k outside x (the load is clamped to valid memory, not skipped)
__device__ __forceinline__ uint32_t x_bits(const Args& a, int m, int k) {
    const int mc = min(m, a.m - 1), kc = min(k, a.k - 1);
    const uint32_t v = a.x[(size_t)mc * a.ldx + kc];
    return v & opaque((m < a.m && k < a.k) ? 0xFFFFFFFFu : 0u);
}

// Weight codes, exponents and group scales are read once a launch: non-temporal loads (the nt bit) stream them past
// the caches that x and the partial sums reuse. Measured on MI355X against plain loads: the north-star shape 13.3 ->
// 12.3 us, the bfloat4_b GLU pair 16.7 -> 15.1 us, the MFMA kernel 5 % and the LM head 4 % faster.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_stream16(const uint8_t* p) {
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint32_t ld_stream4(const uint8_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
}

template <int PW>
struct Codes {
    uint4 c[PW];
};

template <int I, int MR, int PW>
__device__ __forceinline__ void bfp8_step(float (&acc)[PW][MR], const float (&xs)[PW][MR], const uint4 (&c)[PW]) {
#pragma unroll
    for (int q = 0; q < PW; ++q) {
        const uint32_t w = I / 4 == 0 ? c[q].x : I / 4 == 1 ? c[q].y : I / 4 == 2 ? c[q].z : c[q].w;
        const float f = (float)(int)(signed char)(w >> (8 * (I % 4)));
#pragma unroll
        for (int m = 0; m < MR; ++m) fmac_bcast<I, I == 0>(acc[q][m], xs[q][m], f);
    }
    if constexpr (I + 1 < 16) bfp8_step<I + 1, MR, PW>(acc, xs, c);
}

// ---- x through LDS: a wavefront's rows over its chunk ---------------------------------------------------------------
//
// A wavefront stages the x its chunk needs (MR rows over 512 k) in an LDS window of its own with one 16-byte load a lane
// a row, instead of one 2-byte load a lane per 64-k block: the block loaders then read x from LDS. (Fewer vector
// memory instructions: in a copy of the north-star GEMV on MI355X the small x loads cost 0.3 us of 11.4.) x rows are
// 16-byte aligned and K is a multiple of 32 (the host checks both), so a lane's 8 values lie wholly inside or wholly
// past K.
constexpr int XWIN = 512;  // k a window holds: the longest chunk
template <int MR>
struct XWin {
    uint4 v[MR];
};
// lane l's 16 bytes of each row: k0 + 8 l .. + 7 (zeros past K or past x's rows)
template <int MR>
__device__ __forceinline__ XWin<MR> x_win_load(const Args& a, int k0, int lane) {
    XWin<MR> w;
    const int k = k0 + 8 * lane, kc = min(k, a.k - 8);
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        const int mc = min(m, a.m - 1);
        const uint4 v = *reinterpret_cast<const uint4*>(a.x + (size_t)mc * a.ldx + kc);
        const uint32_t keep = opaque((k < a.k && m < a.m) ? 0xFFFFFFFFu : 0u);
        w.v[m] = make_uint4(v.x & keep, v.y & keep, v.z & keep, v.w & keep);
    }
    return w;
}
// (LDS instructions of one wavefront execute in order: its later reads see these writes)
template <int MR>
__device__ __forceinline__ void x_win_store(const XWin<MR>& w, uint16_t (*xl)[XWIN], int lane) {
#pragma unroll
    for (int m = 0; m < MR; ++m) *reinterpret_cast<uint4*>(&xl[m][8 * lane]) = w.v[m];
}

// ---- the block loaders: rotated slots, a few in flight ---------------------------------------------------------------
//
// A chunk's blocks are loaded and summed in slots: slot u of panel q holds the chunk's block (u + rot_q) mod nb, with
// rot_q = c + (nb_max / 2) (p_q & 1), c = k0 / the chunk length (the chunk's index) and p_q the panel's index in its
// weight. Rotating by the chunk
// spreads the addresses that the wavefronts of the launch request at one time (the first slot of every wavefront is
// not the first block of every chunk), and the half-turn for odd panels spreads a tile's two panels; on MI355X the
// north-star read went 10.3 -> 10.0 us with that order alone. The slots are summed in slot order, a function of the
// chunk and the panel's parity only, so every launch of a weight sums each column in the same order (block lists,
// 16- and 32-column tiles, split K). The first D slots' codes are issued with x and the exponents; slot u + D's are
// issued before slot u is decoded (scheduling barriers keep that order), so a wavefront keeps D slots in flight
// and its data arrives spread over the launch: with all eight issued at once they landed in one burst, and the last
// wavefronts' whole decode came after the last byte (0.3 us of 11.4 in the copy).
// Slots in flight a wavefront: about 6 KB of bfloat8_b codes or 4 KB of bfloat4_b / int4 codes (a slot is one KB a
// panel). Measured on MI355X (alternating builds in one process): the north star (2 panels) 11.71 / 11.66 / 11.86 us
// with 2 / 3 / 4 slots; the bfloat4_b GLU pair (4 panels) 13.79 / 14.02 / 14.20 / 14.31 us with 1 / 2 / 3 / 4.
template <int PW>
__host__ __device__ constexpr int depth_bfp8() {
    return PW >= 6 ? 1 : 6 / PW;
}
template <int PW>
__host__ __device__ constexpr int depth_bfp4() {
    return PW >= 4 ? 1 : 4 / PW;
}

// bfp8: lane (kq, c) accumulates column c over k = 64 b + 16 kq + i; lane (kq, i) makes x' for that k. One chunk
// [k0, k1) of one or two exponent groups (256 k each). ONEG: every chunk of the launch is one group (256-k chunks), and
// only that group is loaded; otherwise a one-group chunk (the last of a K that is an odd number of groups) loads its
// group twice (the second copy is never used) so that no load sits under a branch.
template <int MR, int PW, bool ONEG = false>
__device__ __forceinline__ void chunk_bfp8(const Args& a, const uint8_t* const* cb, const uint8_t* const* eb,
                                           const int (&par)[PW], int k0, int k1, int lane,
                                           uint16_t (*xl)[XWIN], float (&acc)[PW][MR]) {
    constexpr int NU = ONEG ? 4 : 8;  // 64-k blocks (slots)
    constexpr int D = depth_bfp8<PW>() < NU ? depth_bfp8<PW>() : NU;
    const int g0 = k0 >> 8;
    const bool two = !ONEG && k1 - k0 > 256;
    const int nb = two ? NU : 4;
    int rot[PW];
#pragma unroll
    for (int q = 0; q < PW; ++q) rot[q] = ((k0 >> (ONEG ? 8 : 9)) + (NU / 2) * par[q]) & (nb - 1);
    const XWin<MR> xw = x_win_load<MR>(a, k0, lane);
    uint64_t e[PW];  // the chunk's exponents of panel q: byte j (of 8, or 4) is block j's, for the lane's k
#pragma unroll
    for (int q = 0; q < PW; ++q) {
        const uint32_t lo = ld_stream4(eb[q] + (uint32_t)(g0 * 256 + 4 * lane));
        const uint32_t hi = ld_stream4(eb[q] + (uint32_t)((two ? g0 + 1 : g0) * 256 + 4 * lane));
        e[q] = (uint64_t)lo | ((uint64_t)hi << 32);
    }
    Codes<PW> c[NU];
    auto issue = [&](int u) {
#pragma unroll
        for (int q = 0; q < PW; ++q) {
            const int b = 4 * g0 + ((u + rot[q]) & (nb - 1));
            c[u].c[q] = ld_stream16(cb[q] + (uint32_t)(b * 1024 + lane * 16));
        }
    };
#pragma unroll
    for (int u = 0; u < D; ++u) issue(u);
    x_win_store<MR>(xw, xl, lane);
#pragma unroll
    for (int u = 0; u < NU; ++u) {
        if (u + D < NU) issue(u + D);
        __builtin_amdgcn_sched_barrier(0);
        if (ONEG || u < nb) {
            float xs[PW][MR];
#pragma unroll
            for (int q = 0; q < PW; ++q) {
                const int b = (u + rot[q]) & (nb - 1);
                const int ev = (int)((uint32_t)(e[q] >> (8 * b)) & 0xFFu) - 133;
#pragma unroll
                for (int m = 0; m < MR; ++m) xs[q][m] = __builtin_ldexpf(bf16_to_f32(xl[m][64 * b + lane]), ev);
            }
            bfp8_step<0, MR, PW>(acc, xs, c[u].c);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

// The nibble u = m + 8 enters a dot2c as the bf16 whose high byte is HI and low byte u (u < 16, so the exponent field
// is 2 (HI & 0x7F) and u the mantissa): HI = 0x43 gives 128 + u = 136 + m (x as it is: int4), HI = 0x3F gives
// (128 + u) / 256 (the folded x' of bfloat4_b, which can be as large as the format allows: its products and their
// excess over x' m stay 2^8 further from fp32's overflow), HI = 0x1F gives (128 + u) 2^-72 (the fold of a panel chunk
// of small shared exponents, whose x' carries the 2^64 taken off here).
constexpr uint32_t BF16_136 = 0x43434343u;
constexpr uint32_t BF16_136_256 = 0x3F3F3F3Fu;
constexpr uint32_t BF16_136_2P72 = 0x1F1F1F1Fu;

template <int D, int MR, int PW>
__device__ __forceinline__ void bfp4_step(float (&acc)[PW][MR], const uint32_t (&xs)[PW][MR], const uint4 (&c)[PW],
                                          const uint32_t (&mg)[PW]) {
#pragma unroll
    for (int q = 0; q < PW; ++q) {
        const uint32_t w = D == 0 ? c[q].x : D == 1 ? c[q].y : D == 2 ? c[q].z : c[q].w;
        const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
        // bf16 pairs of panel q's magic byte above u, for k 8D + (0,1), (2,3) (low nibbles) and (4,5), (6,7) (high)
        const uint32_t a0 = __builtin_amdgcn_perm(mg[q], lo, 0x04010400u);
        const uint32_t a1 = __builtin_amdgcn_perm(mg[q], lo, 0x04030402u);
        const uint32_t a2 = __builtin_amdgcn_perm(mg[q], hi, 0x04010400u);
        const uint32_t a3 = __builtin_amdgcn_perm(mg[q], hi, 0x04030402u);
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            dot2_bcast<4 * D + 0, D == 0>(acc[q][m], xs[q][m], a0);
            dot2_bcast<4 * D + 1, false>(acc[q][m], xs[q][m], a1);
            dot2_bcast<4 * D + 2, false>(acc[q][m], xs[q][m], a2);
            // (every other accumulator has at least 4 more dot2c after its last one)
            if (D == 3 && q == PW - 1 && m == MR - 1)
                dot2_bcast<4 * D + 3, false, true>(acc[q][m], xs[q][m], a3);
            else
                dot2_bcast<4 * D + 3, false>(acc[q][m], xs[q][m], a3);
        }
    }
    if constexpr (D + 1 < 4) bfp4_step<D + 1, MR, PW>(acc, xs, c, mg);
}

// the 128-K block whose codes a bfloat4_b decoder loads for block b: b itself, or where b lies wholly in the padding
// past K, the block before it (K pads to a whole 256-K exponent group, so only an odd block can lie past K). x is
// zero past K, so those codes add nothing; loading the other block's bytes, already in flight, reads no padding.
__device__ __forceinline__ int real_block(int b, int k) { return b * 128 >= k ? b - 1 : b; }

// bfp4: lane (kq, c) accumulates column c over k = 128 b + 32 kq + j (j < 32); lane (kq, i) makes the bf16 pair x'
// for k = 128 b + 32 kq + 2i, +1. Weight values enter as the bf16 (136 + m) / 256 (0x3F00 | u), so acc = sum x' (136 +
// m) / 256 and sx (per lane, the x' it made) gives the (136 / 256) sum x' to take off; the caller scales the chunk's
// difference by 256 (exact: the same value, rounded alike, as with the weights 136 + m, until those would overflow).
// One chunk of one or two exponent groups (two blocks each), loaded as chunk_bfp8 loads its chunk.
//
// x' = x 2^(E - 129) is a bf16 denormal, and loses low bits of x, below E + log2|x| = 3. So a panel whose shared
// exponents in the wavefront's chunk are all below 64 folds x' = x 2^(E - 65) instead, a normal bf16 for any |x| above
// 2^-62, against the weights (136 + m) 2^-72: every product is the same value, and sx, the x' sum, is scaled back by
// 2^-64 at the end. For a chunk of normal values the two folds give the same bits (powers of two scale exactly); the
// choice is one ballot a panel, uniform across the wavefront, so every lane of a row sums one kind of x'. A panel chunk
// with an exponent of 64 or more keeps the plain fold: its products then lie at least 2^60 above any that a denormal x'
// could hold.
template <int MR, int PW, bool ONEG = false>
__device__ __forceinline__ void chunk_bfp4(const Args& a, const uint8_t* const* cb, const uint8_t* const* eb,
                                           const int (&par)[PW], int k0, int k1, int lane,
                                           uint16_t (*xl)[XWIN], float (&acc)[PW][MR], float (&sx)[PW][MR]) {
    constexpr int NU = ONEG ? 2 : 4;  // 128-k blocks (slots)
    constexpr int D = depth_bfp4<PW>() < NU ? depth_bfp4<PW>() : NU;
    const int kq = lane >> 4, i = lane & 15;
    const int g0 = k0 >> 8;
    const bool two = !ONEG && k1 - k0 > 256;
    const int nb = two ? NU : 2;
    int rot[PW];
#pragma unroll
    for (int q = 0; q < PW; ++q) rot[q] = ((k0 >> (ONEG ? 8 : 9)) + (NU / 2) * par[q]) & (nb - 1);
    const XWin<MR> xw = x_win_load<MR>(a, k0, lane);
    uint32_t e0[PW], e1[PW];  // the chunk's exponent dwords of panel q: group g0's, group g0 + 1's (or g0's again)
#pragma unroll
    for (int q = 0; q < PW; ++q) {
        e0[q] = ld_stream4(eb[q] + (uint32_t)(g0 * 256 + 4 * lane));
        e1[q] = ld_stream4(eb[q] + (uint32_t)((two ? g0 + 1 : g0) * 256 + 4 * lane));
    }
    Codes<PW> c[NU];
    auto issue = [&](int u) {
#pragma unroll
        for (int q = 0; q < PW; ++q) {
            const int b = real_block(2 * g0 + ((u + rot[q]) & (nb - 1)), a.k);
            c[u].c[q] = ld_stream16(cb[q] + (uint32_t)(b * 1024 + lane * 16));
        }
    };
#pragma unroll
    for (int u = 0; u < D; ++u) issue(u);
    x_win_store<MR>(xw, xl, lane);
    // the fold of each panel: every shared exponent of the chunk below 64 (no byte with either of its top two bits set)
    uint32_t mg[PW];
    int eb0[PW];
    bool small[PW];
#pragma unroll
    for (int q = 0; q < PW; ++q) {
        small[q] = __builtin_amdgcn_ballot_w64(((e0[q] | e1[q]) & 0xC0C0C0C0u) != 0u) == 0ull;
        mg[q] = small[q] ? BF16_136_2P72 : BF16_136_256;
        eb0[q] = small[q] ? 65 : 129;
    }
#pragma unroll
    for (int u = 0; u < NU; ++u) {
        if (u + D < NU) issue(u + D);
        __builtin_amdgcn_sched_barrier(0);
        if (ONEG || u < nb) {
            uint32_t xs[PW][MR];
#pragma unroll
            for (int q = 0; q < PW; ++q) {
                const int b = (u + rot[q]) & (nb - 1);
                const uint32_t ep = ((b >> 1) ? e1[q] : e0[q]) >> (16 * (b & 1));
#pragma unroll
                for (int m = 0; m < MR; ++m) {
                    const uint32_t xp = *reinterpret_cast<const uint32_t*>(&xl[m][128 * b + 32 * kq + 2 * i]);
                    const float f0 = __builtin_ldexpf(bf16_to_f32(xp & 0xFFFFu), (int)(ep & 0xFFu) - eb0[q]);
                    const float f1 = __builtin_ldexpf(bf16_to_f32(xp >> 16), (int)((ep >> 8) & 0xFFu) - eb0[q]);
                    // exact: x has 8 significant bits and a power of two keeps them (a denormal result may lose some;
                    // sx then adds the same truncated values the dot products see)
                    const uint32_t pr = (__float_as_uint(f0) >> 16) | (__float_as_uint(f1) & 0xFFFF0000u);
                    xs[q][m] = pr;
                    sx[q][m] += bf16_to_f32(pr & 0xFFFFu) + bf16_to_f32(pr >> 16);
                }
            }
            bfp4_step<0, MR, PW>(acc, xs, c[u].c, mg);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    dot_fence(acc);
#pragma unroll
    for (int q = 0; q < PW; ++q)
#pragma unroll
        for (int m = 0; m < MR; ++m) sx[q][m] = __builtin_ldexpf(sx[q][m], small[q] ? -64 : 0);
}

// a bfloat4_b chunk's column sum (the wavefront's lanes reduced) less the excess: (acc - (136 / 256) sum x') * 256
__device__ __forceinline__ float bfp4_chunk_sum(float acc, float sx) { return (acc - 0.53125f * sx) * 256.f; }

// DR_BFP4_KB: bfp4_step with the lane's two 16-k exponent groups apart: dwords 0 and 1 (k 0..15 of the lane's 32)
// into t0, dwords 2 and 3 into t1 (the same hazard rules; t0's last dot lies at least eight dot2c before any reader)
template <int D, int MR, int PW>
__device__ __forceinline__ void bfp4k_step(float (&t0)[PW][MR], float (&t1)[PW][MR], const uint32_t (&xs)[PW][MR],
                                           const uint4 (&c)[PW]) {
    constexpr uint32_t MAGIC = 0x43434343u;
#pragma unroll
    for (int q = 0; q < PW; ++q) {
        const uint32_t w = D == 0 ? c[q].x : D == 1 ? c[q].y : D == 2 ? c[q].z : c[q].w;
        const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
        const uint32_t a0 = __builtin_amdgcn_perm(MAGIC, lo, 0x04010400u);
        const uint32_t a1 = __builtin_amdgcn_perm(MAGIC, lo, 0x04030402u);
        const uint32_t a2 = __builtin_amdgcn_perm(MAGIC, hi, 0x04010400u);
        const uint32_t a3 = __builtin_amdgcn_perm(MAGIC, hi, 0x04030402u);
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            float& acc = D < 2 ? t0[q][m] : t1[q][m];
            dot2_bcast<4 * D + 0, D == 0>(acc, xs[q][m], a0);
            dot2_bcast<4 * D + 1, false>(acc, xs[q][m], a1);
            dot2_bcast<4 * D + 2, false>(acc, xs[q][m], a2);
            if (D == 3 && q == PW - 1 && m == MR - 1)
                dot2_bcast<4 * D + 3, false, true>(acc, xs[q][m], a3);
            else
                dot2_bcast<4 * D + 3, false>(acc, xs[q][m], a3);
        }
    }
    if constexpr (D + 1 < 4) bfp4k_step<D + 1, MR, PW>(t0, t1, xs, c);
}

// DR_BFP4_KB, one chunk of up to two exponent groups (4 blocks of 128 k). A lane (kq, c) of a block holds 32
// consecutive k of column c, two exponent groups of 16: its dot products over each group take x as it is (bf16 pairs,
// broadcast across the row of 16 lanes) against the bf16 136 + m; less 136 times the group's x sum (the row's lanes
// 0..7 or 8..15 hold its pairs), times 2^(E - 129) of the lane's group, added to the lane's sum: two FMAs a block.
template <int MR, int PW, bool ONEG = false>
__device__ __forceinline__ void chunk_bfp4k(const Args& a, const uint8_t* const* cb, const uint8_t* const* eb, int k0,
                                            int k1, int lane, float (&acc)[PW][MR]) {
    constexpr int NU = ONEG ? 2 : 4;  // 128-k blocks loaded
    const int kq = lane >> 4, i = lane & 15;
    const int g0 = k0 >> 8;
    const bool two = !ONEG && k1 - k0 > 256;
    const int g1 = two ? g0 + 1 : g0;
    uint32_t xp[NU][MR];
    uint32_t ex[NU][PW];
    Codes<PW> c[NU];
#pragma unroll
    for (int u = 0; u < NU; ++u) {
        const int b = 2 * (u < 2 ? g0 : g1) + (u & 1);
        const int kp = b * 128 + kq * 32 + 2 * i;
        const int kc = min(kp, a.k - 2);
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            const int mc = min(m, a.m - 1);
            const uint32_t v = *reinterpret_cast<const uint32_t*>(a.x + (size_t)mc * a.ldx + kc);
            xp[u][m] = v & opaque((kp < a.k && m < a.m) ? 0xFFFFFFFFu : 0u);
        }
    }
#pragma unroll
    for (int u = 0; u < NU; ++u) {
        const int b = real_block(2 * (u < 2 ? g0 : g1) + (u & 1), a.k);
#pragma unroll
        for (int q = 0; q < PW; ++q)
            ex[u][q] = __builtin_nontemporal_load(reinterpret_cast<const uint16_t*>(eb[q] + (size_t)b * 128) + lane);
    }
#pragma unroll
    for (int u = 0; u < NU; ++u) {
        const int b = real_block(2 * (u < 2 ? g0 : g1) + (u & 1), a.k);
#pragma unroll
        for (int q = 0; q < PW; ++q) c[u].c[q] = ld_stream16(cb[q] + (uint32_t)(b * 1024 + lane * 16));
    }
#pragma unroll
    for (int u = 0; u < NU; ++u) {
        if (u == 2 && !two) break;
        uint32_t xs[PW][MR];
        float rs0[MR], rs1[MR];  // 136 times the row's x sums over the two groups
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            const float v = bf16_to_f32(xp[u][m] & 0xFFFFu) + bf16_to_f32(xp[u][m] >> 16);
            // the sum over this lane's half of the row (lanes 0..7: group 0, 8..15: group 1), then the other half's
            const float mine = wsel::add_xor<4>(wsel::add_xor<2>(wsel::add_xor<1>(v)));
            const float other = __uint_as_float(wsel::dpp_xor<8>(__float_as_uint(mine)));
            rs0[m] = 136.f * (i < 8 ? mine : other);
            rs1[m] = 136.f * (i < 8 ? other : mine);
#pragma unroll
            for (int q = 0; q < PW; ++q) xs[q][m] = xp[u][m];
        }
        float t0[PW][MR], t1[PW][MR];
#pragma unroll
        for (int q = 0; q < PW; ++q)
#pragma unroll
            for (int m = 0; m < MR; ++m) t0[q][m] = t1[q][m] = 0.f;
        bfp4k_step<0, MR, PW>(t0, t1, xs, c[u].c);
        dot_fence(t0);
        dot_fence(t1);
#pragma unroll
        for (int q = 0; q < PW; ++q) {
            const float s0 = __builtin_ldexpf(1.f, (int)(ex[u][q] & 0xFFu) - 129);
            const float s1 = __builtin_ldexpf(1.f, (int)((ex[u][q] >> 8) & 0xFFu) - 129);
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                acc[q][m] = __builtin_fmaf(t0[q][m] - rs0[m], s0, acc[q][m]);
                acc[q][m] = __builtin_fmaf(t1[q][m] - rs1[m], s1, acc[q][m]);
            }
        }
    }
}

// int4 (W4A16): the bfloat4_b code layout with no exponents (every value q = u - 8) and a bf16 scale per column and 32
// k (int4/w4a16.py:1-19). Lane (kq, c)'s 32 k of a block are one scale group, so the lane's block sum is a group sum:
// bf16 dot2 of x pairs (as they are) against 136 + q, less 136 times the row's x sum, times the lane's scale. Loads as
// chunk_bfp4: x first, then the scales, then the codes.
template <int MR, int PW, bool ONEG = false>
__device__ __forceinline__ void chunk_int4(const Args& a, const uint8_t* const* cb, const uint16_t* const* gs,
                                           const int (&par)[PW], int k0, int k1, int lane,
                                           uint16_t (*xl)[XWIN], float (&acc)[PW][MR]) {
    constexpr int NU = ONEG ? 2 : 4;  // 128-k blocks (slots)
    constexpr int D = depth_bfp4<PW>() < NU ? depth_bfp4<PW>() : NU;
    const int kq = lane >> 4, i = lane & 15;
    const int g0 = k0 >> 8;
    const bool two = !ONEG && k1 - k0 > 256;
    const int nb = two ? NU : 2;
    int rot[PW];
#pragma unroll
    for (int q = 0; q < PW; ++q) rot[q] = ((k0 >> (ONEG ? 8 : 9)) + (NU / 2) * par[q]) & (nb - 1);
    const XWin<MR> xw = x_win_load<MR>(a, k0, lane);
    uint32_t sc[NU][PW];
#pragma unroll
    for (int u = 0; u < NU; ++u)
#pragma unroll
        for (int q = 0; q < PW; ++q) {
            const int b = 2 * g0 + ((u + rot[q]) & (nb - 1));
            sc[u][q] = __builtin_nontemporal_load(gs[q] + (size_t)b * 64 + lane);
        }
    Codes<PW> c[NU];
    auto issue = [&](int u) {
#pragma unroll
        for (int q = 0; q < PW; ++q) {
            const int b = 2 * g0 + ((u + rot[q]) & (nb - 1));
            c[u].c[q] = ld_stream16(cb[q] + (uint32_t)(b * 1024 + lane * 16));
        }
    };
#pragma unroll
    for (int u = 0; u < D; ++u) issue(u);
    x_win_store<MR>(xw, xl, lane);
#pragma unroll
    for (int u = 0; u < NU; ++u) {
        if (u + D < NU) issue(u + D);
        __builtin_amdgcn_sched_barrier(0);
        if (ONEG || u < nb) {
            uint32_t xs[PW][MR];
            float rs[PW][MR];  // the row's x sum (the 16 lanes' pairs) of panel q's block: 136 times it is in every dot
#pragma unroll
            for (int q = 0; q < PW; ++q) {
                const int b = (u + rot[q]) & (nb - 1);
#pragma unroll
                for (int m = 0; m < MR; ++m) {
                    const uint32_t xp = *reinterpret_cast<const uint32_t*>(&xl[m][128 * b + 32 * kq + 2 * i]);
                    float v = bf16_to_f32(xp & 0xFFFFu) + bf16_to_f32(xp >> 16);
                    v = wsel::add_xor<8>(wsel::add_xor<4>(wsel::add_xor<2>(wsel::add_xor<1>(v))));  // (over the 16 lanes)
                    rs[q][m] = 136.f * v;
                    xs[q][m] = xp;
                }
            }
            float t[PW][MR];
#pragma unroll
            for (int q = 0; q < PW; ++q)
#pragma unroll
                for (int m = 0; m < MR; ++m) t[q][m] = 0.f;
            uint32_t mg[PW];
#pragma unroll
            for (int q = 0; q < PW; ++q) mg[q] = BF16_136;
            bfp4_step<0, MR, PW>(t, xs, c[u].c, mg);
            dot_fence(t);
#pragma unroll
            for (int q = 0; q < PW; ++q)
#pragma unroll
                for (int m = 0; m < MR; ++m)
                    acc[q][m] = __builtin_fmaf(t[q][m] - rs[q][m], bf16_to_f32(sc[u][q]), acc[q][m]);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

// bf16: lane (kq, c) accumulates column c over k = 32 b + 8 kq + j; x pairs are read as they are (the 16 lanes of a
// row read the same 16 bytes)
template <int MR, int PW>
__device__ __forceinline__ void chunk_bf16(const Args& a, const uint8_t* const* cb, int k0, int k1, int lane,
                                           float (&acc)[PW][MR]) {
    constexpr int G = 8 / PW;  // blocks a group (256 k is 8 blocks: 8 / G groups)
    const int kq = lane >> 4;
    for (int gb = k0 / 32; gb < k1 / 32; gb += G) {
        // x first, then the codes (waits are in issue order)
        uint4 c[G][PW];
        uint4 xq[G][MR];
#pragma unroll
        for (int u = 0; u < G; ++u) {
            const int b = gb + u;
            const int kx = b * 32 + kq * 8;
            const int kc = min(kx, a.k - 8);
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const int mc = min(m, a.m - 1);
                const uint4 v = *reinterpret_cast<const uint4*>(a.x + (size_t)mc * a.ldx + kc);
                const uint32_t keep = opaque((kx < a.k && m < a.m) ? 0xFFFFFFFFu : 0u);
                xq[u][m] = make_uint4(v.x & keep, v.y & keep, v.z & keep, v.w & keep);
            }
        }
#pragma unroll
        for (int u = 0; u < G; ++u)
#pragma unroll
            for (int q = 0; q < PW; ++q)
                c[u][q] = ld_stream16(cb[q] + (uint32_t)((gb + u) * 1024 + lane * 16));
#pragma unroll
        for (int u = 0; u < G; ++u)
#pragma unroll
            for (int q = 0; q < PW; ++q)
#pragma unroll
                for (int m = 0; m < MR; ++m) {
                    float v = acc[q][m];
                    v = dot2(c[u][q].x, xq[u][m].x, v);
                    v = dot2(c[u][q].y, xq[u][m].y, v);
                    v = dot2(c[u][q].z, xq[u][m].z, v);
                    v = dot2(c[u][q].w, xq[u][m].w, v);
                    acc[q][m] = v;
                }
    }
}

__device__ __forceinline__ float load_scale(const void* s, int f32, int col) {
    if (s == nullptr) return 1.f;
    return f32 ? reinterpret_cast<const float*>(s)[col] : bf16_to_f32(reinterpret_cast<const uint16_t*>(s)[col]);
}

// The epilogue's operands from memory (column scales, residual), read before the K loop so that their latency hides
// under it instead of adding to the workgroup's end: thread c < TW (the tile's width) the scales of the tile's output
// column c (gate and up with a GLU), thread e the residual of its first epilogue element (row e / TW, column e % TW).
// After the K loop they go to LDS (pre: [0, TILE) the scale or gate scale, [TILE, 2 TILE) the up scale, from PRE_RES
// the residual by thread), where the epilogue takes them. Only kernels of at most MAXW wavefronts stage into it (the
// 16-wavefront MoE down kernels have no scales or residual and pass no pre).
constexpr int PRE_RES = 2 * TILE;
constexpr int PRE_FLOATS = PRE_RES + 64 * MAXW;

struct EpiPre {
    float sg, su, res;
};

template <int ROWS, int PW>
__device__ __forceinline__ EpiPre epi_prefetch(const Args& a, const SegDev& sg, int t) {
    constexpr int TW = tile_w<PW>();
    EpiPre p{1.f, 1.f, 0.f};
    const int e = threadIdx.x;
    if (e < TW) {
        const int oc = t * TW + e;
        if (oc < sg.n_out) {
            if (PW == 4) {
                if (sg.glu == 1) {
                    p.sg = load_scale(sg.scale, sg.scale_f32, 2 * t * TILE + e);
                    p.su = load_scale(sg.scale, sg.scale_f32, 2 * t * TILE + TILE + e);
                } else {
                    p.sg = load_scale(sg.scale, sg.scale_f32, oc);
                    p.su = load_scale(sg.scale_up, sg.scale_f32, oc);
                }
            } else {
                p.sg = load_scale(sg.scale, sg.scale_f32, oc);
            }
        }
    }
    if (PW <= 2 && a.res != nullptr && e < ROWS * TW) {
        const int m = e / TW, oc = t * TW + e % TW;
        if (m < min(a.m, ROWS) && oc < sg.n_out) p.res = bf16_to_f32(a.res[(size_t)m * a.ldr + sg.col0 + oc]);
    }
    return p;
}

__device__ __forceinline__ void epi_stage(const EpiPre& p, float* pre) {
    const int e = threadIdx.x;
    if (e < TILE) {
        pre[e] = p.sg;
        pre[TILE + e] = p.su;
    }
    pre[PRE_RES + e] = p.res;
}

// the dense GLU's activation: silu(g) = g * sigmoid(g); gelu_tanh(g) = g * sigmoid(1.5957691216 g + 0.0713548162 g^3)
// (dense_ops.h:46-59)
__device__ __forceinline__ float act_glu(float g, int act) {
    const float z = act == DR_ACT_GELU_TANH ? g * (1.5957691216f + 0.0713548162f * (g * g)) : g;
    return g / (1.f + __expf(-z));
}

// the experts' act(g) * u: act_glu's two, or swiglu_oai min(g, 7) * sigmoid(1.702 min(g, 7)) * (clamp(u, -7, 7) + 1)
// (dense_ops.h:90-118), a NaN passing through the clamps as it does there (the dense GLU keeps act_glu alone: the
// third branch in its epilogue costs the dense K loop registers)
__device__ __forceinline__ float glu(float g, float u, int act) {
    if (act == DR_ACT_SWIGLU_OAI) {
        const float gc = g > 7.f ? 7.f : g;
        const float uc = u > 7.f ? 7.f : (u < -7.f ? -7.f : u);
        return gc / (1.f + __expf(-(1.702f * gc))) * (uc + 1.f);
    }
    return act_glu(g, act) * u;
}

// the reference's top-k key of a bf16 (dense_writer.cpp:215): a monotonic uint16, 0 below everything
__device__ __forceinline__ uint32_t key_bf16(uint32_t b) { return b ^ (0x8000u | (0x7FFFu & (0u - (b >> 15)))); }
__device__ __forceinline__ uint32_t key_f32(float f) {
    const uint32_t u = __float_as_uint(f);
    return u ^ ((u >> 31) ? 0xFFFFFFFFu : 0x80000000u);
}

// ---- top-k records of tile groups ------------------------------------------------------------------------------------
//
// A launch with more tiles than the caller's records writes one record a group of tk_group consecutive tiles (the
// reference writes one a core, each core's columns ranked together, dense_writer.cpp:185-232). Every tile ranks its
// own 32 columns into a staging record in the workspace; a second kernel on the same stream (dr_group_k, no atomics:
// the stream orders it after the matmul) ranks each group's candidates by a 64-bit key, the record's key above the id
// complemented (0 empty), so the order is the tiles' own: highest first, ties to the lower id.

__device__ __forceinline__ unsigned long long cand_key(uint32_t word, uint32_t id, bool fp32) {
    if (id == 0xFFFFFFFFu || (!fp32 && word == 0u)) return 0ull;
    const uint32_t ok = fp32 ? key_f32(__uint_as_float(word)) : word;
    return ((unsigned long long)ok << 32) | (unsigned long long)(0xFFFFFFFFu - id);
}

constexpr int GROUP_WAVES = 4;      // dr_group_k: a wavefront a row, rows in turn
constexpr int GROUP_MAXCAND = 1024;  // candidates a row of a grouped record at most (tiles a record x k)

// one workgroup a record: rows [row0, row1) of the group's staged tile records, each row's best k of the tiles' k.
// A wavefront takes a row: its lanes load the candidates (word, id) and write each one's 64-bit key to LDS, then each
// candidate's rank is the count of larger keys (the keys are distinct but for the empty 0).
__global__ __launch_bounds__(64 * GROUP_WAVES) void dr_group_k(const uint32_t* __restrict__ stage,
                                                              uint32_t* __restrict__ rec, int tiles, int G, int K, int R,
                                                              int slot0, int row0, int row1, int fp32) {
    extern __shared__ unsigned long long keys[];  // [GROUP_WAVES][G * K]
    const int grp = blockIdx.x, t0 = grp * G, members = min(G, tiles - t0), n = members * K;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const size_t rlen = 2 * (size_t)R * K;
    uint32_t* out = rec + (size_t)(slot0 + grp) * rlen;
    unsigned long long* kw = keys + (size_t)wave * G * K;
    constexpr int PER = GROUP_MAXCAND / 64;  // candidates a lane at most
    for (int r = row0 + wave; r < row1; r += GROUP_WAVES) {
        uint32_t word[PER], id[PER];
        unsigned long long key[PER];
        // every load issued before any is used (slots past n read the last candidate again and are dropped)
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            const int i = min(lane + 64 * q, n - 1);
            const uint32_t* src = stage + (size_t)(t0 + i / K) * rlen + (size_t)r * K + i % K;
            word[q] = src[0];
            id[q] = src[(size_t)R * K];
        }
        int nval = 0;
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            const int i = lane + 64 * q;
            key[q] = i < n ? cand_key(word[q], id[q], fp32 != 0) : 0ull;
            if (i < n) kw[i] = key[q];
            nval += __popcll(__ballot(key[q] != 0ull));
        }
        __builtin_amdgcn_s_waitcnt(0);  // (the wavefront's own LDS writes, read back by its other lanes)
        __builtin_amdgcn_wave_barrier();
        int rank[PER];
#pragma unroll
        for (int q = 0; q < PER; ++q) rank[q] = 0;
        const int qn = (n + 63) / 64;  // (the lanes' candidate slots in use, uniform)
#pragma unroll 8
        for (int j = 0; j < n; ++j) {
            const unsigned long long kj = kw[j];
#pragma unroll
            for (int q = 0; q < PER; ++q)
                if (q < qn) rank[q] += kj > key[q];
        }
#pragma unroll
        for (int q = 0; q < PER; ++q)
            if (key[q] != 0ull && rank[q] < K) {
                out[(size_t)r * K + rank[q]] = word[q];
                out[(size_t)R * K + (size_t)r * K + rank[q]] = id[q];
            }
        for (int q = nval + lane; q < K; q += 64) {
            out[(size_t)r * K + q] = fp32 ? 0xFF800000u : 0u;
            out[(size_t)R * K + (size_t)r * K + q] = 0xFFFFFFFFu;
        }
        __builtin_amdgcn_wave_barrier();  // (this row's keys read before the next row's overwrite them)
    }
}

// ---- expert gather: ids, the union of the rows' ids ----------------------------------------------------------------

// expert id j of row r, or -1 when it is not below the expert count (it chooses nothing)
__device__ __forceinline__ int moe_id(const MoeArgs& a, int r, int j) {
    const size_t i = (size_t)r * a.ld_ids + j;
    const uint32_t e = a.ids32 ? reinterpret_cast<const uint32_t*>(a.ids)[i] : reinterpret_cast<const uint16_t*>(a.ids)[i];
    return e < (uint32_t)a.experts ? (int)e : -1;
}

// the distinct ids below the expert count of the ids' rows, in increasing order (moe/kernels/moe8_rows.h's union)
struct UnionLds {
    uint32_t bits[32];
    uint16_t list[1024];
    int count;
};

// the workgroup's threads: every launch of these kernels has 64 * a.waves. (blockDim.x reads the dispatch's implicit
// arguments, on a line of the argument block nothing else touches: in an epilogue, a scalar-cache miss and a round
// trip after the K loop.)
__device__ __forceinline__ int wg_threads(const Args& a) { return 64 * a.waves; }

template <int MOE>
__device__ __forceinline__ UnionLds* union_lds() {
    __shared__ UnionLds u;
    return &u;
}

// every thread of the workgroup calls it: a bitmap of the ids, then wavefront 0 lists its set bits in order
__device__ __forceinline__ void moe_union(const MoeArgs& a, UnionLds& u) {
    for (int i = threadIdx.x; i < 32; i += wg_threads(a)) u.bits[i] = 0u;
    __syncthreads();
    for (int i = threadIdx.x; i < a.id_rows * a.slots; i += wg_threads(a)) {
        const int e = moe_id(a, i / a.slots, i % a.slots);
        if (e >= 0) atomicOr(&u.bits[e >> 5], 1u << (e & 31));
    }
    __syncthreads();
    if (threadIdx.x < 64) {
        const int l = threadIdx.x;
        const uint32_t w = l < 32 ? u.bits[l] : 0u;
        const int c = __popc(w);
        int incl = c;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int v = __shfl_up(incl, o);
            if (l >= o) incl += v;
        }
        int pos = incl - c;
        for (uint32_t m = w; m != 0u; m &= m - 1u) u.list[pos++] = (uint16_t)(32 * l + __ffs(m) - 1);
        if (l == 63) u.count = incl;
    }
    __syncthreads();
}

// ---- the workgroup's tile: its segment, its panels -------------------------------------------------------------------

template <bool ONE>
__device__ __forceinline__ int find_segment(const Args& a, int g) {
    int s = 0;  // (ONE: a single segment, found without reading the others' bounds first)
    if (!ONE) {
#pragma unroll
        for (int j = 1; j < 4; ++j)
            if (j < a.nseg && g >= a.seg[j].tile_begin) s = j;
    }
    return s;
}

// the code and exponent bases of the tile's PW panels, and each panel's parity (of its index in its weight): plain
// weights the tile's two panels; interleave_glu weights the gate tile's two panels then the up tile's; gate and up
// weights apart their tile's two panels each
// GU (the expert gather's gate/up launches, gate and up apart): PW = 2 is a 16-column tile's gate panel and up panel.
template <int PW, bool GU = false>
__device__ __forceinline__ void panel_ptrs(const SegDev& sg, int t, int k_pad, const uint8_t* (&cb)[PW],
                                           const uint8_t* (&eb)[PW], int (&par)[PW]) {
#pragma unroll
    for (int q = 0; q < PW; ++q) {
        int p;
        const uint8_t* cbase = sg.codes;
        const uint8_t* ebase = sg.exps;
        if (GU && PW == 2) {
            p = t;
            if (q == 1) {
                cbase = sg.codes_up;
                ebase = sg.exps_up;
            }
        } else if (PW <= 2) {
            p = PW * t + q;  // (a narrow launch: the tile is one panel)
        } else if (sg.glu == 1) {
            p = 4 * t + q;  // interleave_glu: gate tile 2t, up tile 2t + 1
        } else {
            p = 2 * t + (q & 1);
            if (q >= 2) {
                cbase = sg.codes_up;
                ebase = sg.exps_up;
            }
        }
        cb[q] = cbase + (size_t)p * sg.pstride;
        eb[q] = ebase + (size_t)p * k_pad;
        par[q] = p & 1;  // (the panel's parity: its half-turn of the block loaders' slots)
    }
}
template <int PW, bool GU = false>
__device__ __forceinline__ void panel_ptrs(const SegDev& sg, int t, int k_pad, const uint8_t* (&cb)[PW],
                                           const uint8_t* (&eb)[PW]) {
    int par[PW];
    panel_ptrs<PW, GU>(sg, t, k_pad, cb, eb, par);
}

// v + p[0] + p[stride] + ... + p[(n - 1) * stride], added in that order, the LDS reads of 8 terms issued together
// before any is added (one LDS round trip for 8 terms, where a loop of read-then-add waits for each read in turn).
// Used by the general and split-K epilogues; the GEMV's plain epilogue keeps its one-term loop, measured faster there.
__device__ __forceinline__ float sum_parts(float v, const float* p, int n, int stride) {
    for (int w0 = 0; w0 < n; w0 += 8) {
        float t[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) t[j] = w0 + j < n ? p[(w0 + j) * stride] : 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (w0 + j < n) v += t[j];
    }
    return v;
}

// ---- the epilogue: the wavefronts' partial sums to the output stages ---------------------------------------------
//
// part [nparts][PW][ROWS][16]: column sums of panel q, added in order (the wavefronts', or with split K the
// workgroups'). Thread (m, col) of the 32-column output tile applies the scales, the GLU, the residual, writes y and keeps
// the tile for the top-k ranking.
template <int ROWS, int PW>
__device__ __forceinline__ void epilogue(const Args& a, const SegDev& sg, int t, const float* part, int nparts,
                                         float (*tval)[TILE], uint32_t (*tkey)[TILE], int wave, int lane,
                                         const float* pre = nullptr) {
    constexpr int TW = tile_w<PW>();
    const int mrows = min(a.m, ROWS);
    const bool topk = a.rec != nullptr;  // (never with PW = 1)
    for (int e = threadIdx.x; e < TW * ROWS; e += wg_threads(a)) {
        const int m = e / TW, col = e % TW;
        const int oc = t * TW + col;  // output column of this segment
        const bool valid = m < mrows && oc < sg.n_out;
        float v = 0.f;
        const int cq = col >> 4, cc = col & 15;
        if (PW == 4) {
            const float gsum = sum_parts(0.f, part + (cq * ROWS + m) * 16 + cc, nparts, PW * ROWS * 16);
            const float usum = sum_parts(0.f, part + ((2 + cq) * ROWS + m) * 16 + cc, nparts, PW * ROWS * 16);
            float sgv = 1.f, suv = 1.f;
            if (valid) {
                if (pre != nullptr) {
                    sgv = pre[col];
                    suv = pre[TILE + col];
                } else if (sg.glu == 1) {
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
            // (the residual: prefetched for the thread's first element)
            const bool rpre = pre != nullptr && e == (int)threadIdx.x;
            float rv = 0.f;
            if (valid && a.res != nullptr) rv = rpre ? pre[PRE_RES + e] : bf16_to_f32(a.res[(size_t)m * a.ldr + ycol]);
            if (valid && a.res != nullptr && a.res_mode == 2) v = rv;
            v = sum_parts(v, part + (cq * ROWS + m) * 16 + cc, nparts, PW * ROWS * 16);
            if (valid) {
                v *= pre != nullptr ? pre[col] : load_scale(sg.scale, sg.scale_f32, oc);
                if (a.res != nullptr && a.res_mode == 1) v += rv;
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
        }
    }
    if (!topk) return;
    __syncthreads();
    // the workgroup's wavefronts rank the rows, two a wavefront (a 32-lane half each; one wavefront walking every row in
    // turn had kept the workgroup ≈ 1 µs a 4-row tile: C5's records cost 19 of its 103 µs): each row's 32 keys, the
    // best k, highest first, ties to the lower column. The record goes to its slot, or with grouped records to the
    // tile's staging record (dr_group_k ranks the groups afterwards).
    {
        const int K = a.tk_k, R = a.tk_rows;
        const size_t rlen = 2 * (size_t)R * K;
        uint32_t* rec = a.rec_out + (size_t)t * rlen;
        auto put = [](uint32_t* p, uint32_t v) { *p = v; };
        const int nw = a.waves, c = lane & 31;
        for (int m = 2 * wave + (lane >> 5); m < mrows && a.row0 + m < R; m += 2 * nw) {
            const int r = a.row0 + m;
            const uint32_t key = tkey[m][c];
            // rank: the columns ahead of c, by key then the lower column first (one 64-bit compare a column: the
            // key above the column complemented)
            const unsigned long long me = ((unsigned long long)key << 32) | (uint32_t)(TILE - 1 - c);
            // (the row's 32 keys in eight 16-byte reads, all issued before the first compare: one read a key had
            // kept each workgroup ranking ≈ 0.2 us longer, C5 87.2 -> 85.5 us)
            int rank = 0, nval = 0;
            const uint4* kr = reinterpret_cast<const uint4*>(&tkey[m][0]);
            uint4 q[TILE / 4];
#pragma unroll
            for (int j4 = 0; j4 < TILE / 4; ++j4) q[j4] = kr[j4];
#pragma unroll
            for (int j = 0; j < TILE; ++j) {
                const uint4 w = q[j >> 2];
                const uint32_t kj = (j & 3) == 0 ? w.x : (j & 3) == 1 ? w.y : (j & 3) == 2 ? w.z : w.w;
                nval += kj != 0u;
                rank += (((unsigned long long)kj << 32) | (uint32_t)(TILE - 1 - j)) > me;
            }
            if (key != 0u && rank < K) {
                const float val = tval[m][c];
                put(rec + (size_t)r * K + rank, a.tk_fp32 ? __float_as_uint(val) : key);
                put(rec + (size_t)R * K + (size_t)r * K + rank, (uint32_t)(a.base + (long long)t * TILE + c));
            }
            if (c >= nval && c < K) {
                put(rec + (size_t)r * K + c, a.tk_fp32 ? 0xFF800000u : 0u);
                put(rec + (size_t)R * K + (size_t)r * K + c, 0xFFFFFFFFu);
            }
        }
    }
}

// the gate/up modes' epilogue: thread (m, col) of the tile adds the bias, applies the GLU and the row's routing weight
// for the expert (the slot's in DR_MOE_GATE_UP; 0 where the row did not choose it in DR_MOE_GATE_UP_ROWS) and writes
// the unit's columns of y (moe_gu_compute.cpp: the GLU in dest, then times the weight's tile). The tile is PW / 2 gate
// panels then as many up panels: 32 columns, or 16 in a narrow launch (PW = 2).
template <int ROWS, int PW, int MOE>
__device__ __forceinline__ void epilogue_moe(const MoeArgs& a, int t, int unit, int ex, const float* part, int nparts,
                                             float wunit) {
    constexpr int TW = 8 * PW, H = PW / 2;
    __shared__ float coef[ROWS];
    const int mrows = min(a.m, ROWS);
    if (threadIdx.x < ROWS) {
        const int m = threadIdx.x, r = a.row0 + m;
        float c = 0.f;
        if (m < mrows) {
            if (MOE == DR_MOE_GATE_UP) {
                c = wunit;  // (the slot's weight, read or routed at the workgroup's start)
            } else if (r < a.id_rows) {
                for (int j = 0; j < a.slots; ++j)
                    if (moe_id(a, r, j) == ex) c = bf16_to_f32(a.rw[(size_t)r * a.ld_rw + j]);
            }
        }
        coef[m] = c;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < TW * ROWS; e += wg_threads(a)) {
        const int m = e / TW, col = e % TW;
        const int oc = t * TW + col;  // the column within the expert's
        if (m >= mrows || oc >= a.en) continue;
        const int cq = col >> 4, cc = col & 15;
        float gsum = sum_parts(0.f, part + (cq * ROWS + m) * 16 + cc, nparts, PW * ROWS * 16);
        float usum = sum_parts(0.f, part + ((H + cq) * ROWS + m) * 16 + cc, nparts, PW * ROWS * 16);
        if (a.bias != nullptr) {
            gsum += bf16_to_f32(a.bias[((size_t)ex * 2 + 0) * a.en + oc]);
            usum += bf16_to_f32(a.bias[((size_t)ex * 2 + 1) * a.en + oc]);
        }
        const float v = glu(gsum, usum, a.act) * coef[m];
        reinterpret_cast<uint16_t*>(a.y)[(size_t)m * a.ldy + (size_t)unit * a.en + oc] = (uint16_t)f32_to_bf16(v);
    }
}

// DR_MOE_GATE_UP with an id past the experts: the slot's columns of this tile are zeros
template <int PW>
__device__ __forceinline__ void moe_zero(const MoeArgs& a, int t, int unit) {
    constexpr int TW = 8 * PW;
    for (int col = threadIdx.x; col < TW; col += wg_threads(a)) {
        const int oc = t * TW + col;
        if (oc < a.en) reinterpret_cast<uint16_t*>(a.y)[(size_t)unit * a.en + oc] = 0;
    }
}

// The epilogue of a plain launch (one weight, bf16 y, no residual, top-k records or split K): the general epilogue's
// arithmetic in the same order (so the same bits), without its branches for the other stages. On MI355X the general
// one's tail cost the north-star launch 0.4 us and the bfloat4_b GLU pair 0.6 (work-stripped copies, one-process A/B).
template <int ROWS, int PW>
__device__ __forceinline__ void epilogue_plain(const Args& a, const SegDev& sg, int t, const float* part,
                                               const float* pre) {
    constexpr int TW = tile_w<PW>();
    const int e = threadIdx.x;
    if (e >= TW * ROWS) return;
    const int m = e / TW, col = e % TW;
    const int oc = t * TW + col;
    if (m >= min(a.m, ROWS) || oc >= sg.n_out) return;
    const int cq = col >> 4, cc = col & 15;
    float v;
    if (PW == 4) {
        // (one partial a loop turn: measured faster here than sum_parts' batched reads)
        float gsum = 0.f, usum = 0.f;
        for (int w = 0; w < a.waves; ++w) {
            gsum += part[((w * PW + cq) * ROWS + m) * 16 + cc];
            usum += part[((w * PW + 2 + cq) * ROWS + m) * 16 + cc];
        }
        v = act_glu(gsum * pre[col], a.act) * (usum * pre[TILE + col]);
    } else {
        v = 0.f;
        for (int w = 0; w < a.waves; ++w) v += part[((w * PW + cq) * ROWS + m) * 16 + cc];
        v *= pre[col];
    }
    reinterpret_cast<uint16_t*>(a.y)[(size_t)m * a.ldy + sg.col0 + oc] = (uint16_t)f32_to_bf16(v);
}

// ---- split K: the tile's workgroups meet in the workspace ------------------------------------------------------------
//
// With splits > 1 each of a tile's workgroups takes cps chunks; it adds its wavefronts' sums (in order), writes them
// to the workspace and counts itself done; the last one reads every workgroup's sums back, in split order, into part
// and runs the epilogue (so the sum order is fixed: chunks, or the 16-row kernel's groups, within a wavefront,
// wavefronts within a split, splits), then resets the tile's counter for the next launch. Returns the number of
// partial sums now in part, 0 when this workgroup is not the tile's last.
//
// The XCDs' L2 caches are not coherent with each other, and an agent-scope release or acquire fence writes back or
// invalidates a whole L2 (it cost 6x the matmul itself). Instead every workspace access is a device-scope atomic
// (relaxed): such loads and stores go to the device's point of coherence on their own. A workgroup's sums are complete
// there before it counts itself (each thread waits for its stores, then the barrier), and the last workgroup reads
// them only after its count has come back. With relaxed accesses that order is the emitted code's, not the memory
// model's: tests/test_isa_hazards.py checks every kernel's gfx950 code for it (the stores waited for and a barrier
// before the counter atomic, the loads after its result and a second barrier). The counters lie at the workspace's start, SPLIT_MAXTILES of them whatever
// the launch's shape, and the sums after them: a workspace shared by launches of any shape never finds an earlier
// launch's sums where a counter should be zero (a launch of more tiles runs unsplit).
#ifndef DR_SPLIT_MAXTILES
#define DR_SPLIT_MAXTILES 16384
#endif
constexpr int SPLIT_MAXTILES = DR_SPLIT_MAXTILES;  // counters in the workspace: tiles of a split launch at most

__device__ __forceinline__ void st_dev(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_dev(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int ROWS, int PW>
__device__ __forceinline__ int gather_splits(const Args& a, int g, int split, float* part) {
    constexpr int E = PW * ROWS * 16;
    __shared__ int last;
    if (a.splits == 1) return a.waves;
    float* mine = a.wpart + ((size_t)g * a.splits + split) * E;
    for (int e = threadIdx.x; e < E; e += wg_threads(a)) {
        st_dev(mine + e, sum_parts(0.f, part + e, a.waves, E));
    }
    __builtin_amdgcn_s_waitcnt(0);  // this thread's stores have reached the point of coherence
    __syncthreads();
    if (threadIdx.x == 0)
        last = __hip_atomic_fetch_add(a.counters + g, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)(a.splits - 1);
    __syncthreads();
    if (!last) return 0;
    const float* all = a.wpart + (size_t)g * a.splits * E;
    // (4 loads a thread out together: each round trip to the point of coherence is long)
    const int n = a.splits * E, T = wg_threads(a);
    for (int e0 = threadIdx.x; e0 < n; e0 += 4 * T) {
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = e0 + j * T < n ? ld_dev(all + e0 + j * T) : 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (e0 + j * T < n) part[e0 + j * T] = v[j];
    }
    if (threadIdx.x == 0) __hip_atomic_store(a.counters + g, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    return a.splits;
}

// ---- the GEMV kernel (few rows): VALU decode and FMA, one accumulator a lane per panel and row -----------------------
//
// FMT >= 0: every segment has that format (one K loop compiled in: a smaller kernel); FMT < 0: each workgroup
// branches on its segment's format. ONE: a single segment.
template <int MOE>
__device__ __forceinline__ constexpr bool moe_k() {
    return MOE == DR_MOE_DOWN || MOE == DR_MOE_DOWN_ROWS;
}
template <int MOE>
__device__ __forceinline__ constexpr bool moe_n() {
    return MOE == DR_MOE_GATE_UP || MOE == DR_MOE_GATE_UP_ROWS;
}

// ONEG: the launch's chunks are 256 k, one exponent group each, and the loaders read only that group (the dense
// kernel keeps its own instantiation: a runtime choice of loader inside it moved the compiler's scheduling of its K
// loop, NS 12.5 -> 13.1 us)
template <int MR, int PW, int FMT, bool ONE, bool ONEG, bool PLAIN>
__device__ __forceinline__ void gemv_body(const Args a) {
    extern __shared__ float part[];  // [W][PW][MR][16]
    __shared__ float tval[MR][TILE];
    __shared__ __align__(16) uint32_t tkey[MR][TILE];

    // (a plain launch has no split: its workgroup is its tile)
    const int g = PLAIN ? (int)blockIdx.x : (int)(blockIdx.x % a.tiles), split = PLAIN ? 0 : (int)(blockIdx.x / a.tiles);
    const SegDev& sg = a.seg[find_segment<ONE>(a, g)];
    const int t = g - sg.tile_begin;
    // (the wavefront index is uniform across the wavefront; readfirstlane lets the compiler see it, so the chunk
    // bounds and loop trip counts live in SGPRs and the K loops branch on scalars)
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int fmt = FMT >= 0 ? FMT : sg.fmt;
    const uint8_t* cb[PW];
    const uint8_t* eb[PW];
    int par[PW];
    panel_ptrs<PW>(sg, t, a.k_pad, cb, eb, par);
    __shared__ __align__(16) uint16_t xwin[MAXW][MR][XWIN];  // each wavefront's x window

    // the epilogue's scales and residual, read before the K loop so that their latency hides under it; a plain launch
    // reads its scales after the K loop instead: before it, their dependent scalar and vector loads and branches had
    // delayed the launch's first weight loads (the north star 11.56 -> 11.28 us, one-process A/B)
    __shared__ float pre[PRE_FLOATS];
    EpiPre ep{1.f, 1.f, 0.f};
    if constexpr (!PLAIN) ep = epi_prefetch<MR, PW>(a, sg, t);

    float wsum[PW][MR];  // this wavefront's column sums (lanes 0..15), its chunks added in order
#pragma unroll
    for (int q = 0; q < PW; ++q)
#pragma unroll
        for (int m = 0; m < MR; ++m) wsum[q][m] = 0.f;
    const int ch1 = min((split + 1) * a.cps, a.chunks);
    for (int ch = split * a.cps + wave; ch < ch1; ch += a.waves) {
        float acc[PW][MR], corr[PW][MR];
#pragma unroll
        for (int q = 0; q < PW; ++q)
#pragma unroll
            for (int m = 0; m < MR; ++m) acc[q][m] = corr[q][m] = 0.f;
        const int k0 = ch * a.kch, k1 = min(k0 + a.kch, a.k_pad);
        if (fmt == DR_BFP8) {
            chunk_bfp8<MR, PW, ONEG>(a, cb, eb, par, k0, k1, lane, xwin[wave], acc);
        } else if (FMT == DR_INT4) {
            const uint16_t* gs[PW];
#pragma unroll
            for (int q = 0; q < PW; ++q) gs[q] = sg.gscale + (size_t)(PW * t + q) * (a.k_pad / 128) * 64;
            chunk_int4<MR, PW, ONEG>(a, cb, gs, par, k0, k1, lane, xwin[wave], acc);
        } else if (fmt == DR_BFP4) {
            float sx[PW][MR];
#pragma unroll
            for (int q = 0; q < PW; ++q)
#pragma unroll
                for (int m = 0; m < MR; ++m) sx[q][m] = 0.f;
            chunk_bfp4<MR, PW, ONEG>(a, cb, eb, par, k0, k1, lane, xwin[wave], acc, sx);
            // the wavefront's sum of x' (every lane made distinct x'): its excess is taken off every column
#pragma unroll
            for (int q = 0; q < PW; ++q)
#pragma unroll
                for (int m = 0; m < MR; ++m) {
                    float v = wsel::add_xor<8>(wsel::add_xor<4>(wsel::add_xor<2>(wsel::add_xor<1>(sx[q][m]))));
                    corr[q][m] = wsel::add_xor<32>(wsel::add_xor<16>(v));
                }
        } else {
            chunk_bf16<MR, PW>(a, cb, k0, k1, lane, acc);
        }
        // the chunk's column sums: the four quarter-rows of each column, in a fixed order
#pragma unroll
        for (int q = 0; q < PW; ++q)
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                float v = acc[q][m];
                v = wsel::add_xor<32>(wsel::add_xor<16>(v));
                wsum[q][m] += fmt == DR_BFP4 ? bfp4_chunk_sum(v, corr[q][m]) : v;
            }
    }
    if (lane < 16) {
#pragma unroll
        for (int q = 0; q < PW; ++q)
#pragma unroll
            for (int m = 0; m < MR; ++m) part[((wave * PW + q) * MR + m) * 16 + lane] = wsum[q][m];
    }
    if constexpr (PLAIN) ep = epi_prefetch<MR, PW>(a, sg, t);
    epi_stage(ep, pre);
    __syncthreads();
    if constexpr (PLAIN) {
        epilogue_plain<MR, PW>(a, sg, t, part, pre);
        return;
    }
    const int nparts = gather_splits<MR, PW>(a, g, split, part);
    if (nparts) epilogue<MR, PW>(a, sg, t, part, nparts, tval, tkey, wave, lane, pre);
}

// PLAIN: a plain launch (epilogue_plain), one weight of format FMT
template <int MR, int PW, int FMT, bool ONE, bool PLAIN = false>
__global__ __launch_bounds__(512) void dr_gemv(const Args a) {
    gemv_body<MR, PW, FMT, ONE, false, PLAIN>(a);
}

// the same for launches of 256-k chunks (K up to 2048)
template <int MR, int PW, int FMT, bool ONE, bool PLAIN = false>
__global__ __launch_bounds__(512) void dr_gemv_g1(const Args a) {
    gemv_body<MR, PW, FMT, ONE, true, PLAIN>(a);
}


// ---- the expert gather (include/moe.h): the GEMV and MFMA kernels over the chosen experts' bfloat4_b weights ----------
//
// Kernels of their own (the dense kernels stay as they are: a gather branch in them, even compiled out, moved the
// compiler's scheduling of the dense K loop). Gate/up modes: the launch's tiles are units (slots, or the union's
// experts) times the expert's tiles; the workgroup's unit gives its expert, whose weights sit cstride / estride bytes
// per expert further on. Down modes: the launch's K is the units' blocks of ekp rows one after another; a chunk lies in
// one unit (ekp is a multiple of the chunk), whose expert gives that chunk's weights and whose ek values of x sit at
// unit * ek.
template <int MR, int PW, int MOE, bool KB>
__global__ __launch_bounds__((MOE == DR_MOE_DOWN || MOE == DR_MOE_DOWN_ROWS) ? 64 * MAXW_DOWN : 64 * MAXW) void
dr_gemv_moe(const MoeArgs a) {
    extern __shared__ float part[];  // [W][PW][MR][16]
    __shared__ float tval[MR][TILE];
    __shared__ __align__(16) uint32_t tkey[MR][TILE];

    const int g = blockIdx.x % a.tiles, split = blockIdx.x / a.tiles;
    const SegDev& sg = a.seg[0];
    int t = g - sg.tile_begin;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    UnionLds* ul = nullptr;
    if constexpr (MOE == DR_MOE_GATE_UP_ROWS || MOE == DR_MOE_DOWN_ROWS) {
        ul = union_lds<MOE>();
        moe_union(a, *ul);
    }
    int unit = 0, ex = 0;
    float wunit = 0.f;  // DR_MOE_GATE_UP: the slot's routing weight
    __shared__ int r_id[moe_route::MAXK];
    __shared__ uint16_t r_w[moe_route::MAXK];
    if constexpr (MOE == DR_MOE_GATE_UP) {
        if (a.routed) {
            // the token's routing, by wavefront 0 with the router's code (the same picks and weights bit for bit);
            // the other wavefronts wait at the barrier. Workgroup 0 writes them out for the down launch and the caller.
            __shared__ moe_route::RouteLds rl;
            if (wave == 0) {
                int mine;
                uint16_t wbits;
                moe_route::route_row<ROUTE_MAXPER>(a.route, 0, lane, rl, mine, wbits);
                if (lane < a.route.k) {
                    r_id[lane] = mine;
                    r_w[lane] = wbits;
                }
                if (lane == 0 && a.route.slot >= 0) {  // (the slot column: its id at weight 1.0)
                    r_id[a.route.k] = (int)a.route.slot;
                    r_w[a.route.k] = 0x3F80u;
                }
                if (blockIdx.x == 0) moe_route::route_store(a.route, 0, lane, mine, wbits);
            }
            __syncthreads();
        }
    }
    if constexpr (moe_n<MOE>()) {
        unit = t / a.tpe;
        t -= unit * a.tpe;
        if (MOE == DR_MOE_GATE_UP && a.routed) {
            ex = r_id[unit] < a.experts ? r_id[unit] : -1;  // (as moe_id: an id past the experts chooses none)
            wunit = bf16_to_f32(r_w[unit]);
        } else {
            ex = MOE == DR_MOE_GATE_UP ? moe_id(a, 0, unit) : (unit < ul->count ? (int)ul->list[unit] : -1);
            if (MOE == DR_MOE_GATE_UP) wunit = bf16_to_f32(a.rw[unit]);
        }
        ex = __builtin_amdgcn_readfirstlane(ex);
        if (ex < 0) {
            if (MOE == DR_MOE_GATE_UP && split == 0) moe_zero<PW>(a, t, unit);
            return;
        }
    }
    const uint8_t* cb[PW];
    const uint8_t* eb[PW];
    int par[PW];
    panel_ptrs<PW, moe_n<MOE>()>(sg, t, moe_k<MOE>() ? a.ekp : a.k_pad, cb, eb, par);
    __shared__ __align__(16) uint16_t xwin[moe_k<MOE>() ? MAXW_DOWN : MAXW][MR][XWIN];  // each wavefront's x window
    if constexpr (moe_n<MOE>()) {
#pragma unroll
        for (int q = 0; q < PW; ++q) {
            cb[q] += (size_t)ex * a.cstride;
            eb[q] += (size_t)ex * a.estride;
        }
    }

    float wsum[PW][MR];  // this wavefront's column sums (lanes 0..15), its chunks added in order
#pragma unroll
    for (int q = 0; q < PW; ++q)
#pragma unroll
        for (int m = 0; m < MR; ++m) wsum[q][m] = 0.f;
    // one chunk [k0, k1) of x (b) against the panels cbx / ebx, added to wsum
    auto chunk = [&](const Args& b, const uint8_t* const* cbx, const uint8_t* const* ebx, int k0, int k1) {
        float acc[PW][MR], sx[PW][MR];
#pragma unroll
        for (int q = 0; q < PW; ++q)
#pragma unroll
            for (int m = 0; m < MR; ++m) acc[q][m] = sx[q][m] = 0.f;
        if constexpr (KB) {  // (the lanes' sums are already scaled, their x sums taken off)
            chunk_bfp4k<MR, PW>(b, cbx, ebx, k0, k1, lane, acc);
#pragma unroll
            for (int q = 0; q < PW; ++q)
#pragma unroll
                for (int m = 0; m < MR; ++m) wsum[q][m] += wsel::add_xor<32>(wsel::add_xor<16>(acc[q][m]));
            return;
        }
        chunk_bfp4<MR, PW>(b, cbx, ebx, par, k0, k1, lane, xwin[wave], acc, sx);
        // the chunk's column sums less the wavefront's excess, as dr_gemv's
#pragma unroll
        for (int q = 0; q < PW; ++q)
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                float c = wsel::add_xor<8>(wsel::add_xor<4>(wsel::add_xor<2>(wsel::add_xor<1>(sx[q][m]))));
                c = wsel::add_xor<32>(wsel::add_xor<16>(c));
                float v = acc[q][m];
                v = wsel::add_xor<32>(wsel::add_xor<16>(v));
                wsum[q][m] += bfp4_chunk_sum(v, c);
            }
    };
    // DR_MOE_DOWN: every slot's id, lane j slot j, read once (a chunk then takes its unit's id from a lane, not from
    // memory: one dependent round trip fewer a chunk)
    int idv = -1;
    if constexpr (MOE == DR_MOE_DOWN) idv = lane < a.slots ? moe_id(a, 0, lane) : -1;
    const int ch1 = min((split + 1) * a.cps, a.chunks);
    for (int ch = split * a.cps + wave; ch < ch1; ch += a.waves) {
        const int k0 = ch * a.kch, k1 = min(k0 + a.kch, a.k_pad);
        if constexpr (moe_k<MOE>()) {
            const int s = __builtin_amdgcn_readfirstlane(k0 / a.ekp);
            int e = MOE == DR_MOE_DOWN ? __builtin_amdgcn_readlane(idv, s) : (s < ul->count ? (int)ul->list[s] : -1);
            e = __builtin_amdgcn_readfirstlane(e);
            if (e < 0) continue;  // (an id past the experts, or a block past the union: nothing to add)
            Args b = a;  // (the chunk's view of x: the unit's block)
            b.x = a.x + (size_t)s * a.ek;
            b.k = a.ek;
            b.k_pad = a.ekp;
            const uint8_t* cbe[PW];
            const uint8_t* ebe[PW];
#pragma unroll
            for (int q = 0; q < PW; ++q) {
                cbe[q] = cb[q] + (size_t)e * a.cstride;
                ebe[q] = eb[q] + (size_t)e * a.estride;
            }
            chunk(b, cbe, ebe, k0 - s * a.ekp, k1 - s * a.ekp);
        } else {
            chunk(a, cb, eb, k0, k1);
        }
    }
    if (lane < 16) {
#pragma unroll
        for (int q = 0; q < PW; ++q)
#pragma unroll
            for (int m = 0; m < MR; ++m) part[((wave * PW + q) * MR + m) * 16 + lane] = wsum[q][m];
    }
    __syncthreads();
    const int nparts = gather_splits<MR, PW>(a, g, split, part);
    if (!nparts) return;
    if constexpr (moe_n<MOE>())
        epilogue_moe<MR, PW, MOE>(a, t, unit, ex, part, nparts, wunit);
    else
        epilogue<MR, PW>(a, sg, t, part, nparts, tval, tkey, wave, lane);
}

// ---- the MFMA kernel (rows in tiles of 16): 16x16x32 bf16 matrix cores, weights decoded to exact bf16 ---------------
//
// A is x (bf16 as it is: 16 rows of a row tile, 8 k a lane), B the weights: lane (kq, c) already holds column c at
// consecutive k, the k-slots the MFMA wants, so B is its codes decoded in registers -- bf16 weights as they are,
// block-float m * 2^(E - bias) (exact in bf16: at most 7 significant bits), the power of two broadcast across the row
// from the lane that read that k's exponent. Output lane l: rows 4 (l / 16) .. +3 of column l % 16.

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;

// d = broadcast(s from lane I of this row of 16) * f (the same hazard rule as fmac_bcast)
template <int I, bool NOP>
__device__ __forceinline__ float mul_bcast(float s, float f) {
    float d;
    if constexpr (NOP)
        asm volatile("s_nop 1\n\tv_mul_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf"
                     : "=v"(d) : "v"(s), "v"(f), "i"(I));
    else
        asm volatile("v_mul_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf"
                     : "=v"(d) : "v"(s), "v"(f), "i"(I));
    return d;
}

// two fp32 values with at most 8 significant bits as one bf16 pair (truncation is exact)
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
    return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

// 16 bytes of x: row m, columns k .. k + 7 (k a multiple of 8). Rows past x read its last row: they only reach output
// rows that are never written. Columns past K read its last columns and are zeroed by x_kmask (the weights there are
// zero, but x might not be finite)
__device__ __forceinline__ uint4 x_row8(const Args& a, int m, int k) {
    const int mc = min(m, a.m - 1), kc = min(k, a.k - 8);
    return *reinterpret_cast<const uint4*>(a.x + (size_t)mc * a.ldx + kc);
}
__device__ __forceinline__ void x_kmask(uint4& v, const Args& a, int k) {
    if (k >= a.k) v = make_uint4(0u, 0u, 0u, 0u);
}

// 32-row launches stage x through LDS, each wavefront in 8 KB of its own. x_row8's loads give a lane its operand
// directly, but one load then spans 16 rows, 64 bytes of a 128-byte line in each, and at 32 rows x is most of what a
// workgroup reads. XStage::stage copies the 32 rows over k0 .. k0 + 8 NCH - 1 to LDS with buffer loads straight to
// LDS (buffer_load_dwordx4 ... lds: lane l's 16 bytes land at slot 64 i + l of load i), each load 64 / NCH whole rows
// of that range, whole lines; x_lds then reads the operands. Row r's 8-value chunk c sits at slot NCH r + (c ^ s(r)),
// s(r) = r & 15 with 16 chunks a row, (r >> 1) & 7 with 8: the 16 rows of one operand read hit 16 different bank
// groups. A lane's offset into x is fixed for the whole K loop but for the step's k and the load's rows, one add a
// load: for load i its row is 64 i / NCH + l / NCH and its chunk (l % NCH) ^ s(row), which is the lane's chunk of
// load 0 with 4 (i & 3) (16 chunks) or 4 (i & 1) (8 chunks) xored in. The buffer ends with x's last row, so rows past
// x and the columns past the last row's end read as zeros (the rows only reach output rows that are never written;
// the columns past K are zeroed by x_kmask as in x_row8).
constexpr int XS_BYTES = 8192;  // a wavefront's staging: 32 rows x 128 k of bf16
constexpr int PAIR_D = 2;       // dr_mfma_pairs: the steps of codes in flight (bfloat4_b)
constexpr int PAIR_RS = 36;     // dr_mfma_pairs: a column's partial sums, 32 rows and 4 of padding
template <int NCH>
__device__ __forceinline__ int x_swz(int row) {
    static_assert(NCH == 8 || NCH == 16, "x_swz: 8 or 16 chunks a row");
    return NCH == 16 ? (row & 15) : ((row >> 1) & 7);
}
template <int NCH>
struct XStage {
    static_assert(NCH * 16 * 32 <= XS_BYTES, "XStage: the staging holds 32 rows of 8 NCH values");
    static constexpr int RPI = 64 / NCH;  // rows a load covers
    __amdgpu_buffer_rsrc_t r;
    uint32_t off[4];  // the lane's byte offset for loads i with (i & 3) == j (16 chunks) or (i & 1) == j (8)
    uint32_t ldx2;
    // xbytes: the bytes from a.x on that the loads may read (0: m rows of ldx)
    __device__ __forceinline__ XStage(const Args& a, int lane, uint32_t xbytes = 0) {
        ldx2 = 2u * (uint32_t)a.ldx;
        r = __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, (int)(xbytes ? xbytes : ldx2 * (uint32_t)a.m),
                                              0x00020000);
        const int l = (int)opaque((uint32_t)lane);  // (made per chunk, not held across the kernel's chunk loop)
        const int row = l / NCH, c0 = (l % NCH) ^ x_swz<NCH>(row);
#pragma unroll
        for (int j = 0; j < 4; ++j) off[j] = (uint32_t)row * ldx2 + 16u * (uint32_t)(c0 ^ (4 * j));
    }
    __device__ __forceinline__ void stage(int k0, uint4* xs) const {
        // the wavefront's reads of the previous staging have returned before these loads may land on it (s_waitcnt
        // lgkmcnt(0): the loads write LDS when they return, outside the order of the wavefront's own LDS instructions)
        __builtin_amdgcn_s_waitcnt(0xC07F);
        // (opaque: the offsets of all the loads, hoisted out of the K loop, would hold 8 registers)
        uint32_t o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = opaque(off[j]) + 2u * (uint32_t)k0;
#pragma unroll
        for (int i = 0; i < 32 / RPI; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(xs + 64 * i), 16,
                                                     o[NCH == 16 ? (i & 3) : (i & 1)] + (uint32_t)(RPI * i) * ldx2, 0,
                                                     0, 0);
    }
};
// the operand x_row8(a, row, k0 + 8 c) would give, from the staging of k0 (row < 32)
template <int NCH>
__device__ __forceinline__ uint4 x_lds(const uint4* xs, int row, int c) {
    return xs[NCH * row + (c ^ x_swz<NCH>(row))];
}

__device__ __forceinline__ f32x4 mfma(uint4 a, uint4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// B for 8 bfp8 values: bytes 8H .. 8H + 7 of the lane's codes (k-offsets 16 kq + 8H + j), times the broadcast scales
template <int H>
__device__ __forceinline__ uint4 b_bfp8(const uint4& w, float s) {
    const uint32_t w0 = H ? w.z : w.x, w1 = H ? w.w : w.y;
    float v[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = (float)(int)(signed char)(w0 >> (8 * j));
#pragma unroll
    for (int j = 0; j < 4; ++j) v[4 + j] = (float)(int)(signed char)(w1 >> (8 * j));
    float p[8];
    p[0] = mul_bcast<8 * H + 0, H == 0>(s, v[0]);
    p[1] = mul_bcast<8 * H + 1, false>(s, v[1]);
    p[2] = mul_bcast<8 * H + 2, false>(s, v[2]);
    p[3] = mul_bcast<8 * H + 3, false>(s, v[3]);
    p[4] = mul_bcast<8 * H + 4, false>(s, v[4]);
    p[5] = mul_bcast<8 * H + 5, false>(s, v[5]);
    p[6] = mul_bcast<8 * H + 6, false>(s, v[6]);
    p[7] = mul_bcast<8 * H + 7, false>(s, v[7]);
    return make_uint4(pack_bf16(p[0], p[1]), pack_bf16(p[2], p[3]), pack_bf16(p[4], p[5]), pack_bf16(p[6], p[7]));
}

// bfp8, one exponent group (4 blocks of 64 k): MFMA h of block b takes k = 64 b + 16 kq + 8 h + j
template <int MT, int PW>
__device__ __forceinline__ void mgroup_bfp8(const Args& a, const uint8_t* const* cb, const uint8_t* const* eb, int g,
                                            int lane, f32x4 (&acc)[PW][MT]) {
    const int r = lane & 15, kq = lane >> 4;
    uint4 A[4][2][MT];
    uint32_t e[PW];
    uint4 c[4][PW];
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int tt = 0; tt < MT; ++tt) A[b][h][tt] = x_row8(a, 16 * tt + r, (4 * g + b) * 64 + 16 * kq + 8 * h);
#pragma unroll
    for (int q = 0; q < PW; ++q) e[q] = ld_stream4(eb[q] + (uint32_t)(g * 256 + 4 * lane));
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int q = 0; q < PW; ++q)
            c[b][q] = ld_stream16(cb[q] + (uint32_t)((4 * g + b) * 1024 + lane * 16));
    if (a.k != a.k_pad && (g + 1) * 256 > a.k) {  // (a ragged K's last group only)
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int tt = 0; tt < MT; ++tt) x_kmask(A[b][h][tt], a, (4 * g + b) * 64 + 16 * kq + 8 * h);
    }
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int q = 0; q < PW; ++q) {
            // this lane's scale: the exponent of k = 64 b + lane (the lane whose index is that k's offset)
            const float s = __builtin_ldexpf(1.f, (int)((e[q] >> (8 * b)) & 0xFFu) - 133);
            const uint4 B0 = b_bfp8<0>(c[b][q], s);
            const uint4 B1 = b_bfp8<1>(c[b][q], s);
#pragma unroll
            for (int tt = 0; tt < MT; ++tt) {
                acc[q][tt] = mfma(A[b][0][tt], B0, acc[q][tt]);
                acc[q][tt] = mfma(A[b][1][tt], B1, acc[q][tt]);
            }
        }
}

// B for the 8 bfp4 values of dword D (k-offsets 32 kq + 8 D + j): nibble u = m + 8 moved to the top of a byte with
// its top bit flipped is 16 m as a signed byte; s0 / s1 carry 2^(E - 129) / 16 of the even / odd k of each pair,
// broadcast from lane 4 D + j / 2
template <int D>
__device__ __forceinline__ uint4 b_bfp4(uint32_t w, float s0, float s1) {
    const uint32_t lo = ((w << 4) & 0xF0F0F0F0u) ^ 0x80808080u;  // k 8D + 0..3
    const uint32_t hi = (w & 0xF0F0F0F0u) ^ 0x80808080u;         // k 8D + 4..7
    float v[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = (float)(int)(signed char)(lo >> (8 * j));
#pragma unroll
    for (int j = 0; j < 4; ++j) v[4 + j] = (float)(int)(signed char)(hi >> (8 * j));
    float p[8];
    p[0] = mul_bcast<4 * D + 0, D == 0>(s0, v[0]);
    p[1] = mul_bcast<4 * D + 0, D == 0>(s1, v[1]);
    p[2] = mul_bcast<4 * D + 1, false>(s0, v[2]);
    p[3] = mul_bcast<4 * D + 1, false>(s1, v[3]);
    p[4] = mul_bcast<4 * D + 2, false>(s0, v[4]);
    p[5] = mul_bcast<4 * D + 2, false>(s1, v[5]);
    p[6] = mul_bcast<4 * D + 3, false>(s0, v[6]);
    p[7] = mul_bcast<4 * D + 3, false>(s1, v[7]);
    return make_uint4(pack_bf16(p[0], p[1]), pack_bf16(p[2], p[3]), pack_bf16(p[4], p[5]), pack_bf16(p[6], p[7]));
}

// bfp4, one exponent group (2 blocks of 128 k): MFMA D of block b takes k = 128 b + 32 kq + 8 D + j
template <int MT, int PW>
__device__ __forceinline__ void mgroup_bfp4(const Args& a, const uint8_t* const* cb, const uint8_t* const* eb, int g,
                                            int lane, f32x4 (&acc)[PW][MT]) {
    const int r = lane & 15, kq = lane >> 4;
    uint4 A[2][4][MT];
    uint32_t e[PW];
    uint4 c[2][PW];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int d = 0; d < 4; ++d)
#pragma unroll
            for (int tt = 0; tt < MT; ++tt) A[b][d][tt] = x_row8(a, 16 * tt + r, (2 * g + b) * 128 + 32 * kq + 8 * d);
#pragma unroll
    for (int q = 0; q < PW; ++q) e[q] = ld_stream4(eb[q] + (uint32_t)(g * 256 + 4 * lane));
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int q = 0; q < PW; ++q)
            c[b][q] = ld_stream16(cb[q] + (uint32_t)(real_block(2 * g + b, a.k) * 1024 + lane * 16));
    if (a.k != a.k_pad && (g + 1) * 256 > a.k) {  // (a ragged K's last group only)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int d = 0; d < 4; ++d)
#pragma unroll
                for (int tt = 0; tt < MT; ++tt) x_kmask(A[b][d][tt], a, (2 * g + b) * 128 + 32 * kq + 8 * d);
    }
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int q = 0; q < PW; ++q) {
            // this lane's scales: the exponents of the pair k = 128 b + 32 kq + 2 i, + 1 (lane 16 kq + i)
            const uint32_t ep = e[q] >> (16 * b);
            const float s0 = __builtin_ldexpf(1.f, (int)(ep & 0xFFu) - 133);
            const float s1 = __builtin_ldexpf(1.f, (int)((ep >> 8) & 0xFFu) - 133);
            const uint4 B0 = b_bfp4<0>(c[b][q].x, s0, s1);
            const uint4 B1 = b_bfp4<1>(c[b][q].y, s0, s1);
            const uint4 B2 = b_bfp4<2>(c[b][q].z, s0, s1);
            const uint4 B3 = b_bfp4<3>(c[b][q].w, s0, s1);
#pragma unroll
            for (int tt = 0; tt < MT; ++tt) {
                acc[q][tt] = mfma(A[b][0][tt], B0, acc[q][tt]);
                acc[q][tt] = mfma(A[b][1][tt], B1, acc[q][tt]);
                acc[q][tt] = mfma(A[b][2][tt], B2, acc[q][tt]);
                acc[q][tt] = mfma(A[b][3][tt], B3, acc[q][tt]);
            }
        }
}

// DR_BFP4_KB: B for the 8 values of dword D, the lane's own column at its own exponent group (no broadcast): u = m + 8
// moved to the top of a byte with its top bit flipped is 16 m as a signed byte, times s = 2^(E - 133) of the group
template <int D>
__device__ __forceinline__ uint4 b_bfp4k(uint32_t w, float s) {
    const uint32_t lo = ((w << 4) & 0xF0F0F0F0u) ^ 0x80808080u;  // k 8D + 0..3
    const uint32_t hi = (w & 0xF0F0F0F0u) ^ 0x80808080u;         // k 8D + 4..7
    float p[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) p[j] = (float)(int)(signed char)(lo >> (8 * j)) * s;
#pragma unroll
    for (int j = 0; j < 4; ++j) p[4 + j] = (float)(int)(signed char)(hi >> (8 * j)) * s;
    return make_uint4(pack_bf16(p[0], p[1]), pack_bf16(p[2], p[3]), pack_bf16(p[4], p[5]), pack_bf16(p[6], p[7]));
}

// DR_BFP4_KB, one exponent group of 256 k (2 blocks of 128), as mgroup_bfp4: MFMA D of block b takes k = 128 b +
// 32 kq + 8 D + j, in the lane's group D / 2
template <int MT, int PW>
__device__ __forceinline__ void mgroup_bfp4k(const Args& a, const uint8_t* const* cb, const uint8_t* const* eb, int g,
                                             int lane, f32x4 (&acc)[PW][MT]) {
    const int r = lane & 15, kq = lane >> 4;
    uint4 A[2][4][MT];
    uint32_t e[2][PW];
    uint4 c[2][PW];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int d = 0; d < 4; ++d)
#pragma unroll
            for (int tt = 0; tt < MT; ++tt) A[b][d][tt] = x_row8(a, 16 * tt + r, (2 * g + b) * 128 + 32 * kq + 8 * d);
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int q = 0; q < PW; ++q)
            e[b][q] = __builtin_nontemporal_load(
                reinterpret_cast<const uint16_t*>(eb[q] + (size_t)real_block(2 * g + b, a.k) * 128) + lane);
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int q = 0; q < PW; ++q)
            c[b][q] = ld_stream16(cb[q] + (uint32_t)(real_block(2 * g + b, a.k) * 1024 + lane * 16));
    if (a.k != a.k_pad && (g + 1) * 256 > a.k) {  // (a ragged K's last group only)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int d = 0; d < 4; ++d)
#pragma unroll
                for (int tt = 0; tt < MT; ++tt) x_kmask(A[b][d][tt], a, (2 * g + b) * 128 + 32 * kq + 8 * d);
    }
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int q = 0; q < PW; ++q) {
            const float s0 = __builtin_ldexpf(1.f, (int)(e[b][q] & 0xFFu) - 133);
            const float s1 = __builtin_ldexpf(1.f, (int)((e[b][q] >> 8) & 0xFFu) - 133);
            const uint4 B0 = b_bfp4k<0>(c[b][q].x, s0);
            const uint4 B1 = b_bfp4k<1>(c[b][q].y, s0);
            const uint4 B2 = b_bfp4k<2>(c[b][q].z, s1);
            const uint4 B3 = b_bfp4k<3>(c[b][q].w, s1);
#pragma unroll
            for (int tt = 0; tt < MT; ++tt) {
                acc[q][tt] = mfma(A[b][0][tt], B0, acc[q][tt]);
                acc[q][tt] = mfma(A[b][1][tt], B1, acc[q][tt]);
                acc[q][tt] = mfma(A[b][2][tt], B2, acc[q][tt]);
                acc[q][tt] = mfma(A[b][3][tt], B3, acc[q][tt]);
            }
        }
}

// bf16, 4 blocks of 32 k: the lane's 8 values are its B as they are (k = 32 b + 8 kq + j)
template <int MT, int PW>
__device__ __forceinline__ void mgroup_bf16(const Args& a, const uint8_t* const* cb, int b0, int lane,
                                            f32x4 (&acc)[PW][MT]) {
    const int r = lane & 15, kq = lane >> 4;
    uint4 A[4][MT];
    uint4 c[4][PW];
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int tt = 0; tt < MT; ++tt) A[u][tt] = x_row8(a, 16 * tt + r, (b0 + u) * 32 + 8 * kq);
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int q = 0; q < PW; ++q) c[u][q] = ld_stream16(cb[q] + (uint32_t)((b0 + u) * 1024 + lane * 16));
    if (a.k != a.k_pad && (b0 + 4) * 32 > a.k) {  // (a ragged K's last blocks only)
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int tt = 0; tt < MT; ++tt) x_kmask(A[u][tt], a, (b0 + u) * 32 + 8 * kq);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int q = 0; q < PW; ++q)
#pragma unroll
            for (int tt = 0; tt < MT; ++tt) acc[q][tt] = mfma(A[u][tt], c[u][q], acc[q][tt]);
}

// ---- 32 rows: a wavefront's chunk in steps of 128 k, software-pipelined ---------------------------------------------
//
// Step s + 1's x is staged and its codes loaded while step s is decoded and multiplied, so one step's loads are in
// flight during the compute of the step before (without that, every wavefront of a workgroup waits for its loads and
// then computes, together, and the CU idles through half of each). Step s's x operands are read from the staging into
// registers before step s + 1's loads are issued into the same 8 KB, which keeps a workgroup's LDS small enough for
// two workgroups a CU.
//
// A chunk's 128-k units are visited rotated: chunk k0 starts at its unit (k0 / 512) mod 4 and wraps round (bf16's
// 64-k steps: at its step (k0 / 512) mod 8). The wavefronts of a workgroup take one chunk each, so without the
// rotation all of them read the same offset of their chunks at once (every chunk starts on an 8 KB boundary of its
// panel), and those reads pile onto a few of HBM's channels: C4's block list took 16.8 us in the plain order, 15.1
// with the rotation, and a plain read of the same bytes in the two orders 14.0 and 11.9 us. Each accumulator still
// sums its chunk's k in one fixed order, the same in every 32-row kernel of a format (the tile-pair and one-tile
// kernels, bfloat8_b's 64- and 128-k steps), so their results agree bit for bit. bfloat8_b and bf16 are rotated;
// bfloat4_b keeps the plain order, which measured faster for it (the MoE rows' gate_up 131.8 against 140.5 us). The
// 16-row kernel is not rotated either (C3 15.0 -> 15.8 us rotated); its wavefronts take 256-k groups in turn instead
// (dr_mfma), so a row's sums there differ in the last bits from the same row's in a 32-row launch. The rotated
// kernels load a chunk's exponent words (one or two 256-k groups) once, before its first step.
__device__ __forceinline__ int xl_rot(int k0, int units) { return ((k0 >> 9) & 3) % units; }
// the chunk's exponent words of panel q: lo for group k0 / 256, hi for the next (the same one again for a one-group
// chunk, so that no load sits under a branch)
template <int PW>
__device__ __forceinline__ void xl_exps(const uint8_t* const* eb, int k0, int k1, int lane, uint32_t (&lo)[PW],
                                        uint32_t (&hi)[PW]) {
    const int g0 = k0 >> 8, g1 = k1 - k0 > 256 ? g0 + 1 : g0;
#pragma unroll
    for (int q = 0; q < PW; ++q) {
        lo[q] = ld_stream4(eb[q] + (uint32_t)(g0 * 256 + 4 * lane));
        hi[q] = ld_stream4(eb[q] + (uint32_t)(g1 * 256 + 4 * lane));
    }
}

// x operands of one step of 8 NCH k: A[j][tt] = rows 16 tt + r, the 8 values of chunk chunk(j, kq) (zeroed past K)
template <int NCH, int NJ, typename F>
__device__ __forceinline__ void xl_operands(const Args& a, const uint4* xb, int k, int lane, uint4 (&A)[NJ][2], F chunk) {
    const int r = lane & 15, kq = lane >> 4;
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) A[j][tt] = x_lds<NCH>(xb, 16 * tt + r, chunk(j, kq));
    if (a.k != a.k_pad && k + 8 * NCH > a.k) {  // (a ragged K's last step only)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) x_kmask(A[j][tt], a, k + 8 * chunk(j, kq));
    }
}

// D: the steps whose codes are in flight (1 or 2; 2 needs an even step count, xl_chunk takes 1 otherwise). x is staged
// one step ahead in the wavefront's one staging buffer, its loads after the current step's x operands are read out.
// The issue order, x(s), c(s + D - 1), x(s + 1), c(s + D), ..., keeps the waits exact: the compiler waits for the
// newest LDS-bound load before any staging read, which then costs nothing the step did not need (its own codes);
// and every load is issued on every path (the last D steps in a block of their own, issuing no codes), since a load
// issued under a condition makes the compiler's count assume the worst and wait for every load in flight. s counts
// the steps in the order visited; the rotated chunk functions map it to their step (xl_rot). bfloat4_b's, in the
// plain order, loads a 256-k group's exponent word with the group's first step's codes and reads it at that step, so
// one copy of it serves D <= 2.
template <int D, typename IssueX, typename IssueC, typename Step>
__device__ __forceinline__ void xl_steps(int ns, IssueX issue_x, IssueC issue_c, Step step) {
    static_assert(D == 1 || D == 2, "xl_steps: one or two steps of codes in flight");
    issue_x(0);
#pragma unroll
    for (int j = 0; j < D; ++j) issue_c(j, j);
    int s0 = 0;
    for (; s0 + D < ns; s0 += D) {
#pragma unroll
        for (int j = 0; j < D; ++j)
            step(s0 + j, j, [&] {
                issue_x(s0 + j + 1);
                issue_c(s0 + j + D, j);
            });
    }
#pragma unroll
    for (int j = 0; j < D; ++j)
        step(s0 + j, j, [&] {
            if (j + 1 < D) issue_x(s0 + j + 1);  // (j is a constant here)
        });
}

// bfloat8_b: a step is blocks k / 64 and k / 64 + 1 (k0, k1 multiples of 256: a group is two steps); MFMA (b, h) takes
// k = 64 b + 16 kq + 8 h + j of the step
template <int PW, int D = 1>
__device__ __forceinline__ void xl_chunk_bfp8(const Args& a, const uint8_t* const* cb, const uint8_t* const* eb, int k0,
                                              int k1, int lane, f32x4 (&acc)[PW][2], uint4* xs) {
    static_assert(D == 1 || D == 2, "xl_chunk_bfp8: one or two steps in flight");
    const int ns = (k1 - k0) >> 7;
    if constexpr (D > 1) {
        if (ns % D) {
            xl_chunk_bfp8<PW, 1>(a, cb, eb, k0, k1, lane, acc, xs);
            return;
        }
    }
    const XStage<16> xst(a, lane);
    const int rr = xl_rot(k0, ns);
    auto kof = [&](int s) { const int t = s + rr; return k0 + 128 * (t >= ns ? t - ns : t); };
    uint32_t elo[PW], ehi[PW];
    xl_exps<PW>(eb, k0, k1, lane, elo, ehi);
    uint4 cn[D][2][PW];
    auto issue_x = [&](int s) { xst.stage(kof(s), xs); };
    auto issue_c = [&](int s, int slot) {
        const int k = kof(s);
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int q = 0; q < PW; ++q)
                cn[slot][b][q] = ld_stream16(cb[q] + (uint32_t)(((k >> 6) + b) * 1024 + lane * 16));
    };
    auto step = [&](int s, int j, auto next) {
        const int k = kof(s);
        const bool hi = k - k0 >= 256;
        uint4 c[2][PW];
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int q = 0; q < PW; ++q) c[b][q] = cn[j][b][q];
        uint4 A[4][2];  // [2 b + h][tt]
        xl_operands<16, 4>(a, xs, k, lane, A, [](int jj, int kq) { return 8 * (jj >> 1) + 2 * kq + (jj & 1); });
        next();
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int q = 0; q < PW; ++q) {
                const uint32_t ew = hi ? ehi[q] : elo[q];
                const float sc = __builtin_ldexpf(1.f, (int)((ew >> (8 * (((k >> 6) & 3) + b))) & 0xFFu) - 133);
                const uint4 B0 = b_bfp8<0>(c[b][q], sc);
                const uint4 B1 = b_bfp8<1>(c[b][q], sc);
#pragma unroll
                for (int tt = 0; tt < 2; ++tt) {
                    acc[q][tt] = mfma(A[2 * b][tt], B0, acc[q][tt]);
                    acc[q][tt] = mfma(A[2 * b + 1][tt], B1, acc[q][tt]);
                }
            }
    };
    xl_steps<D>(ns, issue_x, issue_c, step);
}

// bfloat8_b one block a step (64 k, its codes 1 KB a panel): half the bytes of a step in flight, for wide tiles
// (dr_mfma_pairs' four panels); MFMA h of the step takes k = 16 kq + 8 h + j. Sums in the order of xl_chunk_bfp8.
template <int PW, int D = 1>
__device__ __forceinline__ void xl_chunk_bfp8_b1(const Args& a, const uint8_t* const* cb, const uint8_t* const* eb,
                                                 int k0, int k1, int lane, f32x4 (&acc)[PW][2], uint4* xs) {
    static_assert(D == 1 || D == 2, "xl_chunk_bfp8_b1: one or two steps in flight");
    const int ns = (k1 - k0) >> 6;
    if constexpr (D > 1) {
        if (ns % D) {
            xl_chunk_bfp8_b1<PW, 1>(a, cb, eb, k0, k1, lane, acc, xs);
            return;
        }
    }
    const XStage<8> xst(a, lane);
    const int rr = 2 * xl_rot(k0, ns >> 1);  // (in 128-k units, as xl_chunk_bfp8)
    auto kof = [&](int s) { const int t = s + rr; return k0 + 64 * (t >= ns ? t - ns : t); };
    uint32_t elo[PW], ehi[PW];
    xl_exps<PW>(eb, k0, k1, lane, elo, ehi);
    uint4 cn[D][PW];
    auto issue_x = [&](int s) { xst.stage(kof(s), xs); };
    auto issue_c = [&](int s, int slot) {
        const int k = kof(s);
#pragma unroll
        for (int q = 0; q < PW; ++q) cn[slot][q] = ld_stream16(cb[q] + (uint32_t)((k >> 6) * 1024 + lane * 16));
    };
    auto step = [&](int s, int j, auto next) {
        const int k = kof(s);
        const bool hi = k - k0 >= 256;
        uint4 c[PW];
#pragma unroll
        for (int q = 0; q < PW; ++q) c[q] = cn[j][q];
        uint4 A[2][2];  // [h][tt]
        xl_operands<8, 2>(a, xs, k, lane, A, [](int jj, int kq) { return 2 * kq + jj; });
        next();
#pragma unroll
        for (int q = 0; q < PW; ++q) {
            const uint32_t ew = hi ? ehi[q] : elo[q];
            const float sc = __builtin_ldexpf(1.f, (int)((ew >> (8 * ((k >> 6) & 3))) & 0xFFu) - 133);
            const uint4 B0 = b_bfp8<0>(c[q], sc);
            const uint4 B1 = b_bfp8<1>(c[q], sc);
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                acc[q][tt] = mfma(A[0][tt], B0, acc[q][tt]);
                acc[q][tt] = mfma(A[1][tt], B1, acc[q][tt]);
            }
        }
    };
    xl_steps<D>(ns, issue_x, issue_c, step);
}

// bfloat4_b: a step is block k / 128; MFMA D takes k = 32 kq + 8 D + j of the step
template <int PW, int D = 1>
__device__ __forceinline__ void xl_chunk_bfp4(const Args& a, const uint8_t* const* cb, const uint8_t* const* eb, int k0,
                                              int k1, int lane, f32x4 (&acc)[PW][2], uint4* xs, uint32_t xbytes = 0) {
    static_assert(D == 1 || D == 2, "xl_chunk_bfp4: one or two steps in flight");
    const int ns = (k1 - k0) >> 7;
    if constexpr (D > 1) {
        if (ns % D) {
            xl_chunk_bfp4<PW, 1>(a, cb, eb, k0, k1, lane, acc, xs, xbytes);
            return;
        }
    }
    const XStage<16> xst(a, lane, xbytes);
    uint4 cn[D][PW];
    uint32_t en[PW], e[PW];
    auto issue_x = [&](int s) { xst.stage(k0 + 128 * s, xs); };
    auto issue_c = [&](int s, int slot) {
        const int k = k0 + 128 * s;
        if (!(s & 1)) {
#pragma unroll
            for (int q = 0; q < PW; ++q) en[q] = ld_stream4(eb[q] + (uint32_t)(k + 4 * lane));
        }
#pragma unroll
        for (int q = 0; q < PW; ++q)
            cn[slot][q] = ld_stream16(cb[q] + (uint32_t)(real_block(k >> 7, a.k) * 1024 + lane * 16));
    };
    auto step = [&](int s, int j, auto next) {
        const int k = k0 + 128 * s;
        uint4 c[PW];
#pragma unroll
        for (int q = 0; q < PW; ++q) c[q] = cn[j][q];
        if (!(s & 1)) {
#pragma unroll
            for (int q = 0; q < PW; ++q) e[q] = en[q];
        }
        uint4 A[4][2];  // [D][tt]
        xl_operands<16, 4>(a, xs, k, lane, A, [](int jj, int kq) { return 4 * kq + jj; });
        next();
#pragma unroll
        for (int q = 0; q < PW; ++q) {
            const uint32_t ep = e[q] >> (16 * (s & 1));
            const float s0f = __builtin_ldexpf(1.f, (int)(ep & 0xFFu) - 133);
            const float s1f = __builtin_ldexpf(1.f, (int)((ep >> 8) & 0xFFu) - 133);
            const uint4 B0 = b_bfp4<0>(c[q].x, s0f, s1f);
            const uint4 B1 = b_bfp4<1>(c[q].y, s0f, s1f);
            const uint4 B2 = b_bfp4<2>(c[q].z, s0f, s1f);
            const uint4 B3 = b_bfp4<3>(c[q].w, s0f, s1f);
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                acc[q][tt] = mfma(A[0][tt], B0, acc[q][tt]);
                acc[q][tt] = mfma(A[1][tt], B1, acc[q][tt]);
                acc[q][tt] = mfma(A[2][tt], B2, acc[q][tt]);
                acc[q][tt] = mfma(A[3][tt], B3, acc[q][tt]);
            }
        }
    };
    xl_steps<D>(ns, issue_x, issue_c, step);
}

// bf16: a step is 64 k, blocks k / 32 and k / 32 + 1 (its 4 KB of codes a panel pair: half the bfloat8_b step's
// registers for a 128-k step's 8 KB); MFMA u takes k = 32 u + 8 kq + j of the step
template <int PW, int D = 1>
__device__ __forceinline__ void xl_chunk_bf16(const Args& a, const uint8_t* const* cb, int k0, int k1, int lane,
                                              f32x4 (&acc)[PW][2], uint4* xs) {
    static_assert(D == 1 || D == 2, "xl_chunk_bf16: one or two steps in flight");
    const int ns = (k1 - k0) >> 6;
    if constexpr (D > 1) {
        if (ns % D) {
            xl_chunk_bf16<PW, 1>(a, cb, k0, k1, lane, acc, xs);
            return;
        }
    }
    const XStage<8> xst(a, lane);
    const int rr = ((k0 >> 9) & 7) % ns;  // (in its 64-k steps: C4 14.9 -> 14.8 us against 128-k units)
    auto kof = [&](int s) { const int t = s + rr; return k0 + 64 * (t >= ns ? t - ns : t); };
    uint4 cn[D][2][PW];
    auto issue_x = [&](int s) { xst.stage(kof(s), xs); };
    auto issue_c = [&](int s, int slot) {
        const int k = kof(s);
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int q = 0; q < PW; ++q)
                cn[slot][u][q] = ld_stream16(cb[q] + (uint32_t)(((k >> 5) + u) * 1024 + lane * 16));
    };
    auto step = [&](int s, int j, auto next) {
        const int k = kof(s);
        uint4 c[2][PW];
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int q = 0; q < PW; ++q) c[u][q] = cn[j][u][q];
        uint4 A[2][2];  // [u][tt]
        xl_operands<8, 2>(a, xs, k, lane, A, [](int jj, int kq) { return 4 * jj + kq; });
        next();
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int q = 0; q < PW; ++q)
#pragma unroll
                for (int tt = 0; tt < 2; ++tt) acc[q][tt] = mfma(A[u][tt], c[u][q], acc[q][tt]);
    };
    xl_steps<D>(ns, issue_x, issue_c, step);
}

template <int MT, int PW, int FMT, bool ONE>
__global__ __launch_bounds__(512, MT == 2 ? 4 : 1) void dr_mfma(const Args a) {  // (32 rows: 4 wavefronts a SIMD, so
                                                                                 // two workgroups a CU)
    constexpr int ROWS = 16 * MT;
    extern __shared__ float part[];  // [W][PW][ROWS][16]
    __shared__ float tval[ROWS][TILE];
    __shared__ __align__(16) uint32_t tkey[ROWS][TILE];

    const int g = blockIdx.x % a.tiles, split = blockIdx.x / a.tiles;
    const SegDev& sg = a.seg[find_segment<ONE>(a, g)];
    const int t = g - sg.tile_begin;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int fmt = FMT >= 0 ? FMT : sg.fmt;
    const uint8_t* cb[PW];
    const uint8_t* eb[PW];
    panel_ptrs<PW>(sg, t, a.k_pad, cb, eb);
    __shared__ float pre[PRE_FLOATS];
    const EpiPre ep = epi_prefetch<ROWS, PW>(a, sg, t);

    f32x4 acc[PW][MT];  // this wavefront's sums over its chunks (16 rows: its groups), in order
#pragma unroll
    for (int q = 0; q < PW; ++q)
#pragma unroll
        for (int tt = 0; tt < MT; ++tt) acc[q][tt] = f32x4{0.f, 0.f, 0.f, 0.f};
    // 32 rows: x through the wavefront's LDS staging, which the partial sums overwrite after the K loop
    constexpr bool XL = MT == 2;
    uint4* xs = reinterpret_cast<uint4*>(part) + wave * (XS_BYTES / 16);
    const int ch1 = min((split + 1) * a.cps, a.chunks);
    if constexpr (XL) {
        for (int ch = split * a.cps + wave; ch < ch1; ch += a.waves) {
            const int k0 = ch * a.kch, k1 = min(k0 + a.kch, a.k_pad);
            if (fmt == DR_BFP8) xl_chunk_bfp8<PW>(a, cb, eb, k0, k1, lane, acc, xs);
            else if (fmt == DR_BFP4) xl_chunk_bfp4<PW>(a, cb, eb, k0, k1, lane, acc, xs);
            else xl_chunk_bf16<PW>(a, cb, k0, k1, lane, acc, xs);
        }
    } else {
        // 16 rows: the wavefronts take the split's 256-k groups in turn (wavefront w groups w, w + W, ...), each one
        // group at a time, so at any moment they read consecutive 4 KB of a panel rather than the same offset of
        // their 512-k chunks (C3 15.0 -> 14.5 us; in a plain read of C3's bytes 10.0 -> 9.6)
        const int g0 = (split * a.cps * a.kch) >> 8, g1 = min(ch1 * a.kch, a.k_pad) >> 8;
        for (int gg = g0 + wave; gg < g1; gg += a.waves) {
            if (fmt == DR_BFP8) mgroup_bfp8<MT, PW>(a, cb, eb, gg, lane, acc);
            else if (fmt == DR_BFP4) mgroup_bfp4<MT, PW>(a, cb, eb, gg, lane, acc);
            else {
                mgroup_bf16<MT, PW>(a, cb, 8 * gg, lane, acc);
                mgroup_bf16<MT, PW>(a, cb, 8 * gg + 4, lane, acc);
            }
        }
    }
    if constexpr (XL) __syncthreads();  // (every wavefront done with its staging before any partial lands on it)
#pragma unroll
    for (int q = 0; q < PW; ++q)
#pragma unroll
        for (int tt = 0; tt < MT; ++tt)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                part[((wave * PW + q) * ROWS + 16 * tt + 4 * (lane >> 4) + j) * 16 + (lane & 15)] = acc[q][tt][j];
    epi_stage(ep, pre);
    __syncthreads();
    const int nparts = gather_splits<ROWS, PW>(a, g, split, part);
    if (nparts) epilogue<ROWS, PW>(a, sg, t, part, nparts, tval, tkey, wave, lane, pre);
}

// ---- 32 rows, two tiles a workgroup -------------------------------------------------------------------------------
//
// A 32-row launch of more tiles than CUs: each workgroup of a block-float segment computes two adjacent 32-column
// tiles (the last pair of an odd count, one). Its wavefronts stage their x once for four panels, so x's traffic into
// the CU and the workgroup's fixed cost (its start, barriers, epilogue) are paid once a pair, and the launch has fewer
// workgroups (C4's 192 bfloat8_b tiles: 96, beside the 128 bf16 tiles: 224 workgroups, one round on 256 CUs, where 64
// CUs had had two tiles one after the other). bf16 segments keep a tile a workgroup: their weights are twice x's bytes
// a tile, and pairing them halved the workgroups for little saved (the NS shape at 32 rows: 28.2 -> 29.9 us, against
// bfloat8_b's 21.5 -> 19.6). Each tile's panels are summed by the same lanes, steps and wavefronts in the same order as
// in dr_mfma<2, 2>, so the results are the same bit for bit. Plain tiles only: no top-k records, GLU, residual or
// split K.
template <int PW, int FMT>  // PW 4: two tiles, 2: one
__device__ __forceinline__ void pair_tiles(const Args& a, const SegDev& sg, int t0, int nt, int fmt, int wave,
                                           int lane, float* part) {
    constexpr int ROWS = 32;
    const uint8_t* cb[PW];
    const uint8_t* eb[PW];
#pragma unroll
    for (int q = 0; q < PW; ++q) {
        const int pan = 2 * (t0 + (nt == 2 ? q >> 1 : 0)) + (q & 1);
        cb[q] = sg.codes + (size_t)pan * sg.pstride;
        eb[q] = sg.exps + (size_t)pan * a.k_pad;
    }
    f32x4 acc[PW][2];
#pragma unroll
    for (int q = 0; q < PW; ++q)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) acc[q][tt] = f32x4{0.f, 0.f, 0.f, 0.f};
    // what the epilogue reads of the arguments, loaded now
    const int n_out = pin(sg.n_out), col0 = pin(sg.col0), mrows = pin(a.m), ldy = pin(a.ldy), y_f32 = pin(a.y_f32);
    void* const y = pin(a.y);
    // the tiles' column scales, read before the K loop (after it, their round trip would end the workgroup)
    __shared__ float psc[2][TILE];
    float sc = 1.f;
    const int su = (int)threadIdx.x >> 5, scol = (int)threadIdx.x & (TILE - 1);
    if (su < nt && (t0 + su) * TILE + scol < sg.n_out) sc = load_scale(sg.scale, sg.scale_f32, (t0 + su) * TILE + scol);
    uint4* xs = reinterpret_cast<uint4*>(part) + wave * (XS_BYTES / 16);
    for (int ch = wave; ch < a.chunks; ch += a.waves) {
        const int k0 = ch * a.kch, k1 = min(k0 + a.kch, a.k_pad);
        if (fmt == DR_BFP8) xl_chunk_bfp8_b1<PW, 1>(a, cb, eb, k0, k1, lane, acc, xs);
        else if (fmt == DR_BFP4) xl_chunk_bfp4<PW, PAIR_D>(a, cb, eb, k0, k1, lane, acc, xs);
        else xl_chunk_bf16<PW, 1>(a, cb, k0, k1, lane, acc, xs);  // (two in flight: C4 14.8 -> 15.0 us)
    }
    __syncthreads();  // (every wavefront done with its staging before any partial lands on it)
    // the partial sums by column: pt[tile][wave][panel][16 columns][PAIR_RS rows] (4 rows of padding: the lanes of a
    // 16-byte access land on distinct banks), each lane's 4 rows of a 16-row block one 16-byte store
    const int W = a.waves;
#pragma unroll
    for (int q = 0; q < PW; ++q)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
            *reinterpret_cast<f32x4*>(part + ((((q >> 1) * W + wave) * 2 + (q & 1)) * 16 + (lane & 15)) * PAIR_RS +
                                      16 * tt + 4 * (lane >> 4)) = acc[q][tt];
    if (su < 2) psc[su][scol] = sc;
    __syncthreads();
    // item (tile u, column c, rows m0 .. m0 + 3), 256 a tile, the workgroup's threads taking them in turn: the
    // wavefronts' sums in order, times the column's scale, to y
    for (int it = (int)threadIdx.x; it < 256 * nt; it += 64 * W) {
        const int u = it >> 8, c = it & 31, m0 = 4 * ((it & 255) >> 5);
        const int oc = (t0 + u) * TILE + c;
        if (oc >= n_out || m0 >= mrows) continue;
        const float* src = part + ((u * W * 2 + (c >> 4)) * 16 + (c & 15)) * PAIR_RS + m0;
        f32x4 v = {0.f, 0.f, 0.f, 0.f};
        for (int w0 = 0; w0 < W; w0 += 8) {
            f32x4 t[8];
#pragma unroll
            for (int j = 0; j < 8; ++j)
                t[j] = w0 + j < W ? *reinterpret_cast<const f32x4*>(src + (size_t)(w0 + j) * 2 * 16 * PAIR_RS) : v;
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (w0 + j < W) {
                    v[0] += t[j][0];
                    v[1] += t[j][1];
                    v[2] += t[j][2];
                    v[3] += t[j][3];
                }
        }
        const float scv = psc[u][c];
        const size_t y0 = (size_t)m0 * ldy + col0 + oc;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (m0 + j >= mrows) break;
            const float o = v[j] * scv;
            if (y_f32)
                reinterpret_cast<float*>(y)[y0 + (size_t)j * ldy] = o;
            else
                reinterpret_cast<uint16_t*>(y)[y0 + (size_t)j * ldy] = (uint16_t)f32_to_bf16(o);
        }
    }
}

template <int FMT, bool ONE>
__global__ __launch_bounds__(512) void dr_mfma_pairs(const Args a) {
    extern __shared__ float part[];  // x staging during the K loop; then [tiles][W][2][16][PAIR_RS]
    const int gp = blockIdx.x;
    int si = 0;
    if (!ONE) {
#pragma unroll
        for (int j = 1; j < 4; ++j)
            if (j < a.nseg && gp >= a.pair_begin[j]) si = j;
    }
    const SegDev& sg = a.seg[si];
    const int per = a.pair_tiles[si];  // (uniform)
    const int t0 = per * (gp - a.pair_begin[si]);
    const int nt = sg.tiles - t0 < per ? sg.tiles - t0 : per;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int fmt = FMT >= 0 ? FMT : sg.fmt;
    if (nt == 2)
        pair_tiles<4, FMT>(a, sg, t0, nt, fmt, wave, lane, part);
    else
        pair_tiles<2, FMT>(a, sg, t0, nt, fmt, wave, lane, part);
}

template <int MT, int PW, int MOE, bool KB>
__global__ __launch_bounds__(512) void dr_mfma_moe(const MoeArgs a) {
    constexpr int ROWS = 16 * MT;
    extern __shared__ float part[];  // [W][PW][ROWS][16]
    __shared__ float tval[ROWS][TILE];
    __shared__ __align__(16) uint32_t tkey[ROWS][TILE];

    const int g = blockIdx.x % a.tiles, split = blockIdx.x / a.tiles;
    const SegDev& sg = a.seg[0];
    int t = g - sg.tile_begin;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    // the expert gather, as dr_gemv_moe's (the rows modes past two rows)
    UnionLds* ul = nullptr;
    if constexpr (MOE == DR_MOE_GATE_UP_ROWS || MOE == DR_MOE_DOWN_ROWS) {
        ul = union_lds<MOE>();
        moe_union(a, *ul);
    }
    int unit = 0, ex = 0;
    if constexpr (moe_n<MOE>()) {
        unit = t / a.tpe;
        t -= unit * a.tpe;
        ex = MOE == DR_MOE_GATE_UP ? moe_id(a, 0, unit) : (unit < ul->count ? (int)ul->list[unit] : -1);
        ex = __builtin_amdgcn_readfirstlane(ex);
        if (ex < 0) {
            if (MOE == DR_MOE_GATE_UP && split == 0) moe_zero<PW>(a, t, unit);
            return;
        }
    }
    const uint8_t* cb[PW];
    const uint8_t* eb[PW];
    panel_ptrs<PW>(sg, t, moe_k<MOE>() ? a.ekp : a.k_pad, cb, eb);
    if constexpr (moe_n<MOE>()) {
#pragma unroll
        for (int q = 0; q < PW; ++q) {
            cb[q] += (size_t)ex * a.cstride;
            eb[q] += (size_t)ex * a.estride;
        }
    }

    f32x4 acc[PW][MT];  // this wavefront's sums over its chunks, in order
#pragma unroll
    for (int q = 0; q < PW; ++q)
#pragma unroll
        for (int tt = 0; tt < MT; ++tt) acc[q][tt] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto chunk = [&](const Args& b, const uint8_t* const* cbx, const uint8_t* const* ebx, int k0, int k1) {
        for (int gg = k0 >> 8; gg < (k1 >> 8); ++gg) {
            if constexpr (KB)
                mgroup_bfp4k<MT, PW>(b, cbx, ebx, gg, lane, acc);
            else
                mgroup_bfp4<MT, PW>(b, cbx, ebx, gg, lane, acc);
        }
    };
    // DR_MOE_DOWN: every slot's id, lane j slot j, read once (a chunk then takes its unit's id from a lane, not from
    // memory: one dependent round trip fewer a chunk)
    int idv = -1;
    if constexpr (MOE == DR_MOE_DOWN) idv = lane < a.slots ? moe_id(a, 0, lane) : -1;
    // 32 rows: x through each wavefront's LDS staging, as the dense 32-row kernel reads it (the same sums; x read in
    // whole lines). The down's chunk views x from its unit's block on, so its staging may read only up to x's end.
    constexpr bool XLG = MOE == DR_MOE_GATE_UP_ROWS && MT == 2 && !KB;
    constexpr bool XLD = MOE == DR_MOE_DOWN_ROWS && MT == 2 && !KB;
    uint4* xs = reinterpret_cast<uint4*>(part) + wave * (XS_BYTES / 16);
    const int ch1 = min((split + 1) * a.cps, a.chunks);
    for (int ch = split * a.cps + wave; ch < ch1; ch += a.waves) {
        const int k0 = ch * a.kch, k1 = min(k0 + a.kch, a.k_pad);
        if constexpr (moe_k<MOE>()) {
            const int s = __builtin_amdgcn_readfirstlane(k0 / a.ekp);
            int e = MOE == DR_MOE_DOWN ? __builtin_amdgcn_readlane(idv, s) : (s < ul->count ? (int)ul->list[s] : -1);
            e = __builtin_amdgcn_readfirstlane(e);
            if (e < 0) continue;
            Args b = a;  // (the chunk's view of x: the unit's block)
            b.x = a.x + (size_t)s * a.ek;
            b.k = a.ek;
            b.k_pad = a.ekp;
            const uint8_t* cbe[PW];
            const uint8_t* ebe[PW];
#pragma unroll
            for (int q = 0; q < PW; ++q) {
                cbe[q] = cb[q] + (size_t)e * a.cstride;
                ebe[q] = eb[q] + (size_t)e * a.estride;
            }
            if constexpr (XLD) {
                const uint32_t xb = 2u * (uint32_t)a.ldx * (uint32_t)a.m - 2u * (uint32_t)(s * a.ek);  // (to x's end)
                xl_chunk_bfp4<PW>(b, cbe, ebe, k0 - s * a.ekp, k1 - s * a.ekp, lane, acc, xs, xb);
            } else {
                chunk(b, cbe, ebe, k0 - s * a.ekp, k1 - s * a.ekp);
            }
        } else {
            if constexpr (XLG)
                xl_chunk_bfp4<PW>(a, cb, eb, k0, k1, lane, acc, xs);
            else
                chunk(a, cb, eb, k0, k1);
        }
    }
    if constexpr (XLG || XLD) __syncthreads();  // (every wavefront done with its staging before any partial lands on it)
#pragma unroll
    for (int q = 0; q < PW; ++q)
#pragma unroll
        for (int tt = 0; tt < MT; ++tt)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                part[((wave * PW + q) * ROWS + 16 * tt + 4 * (lane >> 4) + j) * 16 + (lane & 15)] = acc[q][tt][j];
    __syncthreads();
    const int nparts = gather_splits<ROWS, PW>(a, g, split, part);
    if (!nparts) return;
    if constexpr (moe_n<MOE>())
        epilogue_moe<ROWS, PW, MOE>(a, t, unit, ex, part, nparts, 0.f);
    else
        epilogue<ROWS, PW>(a, sg, t, part, nparts, tval, tkey, wave, lane);
}

// DR_MOE_GATE_UP_ROWS at 32 rows: two adjacent 32-column tiles of one unit's expert a workgroup, so the wavefronts'
// staged x serves both (the unit's tiles in pairs, the last of an odd count alone): the gpt-oss gate/up at 17, 24 and
// 32 rows 122, 135, 148 -> 107, 125, 128 us. Each tile's panels are summed by the same lanes, steps and wavefronts in
// the same order as in dr_mfma_moe<2, 4> (xl_chunk_bfp4 over more panels), so the results do not change.
template <int NT>
__device__ __forceinline__ void moe_pair_tiles(const MoeArgs& a, int t0, int unit, int ex, int wave, int lane,
                                               float* part) {
    constexpr int PW = 4 * NT, ROWS = 32;
    const SegDev& sg = a.seg[0];
    const uint8_t* cb[PW];
    const uint8_t* eb[PW];
#pragma unroll
    for (int u = 0; u < NT; ++u) {
        const uint8_t* c4[4];
        const uint8_t* e4[4];
        panel_ptrs<4>(sg, t0 + u, a.k_pad, c4, e4);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            cb[4 * u + q] = c4[q] + (size_t)ex * a.cstride;
            eb[4 * u + q] = e4[q] + (size_t)ex * a.estride;
        }
    }
    f32x4 acc[PW][2];
#pragma unroll
    for (int q = 0; q < PW; ++q)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) acc[q][tt] = f32x4{0.f, 0.f, 0.f, 0.f};
    uint4* xs = reinterpret_cast<uint4*>(part) + wave * (XS_BYTES / 16);
    for (int ch = wave; ch < a.chunks; ch += a.waves) {
        const int k0 = ch * a.kch, k1 = min(k0 + a.kch, a.k_pad);
        xl_chunk_bfp4<PW>(a, cb, eb, k0, k1, lane, acc, xs);
    }
#pragma unroll
    for (int u = 0; u < NT; ++u) {
        __syncthreads();  // (the staging, or the previous tile's epilogue, done with part)
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    part[((wave * 4 + q) * ROWS + 16 * tt + 4 * (lane >> 4) + j) * 16 + (lane & 15)] = acc[4 * u + q][tt][j];
        __syncthreads();
        epilogue_moe<ROWS, 4, DR_MOE_GATE_UP_ROWS>(a, t0 + u, unit, ex, part, a.waves, 0.f);
    }
}

__global__ __launch_bounds__(512) void dr_mfma_moe_pairs(const MoeArgs a) {
    extern __shared__ float part[];  // the x staging during the K loop; then one tile's [W][4][32][16]
    UnionLds* ul = union_lds<DR_MOE_GATE_UP_ROWS>();
    moe_union(a, *ul);
    const int tp2 = (a.tpe + 1) / 2;
    const int unit = blockIdx.x / tp2, t0 = 2 * (blockIdx.x - unit * tp2);
    const int ex = __builtin_amdgcn_readfirstlane(unit < ul->count ? (int)ul->list[unit] : -1);
    if (ex < 0) return;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (a.tpe - t0 >= 2)
        moe_pair_tiles<2>(a, t0, unit, ex, wave, lane, part);
    else
        moe_pair_tiles<1>(a, t0, unit, ex, wave, lane, part);
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
#pragma unroll
    for (int i = 0; i < 8; ++i) exps[(size_t)p * k_pad + exp_off(FMT, kk0 + i)] = (uint8_t)ex[i];
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

// DR_BFP4_KB: one thread a (column, 16-k group): the group's shared exponent and its 16 codes (bfloat4_b's rounding,
// bfp_face_row, over 16 consecutive K at one N), the codes in bfloat4_b's code layout (two dwords of the lane's four)
__global__ __launch_bounds__(256) void dr_pack_kb_k(const float* __restrict__ w, long long ld_w, int n, int k,
                                                    const float* __restrict__ cdiv, uint8_t* __restrict__ codes,
                                                    uint8_t* __restrict__ exps, int n_pad, int k_pad) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const int kgroups = k_pad / 16;
    if (idx >= (long long)n_pad * kgroups) return;
    const int col = (int)(idx / kgroups), kg = (int)(idx % kgroups);
    const int p = col / 16, c = col % 16, k0 = kg * 16;
    const float d = (cdiv != nullptr && col < n) ? cdiv[col] : 1.f;
    float v[16];
#pragma unroll
    for (int t = 0; t < 16; ++t) {
        const int kk = k0 + t;
        float x = (col < n && kk < k) ? w[(long long)col * ld_w + kk] : 0.f;
        if (cdiv != nullptr && col < n) x = x / d;
        v[t] = x;
    }
    int sm[16];
    const uint32_t ex = bfp_face_row<3>(v, sm);
    exps[(size_t)p * k_pad + exp_off_kb(k0, c)] = (uint8_t)ex;
    const int b = k0 / 128, kq = (k0 % 128) / 32, h = (k0 % 32) / 16;
    uint32_t word[2] = {0u, 0u};
#pragma unroll
    for (int half = 0; half < 2; ++half)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t ulo = (uint32_t)(sm[8 * half + j] + 8), uhi = (uint32_t)(sm[8 * half + 4 + j] + 8);
            word[half] |= (ulo | (uhi << 4)) << (8 * j);
        }
    *reinterpret_cast<uint2*>(codes + (size_t)p * (k_pad / 128) * 1024 + (size_t)b * 1024 + (kq * 16 + c) * 16 + h * 8) =
        make_uint2(word[0], word[1]);
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
        const int e = exps[(size_t)p * k_pad + (FMT == DR_BFP4_KB ? exp_off_kb(kk, c) : exp_off(FMT, kk))];
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

// int4 codes q [n][ldq] (-7..7) to the bfloat4_b code layout (u = q + 8): one thread per (panel, k-block, lane), the
// lane's 16 bytes (dword d: k 8 d + j low, 8 d + 4 + j high, of its 32 k)
__global__ __launch_bounds__(256) void dr_pack_int4_k(const int8_t* __restrict__ q, long long ldq, int n, int k,
                                                      uint8_t* __restrict__ codes, int n_pad, int k_pad) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const int nblk = k_pad / 128;
    if (idx >= (long long)(n_pad / 16) * nblk * 64) return;
    const int lane = (int)(idx & 63), b = (int)((idx >> 6) % nblk), p = (int)((idx >> 6) / nblk);
    const int col = 16 * p + (lane & 15), kb = 128 * b + 32 * (lane >> 4);
    uint32_t w[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        uint32_t v = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int klo = kb + 8 * d + j, khi = klo + 4;
            const uint32_t lo = (col < n && klo < k) ? (uint32_t)(q[(size_t)col * ldq + klo] + 8) : 8u;
            const uint32_t hi = (col < n && khi < k) ? (uint32_t)(q[(size_t)col * ldq + khi] + 8) : 8u;
            v |= ((lo & 15u) | ((hi & 15u) << 4)) << (8 * j);
        }
        w[d] = v;
    }
    *reinterpret_cast<uint4*>(codes + (size_t)p * nblk * 1024 + (size_t)b * 1024 + lane * 16) =
        make_uint4(w[0], w[1], w[2], w[3]);
}

// int4 group scales s [n][lds] bf16 to [panel][k-block][kq][c]: the scale of column 16 p + c and group 4 b + kq
__global__ __launch_bounds__(256) void dr_pack_int4_scales_k(const uint16_t* __restrict__ s, long long lds, int n,
                                                             int k, uint16_t* __restrict__ out, int n_pad, int k_pad) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const int nblk = k_pad / 128;
    if (idx >= (long long)(n_pad / 16) * nblk * 64) return;
    const int lane = (int)(idx & 63), b = (int)((idx >> 6) % nblk), p = (int)((idx >> 6) / nblk);
    const int col = 16 * p + (lane & 15), g = 4 * b + (lane >> 4);
    out[idx] = (col < n && g < k / 32) ? s[(size_t)col * lds + g] : (uint16_t)0;
}

// ---- top-k merge -----------------------------------------------------------------------------------------------------
//
// Every slot of a row becomes a 64-bit key: the record's key (fp32 scores in key_f32's order, or the bf16 key as it
// is) above its id complemented, 0 for an empty slot. The keys are distinct, so the best k_out are one set whatever
// order the work runs in; wave_select.h's select_row finds them over several workgroups a row.

constexpr int MERGE_MAXK = 64;  // k_out at most: one list is one value a lane

using namespace wsel;

template <bool NARROW>  // k_out <= 32
__global__ __launch_bounds__(SEL_T) void dr_merge_k(SelArgs A, int fp32, float* __restrict__ vals,
                                                    int32_t* __restrict__ ids) {
    __shared__ SelShared sh;
    const int r = blockIdx.x % A.rows, sl = blockIdx.x / A.rows;
    const int lane = threadIdx.x & 63;
    unsigned long long list;
    int count;
    const bool mine = select_row<NARROW>(
        A, r, sl,
        [fp32](uint32_t key, uint32_t id, uint32_t) -> unsigned long long {
            if (id == 0xFFFFFFFFu || (!fp32 && key == 0u)) return 0ull;
            const uint32_t ok = fp32 ? key_f32(__uint_as_float(key)) : key;
            return ((unsigned long long)ok << 32) | (unsigned long long)(0xFFFFFFFFu - id);
        },
        sh, list, count);
    if (!mine || threadIdx.x >= 64 || lane >= A.keep) return;
    float val = -__builtin_huge_valf();
    int32_t id = -1;
    if (list != 0ull) {
        const uint32_t ok = (uint32_t)(list >> 32);
        id = (int32_t)(0xFFFFFFFFu - (uint32_t)(list & 0xFFFFFFFFu));
        if (fp32) {
            val = __uint_as_float((ok >> 31) ? (ok ^ 0x80000000u) : ~ok);
        } else {
            const uint32_t bits = ok >= 0x8000u ? (ok & 0x7FFFu) : (~ok & 0xFFFFu);
            val = __uint_as_float(bits << 16);
        }
    }
    vals[(size_t)r * A.keep + lane] = val;
    ids[(size_t)r * A.keep + lane] = id;
}

// ---- the read ceiling (measurement) --------------------------------------------------------------------------------
//
// A plain streaming read with every CU, the ceiling the matmul's weight bandwidth is compared against: one workgroup
// of READ_T threads a READ_T * READ_U * 16-byte slice, each thread's READ_U non-temporal 16-byte loads all issued
// before any is used (of the shapes tried on MI355X -- slices of 32 KB to 128 KB a workgroup, or a persistent grid of
// one or two workgroups a CU looping over the buffer -- the 32 KB slices read fastest). The loaded words are folded and
// compared with a value they never take, so the loads stay and nothing is written.
constexpr int READ_T = 512, READ_U = 4;

__global__ __launch_bounds__(READ_T) void dr_read_k(const u32x4_t* __restrict__ p, long long n16, uint32_t* sink) {
    const long long base = (long long)blockIdx.x * READ_T * READ_U + threadIdx.x;
    u32x4_t v[READ_U];
#pragma unroll
    for (int u = 0; u < READ_U; ++u) {
        const long long i = min(base + (long long)u * READ_T, n16 - 1);
        v[u] = __builtin_nontemporal_load(p + i);
    }
    uint32_t acc = 0;
#pragma unroll
    for (int u = 0; u < READ_U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    if (acc == 0x9E3779B9u && threadIdx.x == 0) sink[0] = acc;
}

inline hipStream_t S(void* s) { return reinterpret_cast<hipStream_t>(s); }

int hip_status(hipError_t e) { return e == hipSuccess ? DR_OK : DR_EHIP; }

// CUs of the current device (read once a device; 256 if it cannot be read)
int cu_count() {
    static std::atomic<int> cus[64];
    int d = 0;
    if (hipGetDevice(&d) != hipSuccess || d < 0 || d >= 64) return 256;
    int v = cus[d].load(std::memory_order_relaxed);
    if (v == 0) {
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, d) != hipSuccess || v <= 0) v = 256;
        cus[d].store(v, std::memory_order_relaxed);
    }
    return v;
}

// whether 16-column tiles lower the most that any CU streams against `tiles` 32-column ones: ceil(2 T / C) halves
// against ceil(T / C) whole tiles (128 tiles: one half against one tile; 360: three halves against two tiles; 448:
// four halves, two tiles, the same)
bool narrow_better(int tiles) {
    const int c = cu_count();
    return (2 * tiles + c - 1) / c < 2 * ((tiles + c - 1) / c);
}

// the K range of one chunk: 512 (two exponent groups) past K = 2048, else 256 (K = 2048: eight wavefronts of one group
// each, rather than four of two: the bfloat8_b GEMV at N = 4096 4.30 -> 4.09 us). The MFMA kernel (16 or 32 rows a
// pass), which walks a chunk's groups one after another, takes 256 up to K = 3072 too, so that a tile has eight
// wavefronts rather than six or fewer (K = 2304 and 3072 at 3-32 rows 2-22 % faster; at K = 3584, seven chunks of 512
// against eight wavefronts with two of 256 for most, 16 rows lost 4-6 %; the GEMV at K = 3072 gains at N = 4096 and
// loses at N = 8192).
#ifndef DR_CHUNK_K
#define DR_CHUNK_K 0
#endif
static_assert(DR_CHUNK_K == 0 || (DR_CHUNK_K % 256 == 0 && DR_CHUNK_K <= 512),
              "a chunk is one or two 256-k exponent groups");

// a workgroup takes at most this many chunks (its MAXW wavefronts two each); more K is split over several workgroups
// a tile, which then meet in the workspace: fewer splits of more chunks beat more of fewer (K = 14336 at M = 8: 2 x 14
// chunks 15.8 us, 4 x 7 17.7 us; the MoE down's K = 12288: 2 x 12 9.0 us, 3 x 8 9.9 us)
#ifndef DR_SPLIT_CHUNKS
#define DR_SPLIT_CHUNKS 16
#endif

// the split of a padded K into chunks of ch
void plan_chunks(int k_pad, int ch, int* chunks, int* kch, int* waves, int* splits, int* cps) {
    *kch = ch;
    *chunks = (k_pad + ch - 1) / ch;
    *splits = (*chunks + DR_SPLIT_CHUNKS - 1) / DR_SPLIT_CHUNKS;
    *cps = (*chunks + *splits - 1) / *splits;
    *waves = *cps < MAXW ? *cps : MAXW;
}

void plan(int k, bool mfma, int* chunks, int* kch, int* waves, int* splits, int* cps) {
    const int k_pad = (k + KALIGN - 1) / KALIGN * KALIGN;
    const int ch = DR_CHUNK_K ? DR_CHUNK_K : (k_pad > (mfma ? 3072 : 2048) ? 512 : 256);
    plan_chunks(k_pad, ch, chunks, kch, waves, splits, cps);
}

// a launch of more tiles than the workspace has counters for runs unsplit
void limit_splits(Args& a) {
    if (a.splits > 1 && a.tiles > SPLIT_MAXTILES) {
        a.splits = 1;
        a.cps = a.chunks;
        a.waves = a.cps < MAXW ? a.cps : MAXW;
    }
}

// the MFMA kernel from this many rows on; below it the GEMV kernel's rows a pass
#ifndef DR_MFMA_MIN_M
#define DR_MFMA_MIN_M 3
#endif

int rows_per_pass(int m) {
    if (m >= DR_MFMA_MIN_M) return m <= 16 ? 16 : 32;
    return m <= 1 ? 1 : m <= 2 ? 2 : m <= 4 ? 4 : 8;
}

// Set by dr_launch_plan while it walks the launch path: the dense launches then store their kernel's LDS bytes (static
// plus dynamic) here instead of launching it.
thread_local size_t* lds_query = nullptr;

template <typename F>
void fire(F kernel, dim3 grid, dim3 block, size_t lds, hipStream_t st, const Args& a) {
    if (lds_query != nullptr) {
        hipFuncAttributes at{};
        const bool got = hipFuncGetAttributes(&at, reinterpret_cast<const void*>(kernel)) == hipSuccess;
        *lds_query = lds + (got ? at.sharedSizeBytes : 0);
        return;
    }
    hipLaunchKernelGGL(kernel, grid, block, lds, st, a);
}

// dynamic LDS of a dense launch: the partial sums, and at 32 rows (the MFMA kernel) the wavefronts' x staging
size_t dense_lds(const Args& a, int pw, int rows) {
    const size_t part = (size_t)max(a.waves, a.splits) * pw * rows * 16 * sizeof(float);
    return rows == 32 ? max(part, (size_t)a.waves * XS_BYTES) : part;
}

template <int MR, int PW>
void launch_gemv(const Args& a, int grid, hipStream_t st) {
    const dim3 b(64 * a.waves);
    const size_t lds = dense_lds(a, PW, MR);
    const bool g1 = a.kch == 256;
    if (a.nseg > 1) {
        if (g1)
            fire((dr_gemv_g1<MR, PW, -1, false>), dim3(grid), b, lds, st, a);
        else
            fire((dr_gemv<MR, PW, -1, false>), dim3(grid), b, lds, st, a);
        return;
    }
    // a plain launch (one weight, bf16 y, no residual, top-k records or split K) takes the plain epilogue
    const bool plain = MR <= 2 && a.rec == nullptr && a.res == nullptr && !a.y_f32 && a.splits == 1;
    switch (a.seg[0].fmt) {
        case DR_BFP8:
            if constexpr (MR <= 2) {
                if (plain) {
                    if (g1)
                        fire((dr_gemv_g1<MR, PW, DR_BFP8, true, true>), dim3(grid), b, lds, st, a);
                    else
                        fire((dr_gemv<MR, PW, DR_BFP8, true, true>), dim3(grid), b, lds, st, a);
                    break;
                }
            }
            if (g1)
                fire((dr_gemv_g1<MR, PW, DR_BFP8, true>), dim3(grid), b, lds, st, a);
            else
                fire((dr_gemv<MR, PW, DR_BFP8, true>), dim3(grid), b, lds, st, a);
            break;
        case DR_BFP4:
            if constexpr (MR <= 2) {
                if (plain) {
                    if (g1)
                        fire((dr_gemv_g1<MR, PW, DR_BFP4, true, true>), dim3(grid), b, lds, st, a);
                    else
                        fire((dr_gemv<MR, PW, DR_BFP4, true, true>), dim3(grid), b, lds, st, a);
                    break;
                }
            }
            if (g1)
                fire((dr_gemv_g1<MR, PW, DR_BFP4, true>), dim3(grid), b, lds, st, a);
            else
                fire((dr_gemv<MR, PW, DR_BFP4, true>), dim3(grid), b, lds, st, a);
            break;
        case DR_INT4:
            if constexpr (PW <= 2 && MR <= 2) {
                if (plain) {
                    if (g1)
                        fire((dr_gemv_g1<MR, PW, DR_INT4, true, true>), dim3(grid), b, lds, st, a);
                    else
                        fire((dr_gemv<MR, PW, DR_INT4, true, true>), dim3(grid), b, lds, st, a);
                    break;
                }
                if (g1)
                    fire((dr_gemv_g1<MR, PW, DR_INT4, true>), dim3(grid), b, lds, st, a);
                else
                    fire((dr_gemv<MR, PW, DR_INT4, true>), dim3(grid), b, lds, st, a);
            }
            break;
        default:  // (bf16 chunks have no exponent groups: one kernel serves every chunk size)
            fire((dr_gemv<MR, PW, DR_BF16, true>), dim3(grid), b, lds, st, a);
            break;
    }
}

template <int MT, int PW>
void launch_mfma(const Args& a, int grid, hipStream_t st) {
    const dim3 b(64 * a.waves);
    const size_t lds = dense_lds(a, PW, 16 * MT);
    if (a.nseg > 1) {
        fire((dr_mfma<MT, PW, -1, false>), dim3(grid), b, lds, st, a);
        return;
    }
    switch (a.seg[0].fmt) {
        case DR_BFP8: fire((dr_mfma<MT, PW, DR_BFP8, true>), dim3(grid), b, lds, st, a); break;
        case DR_BFP4: fire((dr_mfma<MT, PW, DR_BFP4, true>), dim3(grid), b, lds, st, a); break;
        default: fire((dr_mfma<MT, PW, DR_BF16, true>), dim3(grid), b, lds, st, a); break;
    }
}

template <int MR, int PW, int MOE>
void launch_gemv_moe(const MoeArgs& a, int grid, hipStream_t st) {
    const dim3 b(64 * a.waves);
    const size_t lds = (size_t)max(a.waves, a.splits) * PW * MR * 16 * sizeof(float);
    if (a.seg[0].fmt == DR_BFP4_KB)
        hipLaunchKernelGGL((dr_gemv_moe<MR, PW, MOE, true>), dim3(grid), b, lds, st, a);
    else
        hipLaunchKernelGGL((dr_gemv_moe<MR, PW, MOE, false>), dim3(grid), b, lds, st, a);
}

template <int MT, int PW, int MOE>
void launch_mfma_moe(const MoeArgs& a, int grid, hipStream_t st) {
    const dim3 b(64 * a.waves);
    size_t lds = (size_t)max(a.waves, a.splits) * PW * 16 * MT * 16 * sizeof(float);
    if ((MOE == DR_MOE_GATE_UP_ROWS || MOE == DR_MOE_DOWN_ROWS) && MT == 2)
        lds = max(lds, (size_t)a.waves * XS_BYTES);  // (the x staging)
    if (a.seg[0].fmt == DR_BFP4_KB)
        hipLaunchKernelGGL((dr_mfma_moe<MT, PW, MOE, true>), dim3(grid), b, lds, st, a);
    else
        hipLaunchKernelGGL((dr_mfma_moe<MT, PW, MOE, false>), dim3(grid), b, lds, st, a);
}

// one pass of an expert-gathered launch (bfloat4_b, or its kblock packs): the one-row modes on the GEMV; the rows modes on the GEMV up to
// two rows, else the MFMA kernel (16 rows a pass for gate/up, 16 or 32 for down)
hipError_t launch_moe(const MoeArgs& a, int mode, int rows, int pw, int grid, hipStream_t st) {
    const bool narrow = pw == 2;  // (gate/up modes: 16-column tiles; down modes: pw 1)
    switch (mode) {
        case DR_MOE_GATE_UP:
            narrow ? launch_gemv_moe<1, 2, DR_MOE_GATE_UP>(a, grid, st) : launch_gemv_moe<1, 4, DR_MOE_GATE_UP>(a, grid, st);
            break;
        case DR_MOE_DOWN:
            pw == 1 ? launch_gemv_moe<1, 1, DR_MOE_DOWN>(a, grid, st) : launch_gemv_moe<1, 2, DR_MOE_DOWN>(a, grid, st);
            break;
        case DR_MOE_GATE_UP_ROWS:
            if (rows == 1)
                narrow ? launch_gemv_moe<1, 2, DR_MOE_GATE_UP_ROWS>(a, grid, st)
                       : launch_gemv_moe<1, 4, DR_MOE_GATE_UP_ROWS>(a, grid, st);
            else if (rows == 2)
                narrow ? launch_gemv_moe<2, 2, DR_MOE_GATE_UP_ROWS>(a, grid, st)
                       : launch_gemv_moe<2, 4, DR_MOE_GATE_UP_ROWS>(a, grid, st);
            else if (rows == 16)
                launch_mfma_moe<1, 4, DR_MOE_GATE_UP_ROWS>(a, grid, st);
            else if (a.seg[0].fmt != DR_BFP4_KB && a.splits == 1) {
                const size_t lds = max((size_t)a.waves * XS_BYTES, (size_t)a.waves * 4 * 32 * 16 * sizeof(float));
                hipLaunchKernelGGL(dr_mfma_moe_pairs, dim3(a.tiles / a.tpe * ((a.tpe + 1) / 2)), dim3(64 * a.waves), lds,
                                   st, a);
            } else
                launch_mfma_moe<2, 4, DR_MOE_GATE_UP_ROWS>(a, grid, st);
            break;
        default:
            if (rows == 1)
                pw == 1 ? launch_gemv_moe<1, 1, DR_MOE_DOWN_ROWS>(a, grid, st)
                        : launch_gemv_moe<1, 2, DR_MOE_DOWN_ROWS>(a, grid, st);
            else if (rows == 2)
                pw == 1 ? launch_gemv_moe<2, 1, DR_MOE_DOWN_ROWS>(a, grid, st)
                        : launch_gemv_moe<2, 2, DR_MOE_DOWN_ROWS>(a, grid, st);
            else if (rows == 16)
                launch_mfma_moe<1, 2, DR_MOE_DOWN_ROWS>(a, grid, st);
            else
                launch_mfma_moe<2, 2, DR_MOE_DOWN_ROWS>(a, grid, st);
            break;
    }
    return hipGetLastError();
}

// one pass of up to `rows` rows
void launch_pairs(const Args& a, hipStream_t st) {
    const dim3 b(64 * a.waves);
    const size_t lds = max((size_t)a.waves * XS_BYTES, (size_t)2 * a.waves * 2 * 16 * PAIR_RS * sizeof(float));
    if (a.nseg > 1) {
        fire((dr_mfma_pairs<-1, false>), dim3(a.pairs), b, lds, st, a);
        return;
    }
    switch (a.seg[0].fmt) {
        case DR_BFP8: fire((dr_mfma_pairs<DR_BFP8, true>), dim3(a.pairs), b, lds, st, a); break;
        case DR_BFP4: fire((dr_mfma_pairs<DR_BFP4, true>), dim3(a.pairs), b, lds, st, a); break;
        default: fire((dr_mfma_pairs<DR_BF16, true>), dim3(a.pairs), b, lds, st, a); break;
    }
}

hipError_t launch_rows(const Args& a, int rows, int pw, int grid, hipStream_t st) {
    if (rows == 32 && a.pairs > 0) {
        launch_pairs(a, st);
        return hipGetLastError();
    }
    switch (rows) {
        case 1: pw == 1 ? launch_gemv<1, 1>(a, grid, st) : pw == 2 ? launch_gemv<1, 2>(a, grid, st) : launch_gemv<1, 4>(a, grid, st); break;
        case 2: pw == 1 ? launch_gemv<2, 1>(a, grid, st) : pw == 2 ? launch_gemv<2, 2>(a, grid, st) : launch_gemv<2, 4>(a, grid, st); break;
        case 4: pw == 2 ? launch_gemv<4, 2>(a, grid, st) : launch_gemv<4, 4>(a, grid, st); break;
        case 8: launch_gemv<8, 2>(a, grid, st); break;  // (a GLU pass takes at most 4 GEMV rows)
        case 16: pw == 1 ? launch_mfma<1, 1>(a, grid, st) : pw == 2 ? launch_mfma<1, 2>(a, grid, st) : launch_mfma<1, 4>(a, grid, st); break;
        default: pw == 1 ? launch_mfma<2, 1>(a, grid, st) : launch_mfma<2, 2>(a, grid, st); break;  // (a GLU pass takes at most 16 MFMA rows)
    }
    return hipGetLastError();
}

}  // namespace

extern "C" {

int64_t dr_codes_bytes(int fmt, int k_pad, int n_pad) {
    const int64_t v = (int64_t)k_pad * n_pad;
    return fmt == DR_BFP8 ? v : (fmt == DR_BFP4 || fmt == DR_INT4 || fmt == DR_BFP4_KB) ? v / 2 : 2 * v;
}

int64_t dr_exps_bytes(int fmt, int k_pad, int n_pad) {
    return (fmt == DR_BFP8 || fmt == DR_BFP4 || fmt == DR_BFP4_KB) ? (int64_t)k_pad * n_pad / 16 : 0;
}

int64_t dr_int4_scales_bytes(int k_pad, int n_pad) { return (int64_t)(k_pad / 128) * 4 * n_pad * 2; }

int dr_pack_int4(const int8_t* q, int64_t ld_q, int n, int k, void* codes, int n_pad, int k_pad, void* stream) {
    if (q == nullptr || codes == nullptr || n <= 0 || k <= 0 || k % 32 || n_pad < n || n_pad % 32 || k_pad < k ||
        k_pad % KALIGN || ld_q < k)
        return DR_EINVAL;
    const long long threads = (long long)(n_pad / 16) * (k_pad / 128) * 64;
    hipLaunchKernelGGL(dr_pack_int4_k, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, S(stream), q,
                       (long long)ld_q, n, k, reinterpret_cast<uint8_t*>(codes), n_pad, k_pad);
    return hip_status(hipGetLastError());
}

int dr_pack_int4_scales(const uint16_t* s, int64_t ld_s, int n, int k, void* out, int n_pad, int k_pad, void* stream) {
    if (s == nullptr || out == nullptr || n <= 0 || k <= 0 || k % 32 || n_pad < n || n_pad % 32 || k_pad < k ||
        k_pad % KALIGN || ld_s < k / 32)
        return DR_EINVAL;
    const long long threads = (long long)(n_pad / 16) * (k_pad / 128) * 64;
    hipLaunchKernelGGL(dr_pack_int4_scales_k, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, S(stream), s,
                       (long long)ld_s, n, k, reinterpret_cast<uint16_t*>(out), n_pad, k_pad);
    return hip_status(hipGetLastError());
}

int dr_pack(const float* w, int64_t ld_w, int n, int k, int fmt, const float* col_div, void* codes, void* exps,
            int n_pad, int k_pad, void* stream) {
    if (w == nullptr || codes == nullptr || n <= 0 || k <= 0 || n_pad < n || n_pad % 32 || k_pad < k ||
        k_pad % KALIGN || ld_w < k || (fmt != DR_BF16 && exps == nullptr) || fmt < 0 || fmt > DR_BFP4_KB ||
        fmt == DR_INT4)
        return DR_EINVAL;
    const long long total = (long long)(n_pad / 16) * (k_pad / 8);
    const int grid = (int)((total + 255) / 256);
    auto* c8 = reinterpret_cast<uint8_t*>(codes);
    auto* e8 = reinterpret_cast<uint8_t*>(exps);
    if (fmt == DR_BFP4_KB) {
        const long long tk = (long long)n_pad * (k_pad / 16);
        hipLaunchKernelGGL(dr_pack_kb_k, dim3((int)((tk + 255) / 256)), dim3(256), 0, S(stream), w, (long long)ld_w, n, k,
                           col_div, c8, e8, n_pad, k_pad);
    } else if (fmt == DR_BFP8)
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
        n_pad % 32 || ld_out < n || (fmt != DR_BF16 && exps == nullptr) || fmt < 0 || fmt > DR_BFP4_KB || fmt == DR_INT4)
        return DR_EINVAL;
    const long long total = (long long)n * k;
    const int grid = (int)((total + 255) / 256);
    auto* c8 = reinterpret_cast<const uint8_t*>(codes);
    auto* e8 = reinterpret_cast<const uint8_t*>(exps);
    if (fmt == DR_BFP8)
        hipLaunchKernelGGL(dr_unpack_k<DR_BFP8>, dim3(grid), dim3(256), 0, S(stream), c8, e8, n, k, k_pad, out, (long long)ld_out);
    else if (fmt == DR_BFP4)
        hipLaunchKernelGGL(dr_unpack_k<DR_BFP4>, dim3(grid), dim3(256), 0, S(stream), c8, e8, n, k, k_pad, out, (long long)ld_out);
    else if (fmt == DR_BFP4_KB)
        hipLaunchKernelGGL(dr_unpack_k<DR_BFP4_KB>, dim3(grid), dim3(256), 0, S(stream), c8, e8, n, k, k_pad, out, (long long)ld_out);
    else
        hipLaunchKernelGGL(dr_unpack_k<DR_BF16>, dim3(grid), dim3(256), 0, S(stream), c8, e8, n, k, k_pad, out, (long long)ld_out);
    return hip_status(hipGetLastError());
}

int dr_plan(int k, int m, int32_t* chunks, int32_t* kch, int32_t* rpp) {
    if (k <= 0 || m <= 0) return DR_EINVAL;
    int c, ch, w, sp, cps;
    plan(k, rows_per_pass(m) >= 16, &c, &ch, &w, &sp, &cps);
    if (chunks) *chunks = c;
    if (kch) *kch = ch;
    if (rpp) *rpp = rows_per_pass(m);
    return DR_OK;
}

}  // extern "C"

namespace {

// the launch's arguments, its panel width, tiles and rows a pass (shared by dr_matmul and dr_workspace_bytes; for the
// expert gather, gather = true: no 16-column tiles here, and the kblock format allowed)
int prepare(const dr_launch* L, Args& a, int& pw, int& tiles, int& mr, bool gather = false) {
    // x rows are read 16 bytes at a time: the rows start 16-byte aligned
    if (L == nullptr || L->x == nullptr || L->y == nullptr || L->m <= 0 || L->k <= 0 || L->k % 32 ||
        L->ldx < L->k || L->ldx % 8 || (reinterpret_cast<uintptr_t>(L->x) & 15) || L->nseg < 1 || L->nseg > 4)
        return DR_EINVAL;
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
    if (a.act < DR_ACT_SILU || a.act > DR_ACT_SWIGLU_OAI) return DR_EINVAL;  // (swiglu_oai: the expert gather only)
    a.nseg = L->nseg;
    pw = L->seg[0].glu ? 4 : 2;
    tiles = 0;
    for (int i = 0; i < L->nseg; ++i) {
        const dr_segment& s = L->seg[i];
        SegDev& d = a.seg[i];
        const bool bfp = s.fmt == DR_BFP8 || s.fmt == DR_BFP4 || s.fmt == DR_BFP4_KB;
        if (s.fmt < 0 || s.fmt > (gather ? DR_BFP4_KB : DR_INT4) || s.n <= 0 || s.n_pad < s.n || s.n_pad % 32 || s.col0 < 0 || s.col0 % 32 ||
            s.codes == nullptr || (bfp && s.exps == nullptr) || s.glu < 0 || s.glu > 2 || (s.glu ? 4 : 2) != pw)
            return DR_EINVAL;
        // an int4 weight alone: one segment, no GLU, residual or top-k, its group scales given
        if (s.fmt == DR_INT4 && (L->nseg != 1 || s.glu || s.scale == nullptr || L->residual || L->topk.records))
            return DR_EINVAL;
        if (s.glu == 1 && s.n % 64) return DR_EINVAL;
        if (s.glu == 2 && (s.codes_up == nullptr || (s.fmt != DR_BF16 && s.exps_up == nullptr))) return DR_EINVAL;
        d.codes = reinterpret_cast<const uint8_t*>(s.codes);
        d.exps = reinterpret_cast<const uint8_t*>(s.exps);
        d.codes_up = reinterpret_cast<const uint8_t*>(s.codes_up);
        d.exps_up = reinterpret_cast<const uint8_t*>(s.exps_up);
        d.scale = s.fmt == DR_INT4 ? nullptr : s.scale;
        d.gscale = s.fmt == DR_INT4 ? reinterpret_cast<const uint16_t*>(s.scale) : nullptr;
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
        d.pstride = (unsigned)((a.k_pad / kblk(s.fmt)) * 1024);
        tiles += d.tiles;
        if ((int64_t)s.col0 + d.n_out > L->ldy) return DR_EINVAL;
    }
    // A block list's segments in order of the bytes a tile reads (bf16, then bfloat8_b, then bfloat4_b; stable): the
    // lowest workgroup indices start first, so the heaviest tiles do not queue for a CU behind lighter ones (each
    // segment keeps its own output columns; the order changes no result).
    if (a.nseg > 1) {
        auto heavier = [](int f, int g) { return (f == DR_BF16 ? 3 : f == DR_BFP8 ? 2 : 1) > (g == DR_BF16 ? 3 : g == DR_BFP8 ? 2 : 1); };
        for (int i = 1; i < a.nseg; ++i) {
            const SegDev v = a.seg[i];
            int j = i - 1;
            for (; j >= 0 && heavier(v.fmt, a.seg[j].fmt); --j) a.seg[j + 1] = a.seg[j];
            a.seg[j + 1] = v;
        }
        int tb = 0;
        for (int i = 0; i < a.nseg; ++i) {
            a.seg[i].tile_begin = tb;
            tb += a.seg[i].tiles;
        }
    }
    if (a.res != nullptr && (L->ldr < a.seg[0].col0 + a.seg[0].n_out || L->nseg != 1 || pw != 2)) return DR_EINVAL;
    const dr_topk& T = L->topk;
    a.rec = reinterpret_cast<uint32_t*>(T.records);
    a.tk_group = 1;
    if (a.rec != nullptr) {
        if (T.k < 1 || T.k > 32 || T.rows < 1 || T.rows > 32 || T.rows > L->m || T.slot0 < 0 || L->nseg != 1 ||
            pw != 2 || T.n_valid < 0 || T.max_records < 0)
            return DR_EINVAL;
        // tiles in groups so that the launch writes at most max_records records
        if (T.max_records > 0 && tiles > T.max_records) a.tk_group = (tiles + T.max_records - 1) / T.max_records;
        const int records = (tiles + a.tk_group - 1) / a.tk_group;
        if ((int64_t)T.slot0 + records > T.records_cap) return DR_EINVAL;
        if (a.tk_group > 1 && a.tk_group * T.k > GROUP_MAXCAND) return DR_ERANGE;
        a.tk_k = T.k;
        a.tk_rows = T.rows;
        a.slot0 = T.slot0;
        a.rec_out = a.rec + (size_t)T.slot0 * 2 * T.rows * T.k;  // (grouped: the staging, once the workspace is bound)
        a.n_valid = T.n_valid;
        a.base = T.base;
        a.write_y = T.write_y != 0;
        a.tk_fp32 = T.fp32 != 0;
    }
    mr = rows_per_pass(L->m);
    if (pw == 4 && mr == 8) mr = 4;    // (GLU: at most 4 GEMV rows or 16 MFMA rows a pass, for the registers
    if (pw == 4 && mr == 32) mr = 16;  // and the LDS)
    if (a.seg[0].fmt == DR_INT4) mr = L->m >= 2 ? 2 : 1;  // (int4: the GEMV, two rows a pass)
    plan(L->k, !gather && mr >= 16, &a.chunks, &a.kch, &a.waves, &a.splits, &a.cps);  // (the expert gather: as before)
    a.tiles = tiles;
    limit_splits(a);
    // A GEMV launch takes 16-column tiles (one panel a workgroup) where they lower the most any CU streams (fewer
    // 32-column tiles than CUs, or a count just past a multiple of the CUs): each column's sums are made by the same
    // lanes in the same order whatever the tile width, so the results are the same bit for bit. (Not with top-k
    // records, one a 32-column tile, nor a GLU's pairs.)
    // The MFMA kernel (unsplit) takes them where even the 16-column tiles are at most one a CU: each reads all of x, so
    // two on a CU cost more than one 32-column tile (bfloat8_b K = 4096 at 3-16 rows, N = 2048 and 4096: 16-19 %
    // faster; the same sums a column, as the GEMV's).
    if (!gather && pw == 2 && a.rec == nullptr &&
        (mr <= 2 ? narrow_better(tiles) : (mr >= 16 && a.splits == 1 && 2 * tiles <= cu_count()))) {
        pw = 1;
        tiles = 0;
        for (int i = 0; i < a.nseg; ++i) {
            a.seg[i].tiles = (a.seg[i].n_out + 15) / 16;
            a.seg[i].tile_begin = tiles;
            tiles += a.seg[i].tiles;
        }
        a.tiles = tiles;
        plan(L->k, mr >= 16, &a.chunks, &a.kch, &a.waves, &a.splits, &a.cps);
        limit_splits(a);
    }
    // 32 rows, plain tiles, more tiles than CUs: block-float segments in tile pairs (dr_mfma_pairs)
    a.pairs = 0;
    bool pairable = false;
    for (int i = 0; i < a.nseg; ++i) pairable |= a.seg[i].fmt != DR_BF16;
    if (!gather && pairable && mr == 32 && pw == 2 && a.splits == 1 && a.rec == nullptr && a.res == nullptr &&
        tiles > cu_count()) {
        // here a workgroup's bytes order the segments (a bfloat8_b pair 2 x 1088 B a 32-k step, a bf16 tile 2048, a
        // bfloat4_b pair 2 x 576; stable), so the heaviest workgroups start first: C4 14.80 -> 14.70 us against the
        // tiles' order above (its bf16 tiles first)
        auto wg_bytes = [](int f) { return f == DR_BFP8 ? 2176 : f == DR_BF16 ? 2048 : 1152; };
        for (int i = 1; i < a.nseg; ++i) {
            const SegDev v = a.seg[i];
            int j = i - 1;
            for (; j >= 0 && wg_bytes(v.fmt) > wg_bytes(a.seg[j].fmt); --j) a.seg[j + 1] = a.seg[j];
            a.seg[j + 1] = v;
        }
        int tb = 0;
        for (int i = 0; i < a.nseg; ++i) {
            a.seg[i].tile_begin = tb;
            tb += a.seg[i].tiles;
            a.pair_tiles[i] = a.seg[i].fmt == DR_BF16 ? 1 : 2;
            a.pair_begin[i] = a.pairs;
            a.pairs += (a.seg[i].tiles + a.pair_tiles[i] - 1) / a.pair_tiles[i];
        }
    }
    return DR_OK;
}

// The workspace: SPLIT_MAXTILES split-K counters at a fixed place (so that launches of any shape can share one), then
// split K's column sums (every workgroup's), then the grouped records' staging (every tile's record).
constexpr int64_t WS_COUNTERS = (int64_t)SPLIT_MAXTILES * 4;

int64_t split_sums_bytes(const Args& a, int pw, int mr) {
    return a.splits > 1 ? (int64_t)a.tiles * a.splits * pw * mr * 16 * 4 : 0;
}

int64_t workspace_bytes(const Args& a, int pw, int mr) {
    if (a.splits == 1 && a.tk_group <= 1) return 0;
    const int64_t stage = a.tk_group > 1 ? (int64_t)a.tiles * 2 * a.tk_rows * a.tk_k * 4 : 0;
    return WS_COUNTERS + split_sums_bytes(a, pw, mr) + stage;
}

void bind_split(Args& a, void* workspace, int pw, int mr) {
    uint8_t* w = reinterpret_cast<uint8_t*>(workspace);
    a.counters = reinterpret_cast<uint32_t*>(w);
    a.wpart = reinterpret_cast<float*>(w + WS_COUNTERS);
    a.tstage = reinterpret_cast<uint32_t*>(w + WS_COUNTERS + split_sums_bytes(a, pw, mr));
    if (a.rec != nullptr && a.tk_group > 1) a.rec_out = a.tstage;
}

// dr_matmul's launches: one pass of up to mr rows each (the passes a top-k launch needs, not y, skipped)
int run_passes(const dr_launch* L, const Args& a, int tiles, int mr, int pw, hipStream_t st) {
    const size_t ysz = a.y_f32 ? 4 : 2;
    for (int r0 = 0; r0 < L->m; r0 += mr) {
        Args p = a;
        p.m = L->m - r0 < mr ? L->m - r0 : mr;
        p.x = a.x + (size_t)r0 * a.ldx;
        p.y = reinterpret_cast<uint8_t*>(L->y) + (size_t)r0 * a.ldy * ysz;
        if (a.res) p.res = a.res + (size_t)r0 * a.ldr;
        p.row0 = r0;
        if (a.rec != nullptr && r0 >= a.tk_rows && !a.write_y) continue;
        // a last pass of at most 16 rows of a 32-row launch runs the 16-row MFMA kernel: the same plan, and each row's
        // sums the same bit for bit, at less cost (bfloat8_b K = 2048 N = 4096: 16 rows 7.4 us against 9.2 at 32)
        const int rows = (mr == 32 && p.m <= 16) ? 16 : mr;
        hipError_t e = launch_rows(p, rows, pw, tiles * a.splits, st);
        if (e == hipSuccess && a.rec != nullptr && a.tk_group > 1 && r0 < a.tk_rows) {
            const int records = (tiles + a.tk_group - 1) / a.tk_group;
            const size_t lds = (size_t)GROUP_WAVES * a.tk_group * a.tk_k * sizeof(unsigned long long);
            hipLaunchKernelGGL(dr_group_k, dim3(records), dim3(64 * GROUP_WAVES), lds, st, a.tstage, a.rec, tiles,
                               a.tk_group, a.tk_k, a.tk_rows, a.slot0, r0, min(r0 + p.m, a.tk_rows), a.tk_fp32);
            e = hipGetLastError();
        }
        if (e != hipSuccess) return DR_EHIP;
    }
    return DR_OK;
}

// ---- the library's own workspace, for dr_matmul_noalloc ---------------------------------------------------------------
//
// A file-scope device array, one copy on every GPU the library runs on, held until the process ends. Host code never
// uses its name as an address (on the host it is only a stand-in for the symbol): each device's address comes from
// hipGetSymbolAddress, once per device with that device current, and that address is what kernels and fills get.
// It serves as dr_matmul's workspace: the split-K counters must start at zero (a fill kernel clears them on a device's
// first call; every launch leaves them at zero), the partial sums and the records' staging need no clearing.
static __device__ __align__(256) uint8_t scratch[DR_SCRATCH_BYTES];

__global__ __launch_bounds__(256) void dr_zero_k(uint32_t* __restrict__ p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

constexpr int SCRATCH_DEVICES = 64;
std::mutex scratch_mu;
void* scratch_addr[SCRATCH_DEVICES];  // (guarded by scratch_mu)

// The scratch of the launch stream's device, or null with `status` set. The stream must belong to the current device
// (the array's address is looked up with its device current; another device's stream is refused, DR_EINVAL). On a
// device's first call the counters are cleared by a fill on a stream of the library's own, and the host waits for it
// before the address is published: a call on any stream then finds them zero. That first call must not be made
// under stream capture (the fill would be captured, not run): it is refused (DR_EINVAL) and nothing is enqueued, so
// a caller that captures makes one eager call first.
void* scratch_for_stream(hipStream_t st, int& status) {
    int cur = 0;
    if (hipGetDevice(&cur) != hipSuccess || cur < 0 || cur >= SCRATCH_DEVICES) {
        status = DR_EHIP;
        return nullptr;
    }
    int sd = cur;
    if (st != nullptr && hipStreamGetDevice(st, &sd) != hipSuccess) {
        status = DR_EHIP;
        return nullptr;
    }
    if (sd != cur) {
        status = DR_EINVAL;
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(scratch_mu);
    if (scratch_addr[cur] == nullptr) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(st, &cs) != hipSuccess) {
            status = DR_EHIP;
            return nullptr;
        }
        if (cs != hipStreamCaptureStatusNone) {
            status = DR_EINVAL;
            return nullptr;
        }
        void* ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr) {
            status = DR_EHIP;
            return nullptr;
        }
        constexpr int n = (int)(WS_COUNTERS / 4);  // the split-K counters
        hipStream_t z = nullptr;
        if (hipStreamCreateWithFlags(&z, hipStreamNonBlocking) != hipSuccess) {
            status = DR_EHIP;
            return nullptr;
        }
        hipLaunchKernelGGL(dr_zero_k, dim3((n + 255) / 256), dim3(256), 0, z, reinterpret_cast<uint32_t*>(ptr), n);
        const bool ok = hipGetLastError() == hipSuccess && hipStreamSynchronize(z) == hipSuccess;
        hipStreamDestroy(z);
        if (!ok) {
            status = DR_EHIP;
            return nullptr;
        }
        scratch_addr[cur] = ptr;
    }
    return scratch_addr[cur];
}


}  // namespace

extern "C" {

int64_t dr_workspace_bytes(const dr_launch* L) {
    Args a{};
    int pw, tiles, mr;
    if (L != nullptr && L->act == DR_ACT_SWIGLU_OAI) return -1;  // (the dense GLU: silu or gelu_tanh)
    if (prepare(L, a, pw, tiles, mr) != DR_OK) return -1;
    return workspace_bytes(a, pw, mr);
}

int dr_matmul(const dr_launch* L) {
    Args a{};
    int pw, tiles, mr;
    if (L != nullptr && L->act == DR_ACT_SWIGLU_OAI) return DR_EINVAL;  // (the dense GLU: silu or gelu_tanh)
    const int st0 = prepare(L, a, pw, tiles, mr);
    if (st0 != DR_OK) return st0;
    const int64_t need = workspace_bytes(a, pw, mr);
    if (need > 0) {
        // split K needs the workspace: its counters start at zero (the caller zeroes it once; each launch leaves
        // them at zero)
        if (L->workspace == nullptr || L->workspace_bytes < need) return DR_EINVAL;
        bind_split(a, L->workspace, pw, mr);
    }
    return run_passes(L, a, tiles, mr, pw, S(L->stream));
}

int64_t dr_scratch_bytes(void) { return DR_SCRATCH_BYTES; }

int dr_stream_read(const void* p, int64_t bytes, uint32_t* sink, void* stream) {
    if (p == nullptr || sink == nullptr || bytes < 16 || bytes % 16 || (reinterpret_cast<uintptr_t>(p) & 15)) return DR_EINVAL;
    const long long n16 = bytes / 16;
    const long long per = (long long)READ_T * READ_U;
    hipLaunchKernelGGL(dr_read_k, dim3((unsigned)((n16 + per - 1) / per)), dim3(READ_T), 0, S(stream),
                       reinterpret_cast<const u32x4_t*>(p), n16, sink);
    return hip_status(hipGetLastError());
}

int dr_matmul_noalloc(const dr_launch* L) {
    Args a{};
    int pw, tiles, mr;
    if (L != nullptr && L->act == DR_ACT_SWIGLU_OAI) return DR_EINVAL;
    const int st0 = prepare(L, a, pw, tiles, mr);
    if (st0 != DR_OK) return st0;
    const int64_t need = workspace_bytes(a, pw, mr);
    if (need > DR_SCRATCH_BYTES) return DR_ERANGE;  // (checked before any device call)
    hipStream_t st = S(L->stream);
    if (need > 0) {
        int status = DR_OK;
        void* ws = scratch_for_stream(st, status);
        if (ws == nullptr) return status;
        bind_split(a, ws, pw, mr);
    }
    return run_passes(L, a, tiles, mr, pw, st);
}

int dr_launch_plan(const dr_launch* L, dr_launch_info* info) {
    Args a{};
    int pw, tiles, mr;
    if (info == nullptr) return DR_EINVAL;
    if (L != nullptr && L->act == DR_ACT_SWIGLU_OAI) return DR_EINVAL;
    const int st = prepare(L, a, pw, tiles, mr);
    if (st != DR_OK) return st;
    *info = dr_launch_info{};
    info->kernel = (mr >= 16) ? 1 : 0;
    info->rows_per_pass = mr;
    info->tile_cols = pw == 1 ? 16 : TILE;
    info->tiles = tiles;
    info->chunks = a.chunks;
    info->kch = a.kch;
    info->splits = a.splits;
    info->workgroups = a.pairs > 0 ? a.pairs : tiles * a.splits;
    info->tiles_per_workgroup = a.pairs > 0 ? 2 : 1;  // (block-float segments; a launch's bf16 segments take 1)
    int passes = 0;
    for (int r0 = 0; r0 < L->m; r0 += mr)
        if (!(a.rec != nullptr && r0 >= a.tk_rows && !a.write_y)) ++passes;
    info->passes = passes;
    info->records = a.rec != nullptr ? (tiles + a.tk_group - 1) / a.tk_group : 0;
    info->tiles_per_record = a.rec != nullptr ? a.tk_group : 0;
    info->waves = a.waves;
    // the first pass's kernel, walked without launching: its LDS a workgroup (0 where no device answers)
    size_t lds = 0;
    Args p = a;
    p.m = L->m < mr ? L->m : mr;
    lds_query = &lds;
    launch_rows(p, (mr == 32 && p.m <= 16) ? 16 : mr, pw, tiles * a.splits, S(L->stream));
    lds_query = nullptr;
    (void)hipGetLastError();
    info->lds_bytes = (int32_t)lds;
    return DR_OK;
}

int dr_launch_work(const dr_launch* L, int32_t* work, int max_workgroups) {
    Args a{};
    int pw, tiles, mr;
    if (work == nullptr || max_workgroups < 0) return DR_EINVAL;
    if (L != nullptr && L->act == DR_ACT_SWIGLU_OAI) return DR_EINVAL;
    const int st = prepare(L, a, pw, tiles, mr);
    if (st != DR_OK) return st;
    const int wgs = a.pairs > 0 ? a.pairs : tiles * a.splits;
    if (wgs > max_workgroups) return DR_ERANGE;
    const int cols = pw == 1 ? 16 : TILE;
    for (int i = 0; i < wgs; ++i) {
        // the kernels' own mapping of blockIdx.x (dr_mfma_pairs: pair_begin / pair_tiles; the others: find_segment)
        int si = 0, t0, nt = 1, split = 0;
        if (a.pairs > 0) {
            for (int j = 1; j < a.nseg; ++j)
                if (i >= a.pair_begin[j]) si = j;
            t0 = a.pair_tiles[si] * (i - a.pair_begin[si]);
            nt = min(a.pair_tiles[si], a.seg[si].tiles - t0);
        } else {
            const int g = i % tiles;
            split = i / tiles;
            for (int j = 1; j < a.nseg; ++j)
                if (g >= a.seg[j].tile_begin) si = j;
            t0 = g - a.seg[si].tile_begin;
        }
        const SegDev& s = a.seg[si];
        int block = 0;  // (prepare orders a block list's segments by weight; the caller's index of this one)
        for (int j = 0; j < L->nseg; ++j)
            if (L->seg[j].codes == s.codes && L->seg[j].col0 == s.col0) block = j;
        int32_t* o = work + 5 * (size_t)i;
        o[0] = block;
        o[1] = t0;
        o[2] = nt;
        o[3] = split;
        o[4] = s.col0 + t0 * cols;
    }
    return DR_OK;
}

int64_t dr_topk_merge_workspace_bytes(int n_records, int rows, int k) {
    if (n_records < 1 || rows < 1 || rows > SEL_MAXROWS || k < 1) return -1;
    return select_workspace_bytes(n_records, rows, k);
}

int dr_topk_merge(const void* records, int n_records, int rows, int k, int fp32, int k_out, float* vals,
                  int32_t* ids, void* workspace, int64_t workspace_bytes, void* stream) {
    if (records == nullptr || vals == nullptr || ids == nullptr || n_records < 1 || rows < 1 || rows > SEL_MAXROWS ||
        k < 1 || k_out < 1 || k_out > MERGE_MAXK)
        return DR_EINVAL;
    if ((int64_t)n_records * k > ((int64_t)1 << 40)) return DR_ERANGE;
    SelArgs A{reinterpret_cast<const uint32_t*>(records), n_records, rows, k, k_out, 1, 0, nullptr, nullptr, nullptr};
    select_plan(n_records, k, &A.slices, &A.cs);
    if (!select_bind(A, workspace, workspace_bytes)) return DR_EINVAL;
    if (k_out <= 32)
        hipLaunchKernelGGL(dr_merge_k<true>, dim3(rows * A.slices), dim3(SEL_T), 0, S(stream), A, fp32, vals, ids);
    else
        hipLaunchKernelGGL(dr_merge_k<false>, dim3(rows * A.slices), dim3(SEL_T), 0, S(stream), A, fp32, vals, ids);
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

// ---- the expert-gathered launches (include/moe.h) --------------------------------------------------------------------

namespace {

// the base launch's arguments (prepare), then the gather's: the tiles of the gate/up modes, the gathered K of the
// down modes, the rows a pass
int prepare_moe(const dr_launch* L, const dr_moe* M, MoeArgs& a, int& pw, int& tiles, int& mr) {
    if (L == nullptr || M == nullptr || M->mode < DR_MOE_GATE_UP || M->mode > DR_MOE_DOWN_ROWS) return DR_EINVAL;
    const int mode = M->mode;
    const bool nmode = mode == DR_MOE_GATE_UP || mode == DR_MOE_GATE_UP_ROWS;
    const bool rows = mode == DR_MOE_GATE_UP_ROWS || mode == DR_MOE_DOWN_ROWS;
    if (M->ids == nullptr || M->slots < 1 || M->slots > 16 || M->ld_ids < M->slots || M->id_rows < 1 ||
        M->id_rows > 32 || (!rows && M->id_rows != 1) || M->experts < 1 || (rows && M->experts > 1024) ||
        M->codes_stride <= 0 || M->exps_stride <= 0)
        return DR_EINVAL;
    const dr_segment& s0 = L->seg[0];
    if (L->nseg != 1 || L->residual != nullptr || L->topk.records != nullptr || (s0.fmt != DR_BFP4 && s0.fmt != DR_BFP4_KB) ||
        s0.scale != nullptr || s0.scale_up != nullptr || s0.col0 != 0 || (s0.glu == 2) != nmode || (!nmode && s0.glu))
        return DR_EINVAL;
    if (L->m < 1 || L->m > (rows ? M->id_rows : 1)) return DR_EINVAL;
    const int units = rows ? std::min(M->experts, M->id_rows * M->slots) : M->slots;
    dr_launch B = *L;
    int ekp = 0;
    if (nmode) {
        if (M->w == nullptr || M->ld_w < M->slots || M->expert_n != s0.n || L->y_f32 ||
            (int64_t)L->ldy < (int64_t)units * M->expert_n)
            return DR_EINVAL;
    } else {
        if (M->expert_k <= 0 || M->expert_k % 32 || L->k != units * M->expert_k) return DR_EINVAL;
        ekp = (M->expert_k + KALIGN - 1) / KALIGN * KALIGN;
        B.k = units * ekp;  // (the gathered K, each unit's block padded)
        B.ldx = std::max(L->ldx, B.k);
    }
    const int st = prepare(&B, a, pw, tiles, mr, true);
    if (st != DR_OK) return st;
    a.ldx = L->ldx;
    a.ids = M->ids;
    a.ids32 = M->ids32 != 0;
    a.ld_ids = M->ld_ids;
    a.slots = M->slots;
    a.id_rows = M->id_rows;
    a.experts = M->experts;
    a.rw = reinterpret_cast<const uint16_t*>(M->w);
    a.ld_rw = M->ld_w;
    a.cstride = M->codes_stride;
    a.estride = M->exps_stride;
    a.bias = reinterpret_cast<const uint16_t*>(M->bias);
    if (!rows)
        mr = 1;
    else if (L->m <= 2)
        mr = L->m;
    else
        // (gate/up too: one 32-row pass, x staged through LDS, rather than two of 16, whose second streams every
        // weight again: 17, 24 and 32 rows 155, 177, 188 -> 121, 134, 149 us at the gpt-oss shape)
        mr = L->m <= 16 ? 16 : 32;
    if (nmode) {
        // the MFMA rows of gate/up: 256-k chunks up to K = 3072, as the dense MFMA kernel's (the gpt-oss gate/up at 3,
        // 8, 16 and 32 rows 44.2, 80.3, 93.9, 225 -> 32.6, 69.8, 79.0, 188 us)
        if (mr >= 16 && !DR_CHUNK_K && a.k_pad <= 3072 && a.kch != 256)
            plan_chunks(a.k_pad, 256, &a.chunks, &a.kch, &a.waves, &a.splits, &a.cps);
        a.en = M->expert_n;
        a.tpe = (a.en + TILE - 1) / TILE;
        // the GEMV's 16-column tiles (a gate panel and an up panel) where they lower the most a CU streams
        if (mr <= 2 && narrow_better(units * a.tpe)) {
            pw = 2;
            a.tpe = (a.en + 15) / 16;
        }
        tiles = units * a.tpe;
        a.seg[0].tiles = tiles;
        a.tiles = tiles;
    } else {
        a.ek = M->expert_k;
        a.ekp = ekp;
        a.seg[0].pstride = (unsigned)((ekp / kblk(DR_BFP4)) * 1024);
        if (ekp % a.kch) plan_chunks(a.k_pad, 256, &a.chunks, &a.kch, &a.waves, &a.splits, &a.cps);  // (a chunk in one unit)
        // The GEMV's tile width and K splits (the down modes have no block lists, so they may depend on N): the pair
        // of the lowest cost, ceil(workgroups / CUs) rounds of cps chunks x the width each plus a workgroup's fixed
        // cost (its start, barrier and epilogue: about two 16-column chunks), plus the splits' meeting (about four);
        // ties to fewer splits, then to 32 columns. The gpt-oss-shaped down, 90 tiles x 24 chunks: 16 columns unsplit,
        // 180 workgroups of 3 chunks a wavefront (7.4 us; in 4 splits of 6 chunks, 720 workgroups, 8.0 us, the
        // choice without those terms; 2 splits 8.2, 3 8.1).
        if (mr <= 2) {
            const int c = cu_count(), t32 = a.seg[0].tiles, t16 = (a.seg[0].n_out + 15) / 16;
            long best = -1;
            int bw = 32, bcps = a.cps;
            for (int s = 1; s <= 8 && s <= a.chunks; ++s) {
                const int cps = (a.chunks + s - 1) / s, sp = (a.chunks + cps - 1) / cps;
                for (int w = 16; w <= 32; w += 16) {
                    const long wg = (long)(w == 16 ? t16 : t32) * sp;
                    if ((w == 16 ? t16 : t32) > SPLIT_MAXTILES) continue;
                    const long cost = (wg + c - 1) / c * ((long)cps * w + 32) + (sp > 1 ? 64 : 0);
                    if (best < 0 || cost < best || (cost == best && (sp < (a.chunks + bcps - 1) / bcps ||
                                                                     (sp == (a.chunks + bcps - 1) / bcps && w > bw)))) {
                        best = cost;
                        bw = w;
                        bcps = cps;
                    }
                }
            }
            a.cps = bcps;
            a.splits = (a.chunks + bcps - 1) / bcps;
            a.waves = bcps < MAXW_DOWN ? bcps : MAXW_DOWN;
            if (bw == 16) {
                pw = 1;
                tiles = t16;
                a.seg[0].tiles = t16;
                a.tiles = t16;
            }
        }
    }
    limit_splits(a);
    return DR_OK;
}

}  // namespace

extern "C" {

int64_t dr_moe_workspace_bytes(const dr_launch* L, const dr_moe* M) {
    MoeArgs a{};
    int pw, tiles, mr;
    if (prepare_moe(L, M, a, pw, tiles, mr) != DR_OK) return -1;
    return workspace_bytes(a, pw, mr);
}

int dr_moe_matmul(const dr_launch* L, const dr_moe* M) {
    MoeArgs a{};
    int pw, tiles, mr;
    const int st0 = prepare_moe(L, M, a, pw, tiles, mr);
    if (st0 != DR_OK) return st0;
    const int64_t need = workspace_bytes(a, pw, mr);
    if (need > 0) {
        if (L->workspace == nullptr || L->workspace_bytes < need) return DR_EINVAL;
        bind_split(a, L->workspace, pw, mr);
    }
    hipStream_t st = S(L->stream);
    const size_t ysz = a.y_f32 ? 4 : 2;
    for (int r0 = 0; r0 < L->m; r0 += mr) {
        MoeArgs p = a;
        p.m = L->m - r0 < mr ? L->m - r0 : mr;
        p.x = a.x + (size_t)r0 * a.ldx;
        p.y = reinterpret_cast<uint8_t*>(L->y) + (size_t)r0 * a.ldy * ysz;
        p.row0 = r0;
        const hipError_t e = launch_moe(p, M->mode, mr, pw, tiles * a.splits, st);
        if (e != hipSuccess) return DR_EHIP;
    }
    return DR_OK;
}

int dr_moe_route_gate_up(const dr_launch* L, const dr_moe* M, const dr_route* R) {
    moe_route::RouteArgs A;
    const int sr = moe_route::route_args(R, A);
    if (sr != DR_OK) return sr;
    if (R->experts > 64 * ROUTE_MAXPER) return DR_ERANGE;  // (more experts: dr_moe_route, then dr_moe_matmul)
    // one token routed into the buffers the gather then reads: the same ids, weights and experts
    if (M == nullptr || M->mode != DR_MOE_GATE_UP || R->rows != 1 || R->ids != M->ids || R->w != M->w ||
        (R->ids32 != 0) != (M->ids32 != 0) || R->experts != M->experts || M->slots != R->k + (R->slot >= 0 ? 1 : 0))
        return DR_EINVAL;
    MoeArgs a{};
    int pw, tiles, mr;
    const int st0 = prepare_moe(L, M, a, pw, tiles, mr);
    if (st0 != DR_OK) return st0;
    a.routed = 1;
    a.route = A;
    const int64_t need = workspace_bytes(a, pw, mr);
    if (need > 0) {
        if (L->workspace == nullptr || L->workspace_bytes < need) return DR_EINVAL;
        bind_split(a, L->workspace, pw, mr);
    }
    const hipError_t e = launch_moe(a, M->mode, mr, pw, tiles * a.splits, S(L->stream));
    return e == hipSuccess ? DR_OK : DR_EHIP;
}

}  // extern "C"
