// tbq_moe_prefill.hip -- batched (prefill) MoE experts on gfx950 fp16 MFMA.
//
// After routing (exact, as in decode), the (token, slot) pairs are grouped by
// expert and every expert's products run as dense tiles:
//
//   k_dispatch        per-expert histogram, prefix sum and permutation of the
//                     pairs in LDS (one workgroup), plus a tile list of
//                     (expert, first pair, pairs in tile) entries of <= 128
//                     pairs; order inside an expert does not affect results.
//   k_rows_f16        a matrix of fp32 rows to fp16, each row scaled by a
//                     power of two that puts its max |value| in [2^14, 2^15)
//                     (exact, undone in the GEMM epilogues): x for gate/up,
//                     the SwiGLU activations for down.
//   k_moe_f16<0,NS>   act[p] = swiglu(x_t . W_gate[e], x_t . W_up[e]) for a
//                     tile of <= 128 pairs x 128 columns (256 weight rows:
//                     128 gate and 128 up rows), K = H, fp32 out.
//   k_moe_f16<1,NS>   y[p] = act[p] . W_down[e] for <= 128 pairs x 256 rows,
//                     K = F.
//   (k_combine)       out = resid + sum over slots in slot order (tbq_moe.hip).
//
// Weights never pass through LDS.  Each lane dequantises its own MFMA A
// operands in registers: in v_mfma_f32_32x32x16_f16, lane l supplies row
// l % 32 and eight consecutive k of the 16 per step, the half h = l / 32
// choosing which eight.  Within a 128-column chunk the k order is permuted
// (the products are summed over k, so any order shared by both operands
// gives the same sum): step ks, half h covers chunk columns 64h + 8ks .. +8,
// so a lane's 64 weights per chunk are two whole Q4_K sub-blocks -- 32
// contiguous quant bytes and one scale/min pair each.  Only the activation
// tile is shared by the workgroup's 8 waves: it is staged in LDS, double
// buffered, one barrier per chunk.  Weight loads run two chunks ahead,
// activation loads one.
//
// Dequantisation to fp16.  A nibble q becomes the fp16 number 1 + q/16 by
// placing q in the mantissa (0x3C00 | q << 6), for two weights per dword:
// one 24-bit multiply spreads a quant byte's two nibbles into the two
// halves, one three-input bit operation (v_bitop3, (a & b) | c) masks them
// and sets the exponent; one v_pk_fma_f16 with (16 S, C = -16 S - M) gives
// 16 S (1 + q/16) + C = S q - M: three VALU per two weights.  The fma's
// product and sum are exact before its one rounding, so the fp16 roundings
// are those of 16 S, of C (at most ulp(16 S + M) / 2, a per-sub-block
// constant) and of the result.
//
// Accuracy: fp16 weights and activations (11-bit mantissa), fp32
// accumulation; outputs land within 1e-2 relative L2 of the fp32 reference.
// The weights' fp16 form needs 16 * 63 * d + 63 * dmin below 65504.
#include "tbq_kernels.h"
#include "tbq_kquant.hpp"

namespace tbq {

// The int8 prefill decodes Q4_K in the reference's layout for all three
// expert tensors; the fp16 one also takes all three in ggml's layout.
static bool prefill_q4k_layer(const MoeArgs &a) { return a.qg == QT_Q4_K && a.qu == QT_Q4_K && a.qd == QT_Q4_K; }
static bool prefill_gq4k_layer(const MoeArgs &a) {
    return a.qg == QT_GQ4_K && a.qu == QT_GQ4_K && a.qd == QT_GQ4_K;
}

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
// native vectors: HIP's uint4 struct is copied with memcpy, which keeps
// register arrays in scratch memory
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int PF_MT = 128;         // pairs per tile (four 32-pair MFMA sub-tiles)
constexpr int PF_KC = 128;         // K columns per chunk (half a Q4_K super-block)
constexpr int PF_LD = PF_KC + 8;   // LDS row stride in halves (padding breaks bank aliasing)
#ifndef PF_WAVES
#define PF_WAVES 8
#endif
constexpr int PF_THREADS = 64 * PF_WAVES;   // 32 weight rows per wave
constexpr int PF_ROWS = 32 * PF_WAVES;      // weight rows per workgroup
constexpr int PF_COLS = PF_ROWS / 2;        // gate/up columns per workgroup
constexpr size_t PF_LDS_BYTES = (size_t)2 * PF_MT * PF_LD * 2 + PF_MT * 8;   // two activation tiles, pair ids, scales

struct PfTile {
    int e, n;
};

// a tile's count of 32-pair sub-tiles as a type, for the per-count copies of
// the expert GEMM's chunk loop
template <int N>
struct PfSub {
    static constexpr int value = N;
};

// ---------------------------------------------------------------------------
// Dispatch: one workgroup of 1024 threads.  pairs p = t*k + s.  Tiles are
// listed heaviest first (by 32-pair sub-tile count), so the
// longest workgroups start first and the grid's tail is short; tile T's
// pairs are tpair[128T .. 128T + n) (-1 after), its activation rows ttok
// (= pair / k, the token).
// ---------------------------------------------------------------------------
constexpr int PF_MAX_TILES = 65536 * 8 / PF_MT + 256;
// up to this many pairs, k_dispatch keeps the expert indices in registers
// (read once) and the permutation in LDS: a permutation in global memory is
// read back, after its own stores, by a loop of dependent round trips
constexpr int PF_LDS_PAIRS = 8192;

__global__ __launch_bounds__(1024) void k_dispatch(const int *__restrict__ sel_idx, int T, int k, int E,
                                                   int *__restrict__ perm, PfTile *__restrict__ tiles,
                                                   int *__restrict__ ntiles, int *__restrict__ tpair,
                                                   int *__restrict__ ttok) {
    constexpr int NQ = PF_MT / 32;   // sub-tile count classes 1..NQ
    static_assert(PF_MT == 128 && NQ == 4, "tile classes");
    __shared__ int hist[256], off[257], cur[256], wsum[4];
    __shared__ int qcnt[NQ + 1], qbase[NQ + 2];
    __shared__ int t_e[PF_MAX_TILES], t_start[PF_MAX_TILES];
    __shared__ int perm_s[PF_LDS_PAIRS];
    constexpr int NE = PF_LDS_PAIRS / 1024;   // expert indices per thread
    const int tid = threadIdx.x, P = T * k;
    const bool small = P <= PF_LDS_PAIRS;   // uniform
    if (tid < 256) { hist[tid] = 0; cur[tid] = 0; }
    if (tid <= NQ) qcnt[tid] = 0;
    int es[NE];
    if (small) {
#pragma unroll
        for (int m = 0; m < NE; m++) {
            const int p = tid + 1024 * m;
            es[m] = p < P ? sel_idx[(p / k) * 8 + p % k] : -1;
        }
    }
    __syncthreads();
    // a pair whose expert index is outside [0, E) (never produced by the
    // router) joins no tile; the combine skips its slot
    if (small) {
#pragma unroll
        for (int m = 0; m < NE; m++)
            if ((unsigned)es[m] < (unsigned)E) atomicAdd(&hist[es[m]], 1);
    } else {
        for (int p = tid; p < P; p += 1024) {
            const int e = sel_idx[(p / k) * 8 + p % k];
            if ((unsigned)e < (unsigned)E) atomicAdd(&hist[e], 1);
        }
    }
    __syncthreads();
    // exclusive prefix sum of hist over 256 experts: a scan within each of
    // the first four waves (shuffles, no barrier), then the wave totals.
    // Tiles counted per sub-tile class: expert e has n >> 7 full tiles
    // (class 4) and, if n % 128 > 0, one of class (n % 128 + 31) / 32;
    // per wave by ballot counts, one LDS atomic per wave and class.
    int incl = 0;
    if (tid < 256) {   // four whole waves
        const int lane = tid & 63, n = hist[tid];   // 0 for experts >= E
        incl = n;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int o = __shfl_up(incl, d, 64);
            if (lane >= d) incl += o;
        }
        if (lane == 63) wsum[tid >> 6] = incl;
        const int rem = n & (PF_MT - 1), rq = (rem + 31) >> 5;   // 0 when rem = 0
        int c4 = (n >> 7) + (rq == NQ ? 1 : 0);
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) c4 += __shfl_xor(c4, d, 64);
        int cq[NQ + 1];
#pragma unroll
        for (int q = 1; q < NQ; q++) cq[q] = (int)__builtin_popcountll(__builtin_amdgcn_ballot_w64(rq == q));
        cq[NQ] = c4;
        if (lane == 0) {
#pragma unroll
            for (int q = 1; q <= NQ; q++)
                if (cq[q]) atomicAdd(&qcnt[q], cq[q]);
        }
    }
    __syncthreads();
    if (tid < 256) {
        int add = 0;
        for (int w = 0; w < (tid >> 6); w++) add += wsum[w];
        off[tid + 1] = incl + add;
    }
    if (tid == 0) {
        off[0] = 0;
        // classes NQ (heaviest) first
        int b = 0;
        for (int q = NQ; q >= 1; q--) {
            qbase[q] = b;
            b += qcnt[q];
            qcnt[q] = 0;
        }
        *ntiles = b;
        // item tickets of the two expert GEMMs (k_moe_f16), taken from 0
        ntiles[1] = 0;
        ntiles[2] = 0;
        qbase[0] = b;
    }
    __syncthreads();
    if (tid < E) {
        const int n = hist[tid];
        for (int s0 = 0; s0 < n; s0 += PF_MT) {
            const int q = (min(PF_MT, n - s0) + 31) / 32;
            const int t = qbase[q] + atomicAdd(&qcnt[q], 1);
            t_e[t] = tid | min(PF_MT, n - s0) << 16;   // expert | pairs in the tile
            t_start[t] = off[tid] + s0;
        }
    }
    if (small) {
#pragma unroll
        for (int m = 0; m < NE; m++) {
            const int e = es[m];
            if ((unsigned)e < (unsigned)E) perm_s[off[e] + atomicAdd(&cur[e], 1)] = tid + 1024 * m;
        }
    } else {
        for (int p = tid; p < P; p += 1024) {
            const int e = sel_idx[(p / k) * 8 + p % k];
            if ((unsigned)e < (unsigned)E) perm[off[e] + atomicAdd(&cur[e], 1)] = p;
        }
    }
    __syncthreads();
    const int nt = qbase[0];
    // the tile's record and first pair are two independent LDS reads
#pragma unroll 4
    for (int i = tid; i < nt * PF_MT; i += 1024) {
        const int t = i >> 7, j = i & (PF_MT - 1), te = t_e[t], st = t_start[t];
        const int e = te & 0xFFFF, n = te >> 16;
        if (j == 0) tiles[t] = PfTile{e, n};
        const int p = j < n ? (small ? perm_s[st + j] : perm[st + j]) : -1;
        tpair[i] = p;
        ttok[i] = p >= 0 ? p / k : -1;
    }
}

// ---------------------------------------------------------------------------
// Rows of n floats to fp16: one workgroup per row; s = 2^(15 - e) with
// max |row| = f * 2^e (f in [0.5, 1)), so |row| * s < 2^15; inv[row] = 1/s.
// n a multiple of 4.
// ---------------------------------------------------------------------------
// RV > 0: the row is held in registers (n <= 1024 RV), read once with
// every load issued before the max; RV = 0: two passes over the row.
template <int RV>
__global__ __launch_bounds__(256) void k_rows_f16(const float *__restrict__ in, int n, _Float16 *__restrict__ out,
                                                  float *__restrict__ inv) {
    __shared__ float part[4];
    const int row = blockIdx.x, tid = threadIdx.x, n4 = n / 4;
    const float4 *r = reinterpret_cast<const float4 *>(in + (long long)row * n);
    float4 v[RV > 0 ? RV : 1];
    float mx = 0.f;
    if constexpr (RV > 0) {
#pragma unroll
        for (int i = 0; i < RV; i++) v[i] = r[min(tid + 256 * i, n4 - 1)];   // clamped: unconditional
#pragma unroll
        for (int i = 0; i < RV; i++)
            if (tid + 256 * i < n4)
                mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
    } else {
        for (int i = tid; i < n4; i += 256) {
            const float4 w = r[i];
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(w.x), fabsf(w.y)), fmaxf(fabsf(w.z), fabsf(w.w))));
        }
    }
    mx = wave_max(mx);
    if ((tid & 63) == 0) part[tid >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(part[0], part[1]), fmaxf(part[2], part[3]));
    int e = 0;
    frexpf(mx, &e);
    int sh = mx > 0.f ? 15 - e : 0;
    sh = sh > 126 ? 126 : (sh < -126 ? -126 : sh);
    const float s = ldexpf(1.f, sh);
    uint2 *o = reinterpret_cast<uint2 *>(out + (long long)row * n);
    auto put = [&](int i, float4 w) {
        const f16x2 a = {(_Float16)(w.x * s), (_Float16)(w.y * s)};
        const f16x2 b = {(_Float16)(w.z * s), (_Float16)(w.w * s)};
        o[i] = make_uint2(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b));
    };
    if constexpr (RV > 0) {
#pragma unroll
        for (int i = 0; i < RV; i++)
            if (tid + 256 * i < n4) put(tid + 256 * i, v[i]);
    } else {
        for (int i = tid; i < n4; i += 256) put(i, r[i]);
    }
    if (tid == 0) inv[row] = ldexpf(1.f, -sh);
}

// ---------------------------------------------------------------------------
// Weight staging.
// ---------------------------------------------------------------------------
// One lane's loads for a 128-column chunk: the 64 weights of sub-blocks j0
// and j0 + 1 of a row's Q4_K super-block (j0 even), and 16 header bytes.
// The header the two chunks of a super-block need is bytes 0..19: d/dmin
// (0..3), the scale and min dwords of sub-blocks 0..3 (4..7, 8..11), the
// scale dword of 4..7 (12..15) and their min dword (16..19, which are quant
// bytes 0..3, layer4/tb_gguf.c:163-168).  The even chunk (j0 < 4) loads
// bytes 0..15 and passes d/dmin and the scale dword of 4..7 on to the odd
// chunk, which loads bytes 16..31 for the min dword: one 16-byte load per
// chunk instead of a dword and a dword pair (weight loads are issued per
// lane, each to its own row's cache lines, and their count is what the
// memory pipeline pays for).
struct Q4Pair {
    u32x4 h, q0, q1;
};

template <bool GG>
__device__ __forceinline__ void q4pair_load(const uint8_t *sb, int j0, Q4Pair &r) {
    // ggml's scales and mins of all eight sub-blocks are in bytes 4..15
    r.h = *reinterpret_cast<const u32x4 *>(sb + (GG || j0 < 4 ? 0 : 16));
    r.q0 = *reinterpret_cast<const u32x4 *>(sb + 16 + 16 * j0);
    r.q1 = *reinterpret_cast<const u32x4 *>(sb + 32 + 16 * j0);
}

__device__ __forceinline__ float h2f(unsigned bits) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)(bits & 0xFFFFu));
}

// Four quant bytes -> eight fp16 weights S q - Mn (low nibble first, the
// reference's order), as one MFMA operand.
__device__ __forceinline__ f16x8 q4dword_f16(unsigned q, f16x2 S16, f16x2 C) {
    unsigned o[4];
#pragma unroll
    for (int b = 0; b < 4; b++) {
        // quant byte (hi << 4 | lo) -> halves (1 + lo/16, 1 + hi/16)
        const unsigned y = (q >> (8 * b)) & 0xFFu;
        const unsigned t = __builtin_amdgcn_bitop3_b32(__umul24(y, 0x40040u), 0x03C003C0u, 0x3C003C00u, 0xEA);   // (a & b) | c
        o[b] = __builtin_bit_cast(unsigned, __builtin_elementwise_fma(__builtin_bit_cast(f16x2, t), S16, C));
    }
    return __builtin_bit_cast(f16x8, u32x4{o[0], o[1], o[2], o[3]});
}

// The lane's four A operands of sub-block j0 + u (steps 4u .. 4u + 3 of the
// chunk use its quant dwords 0..3).
// dd = d/dmin, sw and mw = the scale and min dwords of j0's half.
__device__ __forceinline__ void q4pair_frags(const Q4Pair &r, unsigned dd, unsigned sw, unsigned mw, int j0, int u,
                                             f16x8 *a) {
    const int sh = 8 * ((j0 + u) & 3);
    const float S = h2f(dd) * (float)((sw >> sh) & 63), Mn = h2f(dd >> 16) * (float)((mw >> sh) & 63);
    const _Float16 s16 = (_Float16)(16.f * S), c = (_Float16)(-(float)s16 - Mn);
    const f16x2 S16 = {s16, s16}, C = {c, c};
    const u32x4 q = u ? r.q1 : r.q0;
    a[0] = q4dword_f16(q.x, S16, C);
    a[1] = q4dword_f16(q.y, S16, C);
    a[2] = q4dword_f16(q.z, S16, C);
    a[3] = q4dword_f16(q.w, S16, C);
}

// ggml's layout (QT_GQ4_K): the 32 quant bytes of sub-blocks j0, j0 + 1 (j0
// even) hold sub-block j0's element i in the low nibble of byte i and
// sub-block j0 + 1's in the high nibble; the scale and min of sub-block j
// follow ggml's get_scale_min_k4 over scale bytes 4..15; d and dmin are IEEE
// halves.  Two quant dwords (bytes 8ks .. 8ks + 7) -> the eight fp16 weights
// S q - Mn of step ks: a byte pair's two nibbles are spread into the two
// halves by one 24-bit multiply (bits 6..9 and 22..25 of y * 0x4040, y the
// pair's nibbles at bits 0..3 and 8..11) and one v_bitop3, then the packed
// fma as in the reference's layout.
__device__ __forceinline__ f16x8 gq4dwords_f16(unsigned d0, unsigned d1, bool hi, f16x2 S16, f16x2 C) {
    const unsigned m0 = (hi ? d0 >> 4 : d0) & 0x0F0F0F0Fu, m1 = (hi ? d1 >> 4 : d1) & 0x0F0F0F0Fu;
    const unsigned y[4] = {m0 & 0xFFFFu, m0 >> 16, m1 & 0xFFFFu, m1 >> 16};
    unsigned o[4];
#pragma unroll
    for (int b = 0; b < 4; b++) {
        const unsigned t = __builtin_amdgcn_bitop3_b32(__umul24(y[b], 0x4040u), 0x03C003C0u, 0x3C003C00u, 0xEA);
        o[b] = __builtin_bit_cast(unsigned, __builtin_elementwise_fma(__builtin_bit_cast(f16x2, t), S16, C));
    }
    return __builtin_bit_cast(f16x8, u32x4{o[0], o[1], o[2], o[3]});
}

__device__ __forceinline__ void gq4pair_frags(const Q4Pair &r, int j0, int u, f16x8 *a) {
    const int jj = j0 + u, k = jj & 3;
    const bool hi = jj >= 4;
    const unsigned y = r.h.y >> (8 * k), z = r.h.z >> (8 * k), w = r.h.w >> (8 * k);
    const int sc = hi ? (int)((w & 15u) | (((y >> 6) & 3u) << 4)) : (int)(y & 63u);
    const int mn = hi ? (int)(((w >> 4) & 15u) | (((z >> 6) & 3u) << 4)) : (int)(z & 63u);
    const float S = h2f(r.h.x) * (float)sc, Mn = h2f(r.h.x >> 16) * (float)mn;
    const _Float16 s16 = (_Float16)(16.f * S), c = (_Float16)(-(float)s16 - Mn);
    const f16x2 S16 = {s16, s16}, C = {c, c};
    a[0] = gq4dwords_f16(r.q0.x, r.q0.y, u, S16, C);
    a[1] = gq4dwords_f16(r.q0.z, r.q0.w, u, S16, C);
    a[2] = gq4dwords_f16(r.q1.x, r.q1.y, u, S16, C);
    a[3] = gq4dwords_f16(r.q1.z, r.q1.w, u, S16, C);
}

// ---------------------------------------------------------------------------
// Expert tile GEMM.  Work items are (tile, row block) pairs, tile-major
// (ncb = F/PF_COLS row blocks for MODE 0, H/PF_ROWS for MODE 1), the tiles
// heaviest first; K = NS * 128.  The grid is persistent (one workgroup
// per CU): workgroup b starts with item b, then takes tickets from the
// counter ntiles[1 + MODE] (zeroed by k_dispatch): item grid + ticket, the
// ticket taken two chunks before the end of the current item.  Items thus
// go out heaviest first to whichever workgroup is about to be free (greedy
// list scheduling); a fixed stride over the items left the workgroups that
// drew heavy items 30% busier than the mean.
//   MODE 0: wave w, lane row i = l % 32 is gate (i < 16) or up (i >= 16)
//   column PF_COLS*cb + 16w + i % 16, so a lane's accumulator registers r
//   and r + 8 hold gate and up of the same (column, pair) and SwiGLU needs
//   no data exchange; X rows are tokens (ttok) of x.
//   MODE 1: lane row i is down row PF_ROWS*cb + 32w + i; X rows are pairs
//   (tpair) of act.  xinv[X row] undoes the row's fp16 scaling.
// Activation staging per chunk: segments tid + 512m (m < 4) = (pair it/16,
// 8 halves at 8*(it%16)).  Every global load is unconditional (indices
// clamped, results selected), so the compiler's wait counts stay exact.
// ---------------------------------------------------------------------------
template <int MODE, int NS, bool GG>
__global__ __launch_bounds__(PF_THREADS) void k_moe_f16(const uint8_t *__restrict__ W0, const uint8_t *__restrict__ W1,
                                                        const _Float16 *__restrict__ X, int x_rows,
                                                        const float *__restrict__ xinv, const int *__restrict__ tpair,
                                                        const int *__restrict__ ttok, const PfTile *__restrict__ tiles,
                                                        int *__restrict__ ntiles, int ncb, int H, int F,
                                                        float *__restrict__ out) {
    constexpr int K = NS * PF_KC;
    constexpr int XPT = PF_MT * PF_KC / 8 / PF_THREADS;   // 16-byte activation segments per thread per chunk
    extern __shared__ __attribute__((aligned(16))) _Float16 pf_lds[];   // [2][PF_MT][PF_LD]
    const int nitems = *ntiles * ncb;
    __shared__ int next_item;
    for (int item = blockIdx.x; item < nitems;) {
    // item -> (tile, row block).  The tile record and its row lists are
    // loaded together.
    const int tix = item / ncb, cb = item % ncb;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, li = lane & 31, lh = lane >> 5;
    const int *xrows = (MODE == 0 ? ttok : tpair) + tix * PF_MT;
    int px[XPT];
#pragma unroll
    for (int m = 0; m < XPT; m++) px[m] = xrows[(tid + PF_THREADS * m) >> 4];
    const int po = tid < PF_MT ? tpair[tix * PF_MT + tid] : -1;
    const int pxo = tid < PF_MT ? xrows[tid] : -1;
    const PfTile tl = tiles[tix];
    const long long rb = (long long)(K / 256) * 144;

    const uint8_t *wrow;
    if (MODE == 0) {
        const int col = cb * PF_COLS + 16 * wave + (li & 15);
        wrow = (li < 16 ? W0 : W1) + ((long long)tl.e * F + col) * rb;
    } else {
        wrow = W0 + ((long long)tl.e * H + cb * PF_ROWS + 32 * wave + li) * rb;
    }
    auto wload = [&](Q4Pair &w, int s) { q4pair_load<GG>(wrow + (long long)(s >> 1) * 144, 4 * (s & 1) + 2 * lh, w); };
    Q4Pair w0, w1, w2;

    // activation rows through a range-checked buffer descriptor: rows past
    // the tile's pair count (id -1) get an offset beyond the buffer, which
    // loads zeros without a memory access
    const int xbytes = x_rows * K * 2;
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc((void *)X, (short)0, xbytes, 0x00020000);
    int xoff[XPT];
#pragma unroll
    for (int m = 0; m < XPT; m++) {
        const int it = tid + PF_THREADS * m;
        xoff[m] = px[m] >= 0 ? (px[m] * K + 8 * (it & 15)) * 2 : xbytes;
    }
    u32x4 xr[XPT];
    auto xload = [&](int s) {
#pragma unroll
        for (int m = 0; m < XPT; m++)
            xr[m] = __builtin_amdgcn_raw_buffer_load_b128(xrs, xoff[m] < xbytes ? xoff[m] + s * PF_KC * 2 : xbytes, 0, 0);
    };
    auto xstore = [&](int buf) {
#pragma unroll
        for (int m = 0; m < XPT; m++) {
            const int it = tid + PF_THREADS * m;
            *reinterpret_cast<u32x4 *>(pf_lds + (buf * PF_MT + (it >> 4)) * PF_LD + 8 * (it & 15)) = xr[m];
        }
    };
    // Issue order: chunk 0's activations and the rows' scales, then the
    // weights of chunks 0 and 1, so that staging the activations and
    // storing the scales wait for their own loads only (the wait counter
    // counts loads in issue order); the weights arrive behind them.
    xload(0);
    const float sc = tid < PF_MT && pxo >= 0 ? xinv[pxo] : 0.f;
    wload(w0, 0);
    wload(w1, min(1, NS - 1));
    // the tile's pair ids and activation-row scales, for the epilogue, in
    // LDS behind the two activation buffers
    int *po_s = reinterpret_cast<int *>(pf_lds + 2 * PF_MT * PF_LD);
    float *sc_s = reinterpret_cast<float *>(po_s + PF_MT);
    xstore(0);
    if (tid < PF_MT) {
        po_s[tid] = po;
        sc_s[tid] = sc;
    }
    xload(min(1, NS - 1));
    __syncthreads();

    const _Float16 *xfrag = pf_lds + li * PF_LD + 64 * lh;
    // the workgroup's next item: a ticket taken two chunks before the end of
    // this one (its latency hidden behind them), so items go to workgroups
    // in the order they finish work, heaviest items first
    int nxt = 0;
    // d/dmin and the scale dword of sub-blocks 4..7, from the even chunk's
    // header for the odd chunk of the same super-block
    unsigned kdd = 0, ksw = 0;
    // The chunk loop and the epilogue for a compile-time count of 32-pair
    // sub-tiles (1..4, uniform over the workgroup): one copy per count, so
    // no branch splits a chunk's LDS reads from its MFMAs and the compiler
    // can issue the next operands' reads while the current MFMAs run.
    auto body = [&](auto nsub_c) {
        constexpr int NSUB = decltype(nsub_c)::value;
        f32x16 acc[NSUB];
#pragma unroll
        for (int t = 0; t < NSUB; t++) acc[t] = f32x16{};
        // steps 4u .. 4u + 3 of a chunk for every sub-tile
        auto mma = [&](const f16x8 *a, const _Float16 *xb, int u) {
#pragma unroll
            for (int t = 0; t < NSUB; t++) {
                f16x8 bv[4];
#pragma unroll
                for (int ks = 0; ks < 4; ks++)
                    bv[ks] = *reinterpret_cast<const f16x8 *>(xb + 32 * t * PF_LD + 8 * (4 * u + ks));
#pragma unroll
                for (int ks = 0; ks < 4; ks++)
                    acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[ks], bv[ks], acc[t], 0, 0, 0);
            }
        };
        // chunk s: weights of chunk s + 2 into wn (ring of three named
        // slots, so the loop need not be unrolled to keep them in
        // registers), activations of chunk s + 2 into registers after
        // staging chunk s + 1's into LDS.  Chunks past the end reload the
        // last one and skip the work.  Every path through a chunk issues the
        // same global loads (the compiler merges wait counts over paths, and
        // a path with fewer loads would make it wait for the prefetches too).
        auto chunk = [&](int s, const Q4Pair &wc, Q4Pair &wn) {
            wload(wn, min(s + 2, NS - 1));
            if (s == NS - 2 && tid == 0) nxt = atomicAdd(ntiles + 1 + MODE, 1) + (int)gridDim.x;
            if (s < NS) {
                const int j0 = 4 * (s & 1) + 2 * lh;
                const _Float16 *xb = xfrag + (s & 1) * PF_MT * PF_LD;
                if constexpr (GG) {
#pragma unroll
                    for (int u = 0; u < 2; u++) {
                        f16x8 a[4];
                        gq4pair_frags(wc, j0, u, a);
                        mma(a, xb, u);
                    }
                } else {
                    const bool odd = s & 1;
                    const unsigned dd = odd ? kdd : wc.h.x, sw = odd ? ksw : wc.h.y, mw = odd ? wc.h.x : wc.h.z;
                    kdd = dd;
                    ksw = odd ? ksw : wc.h.w;
#pragma unroll
                    for (int u = 0; u < 2; u++) {
                        f16x8 a[4];
                        q4pair_frags(wc, dd, sw, mw, j0, u, a);
                        mma(a, xb, u);
                    }
                }
                // buffer last read in chunk s - 1, before the previous barrier
                if (s + 1 < NS) xstore((s + 1) & 1);
            }
            xload(min(s + 2, NS - 1));
            if (s < NS) __syncthreads();
        };
        if constexpr (NS == 4 || (GG && NS <= 8)) {
            // two or three trips, not unrolled: unrolled, the compiler
            // overlaps the trips past what the register file holds (spills)
#pragma nounroll
            for (int s = 0; s < NS; s += 3) {
                chunk(s, w0, w2);
                chunk(s + 1, w1, w0);
                chunk(s + 2, w2, w1);
            }
        } else {
            for (int s = 0; s < NS; s += 3) {
                chunk(s, w0, w2);
                chunk(s + 1, w1, w0);
                chunk(s + 2, w2, w1);
            }
        }
        // accumulator register r of lane l: row 8(r/4) + 4(l/32) + r%4 of
        // the wave's 32, pair 32t + l%32 of the tile
#pragma unroll
        for (int t = 0; t < NSUB; t++) {
            const int pr = 32 * t + li;
            if (pr < tl.n) {
                const int p = po_s[pr];
                const float sc = sc_s[pr];
                if (MODE == 0) {
#pragma unroll
                    for (int h = 0; h < 2; h++) {
                        float a[4];
#pragma unroll
                        for (int c = 0; c < 4; c++) {
                            const int r = 4 * h + c;
                            const float g = acc[t][r] * sc, u = acc[t][r + 8] * sc;
                            a[c] = g * u * __builtin_amdgcn_rcpf(1.0f + __expf(-g));
                        }
                        const int col = cb * PF_COLS + 16 * wave + 8 * h + 4 * lh;
                        *reinterpret_cast<float4 *>(out + (long long)p * F + col) = make_float4(a[0], a[1], a[2], a[3]);
                    }
                } else {
#pragma unroll
                    for (int h = 0; h < 4; h++) {
                        const int row = cb * PF_ROWS + 32 * wave + 8 * h + 4 * lh;
                        *reinterpret_cast<float4 *>(out + (long long)p * H + row) =
                            make_float4(acc[t][4 * h] * sc, acc[t][4 * h + 1] * sc, acc[t][4 * h + 2] * sc,
                                        acc[t][4 * h + 3] * sc);
                    }
                }
            }
        }
    };
    switch ((tl.n + 31) / 32) {
    case 1: body(PfSub<1>{}); break;
    case 2: body(PfSub<2>{}); break;
    case 3: body(PfSub<3>{}); break;
    default: body(PfSub<4>{}); break;
    }
    // the next item rewrites the activation buffers and the pair lists
    if (tid == 0) next_item = nxt;
    __syncthreads();
    item = next_item;
    }
}

// ---------------------------------------------------------------------------
// int8 MFMA variant (TBQ_MOE_I8): Q8_K-quantised activations against the
// Q4_K nibbles on v_mfma_i32_32x32x32_i8.
//
// Activations.  k_rows_q8 quantises rows of n floats per 256-element block
// as the Q8_K activation quantiser (tbo_quantize_q8k): d = max|x| / 127,
// q1 = rint(x / d) clamped to +-127 (computed as x * (1/d)).  For the
// prefill it adds a second int8 level for the residual, q2 = rint((x - q1 d)
// * 256 / d) clamped to +-127, so x = d (q1 + q2 / 256) to 2^-16 of the
// block's max: with the first level alone the layer's MoE delta lands 1-2%
// from the fp32 reference on N(0,1) activations (the SwiGLU outputs are
// heavy-tailed), above the 1e-2 bound.  Each level keeps Q8_K's 16-element
// sums (fp16: |sum| <= 2032 is exact).  The int8 rows store the elements of
// every 16-element group in the order 0,2,4,6,1,3,5,7,8,10,12,14,9,11,13,15:
// the order in which one Q4_K quant dword unpacks with two AND masks and a
// shift (the reference's layout puts weights 2i and 2i+1 in the low and high
// nibbles of byte i, layer4/tb_gguf.c:148-180).  The sum over k does not
// depend on the order, which both operands share.
//
// Weights.  Per 32-weight sub-block j of a row the 6-bit scale is split
// sc_j = 8 a_j + b_j (a_j, b_j < 8) and folded into the int8 operands q a_j
// and q b_j (<= 105), so int8 MFMAs accumulate a whole super-block in int32
// with no per-output scaling: four per sub-block, (q a, q b) x (q1, q2).  The
// mins enter once per super-block through two fp16 MFMAs of the row's m_j
// (each twice) against the pair's 16-element sums of q1 and q2 (exact
// integers in fp32).  Per super-block and output, with F_l = 8 acc_a,l +
// acc_b,l and M_l = sum_j m_j S_j,l:
//   y += dx (d (F_1 + F_2 / 256) - dmin (M_1 + M_2 / 256))
// with d, dmin the row's fp16 super-block scales (a1's reading of the
// scale bytes) and dx the pair's block scale; fp32 accumulation.  The
// activations are the MFMAs' A operand and the weights B, so a lane's
// accumulators all belong to its own weight row (its d and dmin, no lane
// exchange per flush) and to 16 pairs, whose block scales are staged in LDS
// per item.
//
// Items: (tile, 32-pair sub-tile, row block), otherwise the layout of
// k_moe_f16 (8 waves x 32 weight rows, MODE 0 gate/up interleaved per wave,
// activation tile double-buffered in LDS, one barrier per chunk); SwiGLU
// takes a gate row's up partner from lane li + 16.
// ---------------------------------------------------------------------------
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

constexpr int I8_MT = 32;                 // pairs per item
#ifndef I8_AHEAD
#define I8_AHEAD 3                        // weight chunks in flight ahead of the one in use (2 or 3)
#endif
constexpr int I8_LD = PF_KC + 16;         // LDS row stride in bytes (one activation level)
// two activation tiles, the pair and row ids, the pairs' block scales (up
// to 16 super-blocks: K <= 4096), the pairs' 16-element sums of both levels
// (K / 8 halves per pair)
constexpr size_t I8_LDS_BYTES = (size_t)2 * I8_MT * 2 * I8_LD + I8_MT * 8 + 16 * I8_MT * 4 + I8_MT * 4096 / 4;

// Position of element e (< 16) of a 16-element group in the stored order.
__device__ __forceinline__ int q8_pos(int e) {
    const int h = e & 8, r = e & 7;
    return h + ((r & 1) << 2) + (r >> 1);
}

// One wave per 256-element block of a float array (blocks of 256
// consecutive floats).  BLOCKS = false: the prefill operand form of a row of
// n floats (int8 levels [row][2][n] in the MFMA order above, block scales
// [row][n/256], fp16 group sums [row][2][n/16]); BLOCKS = true: the
// reference's Q8_K block of the first level only (layer4/tb_gguf.c:281-288:
// f32 d at 0, int8 qs[256] in element order at 4, int16 bsums[16] at 260;
// 292 bytes), written to q8 with n, dq and bs16 unused.
template <bool BLOCKS>
__global__ __launch_bounds__(256) void k_rows_q8(const float *__restrict__ in, int n, long long nblocks,
                                                 int8_t *__restrict__ q8, float *__restrict__ dq,
                                                 _Float16 *__restrict__ bs16) {
    __shared__ int8_t stage[4][2][256];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const long long b0 = (long long)blockIdx.x * 4 + wave;
    const bool valid = b0 < nblocks;   // past the end: redo the last block, store nothing
    const long long b = valid ? b0 : nblocks - 1;
    const float4 v = reinterpret_cast<const float4 *>(in + b * 256)[lane];
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    amax = wave_max(amax);
    const float d = amax / 127.0f;
    const float id = d > 0.0f ? 1.0f / d : 0.0f;
    const float xs[4] = {v.x, v.y, v.z, v.w};
    int s1 = 0, s2 = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float r = rintf(xs[i] * id);
        r = fminf(fmaxf(r, -127.0f), 127.0f);
        const int q1 = (int)r;
        float r2 = rintf((xs[i] - r * d) * (id * 256.0f));
        r2 = fminf(fmaxf(r2, -127.0f), 127.0f);
        const int q2 = (int)r2;
        s1 += q1;
        s2 += q2;
        const int e = 4 * (lane & 3) + i;   // element within the lane's 16-element group
        const int pos = 16 * (lane >> 2) + (BLOCKS ? e : q8_pos(e));
        stage[wave][0][pos] = (int8_t)q1;
        stage[wave][1][pos] = (int8_t)q2;
    }
    // the group's sums over its four lanes
    s1 += __shfl_xor(s1, 1);
    s1 += __shfl_xor(s1, 2);
    s2 += __shfl_xor(s2, 1);
    s2 += __shfl_xor(s2, 2);
    __syncthreads();
    if (!valid) return;
    if constexpr (BLOCKS) {
        uint8_t *blk = reinterpret_cast<uint8_t *>(q8) + b * 292;   // 4-byte aligned
        reinterpret_cast<int *>(blk + 4)[lane] = reinterpret_cast<const int *>(stage[wave][0])[lane];
        if ((lane & 3) == 0) reinterpret_cast<int16_t *>(blk + 260)[lane >> 2] = (int16_t)s1;
        if (lane == 0) *reinterpret_cast<float *>(blk) = d;
    } else {
        const int nb = n / 256;
        const long long row = b / nb, blk = b % nb;
        int8_t *qr = q8 + row * 2 * n + blk * 256;
        reinterpret_cast<int *>(qr)[lane] = reinterpret_cast<const int *>(stage[wave][0])[lane];
        reinterpret_cast<int *>(qr + n)[lane] = reinterpret_cast<const int *>(stage[wave][1])[lane];
        if ((lane & 3) == 0) {
            _Float16 *sr = bs16 + row * 2 * (n / 16) + blk * 16 + (lane >> 2);
            sr[0] = (_Float16)(float)s1;
            sr[n / 16] = (_Float16)(float)s2;
        }
        if (lane == 0) dq[b] = d;
    }
}

// One lane's Q4_K data for a 128-column chunk c of its row: d/dmin, the
// chunk's four scale bytes, the four mins of its half of the super-block
// (for the min MFMA), and 8 quant bytes of each of the chunk's four
// sub-blocks (elements 16 lh .. 16 lh + 15 of sub-block 4 (c & 1) + ks).
// A lane's share of chunk c (half c & 1 of a super-block, sub-blocks
// 4(c & 1) .. +3): half lh of the k range, as two whole sub-blocks, lh and
// 2 + lh of the chunk (two 16-byte loads; MFMA step ks takes sub-block
// 2(ks >> 1) + lh, bytes 8(ks & 1) .. +7, and the activations' groups in
// the same order), d/dmin, the chunk's scale dword and the mins of the
// lane's half.
struct Q4I8 {
    unsigned dd, sw, mw;
    uint4 q[2];
};

__device__ __forceinline__ void q4i8_load(const uint8_t *sb, int c, int lh, Q4I8 &r) {
    r.dd = *reinterpret_cast<const unsigned *>(sb);
    r.sw = *reinterpret_cast<const unsigned *>(sb + ((c & 1) ? 12 : 4));
    r.mw = *reinterpret_cast<const unsigned *>(sb + (lh ? 16 : 8));   // mins 4..7 sit in quant bytes 0..3
    r.q[0] = *reinterpret_cast<const uint4 *>(sb + 16 + 64 * (c & 1) + 16 * lh);
    r.q[1] = *reinterpret_cast<const uint4 *>(sb + 16 + 64 * (c & 1) + 16 * (2 + lh));
}

template <int MODE, int NS>
__global__ __launch_bounds__(PF_THREADS) void k_moe_i8(const uint8_t *__restrict__ W0, const uint8_t *__restrict__ W1,
                                                       const int8_t *__restrict__ X, const float *__restrict__ XD,
                                                       const _Float16 *__restrict__ XB, int x_rows,
                                                       const int *__restrict__ tpair, const int *__restrict__ ttok,
                                                       const PfTile *__restrict__ tiles, const int *__restrict__ ntiles,
                                                       int ncb, int H, int F, float *__restrict__ out) {
    constexpr int K = NS * PF_KC;
    constexpr int NSB = K / 256;
    constexpr int NQ = PF_MT / I8_MT;   // sub-tiles per tile
    // weight chunks loaded ahead: 3 for long rows (two spill at K = 768)
    constexpr int AH = NS >= 8 ? I8_AHEAD : 2;
    extern __shared__ __attribute__((aligned(16))) int8_t i8_lds[];   // [2][I8_MT][2][I8_LD]
    int *po_s = reinterpret_cast<int *>(i8_lds + 2 * I8_MT * 2 * I8_LD);
    int *px_s = po_s + I8_MT;
    float *dx_s = reinterpret_cast<float *>(px_s + I8_MT);   // [NSB][I8_MT] block scale of pair slot
    _Float16 *xb_s = reinterpret_cast<_Float16 *>(dx_s + 16 * I8_MT);   // [I8_MT][K/8] group sums
    static_assert(NSB <= 16, "dx_s holds 16 super-blocks");
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, li = lane & 31, lh = lane >> 5;
    const long long rb = (long long)(K / 256) * 144;
    const int xbytes = x_rows * 2 * K;
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc((void *)X, (short)0, xbytes, 0x00020000);
    const int nitems = *ntiles * NQ * ncb;
    for (int item = blockIdx.x; item < nitems; item += gridDim.x) {
        const int tix = item / (NQ * ncb), qt = (item / ncb) % NQ, cb = item % ncb;
        const PfTile tl = tiles[tix];
        const int n = min(tl.n - I8_MT * qt, I8_MT);   // pairs of this sub-tile (uniform)
        if (n <= 0) continue;                         // uniform: no barrier skipped by part of the group
        const int *xrows = (MODE == 0 ? ttok : tpair) + tix * PF_MT + I8_MT * qt;
        // activation staging: thread -> (pair slot tid >> 4, level (tid >> 3) & 1, 16 bytes at 16 (tid & 7))
        const int xr = xrows[tid >> 4];
        const int xoff = xr >= 0 ? (xr * 2 + ((tid >> 3) & 1)) * K + 16 * (tid & 7) : xbytes;
        if (tid < I8_MT) {
            po_s[tid] = tpair[tix * PF_MT + I8_MT * qt + tid];
            px_s[tid] = xrows[tid];
        }
        const uint8_t *wrow;
        if (MODE == 0) {
            const int col = cb * PF_COLS + 16 * wave + (li & 15);
            wrow = (li < 16 ? W0 : W1) + ((long long)tl.e * F + col) * rb;
        } else {
            wrow = W0 + ((long long)tl.e * H + cb * PF_ROWS + 32 * wave + li) * rb;
        }
        auto wload = [&](Q4I8 &w, int c) {
            c = min(c, NS - 1);
            q4i8_load(wrow + (long long)(c >> 1) * 144, c, lh, w);
        };
        u32x4 xv;
        auto xload = [&](int c) {
            c = min(c, NS - 1);
            xv = __builtin_amdgcn_raw_buffer_load_b128(xrs, xoff < xbytes ? xoff + c * PF_KC : xbytes, 0, 0);
        };
        auto xstore = [&](int buf) {
            *reinterpret_cast<u32x4 *>(i8_lds + ((buf * I8_MT + (tid >> 4)) * 2 + ((tid >> 3) & 1)) * I8_LD +
                                       16 * (tid & 7)) = xv;
        };
        Q4I8 w0, w1, w2, w3;
        wload(w0, 0);
        wload(w1, min(1, NS - 1));
        if constexpr (AH == 3) wload(w2, min(2, NS - 1));
        xload(0);
        __syncthreads();   // po_s / px_s written
        // the pair slots' block scales and group sums into LDS (ordered
        // before the first flush by chunk 0's barrier): the flushes then
        // wait for no global load
        if (tid < NSB * I8_MT) {
            const int ps = tid % I8_MT, sbi = tid / I8_MT, xrw = px_s[ps];
            dx_s[tid] = xrw >= 0 ? XD[(long long)xrw * NSB + sbi] : 0.f;
        }
        {
            constexpr int SEG = K / 64;   // 16-byte segments of a slot's K / 8 halves
#pragma unroll
            for (int i0 = 0; i0 < I8_MT * SEG; i0 += PF_THREADS) {
                const int i = i0 + tid, ps = min(i / SEG, I8_MT - 1), sg = i % SEG, xrw = px_s[ps];
                const u32x4 v = *reinterpret_cast<const u32x4 *>(XB + (long long)(xrw >= 0 ? xrw : 0) * (K / 8) + 8 * sg);
                if (i < I8_MT * SEG)
                    *reinterpret_cast<u32x4 *>(xb_s + ps * (K / 8) + 8 * sg) = xrw >= 0 ? v : u32x4{0u, 0u, 0u, 0u};
            }
        }
        xstore(0);
        xload(1);
        __syncthreads();
        i32x16 aa1 = {}, ab1 = {}, aa2 = {}, ab2 = {};
        f32x16 y = {};
        // The MFMAs take the activations as the A operand and the weights as
        // B, so accumulator register r of lane l holds pair slot
        // 8(r/4) + 4(l/32) + r%4 and the lane's own weight row l%32: the
        // row's d and dmin are the lane's, the pairs' block scales come from
        // LDS.  Super-block flush:
        //   y += dx (d (F1 + F2/256) - dmin (M1 + M2/256))
        auto flush = [&](const Q4I8 &w, int sb) {
            f16x8 am;   // this lane's row's mins m_{4 lh + i}, each twice
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const _Float16 m = (_Float16)(float)((w.mw >> (8 * i)) & 63u);
                am[2 * i] = m;
                am[2 * i + 1] = m;
            }
            const _Float16 *bsr = xb_s + li * (K / 8) + 16 * sb + 8 * lh;   // pair slot li's sums
            const f16x8 b1 = *reinterpret_cast<const f16x8 *>(bsr);
            const f16x8 b2 = *reinterpret_cast<const f16x8 *>(bsr + K / 16);
            const f32x16 m1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(b1, am, f32x16{}, 0, 0, 0);
            const f32x16 m2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(b2, am, f32x16{}, 0, 0, 0);
            const float dw = f16_ref((uint16_t)(w.dd & 0xFFFFu)), mw = f16_ref((uint16_t)(w.dd >> 16));
            const float4 *dxs = reinterpret_cast<const float4 *>(dx_s + sb * I8_MT);
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const float4 dx4 = dxs[2 * c + lh];   // pair slots 8c + 4lh + 0..3
                const float dxv[4] = {dx4.x, dx4.y, dx4.z, dx4.w};
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const int r = 4 * c + q;
                    const float f = fmaf((float)(8 * aa2[r] + ab2[r]), 1.0f / 256.0f, (float)(8 * aa1[r] + ab1[r]));
                    const float mm = fmaf(m2[r], 1.0f / 256.0f, m1[r]);
                    y[r] = fmaf(dxv[q], fmaf(dw, f, -mw * mm), y[r]);
                }
            }
            aa1 = i32x16{};
            ab1 = i32x16{};
            aa2 = i32x16{};
            ab2 = i32x16{};
        };
        auto chunk = [&](int s, const Q4I8 &wc, Q4I8 &wn) {
            wload(wn, s + AH);
            if (s < NS) {
                const int8_t *xb = i8_lds + ((s & 1) * I8_MT + li) * 2 * I8_LD + 32 * lh;
#pragma unroll
                for (int ks = 0; ks < 4; ks++) {
                    const uint4 q4 = wc.q[ks >> 1];
                    const uint2 q = (ks & 1) ? make_uint2(q4.z, q4.w) : make_uint2(q4.x, q4.y);
                    const unsigned sc = (wc.sw >> (8 * (2 * (ks >> 1) + lh))) & 63u;   // sub-block 2(ks>>1) + lh
                    const unsigned short a = (unsigned short)(sc >> 3), b = (unsigned short)(sc & 7u);
                    const unsigned n0 = q.x & 0x0F0F0F0Fu, n1 = (q.x >> 4) & 0x0F0F0F0Fu;
                    const unsigned n2 = q.y & 0x0F0F0F0Fu, n3 = (q.y >> 4) & 0x0F0F0F0Fu;
                    const u16x2 va = {a, a}, vb = {b, b};
                    auto mul = [](unsigned v, u16x2 f) {
                        return __builtin_bit_cast(unsigned, __builtin_bit_cast(u16x2, v) * f);
                    };
                    const i32x4 Aa = {(int)mul(n0, va), (int)mul(n1, va), (int)mul(n2, va), (int)mul(n3, va)};
                    const i32x4 Ab = {(int)mul(n0, vb), (int)mul(n1, vb), (int)mul(n2, vb), (int)mul(n3, vb)};
                    // 16-element group 4(ks >> 1) + 2 lh + (ks & 1) of the chunk
                    const int go = 64 * (ks >> 1) + 16 * (ks & 1);
                    const i32x4 bv1 = *reinterpret_cast<const i32x4 *>(xb + go);
                    const i32x4 bv2 = *reinterpret_cast<const i32x4 *>(xb + I8_LD + go);
                    aa1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(bv1, Aa, aa1, 0, 0, 0);
                    ab1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(bv1, Ab, ab1, 0, 0, 0);
                    aa2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(bv2, Aa, aa2, 0, 0, 0);
                    ab2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(bv2, Ab, ab2, 0, 0, 0);
                }
                if (s & 1) flush(wc, s >> 1);
                if (s + 1 < NS) xstore((s + 1) & 1);
            }
            xload(s + 2);
            if (s < NS) __syncthreads();
        };
        if constexpr (AH == 3) {
            for (int s = 0; s < NS; s += 4) {
                chunk(s, w0, w3);
                chunk(s + 1, w1, w0);
                chunk(s + 2, w2, w1);
                chunk(s + 3, w3, w2);
            }
        } else {
            for (int s = 0; s < NS; s += 3) {
                chunk(s, w0, w2);
                chunk(s + 1, w1, w0);
                chunk(s + 2, w2, w1);
            }
        }
        // accumulator register r of lane l: pair slot 8(r/4) + 4 lh + r%4 of
        // the sub-tile, the wave's weight row li
        if (MODE == 0) {
            // gate (rows li < 16) and up (li + 16) of column 16 wave + li%16:
            // the up value from lane li + 16
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const float uv = __shfl_xor(y[r], 16);
                const int pr = 8 * (r >> 2) + 4 * lh + (r & 3);
                if (li < 16 && pr < n) {
                    const float g = y[r];
                    const float o = g * uv * __builtin_amdgcn_rcpf(1.0f + __expf(-g));
                    out[(long long)po_s[pr] * F + cb * PF_COLS + 16 * wave + li] = o;
                }
            }
        } else {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int pr = 8 * (r >> 2) + 4 * lh + (r & 3);
                if (pr < n) out[(long long)po_s[pr] * H + cb * PF_ROWS + 32 * wave + li] = y[r];
            }
        }
        __syncthreads();   // the next item rewrites the pair lists and the activation buffers
    }
}

template <int MODE>
static hipError_t launch_moe_i8(int ns, unsigned nwg, hipStream_t st, const uint8_t *W0, const uint8_t *W1,
                                const int8_t *X, const float *XD, const _Float16 *XB, int x_rows, const int *tpair,
                                const int *ttok, const PfTile *tiles, const int *ntiles, int ncb, int H, int F,
                                float *out) {
#define TBQ_NS(N)                                                                                                   \
    case N:                                                                                                         \
        hipLaunchKernelGGL((k_moe_i8<MODE, N>), dim3(nwg), dim3(PF_THREADS), I8_LDS_BYTES, st, W0, W1, X, XD, XB,   \
                           x_rows, tpair, ttok, tiles, ntiles, ncb, H, F, out);                                     \
        break;
    switch (ns) {
        TBQ_NS(2) TBQ_NS(4) TBQ_NS(6) TBQ_NS(8) TBQ_NS(12) TBQ_NS(16) TBQ_NS(24) TBQ_NS(32)
    default:
        return hipErrorNotSupported;
    }
#undef TBQ_NS
    return hipGetLastError();
}

size_t prefill_workspace_bytes(int T, int k, int E, int H, int F) {
    const size_t P = (size_t)T * k;
    const size_t max_tiles = (P + PF_MT - 1) / PF_MT + E;
    auto up = [](size_t n) { return (n + 255) & ~(size_t)255; };
    return up(P * 4) + up(max_tiles * sizeof(PfTile)) + 256 + 2 * up(max_tiles * PF_MT * 4) + up(P * F * 2) +
           up((size_t)T * H * 2) + up(P * 4) + up((size_t)T * 4);
}

// Persistent grid of the expert GEMMs: one workgroup per CU (about 200
// VGPRs per lane hold two of the eight waves per SIMD, so a second
// workgroup would only queue behind the first), never more than the item
// count bound.
static unsigned pf_grid(unsigned max_items) {
    const unsigned g = (unsigned)(tbq_cu_count() > 0 ? tbq_cu_count() : 256);
    return max_items < g ? max_items : g;
}

template <int MODE, bool GG>
static hipError_t launch_moe_f16(int ns, unsigned nwg, hipStream_t st, const uint8_t *W0, const uint8_t *W1,
                                 const _Float16 *X, int x_rows, const float *xinv, const int *tpair, const int *ttok,
                                 const PfTile *tiles, int *ntiles, int ncb, int H, int F, float *out) {
    // more than 64 KiB of dynamic LDS is opted into once per kernel
#define TBQ_NS(N)                                                                                                  \
    case N: {                                                                                                      \
        static const hipError_t attr = hipFuncSetAttribute((const void *)k_moe_f16<MODE, N, GG>,                   \
                                                           hipFuncAttributeMaxDynamicSharedMemorySize,             \
                                                           (int)PF_LDS_BYTES);                                     \
        if (attr != hipSuccess) return attr;                                                                       \
        hipLaunchKernelGGL((k_moe_f16<MODE, N, GG>), dim3(nwg), dim3(PF_THREADS), PF_LDS_BYTES, st, W0, W1, X,     \
                           x_rows, xinv, tpair, ttok, tiles, ntiles, ncb, H, F, out);                              \
        break;                                                                                                     \
    }
    switch (ns) {
        TBQ_NS(2) TBQ_NS(4) TBQ_NS(6) TBQ_NS(8) TBQ_NS(12) TBQ_NS(16) TBQ_NS(24) TBQ_NS(32)
    default:
        return hipErrorNotSupported;
    }
#undef TBQ_NS
    return hipGetLastError();
}

// K values the MFMA kernel is instantiated for (K = 128 * NS).
bool gemm_k_supported(int K) {
    const int n = K / PF_KC;
    return K % 256 == 0 && (n == 2 || n == 4 || n == 6 || n == 8 || n == 12 || n == 16 || n == 24 || n == 32);
}

// int8 mode workspace: the dispatch lists of the fp16 mode, then the
// two-level Q8_K activations of x ([T][2][H] int8, block scales [T][H/256],
// fp16 16-element sums [T][2][H/16]) and of the SwiGLU output ([P][2][F],
// the same three).
size_t prefill_i8_workspace_bytes(int T, int k, int E, int H, int F) {
    const size_t P = (size_t)T * k;
    const size_t max_tiles = (P + PF_MT - 1) / PF_MT + E;
    auto up = [](size_t n) { return (n + 255) & ~(size_t)255; };
    return up(P * 4) + up(max_tiles * sizeof(PfTile)) + 256 + 2 * up(max_tiles * PF_MT * 4) +
           up((size_t)T * H * 2) + up((size_t)T * H / 256 * 4) + up((size_t)T * H / 16 * 4) + up(P * F * 2) +
           up(P * F / 256 * 4) + up(P * F / 16 * 4);
}

// Rows of n floats (n a multiple of 256) to Q8_K blocks in the int8 MFMA
// operand order (k_rows_q8).
hipError_t launch_rows_q8(const float *in, long long rows, int n, int8_t *q8, float *dq, _Float16 *bs16,
                          hipStream_t st) {
    const long long nb = rows * (n / 256);
    hipLaunchKernelGGL(k_rows_q8<false>, dim3((unsigned)((nb + 3) / 4)), dim3(256), 0, st, in, n, nb, q8, dq, bs16);
    return hipGetLastError();
}

// n floats (a multiple of 256) to n / 256 Q8_K blocks of 292 bytes.
hipError_t launch_quantize_q8k(const float *in, long long n, void *blocks, hipStream_t st) {
    const long long nb = n / 256;
    hipLaunchKernelGGL(k_rows_q8<true>, dim3((unsigned)((nb + 3) / 4)), dim3(256), 0, st, in, 256, nb,
                       (int8_t *)blocks, nullptr, nullptr);
    return hipGetLastError();
}

hipError_t launch_moe_prefill_q4k_i8(const MoeArgs &a, void *scratch, hipStream_t st) {
    if (!prefill_q4k_layer(a) || !gemm_k_supported(a.H) || !gemm_k_supported(a.F) || a.H % PF_ROWS ||
        a.F % PF_COLS || a.T > 65536 || a.E > 256)
        return hipErrorNotSupported;
    const size_t P = (size_t)a.T * a.k;
    const int max_tiles = (int)((P + PF_MT - 1) / PF_MT + a.E);
    auto up = [](size_t n) { return (n + 255) & ~(size_t)255; };
    char *w = (char *)scratch;
    int *perm = (int *)w; w += up(P * 4);
    PfTile *tiles = (PfTile *)w; w += up((size_t)max_tiles * sizeof(PfTile));
    int *ntiles = (int *)w; w += 256;
    int *tpair = (int *)w; w += up((size_t)max_tiles * PF_MT * 4);
    int *ttok = (int *)w; w += up((size_t)max_tiles * PF_MT * 4);
    int8_t *x8 = (int8_t *)w; w += up((size_t)a.T * a.H * 2);
    float *xd = (float *)w; w += up((size_t)a.T * a.H / 256 * 4);
    _Float16 *xb = (_Float16 *)w; w += up((size_t)a.T * a.H / 16 * 4);
    int8_t *a8 = (int8_t *)w; w += up(P * a.F * 2);
    float *ad = (float *)w; w += up(P * a.F / 256 * 4);
    _Float16 *ab = (_Float16 *)w;
    hipError_t err = launch_rows_q8(a.xn, a.T, a.H, x8, xd, xb, st);
    if (err != hipSuccess) return err;
    hipLaunchKernelGGL(k_dispatch, dim3(1), dim3(1024), 0, st, a.sel_idx, a.T, a.k, a.E, perm, tiles, ntiles, tpair,
                       ttok);
    err = hipGetLastError();
    if (err != hipSuccess) return err;
    const int ncb0 = a.F / PF_COLS, ncb1 = a.H / PF_ROWS;
    err = launch_moe_i8<0>(a.H / PF_KC, pf_grid((unsigned)(PF_MT / I8_MT * max_tiles * ncb0)), st, (const uint8_t *)a.gate,
                           (const uint8_t *)a.up, x8, xd, xb, a.T, tpair, ttok, tiles, ntiles, ncb0, a.H, a.F, a.act);
    if (err != hipSuccess) return err;
    err = launch_rows_q8(a.act, (long long)P, a.F, a8, ad, ab, st);
    if (err != hipSuccess) return err;
    return launch_moe_i8<1>(a.F / PF_KC, pf_grid((unsigned)(PF_MT / I8_MT * max_tiles * ncb1)), st, (const uint8_t *)a.down,
                            nullptr, a8, ad, ab, (int)P, tpair, ttok, tiles, ntiles, ncb1, a.H, a.F, a.y);
}

// Short rows (n <= 64 * 4 * RW floats): one wave per row, four rows per
// workgroup, the row's max by a wave reduction with no LDS or barrier; the
// same scale and conversion as k_rows_f16.
template <int RW>
__global__ __launch_bounds__(256) void k_rows_f16_wave(const float *__restrict__ in, int rows, int n,
                                                       _Float16 *__restrict__ out, float *__restrict__ inv) {
    const int lane = threadIdx.x & 63;
    const int row = min((int)blockIdx.x * 4 + (int)(threadIdx.x >> 6), rows - 1);   // past the end: redo the last
    const bool store = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6) < rows;
    const int n4 = n / 4;
    const float4 *r = reinterpret_cast<const float4 *>(in + (long long)row * n);
    float4 v[RW];
#pragma unroll
    for (int i = 0; i < RW; i++) v[i] = r[min(lane + 64 * i, n4 - 1)];   // clamped: unconditional
    float mx = 0.f;
#pragma unroll
    for (int i = 0; i < RW; i++)
        if (lane + 64 * i < n4)
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
    mx = wave_max(mx);
    int e = 0;
    frexpf(mx, &e);
    int sh = mx > 0.f ? 15 - e : 0;
    sh = sh > 126 ? 126 : (sh < -126 ? -126 : sh);
    const float s = ldexpf(1.f, sh);
    if (!store) return;
    uint2 *o = reinterpret_cast<uint2 *>(out + (long long)row * n);
#pragma unroll
    for (int i = 0; i < RW; i++) {
        if (lane + 64 * i < n4) {
            const f16x2 a = {(_Float16)(v[i].x * s), (_Float16)(v[i].y * s)};
            const f16x2 b = {(_Float16)(v[i].z * s), (_Float16)(v[i].w * s)};
            o[lane + 64 * i] = make_uint2(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b));
        }
    }
    if (lane == 0) inv[row] = ldexpf(1.f, -sh);
}

hipError_t launch_rows_f16(const float *in, int rows, int n, _Float16 *out, float *inv, hipStream_t st) {
    const int rw = (n / 4 + 63) / 64;   // float4 per lane with a wave per row
    const unsigned wgs = (unsigned)((rows + 3) / 4);
    if (rw <= 4) {
        if (rw <= 1) hipLaunchKernelGGL(k_rows_f16_wave<1>, dim3(wgs), dim3(256), 0, st, in, rows, n, out, inv);
        else if (rw <= 2) hipLaunchKernelGGL(k_rows_f16_wave<2>, dim3(wgs), dim3(256), 0, st, in, rows, n, out, inv);
        else if (rw <= 3) hipLaunchKernelGGL(k_rows_f16_wave<3>, dim3(wgs), dim3(256), 0, st, in, rows, n, out, inv);
        else hipLaunchKernelGGL(k_rows_f16_wave<4>, dim3(wgs), dim3(256), 0, st, in, rows, n, out, inv);
        return hipGetLastError();
    }
    const int rv = (n / 4 + 255) / 256;
    switch (rv) {
    case 1: hipLaunchKernelGGL(k_rows_f16<1>, dim3(rows), dim3(256), 0, st, in, n, out, inv); break;
    case 2: hipLaunchKernelGGL(k_rows_f16<2>, dim3(rows), dim3(256), 0, st, in, n, out, inv); break;
    case 3: case 4: hipLaunchKernelGGL(k_rows_f16<4>, dim3(rows), dim3(256), 0, st, in, n, out, inv); break;
    case 5: case 6: case 7: case 8: hipLaunchKernelGGL(k_rows_f16<8>, dim3(rows), dim3(256), 0, st, in, n, out, inv); break;
    case 9: case 10: case 11: case 12: hipLaunchKernelGGL(k_rows_f16<12>, dim3(rows), dim3(256), 0, st, in, n, out, inv); break;
    case 13: case 14: case 15: case 16: hipLaunchKernelGGL(k_rows_f16<16>, dim3(rows), dim3(256), 0, st, in, n, out, inv); break;
    default: hipLaunchKernelGGL(k_rows_f16<0>, dim3(rows), dim3(256), 0, st, in, n, out, inv); break;
    }
    return hipGetLastError();
}

// Experts on MFMA for Q4_K weights; routing already in a.sel_idx/a.sel_w.
// Uses a.act (pairs x F fp32), a.y (pairs x H fp32) and `scratch`
// (prefill_workspace_bytes).  H and F must be 256, 512, 768, 1024, 1536,
// 2048, 3072 or 4096, H a multiple of PF_ROWS and F of PF_COLS; T <= 65536.
void prefill_x16(const MoeArgs &a, void *scratch, _Float16 **x16, float **xinv) {
    const size_t P = (size_t)a.T * a.k;
    const size_t max_tiles = (P + PF_MT - 1) / PF_MT + a.E;
    auto up = [](size_t n) { return (n + 255) & ~(size_t)255; };
    char *w = (char *)scratch;
    w += up(P * 4) + up(max_tiles * sizeof(PfTile)) + 256 + 2 * up(max_tiles * PF_MT * 4) + up(P * a.F * 2);
    *x16 = (_Float16 *)w;
    w += up((size_t)a.T * a.H * 2) + up(P * 4);
    *xinv = (float *)w;
}

hipError_t launch_moe_prefill_q4k(const MoeArgs &a, void *scratch, hipStream_t st, bool x16_done) {
    auto ok_k = [](int K) {
        const int n = K / PF_KC;
        return K % 256 == 0 && gemm_k_supported(K);
    };
    const bool gg = prefill_gq4k_layer(a);
    if (!(prefill_q4k_layer(a) || gg) || !ok_k(a.H) || !ok_k(a.F) || a.H % PF_ROWS || a.F % PF_COLS ||
        a.T > 65536 || a.E > 256)
        return hipErrorNotSupported;
    const size_t P = (size_t)a.T * a.k;
    const int max_tiles = (int)((P + PF_MT - 1) / PF_MT + a.E);
    auto up = [](size_t n) { return (n + 255) & ~(size_t)255; };
    char *w = (char *)scratch;
    int *perm = (int *)w; w += up(P * 4);
    PfTile *tiles = (PfTile *)w; w += up((size_t)max_tiles * sizeof(PfTile));
    int *ntiles = (int *)w; w += 256;
    int *tpair = (int *)w; w += up((size_t)max_tiles * PF_MT * 4);
    int *ttok = (int *)w; w += up((size_t)max_tiles * PF_MT * 4);
    _Float16 *act16 = (_Float16 *)w; w += up(P * a.F * 2);
    _Float16 *x16 = (_Float16 *)w; w += up((size_t)a.T * a.H * 2);
    float *ainv = (float *)w; w += up(P * 4);
    float *xinv = (float *)w;
    if (!x16_done) {
        const hipError_t e = launch_rows_f16(a.xn, a.T, a.H, x16, xinv, st);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(k_dispatch, dim3(1), dim3(1024), 0, st, a.sel_idx, a.T, a.k, a.E, perm, tiles, ntiles, tpair,
                       ttok);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    const int ncb0 = a.F / PF_COLS, ncb1 = a.H / PF_ROWS;
    const unsigned g0 = pf_grid((unsigned)(max_tiles * ncb0)), g1 = pf_grid((unsigned)(max_tiles * ncb1));
    const uint8_t *wg = (const uint8_t *)a.gate, *wu = (const uint8_t *)a.up, *wd = (const uint8_t *)a.down;
    err = gg ? launch_moe_f16<0, true>(a.H / PF_KC, g0, st, wg, wu, x16, a.T, xinv, tpair, ttok, tiles, ntiles, ncb0,
                                       a.H, a.F, a.act)
             : launch_moe_f16<0, false>(a.H / PF_KC, g0, st, wg, wu, x16, a.T, xinv, tpair, ttok, tiles, ntiles,
                                        ncb0, a.H, a.F, a.act);
    if (err != hipSuccess) return err;
    err = launch_rows_f16(a.act, (int)P, a.F, act16, ainv, st);
    if (err != hipSuccess) return err;
    return gg ? launch_moe_f16<1, true>(a.F / PF_KC, g1, st, wd, nullptr, act16, (int)P, ainv, tpair, ttok, tiles,
                                        ntiles, ncb1, a.H, a.F, a.y)
              : launch_moe_f16<1, false>(a.F / PF_KC, g1, st, wd, nullptr, act16, (int)P, ainv, tpair, ttok, tiles,
                                         ntiles, ncb1, a.H, a.F, a.y);
}

}  // namespace tbq
