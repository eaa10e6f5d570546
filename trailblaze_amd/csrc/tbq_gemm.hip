// tbq_gemm.hip -- the batched prefill's weight products on gfx950:
//
//   C[T][N] = X[T][K] . W[N][K]^T      X fp16 rows (a power-of-two scale per
//                                      row, undone by the consumer), W fp16
//                                      rows or Q4_K rows, fp32 accumulate and
//                                      output
//
// Tiling.  A workgroup of 4 waves owns a 128 (n) x 128 (t) tile of C (rows
// past N or T are clamped on load and not stored), two workgroups per CU;
// wave w owns the 64 x 64 block (n half w & 1, t half w >> 1) as 2 x 2
// blocks of v_mfma_f32_32x32x16_f16 (A = 32 weight rows x 16 k, B = 16 k x
// 32 tokens).  Measured alternatives, all slower on the Qwen3-4B prefill
// shapes: 128 x 256 and 256 x 128 tiles of 8 waves (one workgroup per CU),
// 128 x 64 blocks per wave, K steps of 32 with four workgroups per CU.
// K advances 64 columns per step through two LDS stages of both operands
// ([row][64 + 8 halves]: the 8-half pad puts any 8 consecutive rows of a
// 16-byte column read on 8 disjoint 4-bank groups).  Step s+2's global loads
// are issued two steps ahead into one of two register sets and written to
// the other LDS stage after step s's MFMAs, with one barrier per step.
//
// Weights.  fp16 rows are copied.  Q4_K rows (reference layout) are
// dequantised on the way into LDS: per step a thread takes a piece of one
// 32-weight sub-block of one row (its quant bytes, the super-block's d/dmin
// and the sub-block's 6-bit scale and min, with the reference's reading of
// the scale bytes, layer4/tb_gguf.c:148-180) and writes its fp16 weights
// (q4sub_f16).
//
// Split K.  When the n x t tiles are fewer than the CUs can run, K is split
// over gridDim.z slices; slice z writes its partial sums to P[z][T][N] and
// k_gemm_reduce adds the slices in slice order into C.
#include <algorithm>

#include "tbq_kernels.h"
#include "tbq_kquant.hpp"

namespace tbq {

namespace {

typedef _Float16 hg_f16x8 __attribute__((ext_vector_type(8)));
typedef float hg_f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned hg_u32x4 __attribute__((ext_vector_type(4)));

#ifndef TBQ_HG_BT
#define TBQ_HG_BT 128
#endif
#ifndef TBQ_HG_BN
#define TBQ_HG_BN 128
#endif
#ifndef TBQ_HG_BK
#define TBQ_HG_BK 64
#endif
#ifndef TBQ_HG_WPE
#define TBQ_HG_WPE 2
#endif
constexpr int HG_BN = TBQ_HG_BN, HG_BT = TBQ_HG_BT, HG_BK = TBQ_HG_BK;
constexpr int HG_LD = HG_BK + 8;                  // LDS row stride in halves
#ifndef TBQ_HG_WI
#define TBQ_HG_WI 2
#endif
constexpr int HG_WI = TBQ_HG_WI, HG_WJ = 2;       // 32 x 32 blocks per wave along n and t
constexpr int HG_WN = HG_BN / (32 * HG_WI);       // waves along n
constexpr int HG_THREADS = 64 * HG_WN * (HG_BT / (32 * HG_WJ));
constexpr int HG_ASEG = HG_BN * HG_BK / 8 / HG_THREADS;   // 16-byte A segments per thread and step
constexpr int HG_BSEG = HG_BT * HG_BK / 8 / HG_THREADS;   // 16-byte B segments per thread and step
constexpr int HG_SUBS = HG_BK / 32;                        // Q4_K sub-blocks per row and step
// Q4_K tasks: whole sub-blocks (4 quant dwords) when there are no more of
// them than threads, else halves; HG_QTPT tasks per thread and step
constexpr int HG_QD = HG_BN * HG_SUBS >= HG_THREADS ? 4 : 2;
constexpr int HG_QPS = 4 / HG_QD;                          // tasks per sub-block
constexpr int HG_QTPT = HG_BN * HG_SUBS * HG_QPS / HG_THREADS;
static_assert(HG_QTPT >= 1 && HG_QTPT * HG_THREADS == HG_BN * HG_SUBS * HG_QPS, "Q4_K tasks must divide evenly");

struct HgStage {
    _Float16 a[HG_BN * HG_LD];
    _Float16 b[HG_BT * HG_LD];
};

// A Q4_K sub-block of a row, or half of one (HG_QD quant dwords).
struct Q4Sub {
    uint32_t hdr;      // d | dmin << 16
    uint32_t sw, mw;   // the dwords holding this sub-block's scale and min bytes
    uint32_t q[HG_QD]; // its quant dwords
};

__device__ __forceinline__ void q4sub_load(const uint8_t *sb, int j, int piece, Q4Sub &r) {
    r.hdr = *reinterpret_cast<const uint32_t *>(sb);
    // j < 4: scale byte 4 + j, min byte 8 + j; j >= 4: scale byte 8 + j,
    // min byte 12 + j (the block's first quant dword)
    r.sw = *reinterpret_cast<const uint32_t *>(sb + (j < 4 ? 4 : 12));
    r.mw = *reinterpret_cast<const uint32_t *>(sb + (j < 4 ? 8 : 16));
    const uint8_t *q = sb + 16 + 16 * j + 4 * HG_QD * piece;
    if constexpr (HG_QD == 4) {
        const hg_u32x4 v = *reinterpret_cast<const hg_u32x4 *>(q);
        r.q[0] = v.x; r.q[1] = v.y; r.q[2] = v.z; r.q[3] = v.w;
    } else {
        const uint2 v = *reinterpret_cast<const uint2 *>(q);
        r.q[0] = v.x; r.q[1] = v.y;
    }
}

#ifndef TBQ_HG_EXACT
#define TBQ_HG_EXACT 0
#endif
typedef _Float16 hg_f16x2 __attribute__((ext_vector_type(2)));

// The piece's fp16 weights in element order (weights 2i, 2i+1 are the low
// and high nibbles of quant byte i).  A nibble q becomes the fp16 number
// 1 + q/16 by placing it in the mantissa (0x3C00 | q << 6, both nibbles of
// a byte from one 24-bit multiply and one v_bitop3 (a & b) | c), and one
// packed fp16 fma with (16 S, C = -16 S - M) gives 16 S (1 + q/16) + C =
// S q - M (exact before its one rounding): 1.5 VALU per weight, with the
// fp16 roundings of 16 S, C and the result (16 d 63 + dmin 63 must stay
// below 65504).  TBQ_HG_EXACT instead rounds fl(fl(S q) - M) once
// from fp32, as k_dequant_f16_q4k does.
__device__ __forceinline__ void q4sub_f16(const Q4Sub &r, int j, hg_f16x8 (&o)[HG_QD]) {
    const int jb = 8 * (j & 3);
    const float S = f16_ref(r.hdr & 0xFFFFu) * (float)((r.sw >> jb) & 63);
    const float Mn = f16_ref(r.hdr >> 16) * (float)((r.mw >> jb) & 63);
    if constexpr (TBQ_HG_EXACT) {
#pragma unroll
        for (int c = 0; c < HG_QD; c++) {
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int qq = (int)((r.q[c] >> (8 * (i >> 1) + 4 * (i & 1))) & 15);
                const float tt = S * (float)qq;
                o[c][i] = (_Float16)(tt - Mn);
            }
        }
    } else {
        const _Float16 s16 = (_Float16)(16.f * S), cc = (_Float16)(-(float)s16 - Mn);
        const hg_f16x2 S16 = {s16, s16}, C = {cc, cc};
#pragma unroll
        for (int c = 0; c < HG_QD; c++) {
            unsigned w[4];
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const unsigned y = (r.q[c] >> (8 * b)) & 0xFFu;
                const unsigned t = __builtin_amdgcn_bitop3_b32(__umul24(y, 0x40040u), 0x03C003C0u, 0x3C003C00u, 0xEA);   // (a & b) | c
                w[b] = __builtin_bit_cast(unsigned, __builtin_elementwise_fma(__builtin_bit_cast(hg_f16x2, t), S16, C));
            }
            o[c] = __builtin_bit_cast(hg_f16x8, hg_u32x4{w[0], w[1], w[2], w[3]});
        }
    }
}

}  // namespace

// AF: 0 = W fp16 rows, 1 = W Q4_K rows (reference layout).  kper = K columns
// per slice (a multiple of HG_BK); out = C with row stride ldo (gridDim.z ==
// 1) or the slice partials P[z][T][N] (ldo = N).
// GLU (one slice only): W holds N = 2F rows, gate rows then up rows, and
// out[t][c] = silu(g xs[t]) (u xs[t]) with g, u = rows c and F + c of the
// product (xs: the row scales of X).  The A tile's 32-row blocks alternate
// gate and up rows of the same 32 outputs (tile n-block b holds outputs
// 64 b .. 64 b + 63), so a lane's accumulators of blocks 0 and 1 hold the
// gate and up of the same (output, token).
template <int AF, bool GLU = false>
__global__ __launch_bounds__(HG_THREADS) __attribute__((amdgpu_waves_per_eu(TBQ_HG_WPE))) void k_hgemm(const void *__restrict__ Wv, const _Float16 *__restrict__ X,
                                                         int T, int N, int K, int kper, float *__restrict__ out,
                                                         int ldo, const float *__restrict__ xs = nullptr) {
    static_assert(!GLU || HG_WI == 2, "GLU pairs the wave's two 32-row blocks");
    extern __shared__ __attribute__((aligned(16))) unsigned char hg_lds[];   // two HgStage (72 KiB)
    HgStage *st = reinterpret_cast<HgStage *>(hg_lds);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, li = lane & 31, lh = lane >> 5;
    const int n0 = blockIdx.x * HG_BN, t0 = blockIdx.y * HG_BT;
    const int kb = blockIdx.z * kper, ke = min(K, kb + kper), nsteps = (ke - kb) / HG_BK;
    const int wn = (wave % HG_WN) * 32 * HG_WI, wt = (wave / HG_WN) * 32 * HG_WJ;

    // fp16 loaders: segment i of this thread = row tid / SPR + RSTEP i, 8
    // halves at 8 (tid % SPR)
    constexpr int SPR = HG_BK / 8, RSTEP = HG_THREADS / SPR;
    const int lrow = tid / SPR, lcol = 8 * (tid % SPR);
    const int xbytes = T * K * 2;
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc((void *)X, (short)0, xbytes, 0x00020000);
    int xoff[HG_BSEG];
#pragma unroll
    for (int i = 0; i < HG_BSEG; i++) {
        const int t = t0 + lrow + RSTEP * i;   // rows past T load zeros (offset beyond the buffer)
        xoff[i] = t < T ? (t * K + kb + lcol) * 2 : xbytes;
    }
    // A loader (AF 0: fp16 segments as the B loader; AF 1: row, sub-block of
    // the step's pair, piece)
    const _Float16 *Wh = reinterpret_cast<const _Float16 *>(Wv);
    const uint8_t *Wq = reinterpret_cast<const uint8_t *>(Wv);
    const long long rbq = (long long)(K / 256) * 144;
    // weight row of tile row rho (rows past N clamp to the last)
    auto wrow = [&](int rho) {
        if constexpr (GLU) {
            const int F = N / 2, b = rho >> 5;
            return min((b & 1 ? F : 0) + (n0 >> 1) + 32 * (b >> 1) + (rho & 31), N - 1);
        } else {
            return min(n0 + rho, N - 1);
        }
    };
    // Q4_K task tk = tid + HG_THREADS i: row tk / (QPS SUBS), sub-block
    // (tk / QPS) % SUBS of the step, piece tk % QPS
    auto qtask = [&](int i, int &row, int &sub, int &pc) {
        const int tk = tid + HG_THREADS * i;
        row = tk / (HG_QPS * HG_SUBS);
        sub = (tk / HG_QPS) % HG_SUBS;
        pc = tk % HG_QPS;
    };

    // One step's operands in registers, between their global loads and
    // their LDS stores.  Two sets: the loads of step s + 2 are in flight
    // while step s + 1's are stored.
    struct Regs {
        hg_u32x4 xr[HG_BSEG];
        hg_u32x4 wr[HG_ASEG];
        Q4Sub wq[HG_QTPT];
    };
    auto load = [&](Regs &r, int s) {
        const int k = kb + s * HG_BK;
#pragma unroll
        for (int i = 0; i < HG_BSEG; i++)
            r.xr[i] = __builtin_bit_cast(hg_u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                       xrs, xoff[i] < xbytes ? xoff[i] + s * HG_BK * 2 : xbytes, 0, 0));
        if constexpr (AF == 0) {
#pragma unroll
            for (int i = 0; i < HG_ASEG; i++)
                r.wr[i] = *reinterpret_cast<const hg_u32x4 *>(Wh + (long long)wrow(lrow + RSTEP * i) * K + k + lcol);
        } else {
#pragma unroll
            for (int i = 0; i < HG_QTPT; i++) {
                int row, sub, pc;
                qtask(i, row, sub, pc);
                q4sub_load(Wq + (long long)wrow(row) * rbq + (long long)(k >> 8) * 144,
                           ((k & 255) >> 5) + sub, pc, r.wq[i]);
            }
        }
    };
    auto store = [&](const Regs &r, int buf, int s) {
#pragma unroll
        for (int i = 0; i < HG_BSEG; i++)
            *reinterpret_cast<hg_u32x4 *>(&st[buf].b[(lrow + RSTEP * i) * HG_LD + lcol]) = r.xr[i];
        if constexpr (AF == 0) {
#pragma unroll
            for (int i = 0; i < HG_ASEG; i++)
                *reinterpret_cast<hg_u32x4 *>(&st[buf].a[(lrow + RSTEP * i) * HG_LD + lcol]) = r.wr[i];
        } else {
#pragma unroll
            for (int i = 0; i < HG_QTPT; i++) {
                int row, sub, pc;
                qtask(i, row, sub, pc);
                hg_f16x8 o[HG_QD];
                q4sub_f16(r.wq[i], (((kb + s * HG_BK) & 255) >> 5) + sub, o);
#pragma unroll
                for (int c = 0; c < HG_QD; c++)
                    *reinterpret_cast<hg_f16x8 *>(&st[buf].a[row * HG_LD + 32 * sub + 8 * (HG_QD * pc + c)]) = o[c];
            }
        }
    };

    hg_f32x16 acc[HG_WI][HG_WJ];
#pragma unroll
    for (int i = 0; i < HG_WI; i++)
#pragma unroll
        for (int jx = 0; jx < HG_WJ; jx++) acc[i][jx] = hg_f32x16{};
#ifndef TBQ_HG_ALLREAD
#define TBQ_HG_ALLREAD 0
#endif
    auto compute = [&](int buf) {
        const _Float16 *A = st[buf].a + (wn + li) * HG_LD + 8 * lh;
        const _Float16 *B = st[buf].b + (wt + li) * HG_LD + 8 * lh;
        if constexpr (TBQ_HG_ALLREAD) {
            // every operand of the step read first, then the 16 MFMAs back to back
            hg_f16x8 a[HG_BK / 16][HG_WI], b[HG_BK / 16][HG_WJ];
#pragma unroll
            for (int kk = 0; kk < HG_BK / 16; kk++) {
#pragma unroll
                for (int i = 0; i < HG_WI; i++) a[kk][i] = *reinterpret_cast<const hg_f16x8 *>(A + 32 * i * HG_LD + 16 * kk);
#pragma unroll
                for (int i = 0; i < HG_WJ; i++) b[kk][i] = *reinterpret_cast<const hg_f16x8 *>(B + 32 * i * HG_LD + 16 * kk);
            }
#pragma unroll
            for (int kk = 0; kk < HG_BK / 16; kk++)
#pragma unroll
                for (int i = 0; i < HG_WI; i++)
#pragma unroll
                    for (int jx = 0; jx < HG_WJ; jx++)
                        acc[i][jx] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[kk][i], b[kk][jx], acc[i][jx], 0, 0, 0);
            return;
        }
#pragma unroll
        for (int kk = 0; kk < HG_BK / 16; kk++) {
            hg_f16x8 a[HG_WI], b[HG_WJ];
#pragma unroll
            for (int i = 0; i < HG_WI; i++) a[i] = *reinterpret_cast<const hg_f16x8 *>(A + 32 * i * HG_LD + 16 * kk);
#pragma unroll
            for (int i = 0; i < HG_WJ; i++) b[i] = *reinterpret_cast<const hg_f16x8 *>(B + 32 * i * HG_LD + 16 * kk);
#pragma unroll
            for (int i = 0; i < HG_WI; i++)
#pragma unroll
                for (int jx = 0; jx < HG_WJ; jx++)
                    acc[i][jx] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[jx], acc[i][jx], 0, 0, 0);
        }
    };
    // Loads are unconditional (steps past the end reload the last one, whose
    // stores land in a stage no later step reads), so every path through a
    // step issues the same loads and the compiler's wait counts stay exact.
    const int last = nsteps - 1;
    // sched_barrier(0) pins the order: each step's global loads go out
    // before its MFMAs (the scheduler would otherwise sink them next to
    // their LDS stores and expose their whole latency).
#ifndef TBQ_HG_DEPTH
#define TBQ_HG_DEPTH 2
#endif
    if constexpr (TBQ_HG_DEPTH == 1) {
        Regs r;
        load(r, 0);
        store(r, 0, 0);
        __syncthreads();
        for (int s = 0; s < nsteps; s++) {
            load(r, min(s + 1, last));
            __builtin_amdgcn_sched_barrier(0);
            compute(s & 1);
            __builtin_amdgcn_sched_barrier(0);
            store(r, (s + 1) & 1, min(s + 1, last));   // the other stage was last read in step s - 1
            __syncthreads();
        }
    } else {
        // two register sets: step s + 2's loads are issued at the start of
        // step s, step s + 1's (issued a step earlier) are stored at its end
        Regs r0, r1;
        load(r0, 0);
        load(r1, min(1, last));
        store(r0, 0, 0);
        __syncthreads();
        for (int s = 0; s < nsteps; s += 2) {
            load(r0, min(s + 2, last));
            __builtin_amdgcn_sched_barrier(0);
            compute(0);
            __builtin_amdgcn_sched_barrier(0);
            store(r1, 1, min(s + 1, last));   // stage 1 was last read in step s - 1
            __syncthreads();
            if (s + 1 >= nsteps) break;       // uniform
            load(r1, min(s + 3, last));
            __builtin_amdgcn_sched_barrier(0);
            compute(1);
            __builtin_amdgcn_sched_barrier(0);
            store(r0, 0, min(s + 2, last));
            __syncthreads();
        }
    }
    // accumulator register r of lane l: weight row 8(r/4) + 4(l/32) + r%4 of
    // the 32-row block, token l % 32 of the 32-token block
    if constexpr (GLU) {
        // outputs 64 blockIdx.x + wn / 2 + 8g + 4(l/32) + r%4 of register r
#pragma unroll
        for (int jx = 0; jx < HG_WJ; jx++) {
            const int t = t0 + wt + 32 * jx + li;
            if (t >= T) continue;
            const float sx = xs[t];
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int c = (n0 >> 1) + (wn >> 1) + 8 * g + 4 * lh;
                if (c >= N / 2) continue;
                float a[4];
#pragma unroll
                for (int r = 0; r < 4; r++) a[r] = pro_swiglu(acc[0][jx][4 * g + r] * sx, acc[1][jx][4 * g + r] * sx);
                *reinterpret_cast<float4 *>(out + (long long)t * ldo + c) = make_float4(a[0], a[1], a[2], a[3]);
            }
        }
        return;
    }
    float *o = out + (long long)blockIdx.z * T * N;   // z > 0 only for partials (ldo = N)
#pragma unroll
    for (int jx = 0; jx < HG_WJ; jx++) {
        const int t = t0 + wt + 32 * jx + li;
        if (t >= T) continue;
#pragma unroll
        for (int i = 0; i < HG_WI; i++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int n = n0 + wn + 32 * i + 8 * g + 4 * lh;
                if (n >= N) continue;   // rows past N (clamped loads) are not stored
                *reinterpret_cast<float4 *>(o + (long long)t * ldo + n) =
                    make_float4(acc[i][jx][4 * g], acc[i][jx][4 * g + 1], acc[i][jx][4 * g + 2], acc[i][jx][4 * g + 3]);
            }
    }
}

// C[t][n] (row stride ldc) = sum over the S slices of P[z][t][n], in slice order.
__global__ __launch_bounds__(256) void k_gemm_reduce(const float *__restrict__ P, int S, int T, int N,
                                                     float *__restrict__ C, int ldc) {
    const long long n4 = (long long)T * N / 4;
    const int N4 = N / 4;
    for (long long i = blockIdx.x * 256ll + threadIdx.x; i < n4; i += (long long)gridDim.x * 256) {
        float4 a = reinterpret_cast<const float4 *>(P)[i];
        for (int z = 1; z < S; z++) {
            const float4 b = reinterpret_cast<const float4 *>(P)[z * n4 + i];
            a.x = a.x + b.x;
            a.y = a.y + b.y;
            a.z = a.z + b.z;
            a.w = a.w + b.w;
        }
        const long long t = i / N4, c = i - t * N4;
        *reinterpret_cast<float4 *>(C + t * ldc + 4 * c) = a;
    }
}

// CUs the slicing plans for (the device's, at most 256, so that workspace
// sizes computed before and after initialisation agree on this part).
int hgemm_cus() {
    const int c = tbq_cu_count();
    return c > 0 && c < 256 ? c : 256;
}

// K slices for a T x N product: enough workgroups for one per CU (two per
// CU measured slower: the extra partial sums cost more in k_gemm_reduce
// than the occupancy gains), each slice at least 8 steps.
int hgemm_slices(int T, int N, int K, int n_cu) {
    const int tiles = ((N + HG_BN - 1) / HG_BN) * ((T + HG_BT - 1) / HG_BT);
#ifndef TBQ_HG_SPLIT_WG
#define TBQ_HG_SPLIT_WG 1
#endif
    int s = (TBQ_HG_SPLIT_WG * n_cu + tiles - 1) / tiles;
    s = std::min(s, std::max(1, K / (8 * HG_BK)));
    return std::max(1, std::min(s, 8));
}

size_t hgemm_partial_bytes(int T, int N, int K, int n_cu) {
    const int s = hgemm_slices(T, N, K, n_cu);
    return s > 1 ? (size_t)s * T * N * 4 : 0;
}

bool hgemm_supported(int wqt, int N, int K) {
    return (wqt == QT_F16 || wqt == QT_Q4_K) && N > 0 && N % 4 == 0 && K > 0 && K % 256 == 0;
}

// The gate/up product with SwiGLU in the epilogue (k_hgemm GLU mode): W
// holds 2F rows (gate then up), A[T][F] (row stride lda) = silu(g xs) (u
// xs).  hipErrorNotSupported where the product would be split over K (the
// SwiGLU of partial sums is not defined) or F is not a multiple of 64.
hipError_t launch_hgemm_glu(int wqt, const void *W, const _Float16 *X, const float *xs, int T, int F, int K,
                            float *A, int lda, int n_cu, hipStream_t st) {
    const int N = 2 * F;
    if (!hgemm_supported(wqt, N, K) || F % 64 || T <= 0 || (long long)T * K * 2 >= (1ll << 31) ||
        hgemm_slices(T, N, K, n_cu) != 1)
        return hipErrorNotSupported;
    dim3 grid(N / HG_BN, (T + HG_BT - 1) / HG_BT, 1);
    constexpr size_t lds = 2 * sizeof(HgStage);
    static const hipError_t a0 =
        hipFuncSetAttribute((const void *)k_hgemm<0, true>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    static const hipError_t a1 =
        hipFuncSetAttribute((const void *)k_hgemm<1, true>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (a0 != hipSuccess) return a0;
    if (a1 != hipSuccess) return a1;
    if (wqt == QT_F16)
        hipLaunchKernelGGL((k_hgemm<0, true>), grid, dim3(HG_THREADS), lds, st, W, X, T, N, K, K, A, lda, xs);
    else
        hipLaunchKernelGGL((k_hgemm<1, true>), grid, dim3(HG_THREADS), lds, st, W, X, T, N, K, K, A, lda, xs);
    return hipGetLastError();
}

// wqt: QT_F16 (IEEE fp16 rows, as k_dequant_f16 writes them) or QT_Q4_K.
// C: T rows of N floats at row stride ldc.  part: hgemm_partial_bytes() of
// device memory (unused with one slice).
hipError_t launch_hgemm(int wqt, const void *W, const _Float16 *X, int T, int N, int K, float *C, int ldc,
                        float *part, int n_cu, hipStream_t st, int *nslices) {
    if (!hgemm_supported(wqt, N, K) || T <= 0 || (long long)T * K * 2 >= (1ll << 31)) return hipErrorNotSupported;
    const int S = hgemm_slices(T, N, K, n_cu);
    const int steps = K / HG_BK, per = (steps + S - 1) / S;
    const int Sx = (steps + per - 1) / per;   // slices actually used
    dim3 grid((N + HG_BN - 1) / HG_BN, (T + HG_BT - 1) / HG_BT, Sx);
    float *out = Sx > 1 ? part : C;
    if (Sx > 1 && !part) return hipErrorInvalidValue;
    if (nslices && Sx > 1 && ldc != N) return hipErrorInvalidValue;   // slices are packed at row stride N
    // more than 64 KiB of dynamic LDS is opted into once per kernel
    constexpr size_t lds = 2 * sizeof(HgStage);
    static const hipError_t a0 =
        hipFuncSetAttribute((const void *)k_hgemm<0>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    static const hipError_t a1 =
        hipFuncSetAttribute((const void *)k_hgemm<1>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (a0 != hipSuccess) return a0;
    if (a1 != hipSuccess) return a1;
    if (wqt == QT_F16)
        hipLaunchKernelGGL(k_hgemm<0>, grid, dim3(HG_THREADS), lds, st, W, X, T, N, K, per * HG_BK, out,
                           Sx > 1 ? N : ldc);
    else
        hipLaunchKernelGGL(k_hgemm<1>, grid, dim3(HG_THREADS), lds, st, W, X, T, N, K, per * HG_BK, out,
                           Sx > 1 ? N : ldc);
    hipError_t err = hipGetLastError();
    if (nslices) *nslices = Sx;
    if (err != hipSuccess || Sx == 1 || nslices) return err;
    const long long n4 = (long long)T * N / 4;
    const int g = (int)std::min<long long>((n4 + 255) / 256, 4096);
    hipLaunchKernelGGL(k_gemm_reduce, dim3(g), dim3(256), 0, st, part, Sx, T, N, C, ldc);
    return hipGetLastError();
}

}  // namespace tbq
