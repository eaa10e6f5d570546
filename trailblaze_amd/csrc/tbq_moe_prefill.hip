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
//                     128-pair x 64-column tile (128 weight rows: 64 gate and
//                     64 up rows), K = H, fp32 out.
//   k_moe_f16<1,NS>   y[p] = act[p] . W_down[e] for 128 pairs x 128 rows, K = F.
//   (k_combine)       out = resid + sum over slots in slot order (tbq_moe.hip).
//
// Dequantisation to fp16.  A nibble q becomes the fp16 number 1 + q/16 by
// placing q in the mantissa (0x3C00 | q << 6), for two weights per dword:
// one 24-bit multiply spreads a quant byte's two nibbles into the two
// halves, one AND-OR masks them and sets the exponent; v_pk_add_f16 with
// -1 (exact) gives q/16, and v_pk_fma_f16 with (16 S, -M) gives S q - M with
// only the fp16 roundings of 16 S, M and the result.  About 2 VALU
// operations per weight, where byte->fp32 conversion + fma + bf16 packing
// takes 4.5.
//
// Per 128-column chunk of K each thread dequantises two Q4_K sub-blocks into
// LDS (each weight once per tile) and copies its share of the tile's fp16
// activation rows; v_mfma_f32_32x32x16_f16 accumulates in fp32, each wave
// owning 32 weight rows x up to four 32-pair sub-tiles (sub-tiles past the
// tile's pairs are skipped).  Global loads run one chunk ahead.
//
// Accuracy: fp16 weights and activations (11-bit mantissa), fp32
// accumulation; outputs land within 1e-2 relative L2 of the fp32 reference.
// The weights' fp16 form needs 16 * d * 63 below 65504 (d < 64).
#include "tbq_kernels.h"
#include "tbq_kquant.hpp"

namespace tbq {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
// native vectors: HIP's uint4 struct is copied with memcpy, which keeps
// register arrays in scratch memory
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int PF_MT = 128;         // pairs per tile (four 32-pair MFMA sub-tiles)
constexpr int PF_KC = 128;         // K columns staged per chunk (half a Q4_K super-block)
constexpr int PF_LD = PF_KC + 8;   // LDS row stride in halves (padding breaks bank aliasing)
constexpr int PF_THREADS = 256;
constexpr int PF_ROWS = 128;       // weight rows per workgroup
constexpr size_t PF_LDS_BYTES = (size_t)(PF_ROWS + PF_MT) * PF_LD * 2;   // W and X tiles, single-buffered

struct PfTile {
    int e, start, n;
};

// ---------------------------------------------------------------------------
// Dispatch: one workgroup of 1024 threads.  pairs p = t*k + s.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void k_dispatch(const int *__restrict__ sel_idx, int T, int k, int E,
                                                   int *__restrict__ perm, PfTile *__restrict__ tiles,
                                                   int *__restrict__ ntiles) {
    __shared__ int hist[256], off[257], toff[257], cur[256];
    const int tid = threadIdx.x, P = T * k;
    for (int e = tid; e < 256; e += 1024) { hist[e] = 0; cur[e] = 0; }
    __syncthreads();
    for (int p = tid; p < P; p += 1024) atomicAdd(&hist[sel_idx[(p / k) * 8 + p % k]], 1);
    __syncthreads();
    if (tid == 0) {
        int o = 0, to = 0;
        for (int e = 0; e < E; e++) {
            off[e] = o;
            toff[e] = to;
            o += hist[e];
            to += (hist[e] + PF_MT - 1) / PF_MT;
        }
        off[E] = o;
        toff[E] = to;
        *ntiles = to;
    }
    __syncthreads();
    for (int p = tid; p < P; p += 1024) {
        const int e = sel_idx[(p / k) * 8 + p % k];
        perm[off[e] + atomicAdd(&cur[e], 1)] = p;
    }
    for (int e = tid; e < E; e += 1024) {
        const int n = hist[e];
        for (int i = 0; i * PF_MT < n; i++) {
            PfTile tl;
            tl.e = e;
            tl.start = off[e] + i * PF_MT;
            tl.n = n - i * PF_MT < PF_MT ? n - i * PF_MT : PF_MT;
            tiles[toff[e] + i] = tl;
        }
    }
}

// ---------------------------------------------------------------------------
// Rows of n floats to fp16: one workgroup per row; s = 2^(15 - e) with
// max |row| = f * 2^e (f in [0.5, 1)), so |row| * s < 2^15; inv[row] = 1/s.
// n a multiple of 4.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_rows_f16(const float *__restrict__ in, int n, _Float16 *__restrict__ out,
                                                  float *__restrict__ inv) {
    __shared__ float part[4];
    const int row = blockIdx.x, tid = threadIdx.x;
    const float4 *r = reinterpret_cast<const float4 *>(in + (long long)row * n);
    float mx = 0.f;
    for (int i = tid; i < n / 4; i += 256) {
        const float4 v = r[i];
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
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
    for (int i = tid; i < n / 4; i += 256) {
        const float4 v = r[i];
        const f16x2 a = {(_Float16)(v.x * s), (_Float16)(v.y * s)};
        const f16x2 b = {(_Float16)(v.z * s), (_Float16)(v.w * s)};
        o[i] = make_uint2(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b));
    }
    if (tid == 0) inv[row] = ldexpf(1.f, -sh);
}

// ---------------------------------------------------------------------------
// Staging helpers.
// ---------------------------------------------------------------------------
// Raw bytes of one 32-weight Q4_K sub-block j of a super-block: scale/min
// inputs and the 16 quant bytes.
struct Q4Sub {
    u32x4 hdr, q;
    unsigned mind;
};

__device__ __forceinline__ void q4sub_load(const uint8_t *sb, int j, Q4Sub &r) {
    r.hdr = *reinterpret_cast<const u32x4 *>(sb);
    r.q = *reinterpret_cast<const u32x4 *>(sb + 16 + 16 * j);
    r.mind = *reinterpret_cast<const unsigned *>(sb + 16);
}

// Dequantise (reference scale/min selection, layer4/tb_gguf.c:163-168) and
// write 32 fp16 weights to dst (16-byte aligned).
__device__ __forceinline__ void q4sub_store_f16(const Q4Sub &r, int j, _Float16 *dst) {
    const float d = f16_ref(r.hdr.x & 0xFFFFu), dmin = f16_ref(r.hdr.x >> 16);
    const unsigned sw = j < 4 ? r.hdr.y : r.hdr.w;
    const unsigned mw = j < 4 ? r.hdr.z : r.mind;
    const int sh = 8 * (j & 3);
    const float S = d * (float)((sw >> sh) & 63), Mn = dmin * (float)((mw >> sh) & 63);
    const _Float16 s16 = (_Float16)(16.f * S), nm = (_Float16)(-Mn);
    const f16x2 S16 = {s16, s16}, NM = {nm, nm}, ONE = {(_Float16)1.f, (_Float16)1.f};
    const unsigned qv[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
    unsigned o[16];
#pragma unroll
    for (int i = 0; i < 4; i++) {
#pragma unroll
        for (int b = 0; b < 4; b++) {
            // quant byte (hi << 4 | lo) -> halves (1 + lo/16, 1 + hi/16)
            const unsigned y = (qv[i] >> (8 * b)) & 0xFFu;
            const unsigned t = (__umul24(y, 0x40040u) & 0x03C003C0u) | 0x3C003C00u;
            const f16x2 v = __builtin_bit_cast(f16x2, t) - ONE;
            o[4 * i + b] = __builtin_bit_cast(unsigned, __builtin_elementwise_fma(v, S16, NM));
        }
    }
    u32x4 *d4 = reinterpret_cast<u32x4 *>(dst);
#pragma unroll
    for (int i = 0; i < 4; i++) d4[i] = u32x4{o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]};
}

// ---------------------------------------------------------------------------
// Expert tile GEMM.  grid = (max tiles, F/64) for MODE 0, (max tiles, H/128)
// for MODE 1; K = NS * 128.
//   MODE 0: local weight row r = 32w + j is gate row 16w + j (j < 16) or up
//   row 16w + j - 16 of the workgroup's 64 columns, so a lane's accumulator
//   registers i and i + 8 hold gate and up of the same (column, pair) and
//   SwiGLU needs no data exchange; X rows are tokens (pair / k) of x.
//   MODE 1: local row r is down row 128*blockIdx.y + r; X rows are pairs of
//   act.  xinv[X row] undoes the row's fp16 scaling.
// Thread staging per chunk: W items tid + 256i (i < 2) = (row it/4, sub-block
// it%4 of the chunk); X segments tid + 256i (i < 8) = (pair it/16, 8 halves
// at 8*(it%16)).
// ---------------------------------------------------------------------------
template <int MODE, int NS>
__global__ __launch_bounds__(PF_THREADS, 2) void k_moe_f16(const uint8_t *__restrict__ W0, const uint8_t *__restrict__ W1,
                                                           const _Float16 *__restrict__ X, int x_rows,
                                                           const float *__restrict__ xinv, const int *__restrict__ perm,
                                                           const PfTile *__restrict__ tiles, const int *__restrict__ ntiles,
                                                           int H, int F, int k, float *__restrict__ out) {
    constexpr int K = NS * PF_KC;
    constexpr int XPT = PF_MT * PF_KC / 8 / PF_THREADS;   // 16-byte X segments per thread per chunk
    extern __shared__ __attribute__((aligned(16))) _Float16 pf_lds[];
    _Float16 *Ws = pf_lds;                     // [PF_ROWS][PF_LD]
    _Float16 *Xs = pf_lds + PF_ROWS * PF_LD;   // [PF_MT][PF_LD]
    if ((int)blockIdx.x >= *ntiles) return;
    const PfTile tl = tiles[blockIdx.x];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const long long rb = (long long)(K / 256) * 144;

    const uint8_t *wrow[2];
    int wr_local[2], wj[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int it = tid + PF_THREADS * i, r = it >> 2;
        wr_local[i] = r;
        wj[i] = it & 3;
        if (MODE == 0) {
            const int jj = r & 31, col = blockIdx.y * 64 + 16 * (r >> 5) + (jj & 15);
            wrow[i] = (jj < 16 ? W0 : W1) + ((long long)tl.e * F + col) * rb;
        } else {
            wrow[i] = W0 + ((long long)tl.e * H + blockIdx.y * PF_ROWS + r) * rb;
        }
    }
    // X rows through a range-checked buffer descriptor: rows past the tile's
    // pair count get an offset beyond the buffer, which loads zeros without a
    // memory access, so every load is unconditional (static wait counts)
    const int xbytes = x_rows * K * 2;
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc((void *)X, (short)0, xbytes, 0x00020000);
    int xoff[XPT];
#pragma unroll
    for (int i = 0; i < XPT; i++) {
        const int it = tid + PF_THREADS * i, pr = it >> 4;
        if (pr < tl.n) {
            const int p = perm[tl.start + pr];
            xoff[i] = ((MODE == 0 ? p / k : p) * K + 8 * (it & 15)) * 2;
        } else {
            xoff[i] = xbytes;
        }
    }

    struct Slot {
        Q4Sub w[2];
        u32x4 x[XPT];
    };
    auto load = [&](Slot &sl, int s) {
        const int kc = s * PF_KC;
#pragma unroll
        for (int i = 0; i < 2; i++) q4sub_load(wrow[i] + (long long)(kc / 256) * 144, 4 * (s & 1) + wj[i], sl.w[i]);
#pragma unroll
        for (int i = 0; i < XPT; i++)
            sl.x[i] = __builtin_amdgcn_raw_buffer_load_b128(xrs, xoff[i] < xbytes ? xoff[i] + kc * 2 : xbytes, 0, 0);
    };
    auto store = [&](const Slot &sl, int s) {
#pragma unroll
        for (int i = 0; i < 2; i++) q4sub_store_f16(sl.w[i], 4 * (s & 1) + wj[i], Ws + wr_local[i] * PF_LD + 32 * wj[i]);
#pragma unroll
        for (int i = 0; i < XPT; i++) {
            const int it = tid + PF_THREADS * i;
            *reinterpret_cast<u32x4 *>(Xs + (it >> 4) * PF_LD + 8 * (it & 15)) = sl.x[i];
        }
    };

    const int nsub = (tl.n + 31) / 32;   // 1..4, uniform over the workgroup
    f32x16 acc[4] = {f32x16{}, f32x16{}, f32x16{}, f32x16{}};
    Slot sa, sb;
    load(sa, 0);
    const _Float16 *wb = Ws + (32 * wave + (lane & 31)) * PF_LD + 8 * (lane >> 5);
    const _Float16 *xb = Xs + (lane & 31) * PF_LD + 8 * (lane >> 5);
    // one chunk: prefetch the next into `nxt`, stage `cur`, multiply; the
    // slots are named, not indexed, so the chunk loop need not be unrolled
    // to keep them in registers (NS is even)
    auto chunk = [&](int s, const Slot &cur, Slot &nxt) {
        if (s + 1 < NS) load(nxt, s + 1);
        if (s > 0) __syncthreads();   // the previous chunk's MFMA reads are done
        store(cur, s);
        __syncthreads();
#pragma unroll
        for (int ks = 0; ks < PF_KC; ks += 16) {
            const f16x8 av = *reinterpret_cast<const f16x8 *>(wb + ks);
#pragma unroll
            for (int t = 0; t < 4; t++) {
                if (t < nsub) {
                    const f16x8 bv = *reinterpret_cast<const f16x8 *>(xb + 32 * t * PF_LD + ks);
                    acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bv, acc[t], 0, 0, 0);
                }
            }
        }
    };
#pragma unroll 2
    for (int s = 0; s < NS; s += 2) {
        chunk(s, sa, sb);
        chunk(s + 1, sb, sa);
    }
    // accumulator register i of lane l: row 8(i/4) + 4(l/32) + i%4 of the
    // wave's 32, pair 32t + l%32 of the tile
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const int pr = 32 * t + (lane & 31);
        if (t < nsub && pr < tl.n) {
            const int p = perm[tl.start + pr];
            const float sc = xinv[MODE == 0 ? p / k : p];
            if (MODE == 0) {
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    float a[4];
#pragma unroll
                    for (int c = 0; c < 4; c++) {
                        const int i = 4 * h + c;
                        const float g = acc[t][i] * sc, u = acc[t][i + 8] * sc;
                        a[c] = g / (1.0f + expf_glibc(-g)) * u;
                    }
                    const int col = blockIdx.y * 64 + 16 * wave + 8 * h + 4 * (lane >> 5);
                    *reinterpret_cast<float4 *>(out + (long long)p * F + col) = make_float4(a[0], a[1], a[2], a[3]);
                }
            } else {
#pragma unroll
                for (int h = 0; h < 4; h++) {
                    const int row = blockIdx.y * PF_ROWS + 32 * wave + 8 * h + 4 * (lane >> 5);
                    *reinterpret_cast<float4 *>(out + (long long)p * H + row) =
                        make_float4(acc[t][4 * h] * sc, acc[t][4 * h + 1] * sc, acc[t][4 * h + 2] * sc,
                                    acc[t][4 * h + 3] * sc);
                }
            }
        }
    }
}

size_t prefill_workspace_bytes(int T, int k, int E, int H, int F) {
    const size_t P = (size_t)T * k;
    const size_t max_tiles = (P + PF_MT - 1) / PF_MT + E;
    auto up = [](size_t n) { return (n + 255) & ~(size_t)255; };
    return up(P * 4) + up(max_tiles * sizeof(PfTile)) + 256 + up(P * F * 2) + up((size_t)T * H * 2) + up(P * 4) +
           up((size_t)T * 4);
}

template <int MODE>
static hipError_t launch_moe_f16(int ns, dim3 grid, hipStream_t st, const uint8_t *W0, const uint8_t *W1,
                                 const _Float16 *X, int x_rows, const float *xinv, const int *perm, const PfTile *tiles,
                                 const int *ntiles, int H, int F, int k, float *out) {
    // more than 64 KiB of dynamic LDS is opted into once per kernel
#define TBQ_NS(N)                                                                                                   \
    case N: {                                                                                                       \
        static const hipError_t attr = hipFuncSetAttribute((const void *)k_moe_f16<MODE, N>,                        \
                                                           hipFuncAttributeMaxDynamicSharedMemorySize,              \
                                                           (int)PF_LDS_BYTES);                                      \
        if (attr != hipSuccess) return attr;                                                                        \
        hipLaunchKernelGGL((k_moe_f16<MODE, N>), grid, dim3(PF_THREADS), PF_LDS_BYTES, st, W0, W1, X, x_rows, xinv, \
                           perm, tiles, ntiles, H, F, k, out);                                                      \
        break;                                                                                                      \
    }
    switch (ns) {
        TBQ_NS(2) TBQ_NS(4) TBQ_NS(6) TBQ_NS(8) TBQ_NS(12) TBQ_NS(16) TBQ_NS(24) TBQ_NS(32)
    default:
        return hipErrorNotSupported;
    }
#undef TBQ_NS
    return hipGetLastError();
}

// Experts on MFMA for Q4_K weights; routing already in a.sel_idx/a.sel_w.
// Uses a.act (pairs x F fp32), a.y (pairs x H fp32) and `scratch`
// (prefill_workspace_bytes).  K = H (gate/up) and F (down) must be 256,
// 512, 768, 1024, 1536, 2048, 3072 or 4096.
hipError_t launch_moe_prefill_q4k(const MoeArgs &a, void *scratch, hipStream_t st) {
    auto ok_k = [](int K) {
        const int n = K / PF_KC;
        return K % 256 == 0 && (n == 2 || n == 4 || n == 6 || n == 8 || n == 12 || n == 16 || n == 24 || n == 32);
    };
    if (a.qtype != QT_Q4_K || !ok_k(a.H) || !ok_k(a.F) || a.F % 64 || a.H % PF_ROWS) return hipErrorNotSupported;
    const size_t P = (size_t)a.T * a.k;
    const int max_tiles = (int)((P + PF_MT - 1) / PF_MT + a.E);
    auto up = [](size_t n) { return (n + 255) & ~(size_t)255; };
    char *w = (char *)scratch;
    int *perm = (int *)w; w += up(P * 4);
    PfTile *tiles = (PfTile *)w; w += up((size_t)max_tiles * sizeof(PfTile));
    int *ntiles = (int *)w; w += 256;
    _Float16 *act16 = (_Float16 *)w; w += up(P * a.F * 2);
    _Float16 *x16 = (_Float16 *)w; w += up((size_t)a.T * a.H * 2);
    float *ainv = (float *)w; w += up(P * 4);
    float *xinv = (float *)w;
    hipLaunchKernelGGL(k_rows_f16, dim3(a.T), dim3(256), 0, st, a.xn, a.H, x16, xinv);
    hipLaunchKernelGGL(k_dispatch, dim3(1), dim3(1024), 0, st, a.sel_idx, a.T, a.k, a.E, perm, tiles, ntiles);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    err = launch_moe_f16<0>(a.H / PF_KC, dim3(max_tiles, a.F / 64), st, (const uint8_t *)a.gate, (const uint8_t *)a.up,
                            x16, a.T, xinv, perm, tiles, ntiles, a.H, a.F, a.k, a.act);
    if (err != hipSuccess) return err;
    hipLaunchKernelGGL(k_rows_f16, dim3((unsigned)P), dim3(256), 0, st, a.act, a.F, act16, ainv);
    err = hipGetLastError();
    if (err != hipSuccess) return err;
    return launch_moe_f16<1>(a.F / PF_KC, dim3(max_tiles, a.H / PF_ROWS), st, (const uint8_t *)a.down, nullptr, act16,
                             (int)P, ainv, perm, tiles, ntiles, a.H, a.F, a.k, a.y);
}

}  // namespace tbq
