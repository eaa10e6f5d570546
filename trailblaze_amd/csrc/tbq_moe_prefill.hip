// tbq_moe_prefill.hip -- batched (prefill) MoE experts on gfx950 bf16 MFMA.
//
// After routing (exact, as in decode), the (token, slot) pairs are grouped by
// expert and every expert's products run as dense tiles:
//
//   k_dispatch        per-expert histogram, prefix sum and permutation of the
//                     pairs in LDS (one workgroup), plus a tile list of
//                     (expert, first pair, pairs in tile) entries of <= 128
//                     pairs; order inside an expert does not affect results.
//   k_moe_mfma<0,NS>  act[p] = swiglu(x_t . W_gate[e], x_t . W_up[e]) for a
//                     128-pair x 64-column tile (128 weight rows: 64 gate and
//                     64 up rows), K = H.
//   k_moe_mfma<1,NS>  y[p] = act[p] . W_down[e] for 128 pairs x 128 rows, K = F.
//   (k_combine)       out = resid + sum over slots in slot order (tbq_moe.hip).
//
// Per 128-column chunk of K, each thread dequantises two Q4_K sub-blocks to
// bf16 in LDS (each weight once per tile) and copies its share of the tile's
// bf16 activation rows; v_mfma_f32_32x32x16_bf16 accumulates in fp32, each
// wave owning 32 weight rows x up to 4 32-pair sub-tiles (sub-tiles past the
// tile's pair count are skipped).  Global loads run two chunks ahead.
//
// Accuracy: weights and activations rounded to bf16 (8-bit mantissa), fp32
// accumulation; outputs land within 1e-2 relative L2 of the fp32 reference.
#include "tbq_kernels.h"
#include "tbq_kquant.hpp"

namespace tbq {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
// native vectors: HIP's uint4 struct is copied with memcpy, which keeps
// register arrays in scratch memory
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int PF_MT = 64;          // pairs per tile (two 32-pair MFMA sub-tiles)
constexpr int PF_KC = 128;         // K columns staged per chunk (half a Q4_K super-block)
constexpr int PF_LD = PF_KC + 8;   // LDS row stride in bf16 (padding breaks bank aliasing)
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
// Staging helpers.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    // round to nearest even, as v_cvt_pk_bf16_f32 does
    const __bf16 ha = (__bf16)a, hb = (__bf16)b;
    return (uint32_t)__builtin_bit_cast(uint16_t, ha) | ((uint32_t)__builtin_bit_cast(uint16_t, hb) << 16);
}

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
// write 32 bf16 weights to dst (16-byte aligned).  Per quant dword the low
// and high nibbles are masked once and converted byte-wise; the high
// nibbles keep their x16 position, folded into the scale (exact: power of 2).
__device__ __forceinline__ void q4sub_store_bf16(const Q4Sub &r, int j, __bf16 *dst) {
    const float d = f16_ref(r.hdr.x & 0xFFFFu), dmin = f16_ref(r.hdr.x >> 16);
    const unsigned sw = j < 4 ? r.hdr.y : r.hdr.w;
    const unsigned mw = j < 4 ? r.hdr.z : r.mind;
    const int sh = 8 * (j & 3);
    const float S = d * (float)((sw >> sh) & 63), Mn = dmin * (float)((mw >> sh) & 63);
    const float S16 = S * 0.0625f;
    const unsigned qv[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
    unsigned o[16];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const unsigned lo = qv[i] & 0x0F0F0F0Fu, hi = qv[i] & 0xF0F0F0F0u;
#pragma unroll
        for (int b = 0; b < 4; b++)
            o[4 * i + b] = pack_bf16x2(fmaf(S, (float)((lo >> (8 * b)) & 0xFF), -Mn),
                                       fmaf(S16, (float)((hi >> (8 * b)) & 0xFF), -Mn));
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
//   SwiGLU needs no data exchange; X rows are tokens (pair / k) of x in bf16.
//   MODE 1: local row r is down row 128*blockIdx.y + r; X rows are pairs of
//   act.
// Thread staging per chunk: W items tid + 256i (i < 2) = (row it/4, sub-block
// it%4 of the chunk); X segments tid + 256i (i < 8) = (pair it/16, 8 bf16 at
// 8*(it%16)).
// ---------------------------------------------------------------------------
template <int MODE, int NS>
__global__ __launch_bounds__(PF_THREADS, 2) void k_moe_mfma(const uint8_t *__restrict__ W0, const uint8_t *__restrict__ W1,
                                                            const __bf16 *__restrict__ X, int x_rows,
                                                            const int *__restrict__ perm, const PfTile *__restrict__ tiles,
                                                            const int *__restrict__ ntiles, int H, int F, int k,
                                                            __bf16 *__restrict__ act, float *__restrict__ y) {
    constexpr int K = NS * PF_KC;
    constexpr int XPT = PF_MT * PF_KC / 8 / PF_THREADS;   // 16-byte X segments per thread per chunk
    extern __shared__ __attribute__((aligned(16))) __bf16 pf_lds[];
    __bf16 *Ws = pf_lds;                     // [PF_ROWS][PF_LD]
    __bf16 *Xs = pf_lds + PF_ROWS * PF_LD;   // [PF_MT][PF_LD]
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
        for (int i = 0; i < 2; i++) q4sub_store_bf16(sl.w[i], 4 * (s & 1) + wj[i], Ws + wr_local[i] * PF_LD + 32 * wj[i]);
#pragma unroll
        for (int i = 0; i < XPT; i++) {
            const int it = tid + PF_THREADS * i;
            *reinterpret_cast<u32x4 *>(Xs + (it >> 4) * PF_LD + 8 * (it & 15)) = sl.x[i];
        }
    };

    f32x16 acc[2] = {f32x16{}, f32x16{}};
    Slot sl[3];
    load(sl[0], 0);
    if (NS > 1) load(sl[1], 1);
    const __bf16 *wb = Ws + (32 * wave + (lane & 31)) * PF_LD + 8 * (lane >> 5);
    const __bf16 *xb = Xs + (lane & 31) * PF_LD + 8 * (lane >> 5);
#pragma unroll
    for (int s = 0; s < NS; s++) {
        if (s + 2 < NS) load(sl[(s + 2) % 3], s + 2);
        if (s > 0) __syncthreads();   // the previous chunk's MFMA reads are done
        store(sl[s % 3], s);
        __syncthreads();
        // both 32-pair sub-tiles always run (no branch around the MFMAs); a
        // sub-tile past the tile's pairs reads zero rows and is not stored
#pragma unroll
        for (int ks = 0; ks < PF_KC; ks += 16) {
            const bf16x8 av = *reinterpret_cast<const bf16x8 *>(wb + ks);
            const bf16x8 b0 = *reinterpret_cast<const bf16x8 *>(xb + ks);
            const bf16x8 b1 = *reinterpret_cast<const bf16x8 *>(xb + 32 * PF_LD + ks);
            acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, b0, acc[0], 0, 0, 0);
            acc[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, b1, acc[1], 0, 0, 0);
        }
    }
    const int nsub = (tl.n + 31) / 32;
    // accumulator register i of lane l: row 8(i/4) + 4(l/32) + i%4 of the
    // wave's 32, pair 32t + l%32 of the tile
#pragma unroll
    for (int t = 0; t < 2; t++) {
        const int pr = 32 * t + (lane & 31);
        if (t < nsub && pr < tl.n) {
            const int p = perm[tl.start + pr];
            if (MODE == 0) {
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    unsigned o[2];
#pragma unroll
                    for (int c = 0; c < 2; c++) {
                        float a2[2];
#pragma unroll
                        for (int e = 0; e < 2; e++) {
                            const int i = 4 * h + 2 * c + e;
                            const float g = acc[t][i], u = acc[t][i + 8];
                            a2[e] = g / (1.0f + expf_glibc(-g)) * u;
                        }
                        o[c] = pack_bf16x2(a2[0], a2[1]);
                    }
                    const int col = blockIdx.y * 64 + 16 * wave + 8 * h + 4 * (lane >> 5);
                    *reinterpret_cast<uint2 *>(act + (long long)p * F + col) = make_uint2(o[0], o[1]);
                }
            } else {
#pragma unroll
                for (int h = 0; h < 4; h++) {
                    const int row = blockIdx.y * PF_ROWS + 32 * wave + 8 * h + 4 * (lane >> 5);
                    *reinterpret_cast<float4 *>(y + (long long)p * H + row) =
                        make_float4(acc[t][4 * h], acc[t][4 * h + 1], acc[t][4 * h + 2], acc[t][4 * h + 3]);
                }
            }
        }
    }
}

__global__ __launch_bounds__(256) void k_to_bf16(const float *__restrict__ x, __bf16 *__restrict__ o, long long n4) {
    for (long long i = blockIdx.x * 256ll + threadIdx.x; i < n4; i += (long long)gridDim.x * 256) {
        const float4 v = reinterpret_cast<const float4 *>(x)[i];
        reinterpret_cast<uint2 *>(o)[i] = make_uint2(pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w));
    }
}

size_t prefill_workspace_bytes(int T, int k, int E, int H, int F) {
    const size_t P = (size_t)T * k;
    const size_t max_tiles = (P + PF_MT - 1) / PF_MT + E;
    auto up = [](size_t n) { return (n + 255) & ~(size_t)255; };
    return up(P * 4) + up(max_tiles * sizeof(PfTile)) + 256 + up(P * F * 2) + up((size_t)T * H * 2);
}

template <int MODE>
static hipError_t launch_moe_mfma(int ns, dim3 grid, hipStream_t st, const uint8_t *W0, const uint8_t *W1,
                                  const __bf16 *X, int x_rows, const int *perm, const PfTile *tiles, const int *ntiles, int H, int F,
                                  int k, __bf16 *act, float *y) {
#define TBQ_NS(N)                                                                                                  \
    case N:                                                                                                        \
        hipLaunchKernelGGL((k_moe_mfma<MODE, N>), grid, dim3(PF_THREADS), PF_LDS_BYTES, st, W0, W1, X, x_rows, perm, \
                           tiles, ntiles, H, F, k, act, y);                                                        \
        break;
    switch (ns) {
        TBQ_NS(2) TBQ_NS(4) TBQ_NS(6) TBQ_NS(8) TBQ_NS(12) TBQ_NS(16) TBQ_NS(24) TBQ_NS(32)
    default:
        return hipErrorNotSupported;
    }
#undef TBQ_NS
    return hipGetLastError();
}

// Experts on MFMA for Q4_K weights; routing already in a.sel_idx/a.sel_w.
// Uses a.y (pairs x H fp32) and `scratch` (prefill_workspace_bytes).
// K = H (gate/up) and F (down) must be 256, 512, 768, 1024, 1536, 2048,
// 3072 or 4096.
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
    __bf16 *act = (__bf16 *)w; w += up(P * a.F * 2);
    __bf16 *xb = (__bf16 *)w;
    {
        const long long n4 = (long long)a.T * a.H / 4;
        const int grid = (int)((n4 + 255) / 256 < 2048 ? (n4 + 255) / 256 : 2048);
        hipLaunchKernelGGL(k_to_bf16, dim3(grid), dim3(256), 0, st, a.xn, xb, n4);
    }
    hipLaunchKernelGGL(k_dispatch, dim3(1), dim3(1024), 0, st, a.sel_idx, a.T, a.k, a.E, perm, tiles, ntiles);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    err = launch_moe_mfma<0>(a.H / PF_KC, dim3(max_tiles, a.F / 64), st, (const uint8_t *)a.gate,
                             (const uint8_t *)a.up, xb, a.T, perm, tiles, ntiles, a.H, a.F, a.k, act, nullptr);
    if (err != hipSuccess) return err;
    return launch_moe_mfma<1>(a.F / PF_KC, dim3(max_tiles, a.H / PF_ROWS), st, (const uint8_t *)a.down, nullptr, act,
                              (int)P, perm, tiles, ntiles, a.H, a.F, a.k, nullptr, a.y);
}

}  // namespace tbq
