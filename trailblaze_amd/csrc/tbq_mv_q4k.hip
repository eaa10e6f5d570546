// tbq_mv_q4k.hip -- decode matvec y = W x for Q4_K super-blocks on gfx950,
// built on integer dot products.
//
// (Digit representation and its accuracy: tbq_q4k.hpp.)
//
// Work split: a workgroup stores x's digits in LDS (XD_UNIT layout: 52
// dwords per 64 elements, read free of bank conflicts); x's loads are
// issued before the weight loads so they do not queue behind them; each
// lane owns "units" of two consecutive sub-blocks of one super-block (64
// weights, 4 lanes per super-block) and LPR lanes share a row.  Three
// kernels: k_mv_q4k_xr (K <= 4096, up to 8192 rows: one pass, R rows per
// wave, all weight loads issued before x is staged), k_mv_q4k_xp (K <=
// 4096, taller: persistent waves, the next row's loads in flight while the
// current one is reduced), k_mv_q4k (longer rows: digits read from LDS per
// row, grid-strided rows).
#include "tbq_kernels.h"
#include "tbq_q4k.hpp"

namespace tbq {

constexpr int WG = 1024;        // threads per workgroup (16 waves share one x staging)
#ifndef Q4K_XR_R
#define Q4K_XR_R 2               // rows per lane of the register-x kernel
#endif
#ifndef Q4K_XR_NW
#define Q4K_XR_NW 8              // waves per workgroup of the register-x kernel
#endif
#ifndef Q4K_XP_NW
#define Q4K_XP_NW 16             // waves per workgroup of the persistent kernel (one per CU)
#endif
constexpr int Q4K_XR_MAX_M = 8192;   // taller matrices take the persistent kernel

// One pass of a wave covers RPP = 64/LPR rows; each lane owns UPL units of
// its row.  Rows are grid-strided over all waves; the next pass's loads are
// issued before the current pass is reduced.
template <int LPR, int UPL, bool GG>
__global__ __launch_bounds__(WG) void k_mv_q4k(const uint8_t *__restrict__ W, int M, int K, long long rb,
                                               const float *__restrict__ x, float *__restrict__ y) {
    extern __shared__ uint32_t xd[];
    constexpr int RPP = 64 / LPR;
    const int U = K / 64;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int lr = lane % LPR, rsub = lane / LPR;
    const int stride = gridDim.x * (WG / 64) * RPP;
    int row = (blockIdx.x * (WG / 64) + wave) * RPP + rsub;

    XStager<WG, 2> xs;   // K <= 16384
    xs.load(x, K);
    Q4KUnit cur[UPL], nxt[UPL];
    auto load = [&](Q4KUnit *dst, int r) {
#pragma unroll
        for (int i = 0; i < UPL; i++) {
            const int u = lr + LPR * i;
            if (r < M && u < U) q4k_load<GG>(W + (long long)r * rb, u, dst[i]);
        }
    };
    load(cur, row);
    xs.store(xd, K);
    __syncthreads();
    // every lane of a wave runs the same number of passes: the bound uses the
    // wave's first row, so the shuffles below always see a full wave
    const int wave_row0 = (blockIdx.x * (WG / 64) + wave) * RPP;
    for (int base = wave_row0; base < M; base += stride) {
        const int nrow = row + stride;
        constexpr bool PREFETCH = UPL <= 2;   // keeps UPL 3-4 within 128 VGPRs
        if (PREFETCH && base + stride < M) load(nxt, nrow);
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < UPL; i++) {
            const int u = lr + LPR * i;
            if (row < M && u < U) acc = q4k_unit_dot<GG>(cur[i], u, xd, acc);
        }
        acc = group_sum<LPR>(acc);
        if (lr == 0 && row < M) y[row] = acc;
        if (PREFETCH) {
#pragma unroll
            for (int i = 0; i < UPL; i++) cur[i] = nxt[i];
        } else if (base + stride < M) {
            load(cur, nrow);
        }
        row = nrow;
    }
}

// Rows of up to 64 units (K <= 4096): every lane keeps one unit index for
// all its rows, so it reads that unit's digits from LDS once into registers
// and reuses them for R rows (LDS traffic / R).  A wave covers R passes of
// RPP = 64/LPR rows (rows wave_base + p*RPP + rsub); all R passes' weight
// loads are in flight before x is staged.  No grid-stride loop: the grid
// covers M exactly.
template <int LPR, int R, int NW, int PRO, bool GG>
__global__ __launch_bounds__(NW * 64) void k_mv_q4k_xr(const uint8_t *__restrict__ W, int M, int K, long long rb,
                                                      const float *__restrict__ x, float *__restrict__ y, MvPro pro) {
    extern __shared__ uint32_t xd[];
    constexpr int NT = NW * 64, RPP = 64 / LPR;
    const int U = K / 64;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int lr = lane % LPR, rsub = lane / LPR;
    const bool lv = lr < U;
    const int ul = lv ? lr : 0;
    XStager<NT, (4 * 128 + NT - 1) / NT, (PRO & 3)> xs;   // K <= 4096
    xs.load(x, K, 1, pro);
    // x's loads stay ahead of the weights'.  (The barrier's place in the
    // plain kernel is its measured one: with the base row computed ahead of
    // it, the 4096x4096 matvec took 4.36 instead of 4.22 us.)
    __builtin_amdgcn_sched_barrier(0);
    const int base = (blockIdx.x * NW + wave) * R * RPP + rsub;
    // Unconditional loads (rows past M re-read row M-1, idle lanes unit 0;
    // their results are discarded): under a branch, the compiler would wait
    // for the weights before staging x.
    Q4KUnit w[R];
#pragma unroll
    for (int p = 0; p < R; p++) {
        const int r = min(base + p * RPP, M - 1);
        q4k_load<GG>(W + (long long)r * rb, ul, w[p]);
    }
    // PRO_RES: the rows' residuals, behind the weights (they are used after
    // the dot products, which wait for every weight load anyway)
    float rv[R];
    if constexpr ((PRO & PRO_RES) != 0) {
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int p = 0; p < R; p++) rv[p] = y[min(base + p * RPP, M - 1)];
        __builtin_amdgcn_sched_barrier(0);
    }
    xs.apply(K, pro);
    xs.store(xd, K);
    float *ssred = reinterpret_cast<float *>(xd + (K / 32) * XD_PER_SB);   // PRO_NORMD: NW floats
    if constexpr ((PRO & 3) == PRO_NORMD) pro_ss_put(xs.ss, ssred);
    __syncthreads();
    XUnit xu;
    xunit_load(xd, ul, xu);
    float rn = 1.f;
    if constexpr ((PRO & 3) == PRO_NORMD) rn = pro_ss_scale<NW>(ssred, K, pro.eps);
#pragma unroll
    for (int p = 0; p < R; p++) {
        const int r = base + p * RPP;
        const float v = q4k_unit_dot<GG>(w[p], ul, xu, 0.f);
        const float acc = group_sum<LPR>((r < M && lv) ? v : 0.f);
        if (lr == 0 && r < M) {
            if constexpr ((PRO & PRO_RES) != 0) y[r] = rv[p] + acc;
            else if constexpr ((PRO & 3) == PRO_NORMD) y[r] = acc * rn;
            else y[r] = acc;
        }
    }
}

// Tall matrices (rows of up to 64 units): persistent waves.  Each
// workgroup stages x once; each wave keeps its lanes' x digits in
// registers (fixed unit per lane, as above) and walks rows gridDim.x * NW *
// RPP apart, with the weights of the next D rows in flight while it reduces
// the current one.  Prefetches past the last row re-read row M-1 and are
// discarded, so every load is unconditional.
template <int LPR, int D, int NW, bool GG>
__global__ __launch_bounds__(NW * 64) void k_mv_q4k_xp(const uint8_t *__restrict__ W, int M, int K, long long rb,
                                                      const float *__restrict__ x, float *__restrict__ y) {
    extern __shared__ uint32_t xd[];
    constexpr int NT = NW * 64, RPP = 64 / LPR;
    const int U = K / 64;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int lr = lane % LPR, rsub = lane / LPR;
    const bool lv = lr < U;
    const int ul = lv ? lr : 0;
    XStager<NT, (4 * 128 + NT - 1) / NT> xs;   // K <= 4096
    xs.load(x, K);
    __builtin_amdgcn_sched_barrier(0);   // x's loads stay ahead of the weights'
    const int stride = gridDim.x * NW * RPP;
    const int row0 = (blockIdx.x * NW + wave) * RPP + rsub;
    Q4KUnit buf[D + 1];
#pragma unroll
    for (int i = 0; i < D; i++) q4k_load<GG>(W + (long long)min(row0 + i * stride, M - 1) * rb, ul, buf[i]);
    xs.store(xd, K);
    __syncthreads();
    XUnit xu;
    xunit_load(xd, ul, xu);
    // every lane of a wave runs the same number of passes (bound from the
    // wave's first row), so the reductions always see a full wave
    const int wrow0 = (blockIdx.x * NW + wave) * RPP;
    for (int r0 = wrow0; r0 < M; r0 += stride) {
        const int r = r0 + rsub;
        q4k_load<GG>(W + (long long)min(r + D * stride, M - 1) * rb, ul, buf[D]);
        const float v = q4k_unit_dot<GG>(buf[0], ul, xu, 0.f);
        const float acc = group_sum<LPR>((r < M && lv) ? v : 0.f);
        if (lr == 0 && r < M) y[r] = acc;
#pragma unroll
        for (int i = 0; i < D; i++) buf[i] = buf[i + 1];
    }
}

template <int LPR, int D, int NW, bool GG>
static hipError_t launch_q4k_xp(const void *W, int M, int K, const float *x, float *y, hipStream_t s, int n_cu,
                                int wpc) {
    constexpr int RPW = NW * (64 / LPR);
    const long long need = ((long long)M + RPW - 1) / RPW;
    const long long cap = (long long)n_cu * wpc;
    const int grid = (int)(need < cap ? need : cap);
    const long long rb = (long long)(K / 256) * 144;
    const size_t lds = (size_t)(K / 32) * XD_PER_SB * 4;
    hipLaunchKernelGGL((k_mv_q4k_xp<LPR, D, NW, GG>), dim3(grid), dim3(NW * 64), lds, s, (const uint8_t *)W, M, K,
                       rb, x, y);
    return hipGetLastError();
}

template <int LPR, int R, int NW, int PRO, bool GG>
static hipError_t launch_q4k_xr(const void *W, int M, int K, const float *x, float *y, hipStream_t s,
                                const MvPro &pro) {
    constexpr int ROWS_PER_WG = NW * R * (64 / LPR);
    const int grid = (M + ROWS_PER_WG - 1) / ROWS_PER_WG;
    const long long rb = (long long)(K / 256) * 144;
    const size_t lds = (size_t)(K / 32) * XD_PER_SB * 4 + ((PRO & 3) == PRO_NORMD ? 32 * 4 : 0);
    hipLaunchKernelGGL((k_mv_q4k_xr<LPR, R, NW, PRO, GG>), dim3(grid), dim3(NW * 64), lds, s, (const uint8_t *)W, M, K,
                       rb, x, y, pro);
    return hipGetLastError();
}

template <int PRO, bool GG>
static hipError_t launch_q4k_xr_k(const void *W, int M, int K, const float *x, float *y, hipStream_t s,
                                  const MvPro &pro) {
    const int U = K / 64;
    if (U <= 4) return launch_q4k_xr<4, Q4K_XR_R, Q4K_XR_NW, PRO, GG>(W, M, K, x, y, s, pro);
    if (U <= 8) return launch_q4k_xr<8, Q4K_XR_R, Q4K_XR_NW, PRO, GG>(W, M, K, x, y, s, pro);
    if (U <= 16) return launch_q4k_xr<16, Q4K_XR_R, Q4K_XR_NW, PRO, GG>(W, M, K, x, y, s, pro);
    if (U <= 32) return launch_q4k_xr<32, Q4K_XR_R, Q4K_XR_NW, PRO, GG>(W, M, K, x, y, s, pro);
    // one row per lane where Q4K_XR_R rows per lane would leave between one
    // and two workgroups per CU (256 CUs: 4096 < M < 8192), so every CU gets
    // the same number (6144x4096: 5.3 against 5.9 us; at 4096 rows and
    // below two rows per lane stay faster, 4.24 against 4.31 us)
    constexpr int RW = Q4K_XR_NW * Q4K_XR_R;
    const int n_cu = tbq_cu_count() > 0 ? tbq_cu_count() : 256;
    // 8 to 10 rows per CU (2560 rows on 256 CUs): workgroups of 10 waves of
    // one row, one workgroup per CU, where workgroups of 16 rows left 96 CUs
    // without one (Qwen3-4B's o projection 2560x4096: dense decode 1618 ->
    // 1607 us/token; 5 waves of two rows: 1622)
    if (M > 8LL * n_cu && M <= 10LL * n_cu) return launch_q4k_xr<64, 1, 10, PRO, GG>(W, M, K, x, y, s, pro);
    // 16 to 24 rows per CU with a fused prologue (Qwen3-4B's q|k|v, 6144
    // rows): one workgroup per CU with three rows per wave instead of three
    // workgroups of one row per wave, so x is staged and normalised once per
    // CU (dense decode 1506 -> 1495 us/token; the plain matvec measured
    // 4.77 against 4.86 us in the old shape, which it keeps)
    if (PRO != PRO_NONE && M > 16LL * n_cu && M <= 24LL * n_cu)
        return launch_q4k_xr<64, 3, 8, PRO, GG>(W, M, K, x, y, s, pro);
    const long long wg = ((long long)M + RW - 1) / RW;
    if (Q4K_XR_R > 1 && wg > n_cu && wg < 2LL * n_cu)
        return launch_q4k_xr<64, 1, Q4K_XR_NW, PRO, GG>(W, M, K, x, y, s, pro);
    return launch_q4k_xr<64, Q4K_XR_R, Q4K_XR_NW, PRO, GG>(W, M, K, x, y, s, pro);
}

template <int LPR, int UPL, bool GG>
static hipError_t launch_q4k_t(const void *W, int M, int K, const float *x, float *y, hipStream_t s, int n_cu) {
    constexpr int ROWS_PER_WG = (WG / 64) * (64 / LPR);
    long long need = ((long long)M + ROWS_PER_WG - 1) / ROWS_PER_WG;
    long long cap = 2ll * n_cu;
    int grid = (int)(need < cap ? need : cap);
    long long rb = (long long)(K / 256) * 144;
    size_t lds = (size_t)(K / 32) * XD_PER_SB * 4;
    hipLaunchKernelGGL((k_mv_q4k<LPR, UPL, GG>), dim3(grid), dim3(WG), lds, s, (const uint8_t *)W, M, K, rb, x, y);
    return hipGetLastError();
}

template <bool GG>
static hipError_t launch_q4k_xp_k(const void *W, int M, int K, const float *x, float *y, hipStream_t s, int n_cu) {
    const int U = K / 64;
    constexpr int NW = Q4K_XP_NW;
    if (U <= 4) return launch_q4k_xp<4, 1, NW, GG>(W, M, K, x, y, s, n_cu, 1);
    if (U <= 8) return launch_q4k_xp<8, 1, NW, GG>(W, M, K, x, y, s, n_cu, 1);
    if (U <= 16) return launch_q4k_xp<16, 1, NW, GG>(W, M, K, x, y, s, n_cu, 1);
    if (U <= 32) return launch_q4k_xp<32, 1, NW, GG>(W, M, K, x, y, s, n_cu, 1);
    return launch_q4k_xp<64, 1, NW, GG>(W, M, K, x, y, s, n_cu, 1);
}

template <bool GG>
static hipError_t launch_matvec_q4k_g(const void *W, int M, int K, const float *x, float *y, hipStream_t s, int n_cu) {
    const int U = K / 64;
    if (U <= 64 && M > Q4K_XR_MAX_M) return launch_q4k_xp_k<GG>(W, M, K, x, y, s, n_cu);
    if (U <= 64) return launch_q4k_xr_k<PRO_NONE, GG>(W, M, K, x, y, s, MvPro{});
    if (U <= 128) return launch_q4k_t<64, 2, GG>(W, M, K, x, y, s, n_cu);
    if (U <= 192) return launch_q4k_t<64, 3, GG>(W, M, K, x, y, s, n_cu);
    return launch_q4k_t<64, 4, GG>(W, M, K, x, y, s, n_cu);
}

// Returns hipErrorNotSupported for shapes this kernel does not cover.
// ggml: ggml's Q4_K layout (QT_GQ4_K) instead of the reference's.
hipError_t launch_matvec_q4k(const void *W, int M, int K, const float *x, float *y, hipStream_t s, int n_cu,
                             bool ggml) {
    const int U = K / 64;
    if (K % 256 || U < 4 || U > 256) return hipErrorNotSupported;
    return ggml ? launch_matvec_q4k_g<true>(W, M, K, x, y, s, n_cu) : launch_matvec_q4k_g<false>(W, M, K, x, y, s, n_cu);
}

// With a staging prologue: the register-x kernel only (K <= 4096);
// hipErrorNotSupported otherwise.
hipError_t launch_matvec_q4k_pro(int mode, const MvPro &pro, const void *W, int M, int K, const float *x, float *y,
                                 hipStream_t s, bool ggml) {
    const int U = K / 64;
    if (K % 256 || U < 4 || U > 64) return hipErrorNotSupported;
    switch (mode) {
    case PRO_NONE:
        return ggml ? launch_q4k_xr_k<PRO_NONE, true>(W, M, K, x, y, s, pro)
                    : launch_q4k_xr_k<PRO_NONE, false>(W, M, K, x, y, s, pro);
    case PRO_NORM:
        return ggml ? launch_q4k_xr_k<PRO_NORM, true>(W, M, K, x, y, s, pro)
                    : launch_q4k_xr_k<PRO_NORM, false>(W, M, K, x, y, s, pro);
    case PRO_RES:
        return ggml ? launch_q4k_xr_k<PRO_RES, true>(W, M, K, x, y, s, pro)
                    : launch_q4k_xr_k<PRO_RES, false>(W, M, K, x, y, s, pro);
    case PRO_NORMD:
        return ggml ? launch_q4k_xr_k<PRO_NORMD, true>(W, M, K, x, y, s, pro)
                    : launch_q4k_xr_k<PRO_NORMD, false>(W, M, K, x, y, s, pro);
    default: return hipErrorNotSupported;
    }
}

}  // namespace tbq
