// tbq_matvec.hip -- gfx950 kernels for the bit-exact dequant hook and the
// decode dequant-matvec y = W x (fp32 x, fp32 accumulate) for every block
// format of the reference's dequant table (layer4/tb_gguf.c:293-419), in the
// reference's layouts and in ggml's.
#include "tbq_kquant.hpp"
#include "tbq_kernels.h"

namespace tbq {

// ---------------------------------------------------------------------------
// Dequant: thread t writes weights 8t..8t+7 of the flattened matrix.  Rows
// are whole blocks, so flat weight index / block_weights is the block index.
// ---------------------------------------------------------------------------
template <int QT>
__global__ __launch_bounds__(256) void k_dequant(const uint8_t *__restrict__ W, long long n8,
                                                 float *__restrict__ out) {
    constexpr int BW = block_weights(QT), BB = block_bytes(QT);
    for (long long t = blockIdx.x * 256ll + threadIdx.x; t < n8; t += (long long)gridDim.x * 256) {
        long long e = t * 8;
        float w[8];
        if constexpr (BW == 1) {
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const uint8_t *p = W + (e + i) * BB;
                w[i] = QT == QT_F32 ? __builtin_bit_cast(float, ldu32(p))
                     : QT == QT_F16 ? f16_ref(ldu16(p)) : QT == QT_GF16 ? f16_ieee(ldu16(p))
                     : bf16_ref(ldu16(p));
            }
        } else {
            long long blk = e / BW;
            decode8<QT>(W + blk * BB, (int)(e - blk * BW), w);
        }
        float4 *o = reinterpret_cast<float4 *>(out + e);
        o[0] = make_float4(w[0], w[1], w[2], w[3]);
        o[1] = make_float4(w[4], w[5], w[6], w[7]);
    }
}

// ---------------------------------------------------------------------------
// Generic decode matvec.  x (and its 16-element group sums) are staged once
// per workgroup in LDS; LPR lanes share a row, each striding over the row's
// 32-weight chunks; LPR-wide shuffle reduction; rows grid-strided.
// ---------------------------------------------------------------------------
template <int QT, int LPR>
__global__ __launch_bounds__(256) void k_matvec_generic(const uint8_t *__restrict__ W, int M, int K,
                                                        long long row_bytes, const float *__restrict__ x,
                                                        float *__restrict__ y) {
    extern __shared__ float lds[];
    float *xl = lds;            // K floats (swizzled, see stage_x_swizzled)
    float *xs = lds + K;        // K/16 group sums
    stage_x_swizzled<256>(x, K, xl, xs);
    __syncthreads();
    constexpr int RPW = 256 / LPR;
    const int C = K / 32;
    const int lane = threadIdx.x % LPR, rsub = threadIdx.x / LPR;
    for (int r0 = blockIdx.x * RPW; r0 < M; r0 += gridDim.x * RPW) {
        int r = r0 + rsub;
        float acc = 0.f;
        if (r < M) {
            const uint8_t *row = W + (long long)r * row_bytes;
            for (int c = lane; c < C; c += LPR) {
                float xv[32];
                load_chunk_x(xl, c, xv);
                acc += chunk_dot<QT>(row, c, xv, xs + 2 * c);
            }
        }
        acc = group_sum<LPR>(acc);
        if (lane == 0 && r < M) y[r] = acc;
    }
}

// Rows idx[0..nrows) of a matrix (row stride rb bytes, K weights) to
// out[nrows][K], bit-exact as k_dequant.  grid = (ceil(K / 2048), nrows).
template <int QT>
__global__ __launch_bounds__(256) void k_dequant_rows(const uint8_t *__restrict__ W, long long rb,
                                                      const int *__restrict__ idx, int K, float *__restrict__ out) {
    constexpr int BW = block_weights(QT), BB = block_bytes(QT);
    const uint8_t *row = W + (long long)idx[blockIdx.y] * rb;
    float *o = out + (long long)blockIdx.y * K;
    for (int t = blockIdx.x * 256 + threadIdx.x; t < K / 8; t += gridDim.x * 256) {
        const int e = t * 8;
        float w[8];
        if constexpr (BW == 1) {
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const uint8_t *p = row + (long long)(e + i) * BB;
                w[i] = QT == QT_F32 ? __builtin_bit_cast(float, ldu32(p))
                     : QT == QT_F16 ? f16_ref(ldu16(p)) : QT == QT_GF16 ? f16_ieee(ldu16(p))
                     : bf16_ref(ldu16(p));
            }
        } else {
            decode8<QT>(row + (long long)(e / BW) * BB, e % BW, w);
        }
        float4 *q = reinterpret_cast<float4 *>(o + e);
        q[0] = make_float4(w[0], w[1], w[2], w[3]);
        q[1] = make_float4(w[4], w[5], w[6], w[7]);
    }
}

// W[nrows][K] in format qt to fp16 (the fp32 weight rounded once), for the
// prefill's library GEMMs.  Thread t writes weights 8t..8t+7.
template <int QT>
__global__ __launch_bounds__(256) void k_dequant_f16(const uint8_t *__restrict__ W, long long n8,
                                                     _Float16 *__restrict__ out) {
    constexpr int BW = block_weights(QT), BB = block_bytes(QT);
    for (long long t = blockIdx.x * 256ll + threadIdx.x; t < n8; t += (long long)gridDim.x * 256) {
        const long long e = t * 8;
        float w[8];
        if constexpr (BW == 1) {
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const uint8_t *p = W + (e + i) * BB;
                w[i] = QT == QT_F32 ? __builtin_bit_cast(float, ldu32(p))
                     : QT == QT_F16 ? f16_ref(ldu16(p)) : QT == QT_GF16 ? f16_ieee(ldu16(p))
                     : bf16_ref(ldu16(p));
            }
        } else {
            const long long blk = e / BW;
            decode8<QT>(W + blk * BB, (int)(e - blk * BW), w);
        }
        typedef _Float16 h8 __attribute__((ext_vector_type(8)));
        const h8 v = {(_Float16)w[0], (_Float16)w[1], (_Float16)w[2], (_Float16)w[3],
                      (_Float16)w[4], (_Float16)w[5], (_Float16)w[6], (_Float16)w[7]};
        *reinterpret_cast<h8 *>(out + e) = v;
    }
}

// Q4_K to fp16: thread t writes weights 8t .. 8t + 7 (16 contiguous bytes,
// so a wave's stores are one contiguous run): 64-weight unit u = t / 8
// (super-block u / 4, quant bytes 32p .. 32p + 31, p = u % 4), part
// k = t % 8; the unit's header is read by its 8 threads (cache hits) and
// each reads only its quant dwords.  Values as decode8 rounds them
// (fl(fl(d*s)*q) - fl(dmin*m)), then fp16.  GG: ggml's layout (byte i of
// the run: element i of sub-block 2p low, of 2p+1 high; get_scale_min_k4;
// IEEE fp16 d).
template <bool GG>
__global__ __launch_bounds__(256) void k_dequant_f16_q4k(const uint8_t *__restrict__ W, long long n8,
                                                         _Float16 *__restrict__ out) {
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    for (long long t = blockIdx.x * 256ll + threadIdx.x; t < n8; t += (long long)gridDim.x * 256) {
        const long long u = t >> 3;
        const int k = (int)(t & 7), p = (int)(u & 3);
        const uint8_t *b = W + (u >> 2) * 144;
        const uint4 hdr = *reinterpret_cast<const uint4 *>(b);
        const uint8_t *run = b + 16 + 32 * p;
        int si, mi;
        float d, dmin;
        uint32_t q[2];
        int sh = 0;
        if constexpr (GG) {   // weights 8k + i: bytes 8(k % 4) + i, nibble k / 4
            d = f16_ieee(hdr.x & 0xFFFFu);
            dmin = f16_ieee(hdr.x >> 16);
            gq4k_sm(hdr, p, k >> 2, si, mi);
            const uint2 v = *reinterpret_cast<const uint2 *>(run + 8 * (k & 3));
            q[0] = v.x;
            q[1] = v.y;
            sh = 4 * (k >> 2);
        } else {              // weights 8k + i: byte 4k + i / 2, nibble i % 2
            d = f16_ref(hdr.x & 0xFFFFu);
            dmin = f16_ref(hdr.x >> 16);
            // sub-block j = 2p + k / 4: j < 4 scale byte 4 + j (hdr.y), min
            // byte 8 + j (hdr.z); j >= 4 scale byte 8 + j (hdr.w), min byte
            // 12 + j (the block's first quant dword)
            const int j = 2 * p + (k >> 2), jb = 8 * (j & 3);
            const uint32_t mind = j < 4 ? hdr.z : *reinterpret_cast<const uint32_t *>(b + 16);
            si = (int)(((j < 4 ? hdr.y : hdr.w) >> jb) & 63);
            mi = (int)((mind >> jb) & 63);
            q[0] = *reinterpret_cast<const uint32_t *>(run + 4 * k);
            q[1] = 0;
        }
        const float S = d * (float)si, Mn = dmin * (float)mi;
        h8 v;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int qq = GG ? (int)((q[i >> 2] >> (8 * (i & 3) + sh)) & 15)
                              : (int)((q[0] >> (8 * (i >> 1) + 4 * (i & 1))) & 15);
            const float tt = S * (float)qq;
            v[i] = (_Float16)(tt - Mn);
        }
        *reinterpret_cast<h8 *>(out + t * 8) = v;
    }
}

template <int QT>
static hipError_t launch_dequant_f16_t(const void *W, long long nweights, _Float16 *out, hipStream_t s) {
    if constexpr (QT == QT_Q4_K || QT == QT_GQ4_K) {
        const long long n8 = nweights / 8, blocks = (n8 + 255) / 256;
        const int grid = (int)(blocks < 65536 ? blocks : 65536);
        hipLaunchKernelGGL((k_dequant_f16_q4k<QT == QT_GQ4_K>), dim3(grid), dim3(256), 0, s, (const uint8_t *)W, n8,
                           out);
        return hipGetLastError();
    }
    const long long n8 = nweights / 8, blocks = (n8 + 255) / 256;
    const int grid = (int)(blocks < 65536 ? blocks : 65536);
    hipLaunchKernelGGL((k_dequant_f16<QT>), dim3(grid), dim3(256), 0, s, (const uint8_t *)W, n8, out);
    return hipGetLastError();
}

template <int QT>
static hipError_t launch_dequant_rows_t(const void *W, const int *idx, int nrows, int K, float *out, hipStream_t s) {
    const long long rb = (long long)(K / block_weights(QT)) * block_bytes(QT);
    hipLaunchKernelGGL((k_dequant_rows<QT>), dim3((K / 8 + 255) / 256, nrows), dim3(256), 0, s, (const uint8_t *)W, rb,
                       idx, K, out);
    return hipGetLastError();
}

template <int QT>
static hipError_t launch_dequant_t(const void *W, long long nweights, float *out, hipStream_t s) {
    long long n8 = nweights / 8;
    long long blocks = (n8 + 255) / 256;
    int grid = (int)(blocks < 65536 ? blocks : 65536);
    hipLaunchKernelGGL((k_dequant<QT>), dim3(grid), dim3(256), 0, s, (const uint8_t *)W, n8, out);
    return hipGetLastError();
}

template <int QT, int LPR>
static hipError_t launch_mv(const void *W, int M, int K, const float *x, float *y, hipStream_t s, int n_cu) {
    constexpr int RPW = 256 / LPR;
    long long rb = (long long)(K / block_weights(QT)) * block_bytes(QT);
    int need = (M + RPW - 1) / RPW;
    int cap = n_cu * 4;
    int grid = need < cap ? need : cap;
    size_t lds = (size_t)K * 4 + (size_t)(K / 16) * 4;
    hipLaunchKernelGGL((k_matvec_generic<QT, LPR>), dim3(grid), dim3(256), lds, s, (const uint8_t *)W, M, K, rb, x, y);
    return hipGetLastError();
}

template <int QT>
static hipError_t launch_mv_q(const void *W, int M, int K, const float *x, float *y, hipStream_t s, int n_cu) {
    int C = K / 32;
    // largest power of two <= min(C, 64) that divides C when possible
    int lpr = 64;
    while (lpr > 1 && (lpr > C || C % lpr)) lpr >>= 1;
    if (lpr < 4 && C >= 4) lpr = 4;
    switch (lpr) {
    case 64: return launch_mv<QT, 64>(W, M, K, x, y, s, n_cu);
    case 32: return launch_mv<QT, 32>(W, M, K, x, y, s, n_cu);
    case 16: return launch_mv<QT, 16>(W, M, K, x, y, s, n_cu);
    case 8: return launch_mv<QT, 8>(W, M, K, x, y, s, n_cu);
    case 4: return launch_mv<QT, 4>(W, M, K, x, y, s, n_cu);
    case 2: return launch_mv<QT, 2>(W, M, K, x, y, s, n_cu);
    default: return launch_mv<QT, 1>(W, M, K, x, y, s, n_cu);
    }
}

hipError_t launch_dequant(int qt, const void *W, long long nweights, float *out, hipStream_t s) {
    switch (qt) {
    case QT_F32: return launch_dequant_t<QT_F32>(W, nweights, out, s);
    case QT_F16: return launch_dequant_t<QT_F16>(W, nweights, out, s);
    case QT_BF16: return launch_dequant_t<QT_BF16>(W, nweights, out, s);
    case QT_Q4_0: return launch_dequant_t<QT_Q4_0>(W, nweights, out, s);
    case QT_Q8_0: return launch_dequant_t<QT_Q8_0>(W, nweights, out, s);
    case QT_Q2_K: return launch_dequant_t<QT_Q2_K>(W, nweights, out, s);
    case QT_Q3_K: return launch_dequant_t<QT_Q3_K>(W, nweights, out, s);
    case QT_Q4_K: return launch_dequant_t<QT_Q4_K>(W, nweights, out, s);
    case QT_Q5_K: return launch_dequant_t<QT_Q5_K>(W, nweights, out, s);
    case QT_Q6_K: return launch_dequant_t<QT_Q6_K>(W, nweights, out, s);
    case QT_Q8_K: return launch_dequant_t<QT_Q8_K>(W, nweights, out, s);
    case QT_GF16: return launch_dequant_t<QT_GF16>(W, nweights, out, s);
    case QT_GQ4_0: return launch_dequant_t<QT_GQ4_0>(W, nweights, out, s);
    case QT_GQ8_0: return launch_dequant_t<QT_GQ8_0>(W, nweights, out, s);
    case QT_GQ2_K: return launch_dequant_t<QT_GQ2_K>(W, nweights, out, s);
    case QT_GQ3_K: return launch_dequant_t<QT_GQ3_K>(W, nweights, out, s);
    case QT_GQ4_K: return launch_dequant_t<QT_GQ4_K>(W, nweights, out, s);
    case QT_GQ5_K: return launch_dequant_t<QT_GQ5_K>(W, nweights, out, s);
    case QT_GQ6_K: return launch_dequant_t<QT_GQ6_K>(W, nweights, out, s);
    default: return hipErrorInvalidValue;
    }
}

// nweights (a multiple of 8 and of the block size) of format qt to fp16.
hipError_t launch_dequant_f16(int qt, const void *W, long long nweights, _Float16 *out, hipStream_t s) {
    switch (qt) {
    case QT_F32: return launch_dequant_f16_t<QT_F32>(W, nweights, out, s);
    case QT_F16: return launch_dequant_f16_t<QT_F16>(W, nweights, out, s);
    case QT_BF16: return launch_dequant_f16_t<QT_BF16>(W, nweights, out, s);
    case QT_Q4_0: return launch_dequant_f16_t<QT_Q4_0>(W, nweights, out, s);
    case QT_Q8_0: return launch_dequant_f16_t<QT_Q8_0>(W, nweights, out, s);
    case QT_Q2_K: return launch_dequant_f16_t<QT_Q2_K>(W, nweights, out, s);
    case QT_Q3_K: return launch_dequant_f16_t<QT_Q3_K>(W, nweights, out, s);
    case QT_Q4_K: return launch_dequant_f16_t<QT_Q4_K>(W, nweights, out, s);
    case QT_Q5_K: return launch_dequant_f16_t<QT_Q5_K>(W, nweights, out, s);
    case QT_Q6_K: return launch_dequant_f16_t<QT_Q6_K>(W, nweights, out, s);
    case QT_Q8_K: return launch_dequant_f16_t<QT_Q8_K>(W, nweights, out, s);
    case QT_GF16: return launch_dequant_f16_t<QT_GF16>(W, nweights, out, s);
    case QT_GQ4_0: return launch_dequant_f16_t<QT_GQ4_0>(W, nweights, out, s);
    case QT_GQ8_0: return launch_dequant_f16_t<QT_GQ8_0>(W, nweights, out, s);
    case QT_GQ2_K: return launch_dequant_f16_t<QT_GQ2_K>(W, nweights, out, s);
    case QT_GQ3_K: return launch_dequant_f16_t<QT_GQ3_K>(W, nweights, out, s);
    case QT_GQ4_K: return launch_dequant_f16_t<QT_GQ4_K>(W, nweights, out, s);
    case QT_GQ5_K: return launch_dequant_f16_t<QT_GQ5_K>(W, nweights, out, s);
    case QT_GQ6_K: return launch_dequant_f16_t<QT_GQ6_K>(W, nweights, out, s);
    default: return hipErrorInvalidValue;
    }
}

// Rows idx[i] (device ints, in range) of a [*][K] matrix in format qt.
hipError_t launch_dequant_rows(int qt, const void *W, const int *idx, int nrows, int K, float *out, hipStream_t s) {
    switch (qt) {
    case QT_F32: return launch_dequant_rows_t<QT_F32>(W, idx, nrows, K, out, s);
    case QT_F16: return launch_dequant_rows_t<QT_F16>(W, idx, nrows, K, out, s);
    case QT_BF16: return launch_dequant_rows_t<QT_BF16>(W, idx, nrows, K, out, s);
    case QT_Q4_0: return launch_dequant_rows_t<QT_Q4_0>(W, idx, nrows, K, out, s);
    case QT_Q8_0: return launch_dequant_rows_t<QT_Q8_0>(W, idx, nrows, K, out, s);
    case QT_Q2_K: return launch_dequant_rows_t<QT_Q2_K>(W, idx, nrows, K, out, s);
    case QT_Q3_K: return launch_dequant_rows_t<QT_Q3_K>(W, idx, nrows, K, out, s);
    case QT_Q4_K: return launch_dequant_rows_t<QT_Q4_K>(W, idx, nrows, K, out, s);
    case QT_Q5_K: return launch_dequant_rows_t<QT_Q5_K>(W, idx, nrows, K, out, s);
    case QT_Q6_K: return launch_dequant_rows_t<QT_Q6_K>(W, idx, nrows, K, out, s);
    case QT_Q8_K: return launch_dequant_rows_t<QT_Q8_K>(W, idx, nrows, K, out, s);
    case QT_GF16: return launch_dequant_rows_t<QT_GF16>(W, idx, nrows, K, out, s);
    case QT_GQ4_0: return launch_dequant_rows_t<QT_GQ4_0>(W, idx, nrows, K, out, s);
    case QT_GQ8_0: return launch_dequant_rows_t<QT_GQ8_0>(W, idx, nrows, K, out, s);
    case QT_GQ2_K: return launch_dequant_rows_t<QT_GQ2_K>(W, idx, nrows, K, out, s);
    case QT_GQ3_K: return launch_dequant_rows_t<QT_GQ3_K>(W, idx, nrows, K, out, s);
    case QT_GQ4_K: return launch_dequant_rows_t<QT_GQ4_K>(W, idx, nrows, K, out, s);
    case QT_GQ5_K: return launch_dequant_rows_t<QT_GQ5_K>(W, idx, nrows, K, out, s);
    case QT_GQ6_K: return launch_dequant_rows_t<QT_GQ6_K>(W, idx, nrows, K, out, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_matvec_generic(int qt, const void *W, int M, int K, const float *x, float *y,
                                 hipStream_t s, int n_cu) {
    switch (qt) {
    case QT_F32: return launch_mv_q<QT_F32>(W, M, K, x, y, s, n_cu);
    case QT_F16: return launch_mv_q<QT_F16>(W, M, K, x, y, s, n_cu);
    case QT_BF16: return launch_mv_q<QT_BF16>(W, M, K, x, y, s, n_cu);
    case QT_Q4_0: return launch_mv_q<QT_Q4_0>(W, M, K, x, y, s, n_cu);
    case QT_Q8_0: return launch_mv_q<QT_Q8_0>(W, M, K, x, y, s, n_cu);
    case QT_Q2_K: return launch_mv_q<QT_Q2_K>(W, M, K, x, y, s, n_cu);
    case QT_Q3_K: return launch_mv_q<QT_Q3_K>(W, M, K, x, y, s, n_cu);
    case QT_Q4_K: return launch_mv_q<QT_Q4_K>(W, M, K, x, y, s, n_cu);
    case QT_Q5_K: return launch_mv_q<QT_Q5_K>(W, M, K, x, y, s, n_cu);
    case QT_Q6_K: return launch_mv_q<QT_Q6_K>(W, M, K, x, y, s, n_cu);
    case QT_Q8_K: return launch_mv_q<QT_Q8_K>(W, M, K, x, y, s, n_cu);
    case QT_GF16: return launch_mv_q<QT_GF16>(W, M, K, x, y, s, n_cu);
    case QT_GQ4_0: return launch_mv_q<QT_GQ4_0>(W, M, K, x, y, s, n_cu);
    case QT_GQ8_0: return launch_mv_q<QT_GQ8_0>(W, M, K, x, y, s, n_cu);
    case QT_GQ2_K: return launch_mv_q<QT_GQ2_K>(W, M, K, x, y, s, n_cu);
    case QT_GQ3_K: return launch_mv_q<QT_GQ3_K>(W, M, K, x, y, s, n_cu);
    case QT_GQ4_K: return launch_mv_q<QT_GQ4_K>(W, M, K, x, y, s, n_cu);
    case QT_GQ5_K: return launch_mv_q<QT_GQ5_K>(W, M, K, x, y, s, n_cu);
    case QT_GQ6_K: return launch_mv_q<QT_GQ6_K>(W, M, K, x, y, s, n_cu);
    default: return hipErrorInvalidValue;
    }
}

// Device expf evaluated over a buffer (test hook for the router's expf).
__global__ void k_expf(const float *__restrict__ in, float *__restrict__ out, long long n) {
    for (long long i = blockIdx.x * 256ll + threadIdx.x; i < n; i += (long long)gridDim.x * 256)
        out[i] = expf_glibc(in[i]);
}

__global__ __launch_bounds__(256) void k_add_rows(float *__restrict__ y, const float *__restrict__ part, int nparts,
                                                  int M) {
    for (int i = blockIdx.x * 256 + threadIdx.x; i < M; i += gridDim.x * 256) {
        float a = y[i];
        for (int p = 0; p < nparts; p++) a = a + part[(long long)p * M + i];
        y[i] = a;
    }
}

hipError_t launch_add_rows(float *y, const float *part, int nparts, int M, hipStream_t s) {
    const int blocks = (M + 255) / 256;
    hipLaunchKernelGGL(k_add_rows, dim3(blocks < 4096 ? blocks : 4096), dim3(256), 0, s, y, part, nparts, M);
    return hipGetLastError();
}

hipError_t launch_expf(const float *in, float *out, long long n, hipStream_t s) {
    long long blocks = (n + 255) / 256;
    int grid = (int)(blocks < 16384 ? blocks : 16384);
    if (grid < 1) grid = 1;
    hipLaunchKernelGGL(k_expf, dim3(grid), dim3(256), 0, s, in, out, n);
    return hipGetLastError();
}

}  // namespace tbq
