// kernels_conv.hip - 3x3x3 submanifold sparse convolution for gfx950.
//
// out[i][o] = bias[o] + sum_k sum_c x[nbr[i][k]][c] * W[o][k][c]
// (src/ops/sparse/trellis_sparse_cpu.c:324-373; weight [Co][27][Ci], :361).
//
// Two output-stationary schedules, both writing every output row exactly once
// (no scatter, no atomics, deterministic):
//
//  * generic  - VALU, any channel counts, any storage type.  For each output
//               it follows the reference's operation order exactly: start at
//               the bias, then per valid offset in k order a sequentially
//               rounded fp32 dot product (no fused multiply-add) added to the
//               row.  With fp32 storage the result is bit-identical to the
//               reference CPU backend.
//  * mfma     - bf16/fp16 storage, Ci % 32 == 0, Co % 64 == 0.  Implicit GEMM
//               on v_mfma_f32_16x16x32_{bf16,f16} with fp32 accumulation.  A
//               block owns 64 output rows x 64/128 output channels; each
//               wavefront owns 32 rows x 32/64 channels.  For each offset the
//               lanes gather their source rows straight into MFMA A fragments
//               (16 contiguous bytes per lane) and read pre-packed weight
//               fragments; row groups of 16 with no valid neighbour skip the
//               offset.
#include "tsh_internal.h"

namespace tsh {
namespace {

// Maps a linear block id onto a logical tile so that each of the 8 XCDs
// (which receive block ids round-robin) works on one contiguous range of
// tiles and its L2 sees neighbouring gathers.
__device__ __forceinline__ int64_t xcd_remap(int64_t bid, int64_t grid) {
    constexpr int64_t kXcd = 8;
    const int64_t q = grid / kXcd, r = grid % kXcd;
    const int64_t xcd = bid % kXcd, slot = bid / kXcd;
    return xcd < r ? xcd * (q + 1) + slot : r * (q + 1) + (xcd - r) * q + slot;
}

// ---------------------------------------------------------------------------
// Generic VALU kernel: 32 rows x 64 channels per 256-lane block.
// ---------------------------------------------------------------------------
template <int DT>
__global__ void __launch_bounds__(256) k_conv_generic(const typename Store<DT>::T * __restrict__ x,
                                                      const int32_t * __restrict__ nbr,
                                                      const float * __restrict__ w32,
                                                      const float * __restrict__ bias,
                                                      typename Store<DT>::T * __restrict__ y, int64_t n, int ci,
                                                      int co) {
#pragma clang fp contract(off)
    constexpr int BM = 32, BN = 64, BK = 32;
    __shared__ float s_a[BM][BK + 1];
    __shared__ float s_b[BK][BN];
    __shared__ int32_t s_src[BM];
    const int t = threadIdx.x;
    const int tx = t & 15, ty = t >> 4;
    const int64_t row0 = (int64_t) blockIdx.x * BM;
    const int col0 = blockIdx.y * BN;
    float acc[2][4];
    float part[2][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int col = col0 + tx * 4 + j;
        const float b = (bias != nullptr && col < co) ? bias[col] : 0.0f;
        acc[0][j] = b;
        acc[1][j] = b;
    }
    for (int k = 0; k < 27; ++k) {
        if (t < BM) {
            const int64_t r = row0 + t;
            s_src[t] = r < n ? nbr[r * 27 + k] : -1;
        }
        __syncthreads();
        const bool any = __syncthreads_or(t < BM && s_src[t] >= 0);
        if (!any) {
            continue;
        }
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) part[i][j] = 0.0f;
        for (int c0 = 0; c0 < ci; c0 += BK) {
            // A: 32 rows x 32 channels, 4 per lane.
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int e = t + q * 256;
                const int r = e >> 5, c = e & 31;
                const int32_t src = s_src[r];
                float v = 0.0f;
                if (src >= 0 && c0 + c < ci) {
                    v = Store<DT>::ld(x, (int64_t) src * ci + c0 + c);
                }
                s_a[r][c] = v;
            }
            // B: 32 channels x 64 outputs, 8 per lane.
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const int e = t + q * 256;
                const int c = e >> 6, o = e & 63;
                float v = 0.0f;
                if (c0 + c < ci && col0 + o < co) {
                    v = w32[((int64_t) k * ci + c0 + c) * co + col0 + o];
                }
                s_b[c][o] = v;
            }
            __syncthreads();
            const int kmax = (ci - c0) < BK ? (ci - c0) : BK;
            for (int c = 0; c < kmax; ++c) {
                const float a0 = s_a[ty * 2][c], a1 = s_a[ty * 2 + 1][c];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float b = s_b[c][tx * 4 + j];
                    part[0][j] = part[0][j] + a0 * b;
                    part[1][j] = part[1][j] + a1 * b;
                }
            }
            __syncthreads();
        }
        // Rows without a neighbour at k keep their sum untouched (the
        // reference skips the offset, it does not add a zero).
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            if (s_src[ty * 2 + i] >= 0) {
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = acc[i][j] + part[i][j];
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int64_t r = row0 + ty * 2 + i;
        if (r >= n) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int col = col0 + tx * 4 + j;
            if (col < co) Store<DT>::st(y, r * co + col, acc[i][j]);
        }
    }
}

// ---------------------------------------------------------------------------
// MFMA kernel (bf16 / fp16 storage).
// ---------------------------------------------------------------------------
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

template <int DT> struct Mfma;
template <> struct Mfma<kBF16> {
    typedef bf16x8 V;
    __device__ static f32x4 mac(V a, V b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0); }
};
template <> struct Mfma<kF16> {
    typedef f16x8 V;
    __device__ static f32x4 mac(V a, V b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
};

// Lane layout of v_mfma_f32_16x16x32 (64 lanes): A fragment = row (lane%16),
// 8 consecutive K values starting at 8*(lane/16); B fragment = column
// (lane%16), the same 8 K values; D = rows 4*(lane/16)+i, column lane%16.
// Any consistent K permutation of A and B gives the same product, so only
// the row/column mapping matters for correctness.
template <int DT, int BN>
__global__ void __launch_bounds__(256) k_conv_mfma_masked(const typename Store<DT>::T * __restrict__ x,
                                                          const int32_t * __restrict__ nbr,
                                                          const uint32_t * __restrict__ mask,
                                                          const typename Store<DT>::T * __restrict__ w16,
                                                          const float * __restrict__ bias,
                                                          typename Store<DT>::T * __restrict__ y, int64_t n, int ci,
                                                          int co, int64_t n_col_tiles) {
    using V = typename Mfma<DT>::V;
    constexpr int BM = 64;
    constexpr int WN = BN / 2;      // channels per wavefront
    constexpr int NT = WN / 16;     // 16-wide MFMA column tiles per wavefront
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int wr = wave & 1, wc = wave >> 1;
    const int64_t grid = (int64_t) gridDim.x;
    const int64_t logical = xcd_remap(blockIdx.x, grid);
    const int64_t row_tile = logical / n_col_tiles;
    const int col_tile = (int) (logical % n_col_tiles);
    const int64_t row0 = row_tile * BM + wr * 32;
    const int colw = col_tile * BN + wc * WN;
    const int l16 = lane & 15, lg = lane >> 4;
    const int ci8 = ci >> 3;

    f32x4 acc[2][NT];
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[m][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    int64_t arow[2];
    uint32_t amask[2];
#pragma unroll
    for (int m = 0; m < 2; ++m) {
        arow[m] = row0 + m * 16 + l16;
        amask[m] = arow[m] < n ? mask[arow[m]] : 0u;
    }
    // Offsets any of this wavefront's rows need.
    uint32_t need = amask[0] | amask[1];
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) need |= __shfl_xor(need, d);

    const V zero = V{};
    for (int k = 0; k < 27; ++k) {
        if (((need >> k) & 1u) == 0) {
            continue;
        }
        int32_t src[2];
        bool live[2];
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            src[m] = ((amask[m] >> k) & 1u) ? nbr[arow[m] * 27 + k] : -1;
            live[m] = __ballot(src[m] >= 0) != 0;
        }
        const typename Store<DT>::T * wk = w16 + (int64_t) k * ci8 * co * 8;
        for (int c0 = 0; c0 < ci; c0 += 32) {
            V a[2];
#pragma unroll
            for (int m = 0; m < 2; ++m) {
                a[m] = src[m] >= 0 ? *(const V *) (x + (int64_t) src[m] * ci + c0 + lg * 8) : zero;
            }
            const int g = (c0 >> 3) + lg;
            V b[NT];
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                b[j] = *(const V *) (wk + ((int64_t) g * co + colw + j * 16 + l16) * 8);
            }
#pragma unroll
            for (int m = 0; m < 2; ++m) {
                if (!live[m]) continue;
#pragma unroll
                for (int j = 0; j < NT; ++j) acc[m][j] = Mfma<DT>::mac(a[m], b[j], acc[m][j]);
            }
        }
    }
    // Epilogue: bias, round to storage, store.
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        const int col = colw + j * 16 + l16;
        const float bv = bias != nullptr ? bias[col] : 0.0f;
#pragma unroll
        for (int m = 0; m < 2; ++m) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int64_t r = row0 + m * 16 + lg * 4 + i;
                if (r < n) Store<DT>::st(y, r * co + col, acc[m][j][i] + bv);
            }
        }
    }
}

}  // namespace

hipError_t launch_conv_generic(int dtype, const void * x, const int32_t * nbr, const float * w32, const float * bias,
                               void * y, int64_t n, int ci, int co, hipStream_t s) {
    const dim3 grid((unsigned) ((n + 31) / 32), (unsigned) ((co + 63) / 64));
    switch (dtype) {
        case kF32:
            k_conv_generic<kF32><<<grid, 256, 0, s>>>((const float *) x, nbr, w32, bias, (float *) y, n, ci, co);
            break;
        case kF16:
            k_conv_generic<kF16><<<grid, 256, 0, s>>>((const _Float16 *) x, nbr, w32, bias, (_Float16 *) y, n, ci,
                                                      co);
            break;
        case kBF16:
            k_conv_generic<kBF16><<<grid, 256, 0, s>>>((const uint16_t *) x, nbr, w32, bias, (uint16_t *) y, n, ci,
                                                       co);
            break;
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

bool conv_mfma_supported(int dtype, int ci, int co) {
    return (dtype == kF16 || dtype == kBF16) && ci > 0 && co > 0 && ci % 32 == 0 && co % 64 == 0;
}

hipError_t launch_conv_mfma_masked(int dtype, const void * x, const int32_t * nbr, const uint32_t * mask,
                                   const void * w16, const float * bias, void * y, int64_t n, int ci, int co,
                                   hipStream_t s) {
    if (!conv_mfma_supported(dtype, ci, co)) {
        return hipErrorInvalidValue;
    }
    const int bn = (co % 128 == 0) ? 128 : 64;
    const int64_t row_tiles = (n + 63) / 64;
    const int64_t col_tiles = co / bn;
    const int64_t grid = row_tiles * col_tiles;
    if (grid > 0x7fffffffLL) {
        return hipErrorInvalidValue;
    }
#define TSH_LAUNCH(DTV, TYPE, BNV)                                                                           \
    k_conv_mfma_masked<DTV, BNV><<<(unsigned) grid, 256, 0, s>>>((const TYPE *) x, nbr, mask,               \
                                                                  (const TYPE *) w16, bias, (TYPE *) y, n, ci, \
                                                                  co, col_tiles)
    if (dtype == kBF16) {
        if (bn == 128) TSH_LAUNCH(kBF16, uint16_t, 128);
        else TSH_LAUNCH(kBF16, uint16_t, 64);
    } else {
        if (bn == 128) TSH_LAUNCH(kF16, _Float16, 128);
        else TSH_LAUNCH(kF16, _Float16, 64);
    }
#undef TSH_LAUNCH
    return hipGetLastError();
}

}  // namespace tsh
