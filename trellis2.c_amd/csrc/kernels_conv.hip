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

// ---------------------------------------------------------------------------
// Compacted MFMA kernel (bf16 / fp16 storage).
//
// A block owns TM output rows x BN output channels.  Their fp32 sums live in
// LDS.  For each offset k the block compacts its rows that have a neighbour at
// k into a (src, dst) list (wavefront ballots, destination ascending), so the
// MFMA row dimension runs over valid pairs only: 16-pair row blocks are
// gathered straight into A fragments, multiplied by the k-th weight slice
// (staged through LDS and shared by the four wavefronts) and the 16 x BN
// partial results are added into the LDS sums of their destination rows.
// Within one offset a destination occurs at most once, so no two lanes touch
// the same LDS word; offsets are applied in k order, so the result is
// deterministic.  The tile's rows are written once at the end.
//
// Wavefront w covers channel half (w >> 1) and row blocks (w & 1), +2, +4, +6
// of each pass of eight row blocks.
// ---------------------------------------------------------------------------
template <int DT, int BN, int TM>
__global__ void __launch_bounds__(256) k_conv_mfma_compact(const typename Store<DT>::T * __restrict__ x,
                                                           const int32_t * __restrict__ nbr,
                                                           const uint32_t * __restrict__ mask,
                                                           const typename Store<DT>::T * __restrict__ w16,
                                                           const float * __restrict__ bias,
                                                           typename Store<DT>::T * __restrict__ y, int64_t n,
                                                           int ci, int co, int64_t n_col_tiles) {
    using T = typename Store<DT>::T;
    using V = typename Mfma<DT>::V;
    constexpr int ACC_LD = BN + 4;   // padded fp32 row stride of the LDS sums
    constexpr int BK = 32;           // input channels per K step
    constexpr int WN = BN / 2;       // channels per wavefront
    constexpr int NT = WN / 16;      // MFMA column tiles per wavefront
    constexpr int QB = 4;            // row blocks per wavefront per pass
    constexpr int ROWS_PER_THREAD = (TM + 255) / 256;
    __shared__ float s_acc[TM * ACC_LD];
    __shared__ int32_t s_src[TM];
    __shared__ int32_t s_dst[TM];
    __shared__ int32_t s_wcnt[4 * ROWS_PER_THREAD];
    __shared__ uint32_t s_need;

    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int rh = wave & 1, ch = wave >> 1;
    const int l16 = lane & 15, lg = lane >> 4;
    const int64_t logical = xcd_remap(blockIdx.x, (int64_t) gridDim.x);
    const int64_t row0 = (logical / n_col_tiles) * TM;
    const int col0 = (int) (logical % n_col_tiles) * BN;
    const int ci8 = ci >> 3;
    const uint64_t lt = lane == 0 ? 0ull : (~0ull >> (64 - lane));

    for (int i = t; i < TM * ACC_LD; i += 256) s_acc[i] = 0.0f;
    if (t == 0) s_need = 0u;
    uint32_t m[ROWS_PER_THREAD];
#pragma unroll
    for (int q = 0; q < ROWS_PER_THREAD; ++q) {
        const int local = q * 256 + t;
        const int64_t row = row0 + local;
        m[q] = (local < TM && row < n) ? mask[row] : 0u;
    }
    __syncthreads();
    {
        uint32_t any = 0;
#pragma unroll
        for (int q = 0; q < ROWS_PER_THREAD; ++q) any |= m[q];
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) any |= __shfl_xor(any, d);
        if (lane == 0) atomicOr(&s_need, any);
    }
    __syncthreads();
    const uint32_t need = s_need;

    for (int k = 0; k < 27; ++k) {
        if (((need >> k) & 1u) == 0) continue;
        // Compact this offset's pairs: destination-ascending (src, dst) list.
        int32_t rank[ROWS_PER_THREAD];
#pragma unroll
        for (int q = 0; q < ROWS_PER_THREAD; ++q) {
            const uint64_t bal = __ballot((m[q] >> k) & 1u);
            rank[q] = __popcll(bal & lt);
            if (lane == 0) s_wcnt[q * 4 + wave] = __popcll(bal);
        }
        __syncthreads();
        int c = 0;
#pragma unroll
        for (int q = 0; q < ROWS_PER_THREAD; ++q) {
            int base = c;
            for (int w = 0; w < 4; ++w) {
                base += w < wave ? s_wcnt[q * 4 + w] : 0;
                c += s_wcnt[q * 4 + w];
            }
            if ((m[q] >> k) & 1u) {
                const int local = q * 256 + t;
                s_src[base + rank[q]] = nbr[(row0 + local) * 27 + k];
                s_dst[base + rank[q]] = local;
            }
        }
        __syncthreads();
        const int nb = (c + 15) >> 4;
        const T * wk = w16 + (int64_t) k * ci8 * co * 8;
        for (int pb = 0; pb < nb; pb += 2 * QB) {
            f32x4 acc[QB][NT];
            int32_t src[QB];
            bool live[QB];
#pragma unroll
            for (int q = 0; q < QB; ++q) {
                const int j = pb + rh + 2 * q;
                live[q] = j < nb;
                const int p = j * 16 + l16;
                src[q] = (live[q] && p < c) ? s_src[p] : -1;
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) acc[q][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
            // Operand fragments for K step s, loaded one step ahead into two
            // register sets that alternate (no copies, so a wait only ever
            // covers older loads).  A: gathered source rows (padding slots read
            // row 0; their products are never added).  B: this wavefront's
            // weight columns, read from L2 (the packed weights are L2-resident).
            int64_t abase[QB];
#pragma unroll
            for (int q = 0; q < QB; ++q) abase[q] = (int64_t) (src[q] >= 0 ? src[q] : 0) * ci + lg * 8;
            const T * bbase = wk + ((int64_t) lg * co + col0 + ch * WN + l16) * 8;
            auto load = [&](int s, V * a, V * b) {
#pragma unroll
                for (int q = 0; q < QB; ++q) a[q] = *(const V *) (x + abase[q] + s * BK);
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) b[nt] = *(const V *) (bbase + ((int64_t) s * 4 * co + nt * 16) * 8);
            };
            const int ks = ci / BK;
            auto step = [&](int s, const V * a, const V * b, V * an, V * bn) {
                if (s + 1 < ks) load(s + 1, an, bn);
#pragma unroll
                for (int q = 0; q < QB; ++q) {
                    if (!live[q]) continue;
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt) acc[q][nt] = Mfma<DT>::mac(a[q], b[nt], acc[q][nt]);
                }
            };
            V a0[QB], a1[QB], b0[NT], b1[NT];
            load(0, a0, b0);
            int s = 0;
            for (; s + 1 < ks; s += 2) {
                step(s, a0, b0, a1, b1);
                step(s + 1, a1, b1, a0, b0);
            }
            if (s < ks) step(s, a0, b0, a1, b1);
            // Add the partial products into the destination rows' sums.
#pragma unroll
            for (int q = 0; q < QB; ++q) {
                if (!live[q]) continue;
                const int j = pb + rh + 2 * q;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int p = j * 16 + lg * 4 + i;
                    if (p < c) {
                        float * dst = s_acc + s_dst[p] * ACC_LD + ch * WN + l16;
#pragma unroll
                        for (int nt = 0; nt < NT; ++nt) atomicAdd(dst + nt * 16, acc[q][nt][i]);
                    }
                }
            }
        }
        __syncthreads();
    }
    // Epilogue: bias, round to the storage type, 16-byte coalesced stores.
    constexpr int CHUNKS = BN / 8;
    for (int e = t; e < TM * CHUNKS; e += 256) {
        const int r = e / CHUNKS, cc = (e % CHUNKS) * 8;
        const int64_t row = row0 + r;
        if (row >= n) continue;
        union {
            int4 v;
            T h[8];
        } o;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const float bv = bias != nullptr ? bias[col0 + cc + u] : 0.0f;
            float v = s_acc[r * ACC_LD + cc + u] + bv;
            if constexpr (DT == kBF16) {
                o.h[u] = f32_to_bf16(v);
            } else {
                o.h[u] = (T) v;
            }
        }
        *(int4 *) (y + row * co + col0 + cc) = o.v;
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

hipError_t launch_conv_mfma_compact(int dtype, const void * x, const int32_t * nbr, const uint32_t * mask,
                                    const void * w16, const float * bias, void * y, int64_t n, int ci, int co,
                                    hipStream_t s) {
    if (!conv_mfma_supported(dtype, ci, co)) {
        return hipErrorInvalidValue;
    }
    // Tile shapes (rows x channels): the LDS sums take TM*(BN+4)*4 bytes, so
    // 128x128 and 256x64 leave room for two blocks per CU, 256x128 and 512x64
    // for one.  TRELLIS_HIP_CONV_TILE=1..4 pins a shape for tuning; the shape
    // does not change the order of any sum.
    static const int forced = [] {
        const char * e = getenv("TRELLIS_HIP_CONV_TILE");
        return e != nullptr ? atoi(e) : 0;
    }();
    int shape = forced;
    if (shape < 1 || shape > 4 || ((shape == 1 || shape == 2) && co % 128 != 0)) {
        shape = co % 128 == 0 ? 2 : 3;
    }
    static const int kTm[5] = {0, 256, 128, 256, 512};
    static const int kBn[5] = {0, 128, 128, 64, 64};
    const int tm = kTm[shape], bn = kBn[shape];
    const int64_t row_tiles = (n + tm - 1) / tm;
    const int64_t col_tiles = co / bn;
    const int64_t grid = row_tiles * col_tiles;
    if (grid > 0x7fffffffLL) {
        return hipErrorInvalidValue;
    }
#define TSH_LAUNCH(DTV, TYPE, BNV, TMV)                                                                         \
    k_conv_mfma_compact<DTV, BNV, TMV><<<(unsigned) grid, 256, 0, s>>>((const TYPE *) x, nbr, mask,            \
                                                                        (const TYPE *) w16, bias, (TYPE *) y, n, \
                                                                        ci, co, col_tiles)
#define TSH_SHAPES(DTV, TYPE)                              \
    switch (shape) {                                       \
        case 1: TSH_LAUNCH(DTV, TYPE, 128, 256); break;    \
        case 2: TSH_LAUNCH(DTV, TYPE, 128, 128); break;    \
        case 3: TSH_LAUNCH(DTV, TYPE, 64, 256); break;     \
        default: TSH_LAUNCH(DTV, TYPE, 64, 512); break;    \
    }
    if (dtype == kBF16) {
        TSH_SHAPES(kBF16, uint16_t)
    } else {
        TSH_SHAPES(kF16, _Float16)
    }
#undef TSH_SHAPES
#undef TSH_LAUNCH
    return hipGetLastError();
}

}  // namespace tsh
