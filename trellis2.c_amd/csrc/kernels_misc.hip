// kernels_misc.hip - subdivide, feature broadcast, norms and elementwise ops for gfx950.
//
// Reference semantics:
//   subdivide           src/architectures/sparse_unet_decoder/executor.c:108-154
//                       (child s kept iff logits[p][s] > 0; coord (b, 2x+(s&1), 2y+((s>>1)&1),
//                       2z+((s>>2)&1)); parent-major, s ascending)
//   c2s_gather          src/ops/sparse/trellis_sparse_cpu.c:385-409
//   skip_repeat         src/ops/sparse/trellis_sparse_cpu.c:411-440 (repeat = ceil(8*Co/Ci), clamp)
//   row_norm(_silu)     src/ops/sparse/trellis_sparse_cpu.c:173-232 (two-pass, population variance)
//   silu / add / linear src/ops/sparse/trellis_sparse_cpu.c:234-264, :122-171
// All arithmetic is fp32; storage is fp32, fp16 or bf16.
#include "tsh_internal.h"

namespace tsh {
namespace {

int blocks_for(int64_t count, int block, int cap = 65536) {
    int64_t g = (count + block - 1) / block;
    if (g < 1) g = 1;
    if (g > cap) g = cap;
    return (int) g;
}

#define TSH_GRID_STRIDE(i, count) \
    for (int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; i < (count); i += (int64_t) gridDim.x * blockDim.x)

template <int DT>
__global__ void k_from_f32(const float * __restrict__ src, typename Store<DT>::T * __restrict__ dst, int64_t count) {
    TSH_GRID_STRIDE(i, count) { Store<DT>::st_signed(dst, i, src[i]); }
}

template <int DT>
__global__ void k_to_f32(const typename Store<DT>::T * __restrict__ src, float * __restrict__ dst, int64_t count) {
    TSH_GRID_STRIDE(i, count) { dst[i] = Store<DT>::ld(src, i); }
}

template <int DT>
__global__ void k_silu(typename Store<DT>::T * __restrict__ x, int64_t count) {
    TSH_GRID_STRIDE(i, count) {
        const float v = Store<DT>::ld(x, i);
        Store<DT>::st(x, i, v / (1.0f + expf(-v)));
    }
}

template <int DT>
__global__ void k_add(const typename Store<DT>::T * __restrict__ a, const typename Store<DT>::T * __restrict__ b,
                      typename Store<DT>::T * __restrict__ y, int64_t count) {
    TSH_GRID_STRIDE(i, count) { Store<DT>::st(y, i, Store<DT>::ld(a, i) + Store<DT>::ld(b, i)); }
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d);
    return v;
}

// One wavefront per row: mean, then the sum of squared deviations, then the
// normalised (optionally affine, optionally SiLU) row.
template <int DT>
__global__ void __launch_bounds__(256) k_row_norm(const typename Store<DT>::T * __restrict__ x,
                                                  const float * __restrict__ gamma, const float * __restrict__ beta,
                                                  typename Store<DT>::T * __restrict__ y, int64_t n, int c, float eps,
                                                  int silu) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t) blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= n) return;
    const typename Store<DT>::T * xr = x + row * c;
    float s = 0.0f;
    for (int i = lane; i < c; i += 64) s += Store<DT>::ld(xr, i);
    const float mean = wave_sum(s) / (float) c;
    float q = 0.0f;
    for (int i = lane; i < c; i += 64) {
        const float d = Store<DT>::ld(xr, i) - mean;
        q += d * d;
    }
    const float inv = 1.0f / sqrtf(wave_sum(q) / (float) c + eps);
    typename Store<DT>::T * yr = y + row * c;
    for (int i = lane; i < c; i += 64) {
        float v = (Store<DT>::ld(xr, i) - mean) * inv;
        if (gamma != nullptr) v *= gamma[i];
        if (beta != nullptr) v += beta[i];
        if (silu) v = v / (1.0f + expf(-v));
        Store<DT>::st(yr, i, v);
    }
}

// Dense linear y = bias + x W^T with W^T given as fp32 [ci][co].  Tiled
// 32 rows x 64 outputs per block; each output accumulates from the bias in
// input-channel order without fused multiply-add, the reference order.
template <int DT>
__global__ void __launch_bounds__(256) k_linear(const typename Store<DT>::T * __restrict__ x,
                                                const float * __restrict__ wt, const float * __restrict__ bias,
                                                typename Store<DT>::T * __restrict__ y, int64_t n, int ci, int co,
                                                int silu) {
#pragma clang fp contract(off)
    constexpr int BM = 32, BN = 64, BK = 32;
    __shared__ float s_a[BM][BK + 1];
    __shared__ float s_b[BK][BN];
    const int t = threadIdx.x;
    const int tx = t & 15, ty = t >> 4;
    const int64_t row0 = (int64_t) blockIdx.x * BM;
    const int col0 = blockIdx.y * BN;
    float acc[2][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int col = col0 + tx * 4 + j;
        const float b = (bias != nullptr && col < co) ? bias[col] : 0.0f;
        acc[0][j] = b;
        acc[1][j] = b;
    }
    for (int c0 = 0; c0 < ci; c0 += BK) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int e = t + q * 256;
            const int r = e >> 5, c = e & 31;
            const int64_t row = row0 + r;
            s_a[r][c] = (row < n && c0 + c < ci) ? Store<DT>::ld(x, row * ci + c0 + c) : 0.0f;
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const int e = t + q * 256;
            const int c = e >> 6, o = e & 63;
            s_b[c][o] = (c0 + c < ci && col0 + o < co) ? wt[(int64_t) (c0 + c) * co + col0 + o] : 0.0f;
        }
        __syncthreads();
        const int kmax = (ci - c0) < BK ? (ci - c0) : BK;
        for (int c = 0; c < kmax; ++c) {
            const float a0 = s_a[ty * 2][c], a1 = s_a[ty * 2 + 1][c];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float b = s_b[c][tx * 4 + j];
                acc[0][j] = acc[0][j] + a0 * b;
                acc[1][j] = acc[1][j] + a1 * b;
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
            if (col >= co) continue;
            float v = acc[i][j];
            if (silu) v = v / (1.0f + expf(-v));
            Store<DT>::st_signed(y, r * co + col, v);
        }
    }
}

// Linear with few input channels (Ci <= kSmallK, Co % 8 == 0, Co <= kSmallKCo:
// the encoder's 6 -> 64 input layer): one thread per row and 8 output
// channels, the weights in LDS, one 16-byte store per thread (32 for fp32)
// instead of k_linear's 2-byte stores.  Each output is the bias, then each
// input channel's product added in order, without contraction, and stored
// as k_linear stores it: the outputs are bit-identical to k_linear's.
constexpr int kSmallK = 16;
constexpr int kSmallKCo = 256;

template <int DT>
__global__ void __launch_bounds__(256) k_linear_smallk(const typename Store<DT>::T * __restrict__ x,
                                                       const float * __restrict__ wt, const float * __restrict__ bias,
                                                       typename Store<DT>::T * __restrict__ y, int64_t n, int ci,
                                                       int co, int silu) {
#pragma clang fp contract(off)
    using T = typename Store<DT>::T;
    __shared__ float s_w[kSmallK * kSmallKCo];
    __shared__ float s_b[kSmallKCo];
    for (int e = threadIdx.x; e < ci * co; e += blockDim.x) s_w[e] = wt[e];
    for (int e = threadIdx.x; e < co; e += blockDim.x) s_b[e] = bias != nullptr ? bias[e] : 0.0f;
    __syncthreads();
    const int groups = co / 8;
    const int64_t total = n * groups;
    for (int64_t id = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; id < total;
         id += (int64_t) gridDim.x * blockDim.x) {
        const int64_t row = id / groups;
        const int col = (int) (id - row * groups) * 8;
        float acc[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = s_b[col + j];
        for (int c = 0; c < ci; ++c) {
            const float a = Store<DT>::ld(x, row * ci + c);
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[j] = acc[j] + a * s_w[c * co + col + j];
        }
        union {
            T h[8];
            int4 v[sizeof(T) / 2];
        } o;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            float v = acc[j];
            if (silu) v = v / (1.0f + expf(-v));
            Store<DT>::st_signed(o.h, j, v);
        }
        int4 * dst = (int4 *) (y + row * co + col);
#pragma unroll
        for (int k = 0; k < (int) (sizeof(T) / 2); ++k) dst[k] = o.v[k];
    }
}

template <int DT>
__global__ void k_c2s_count(const typename Store<DT>::T * __restrict__ logits, int64_t n,
                            int32_t * __restrict__ counts) {
    TSH_GRID_STRIDE(p, n) {
        int32_t c = 0;
#pragma unroll
        for (int s = 0; s < 8; ++s) c += Store<DT>::ld(logits, p * 8 + s) > 0.0f ? 1 : 0;
        counts[p] = c;
    }
}

// One lane per (parent, subidx) slot, 8 consecutive lanes per parent: a
// child's place is the parent's offset plus the number of earlier slots of
// the parent that have a child (a ballot over the lane's group of 8), so the
// children a wavefront writes are consecutive in all three outputs.  (One
// lane per parent wrote its children 64 bytes apart from its neighbours'.)
template <int DT>
__global__ void k_c2s_fill(const int4 * __restrict__ coords, const typename Store<DT>::T * __restrict__ logits,
                           const int32_t * __restrict__ offsets, int64_t n, int4 * __restrict__ out_coords,
                           int32_t * __restrict__ parent, int32_t * __restrict__ subidx) {
    const int64_t stride = (int64_t) gridDim.x * blockDim.x;  // a multiple of 64: groups of 8 stay aligned
    const int lane = (int) (threadIdx.x & 63);
    for (int64_t e = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; e < n * 8; e += stride) {
        const int64_t p = e >> 3;
        const int sidx = (int) (e & 7);
        const bool on = Store<DT>::ld(logits, e) > 0.0f;
        const uint32_t grp = (uint32_t) (__ballot(on) >> (lane & 56)) & 0xffu;
        if (on) {
            const int4 c = coords[p];
            const int64_t w = offsets[p] + __popc(grp & ((1u << sidx) - 1u));
            out_coords[w] = make_int4(c.x, 2 * c.y + (sidx & 1), 2 * c.z + ((sidx >> 1) & 1), 2 * c.w + ((sidx >> 2) & 1));
            parent[w] = (int32_t) p;
            subidx[w] = sidx;
        }
    }
}

// ---- exclusive scan (int32), three passes over 2048-element blocks ----------
constexpr int kScanBlock = 256;
constexpr int kScanPer = 8;
constexpr int kScanTile = kScanBlock * kScanPer;

__device__ __forceinline__ int32_t block_exclusive_scan(int32_t v, int32_t * s_wave, int32_t * total) {
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    int32_t incl = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int32_t o = __shfl_up(incl, d);
        if (lane >= d) incl += o;
    }
    if (lane == 63) s_wave[wave] = incl;
    __syncthreads();
    int32_t base = 0, sum = 0;
#pragma unroll
    for (int w = 0; w < kScanBlock / 64; ++w) {
        base += w < wave ? s_wave[w] : 0;
        sum += s_wave[w];
    }
    __syncthreads();
    *total = sum;
    return base + incl - v;
}

__global__ void __launch_bounds__(kScanBlock) k_scan_sums(const int32_t * __restrict__ in, int64_t n,
                                                          int32_t * __restrict__ sums) {
    __shared__ int32_t s_wave[kScanBlock / 64];
    const int64_t base = (int64_t) blockIdx.x * kScanTile + (int64_t) threadIdx.x * kScanPer;
    int32_t v = 0;
#pragma unroll
    for (int q = 0; q < kScanPer; ++q) v += base + q < n ? in[base + q] : 0;
    int32_t total;
    block_exclusive_scan(v, s_wave, &total);
    if (threadIdx.x == 0) sums[blockIdx.x] = total;
}

__global__ void __launch_bounds__(kScanBlock) k_scan_sums_scan(int32_t * __restrict__ sums, int64_t nb,
                                                               int32_t * __restrict__ total_dev) {
    __shared__ int32_t s_wave[kScanBlock / 64];
    int32_t carry = 0;
    for (int64_t b0 = 0; b0 < nb; b0 += kScanBlock) {
        const int64_t i = b0 + threadIdx.x;
        const int32_t v = i < nb ? sums[i] : 0;
        int32_t chunk;
        const int32_t ex = block_exclusive_scan(v, s_wave, &chunk);
        if (i < nb) sums[i] = carry + ex;
        carry += chunk;
    }
    if (threadIdx.x == 0) *total_dev = carry;
}

__global__ void __launch_bounds__(kScanBlock) k_scan_apply(const int32_t * __restrict__ in, int64_t n,
                                                           const int32_t * __restrict__ sums,
                                                           int32_t * __restrict__ out) {
    __shared__ int32_t s_wave[kScanBlock / 64];
    const int64_t base = (int64_t) blockIdx.x * kScanTile + (int64_t) threadIdx.x * kScanPer;
    int32_t vals[kScanPer];
    int32_t v = 0;
#pragma unroll
    for (int q = 0; q < kScanPer; ++q) {
        vals[q] = base + q < n ? in[base + q] : 0;
        v += vals[q];
    }
    int32_t total;
    int32_t run = sums[blockIdx.x] + block_exclusive_scan(v, s_wave, &total);
#pragma unroll
    for (int q = 0; q < kScanPer; ++q) {
        if (base + q < n) out[base + q] = run;
        run += vals[q];
    }
}

// ---- broadcasts ------------------------------------------------------------
template <int DT>
__global__ void k_c2s_gather(const typename Store<DT>::T * __restrict__ x, const int32_t * __restrict__ parent,
                             const int32_t * __restrict__ subidx, typename Store<DT>::T * __restrict__ y,
                             int64_t n_out, int co) {
    using T = typename Store<DT>::T;
    constexpr int kVec = 16 / (int) sizeof(T);
    if (co % kVec == 0) {
        const int vpr = co / kVec;
        TSH_GRID_STRIDE(e, n_out * vpr) {
            const int64_t r = e / vpr;
            const int v = (int) (e % vpr);
            const int64_t from = ((int64_t) parent[r] * 8 + subidx[r]) * co + (int64_t) v * kVec;
            *(int4 *) (y + r * co + (int64_t) v * kVec) = *(const int4 *) (x + from);
        }
    } else {
        TSH_GRID_STRIDE(e, n_out * co) {
            const int64_t r = e / co;
            const int c = (int) (e % co);
            y[e] = x[((int64_t) parent[r] * 8 + subidx[r]) * co + c];
        }
    }
}

constexpr int kIlp = 4;  // chunks per thread and pass in the vectorised broadcasts

// 16-byte chunks with 32-bit indexing, as k_skip_repeat_vec.
template <int DT>
__global__ void __launch_bounds__(256) k_c2s_gather_vec(const typename Store<DT>::T * __restrict__ x,
                                                        const int32_t * __restrict__ parent,
                                                        const int32_t * __restrict__ subidx,
                                                        typename Store<DT>::T * __restrict__ y, int n_out, int co,
                                                        int vpr, int vshift) {
    constexpr int kVec = 16 / (int) sizeof(typename Store<DT>::T);
    const int total = n_out * vpr;
    const int S = gridDim.x * blockDim.x;
    for (int e0 = blockIdx.x * blockDim.x + threadIdx.x; e0 < total; e0 += kIlp * S) {
        int r[kIlp], c0[kIlp];
        int64_t from[kIlp];
#pragma unroll
        for (int u = 0; u < kIlp; ++u) {
            const int e = e0 + u * S < total ? e0 + u * S : e0;
            r[u] = vshift >= 0 ? e >> vshift : e / vpr;
            c0[u] = (e - r[u] * vpr) * kVec;
        }
#pragma unroll
        for (int u = 0; u < kIlp; ++u) from[u] = ((int64_t) parent[r[u]] * 8 + subidx[r[u]]) * co + c0[u];
        int4 v[kIlp];
#pragma unroll
        for (int u = 0; u < kIlp; ++u) v[u] = *(const int4 *) (x + from[u]);
#pragma unroll
        for (int u = 0; u < kIlp; ++u) {
            if (e0 + u * S < total) *(int4 *) (y + (int64_t) r[u] * co + c0[u]) = v[u];
        }
    }
}

template <int DT>
__global__ void k_skip_repeat(const typename Store<DT>::T * __restrict__ x, const int32_t * __restrict__ parent,
                              const int32_t * __restrict__ subidx, typename Store<DT>::T * __restrict__ y,
                              int64_t n_out, int ci, int co, int repeat) {
    TSH_GRID_STRIDE(e, n_out * co) {
        const int64_t r = e / co;
        const int c = (int) (e % co);
        int from = (subidx[r] * co + c) / repeat;
        from = from < ci - 1 ? from : ci - 1;
        y[e] = x[(int64_t) parent[r] * ci + from];
    }
}

// 16-byte output chunks, 32-bit indexing (n_out * co / kVec + kIlp * grid <
// 2^31).  The chunks of a row are consecutive threads: row = e >> vshift when
// the chunk count per row is a power of two (vshift >= 0), else e / vpr.
// Each thread takes kIlp chunks a grid apart with their loads issued
// together, so a row lookup, its source load and the store overlap across
// them instead of running back to back.  kSingle: the repeat count is a
// multiple of the chunk width, so one source element fills the whole chunk
// (repeat-interleave of 8 or more); rshift >= 0: the repeat count is 2^rshift.
typedef int I32x4 __attribute__((ext_vector_type(4)));

template <int DT, bool kSingle>
__global__ void __launch_bounds__(256) k_skip_repeat_vec(const typename Store<DT>::T * __restrict__ x,
                                                         const int32_t * __restrict__ parent,
                                                         const int32_t * __restrict__ subidx,
                                                         typename Store<DT>::T * __restrict__ y, int n_out, int ci,
                                                         int co, int repeat, int rshift, int vpr, int vshift) {
    using T = typename Store<DT>::T;
    constexpr int kVec = 16 / (int) sizeof(T);
    const int total = n_out * vpr;
    const int S = gridDim.x * blockDim.x;
    union Chunk {
        int4 v;
        T e[kVec];
    };
    for (int e0 = blockIdx.x * blockDim.x + threadIdx.x; e0 < total; e0 += kIlp * S) {
        int r[kIlp], c0[kIlp];
#pragma unroll
        for (int u = 0; u < kIlp; ++u) {
            const int e = e0 + u * S < total ? e0 + u * S : e0;
            r[u] = vshift >= 0 ? e >> vshift : e / vpr;
            c0[u] = (e - r[u] * vpr) * kVec;
        }
        const T * xr[kIlp];
        int first[kIlp];
#pragma unroll
        for (int u = 0; u < kIlp; ++u) {
            xr[u] = x + (int64_t) parent[r[u]] * ci;
            first[u] = subidx[r[u]] * co + c0[u];
        }
        Chunk out[kIlp];
#pragma unroll
        for (int u = 0; u < kIlp; ++u) {
            int from = rshift >= 0 ? first[u] >> rshift : first[u] / repeat;
            if constexpr (kSingle) {
                from = from < ci - 1 ? from : ci - 1;
                const T v = xr[u][from];
#pragma unroll
                for (int q = 0; q < kVec; ++q) out[u].e[q] = v;
            } else {
                // One division per chunk; step the quotient/remainder across it.
                int rem = first[u] - from * repeat;
#pragma unroll
                for (int q = 0; q < kVec; ++q) {
                    out[u].e[q] = xr[u][from < ci - 1 ? from : ci - 1];
                    if (++rem == repeat) {
                        rem = 0;
                        ++from;
                    }
                }
            }
        }
#pragma unroll
        for (int u = 0; u < kIlp; ++u) {
            // Non-temporal: the broadcast rows are read back only by the next
            // kernel's gathers, from HBM either way (config 3: 647 MB), and
            // leaving them out of the caches shortened the conv that follows
            // (step 1.990 -> 1.976 ms).
            if (e0 + u * S < total) __builtin_nontemporal_store(__builtin_bit_cast(I32x4, out[u].v), (I32x4 *) (y + (int64_t) r[u] * co + c0[u]));
        }
    }
}

}  // namespace

hipError_t launch_convert_from_f32(int dtype, const float * src, void * dst, int64_t count, hipStream_t s) {
    if (count <= 0) return hipSuccess;
    const int g = blocks_for(count, 256, 16384);
    switch (dtype) {
        case kF32: return hipMemcpyAsync(dst, src, (size_t) count * 4, hipMemcpyDeviceToDevice, s);
        case kF16: k_from_f32<kF16><<<g, 256, 0, s>>>(src, (_Float16 *) dst, count); break;
        case kBF16: k_from_f32<kBF16><<<g, 256, 0, s>>>(src, (uint16_t *) dst, count); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_convert_to_f32(int dtype, const void * src, float * dst, int64_t count, hipStream_t s) {
    if (count <= 0) return hipSuccess;
    const int g = blocks_for(count, 256, 16384);
    switch (dtype) {
        case kF32: return hipMemcpyAsync(dst, src, (size_t) count * 4, hipMemcpyDeviceToDevice, s);
        case kF16: k_to_f32<kF16><<<g, 256, 0, s>>>((const _Float16 *) src, dst, count); break;
        case kBF16: k_to_f32<kBF16><<<g, 256, 0, s>>>((const uint16_t *) src, dst, count); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_silu(int dtype, void * x, int64_t count, hipStream_t s) {
    if (count <= 0) return hipSuccess;
    const int g = blocks_for(count, 256, 16384);
    switch (dtype) {
        case kF32: k_silu<kF32><<<g, 256, 0, s>>>((float *) x, count); break;
        case kF16: k_silu<kF16><<<g, 256, 0, s>>>((_Float16 *) x, count); break;
        case kBF16: k_silu<kBF16><<<g, 256, 0, s>>>((uint16_t *) x, count); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_add(int dtype, const void * a, const void * b, void * y, int64_t count, hipStream_t s) {
    if (count <= 0) return hipSuccess;
    const int g = blocks_for(count, 256, 16384);
    switch (dtype) {
        case kF32: k_add<kF32><<<g, 256, 0, s>>>((const float *) a, (const float *) b, (float *) y, count); break;
        case kF16:
            k_add<kF16><<<g, 256, 0, s>>>((const _Float16 *) a, (const _Float16 *) b, (_Float16 *) y, count);
            break;
        case kBF16:
            k_add<kBF16><<<g, 256, 0, s>>>((const uint16_t *) a, (const uint16_t *) b, (uint16_t *) y, count);
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

namespace {
// 16-bit storage, C = 8 * LPR * CPL: LPR lanes per row, each holding CPL
// 16-byte chunks, so a row is read once into registers, reduced with
// shuffles inside its lane segment (mean, then squared deviations), and
// written back in 16-byte chunks; 64 / LPR rows per wavefront.  SiLU uses the
// hardware exp2 / reciprocal (about 1 ulp each, far inside the 16-bit
// rounding).
template <int DT, int LPR, int CPL>
__global__ void __launch_bounds__(256) k_row_norm_vec(const typename Store<DT>::T * __restrict__ x,
                                                      const float * __restrict__ gamma,
                                                      const float * __restrict__ beta,
                                                      typename Store<DT>::T * __restrict__ y, int64_t n, float eps,
                                                      int silu) {
    using T = typename Store<DT>::T;
    constexpr int C = 8 * LPR * CPL;
    const int lane = threadIdx.x & 63;
    const int li = lane % LPR;
    const int64_t row = ((int64_t) blockIdx.x * 4 + (threadIdx.x >> 6)) * (64 / LPR) + lane / LPR;
    const bool ok = row < n;
    union Chunk {
        int4 v;
        T h[8];
    };
    float v[CPL][8];
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        Chunk ch;
        ch.v = ok ? *(const int4 *) (x + row * C + (li + j * LPR) * 8) : int4{0, 0, 0, 0};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            v[j][e] = Store<DT>::ld(ch.h, e);
            s += v[j][e];
        }
    }
#pragma unroll
    for (int d = LPR / 2; d >= 1; d >>= 1) s += __shfl_xor(s, d);
    const float mean = s / (float) C;
    float q = 0.0f;
#pragma unroll
    for (int j = 0; j < CPL; ++j)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float d = v[j][e] - mean;
            q += d * d;
        }
#pragma unroll
    for (int d = LPR / 2; d >= 1; d >>= 1) q += __shfl_xor(q, d);
    const float inv = 1.0f / sqrtf(q / (float) C + eps);
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int c0 = (li + j * LPR) * 8;
        // The chunk's 8 scale and shift values as two 16-byte loads each.
        float gv[8], bv[8];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const float4 g4 = gamma != nullptr ? *(const float4 *) (gamma + c0 + 4 * h) : float4{1.f, 1.f, 1.f, 1.f};
            const float4 b4 = beta != nullptr ? *(const float4 *) (beta + c0 + 4 * h) : float4{0.f, 0.f, 0.f, 0.f};
            gv[4 * h] = g4.x, gv[4 * h + 1] = g4.y, gv[4 * h + 2] = g4.z, gv[4 * h + 3] = g4.w;
            bv[4 * h] = b4.x, bv[4 * h + 1] = b4.y, bv[4 * h + 2] = b4.z, bv[4 * h + 3] = b4.w;
        }
        Chunk ch;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float o = (v[j][e] - mean) * inv;
            if (gamma != nullptr) o *= gv[e];
            if (beta != nullptr) o += bv[e];
            if (silu) o = o * __builtin_amdgcn_rcpf(1.0f + __expf(-o));
            Store<DT>::st(ch.h, e, o);
        }
        if (ok) *(int4 *) (y + row * C + c0) = ch.v;
    }
}

template <int DT, int LPR, int CPL>
hipError_t launch_row_norm_vec(const void * x, const float * gamma, const float * beta, void * y, int64_t n,
                               float eps, int silu, hipStream_t s) {
    using T = typename Store<DT>::T;
    constexpr int64_t rows_per_block = 4 * (64 / LPR);
    const int64_t g = (n + rows_per_block - 1) / rows_per_block;
    k_row_norm_vec<DT, LPR, CPL><<<(unsigned) g, 256, 0, s>>>((const T *) x, gamma, beta, (T *) y, n, eps, silu);
    return hipGetLastError();
}

template <int DT>
hipError_t launch_row_norm_vec_dt(const void * x, const float * gamma, const float * beta, void * y, int64_t n, int c,
                                  float eps, int silu, hipStream_t s) {
    switch (c) {
        case 64: return launch_row_norm_vec<DT, 8, 1>(x, gamma, beta, y, n, eps, silu, s);
        case 128: return launch_row_norm_vec<DT, 16, 1>(x, gamma, beta, y, n, eps, silu, s);
        case 256: return launch_row_norm_vec<DT, 32, 1>(x, gamma, beta, y, n, eps, silu, s);
        case 512: return launch_row_norm_vec<DT, 64, 1>(x, gamma, beta, y, n, eps, silu, s);
        case 1024: return launch_row_norm_vec<DT, 64, 2>(x, gamma, beta, y, n, eps, silu, s);
        case 2048: return launch_row_norm_vec<DT, 64, 4>(x, gamma, beta, y, n, eps, silu, s);
        default: return hipErrorInvalidValue;
    }
}
}  // namespace

hipError_t launch_row_norm(int dtype, const void * x, const float * gamma, const float * beta, void * y, int64_t n,
                           int c, float eps, int silu, hipStream_t s) {
    // 16-bit storage at the decoder's power-of-two widths: vectorised rows.
    if (dtype != kF32 && (c == 64 || c == 128 || c == 256 || c == 512 || c == 1024 || c == 2048)) {
        return dtype == kBF16 ? launch_row_norm_vec_dt<kBF16>(x, gamma, beta, y, n, c, eps, silu, s)
                              : launch_row_norm_vec_dt<kF16>(x, gamma, beta, y, n, c, eps, silu, s);
    }
    const int64_t g = (n + 3) / 4;
    switch (dtype) {
        case kF32:
            k_row_norm<kF32><<<(unsigned) g, 256, 0, s>>>((const float *) x, gamma, beta, (float *) y, n, c, eps, silu);
            break;
        case kF16:
            k_row_norm<kF16><<<(unsigned) g, 256, 0, s>>>((const _Float16 *) x, gamma, beta, (_Float16 *) y, n, c, eps,
                                                          silu);
            break;
        case kBF16:
            k_row_norm<kBF16><<<(unsigned) g, 256, 0, s>>>((const uint16_t *) x, gamma, beta, (uint16_t *) y, n, c, eps,
                                                           silu);
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_linear(int dtype, const void * x, const float * wt, const float * bias, void * y, int64_t n, int ci,
                         int co, int silu, hipStream_t s) {
    if (ci <= kSmallK && co % 8 == 0 && co <= kSmallKCo) {
        const int g = blocks_for(n * (co / 8), 256, 16384);
        switch (dtype) {
            case kF32:
                k_linear_smallk<kF32><<<g, 256, 0, s>>>((const float *) x, wt, bias, (float *) y, n, ci, co, silu);
                break;
            case kF16:
                k_linear_smallk<kF16><<<g, 256, 0, s>>>((const _Float16 *) x, wt, bias, (_Float16 *) y, n, ci, co,
                                                        silu);
                break;
            case kBF16:
                k_linear_smallk<kBF16><<<g, 256, 0, s>>>((const uint16_t *) x, wt, bias, (uint16_t *) y, n, ci, co,
                                                         silu);
                break;
            default: return hipErrorInvalidValue;
        }
        return hipGetLastError();
    }
    const dim3 grid((unsigned) ((n + 31) / 32), (unsigned) ((co + 63) / 64));
    switch (dtype) {
        case kF32: k_linear<kF32><<<grid, 256, 0, s>>>((const float *) x, wt, bias, (float *) y, n, ci, co, silu); break;
        case kF16:
            k_linear<kF16><<<grid, 256, 0, s>>>((const _Float16 *) x, wt, bias, (_Float16 *) y, n, ci, co, silu);
            break;
        case kBF16:
            k_linear<kBF16><<<grid, 256, 0, s>>>((const uint16_t *) x, wt, bias, (uint16_t *) y, n, ci, co, silu);
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_c2s_count(int dtype, const void * logits, int64_t n, int32_t * counts, hipStream_t s) {
    const int g = blocks_for(n, 256, 16384);
    switch (dtype) {
        case kF32: k_c2s_count<kF32><<<g, 256, 0, s>>>((const float *) logits, n, counts); break;
        case kF16: k_c2s_count<kF16><<<g, 256, 0, s>>>((const _Float16 *) logits, n, counts); break;
        case kBF16: k_c2s_count<kBF16><<<g, 256, 0, s>>>((const uint16_t *) logits, n, counts); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

size_t scan_tmp_bytes(int64_t n) {
    const int64_t nb = (n + kScanTile - 1) / kScanTile;
    return (size_t) (nb + 1) * sizeof(int32_t);
}

hipError_t launch_scan_exclusive(const int32_t * in, int32_t * out, int64_t n, int32_t * total_dev, void * tmp,
                                 hipStream_t s) {
    if (n <= 0) return hipErrorInvalidValue;
    const int64_t nb = (n + kScanTile - 1) / kScanTile;
    int32_t * sums = (int32_t *) tmp;
    k_scan_sums<<<(unsigned) nb, kScanBlock, 0, s>>>(in, n, sums);
    k_scan_sums_scan<<<1, kScanBlock, 0, s>>>(sums, nb, total_dev);
    k_scan_apply<<<(unsigned) nb, kScanBlock, 0, s>>>(in, n, sums, out);
    return hipGetLastError();
}

hipError_t launch_c2s_fill(int dtype, const int32_t * coords, const void * logits, const int32_t * offsets, int64_t n,
                           int32_t * out_coords, int32_t * parent, int32_t * subidx, hipStream_t s) {
    const int g = blocks_for(n * 8, 256, 16384);
    const int4 * c = (const int4 *) coords;
    int4 * oc = (int4 *) out_coords;
    switch (dtype) {
        case kF32: k_c2s_fill<kF32><<<g, 256, 0, s>>>(c, (const float *) logits, offsets, n, oc, parent, subidx); break;
        case kF16:
            k_c2s_fill<kF16><<<g, 256, 0, s>>>(c, (const _Float16 *) logits, offsets, n, oc, parent, subidx);
            break;
        case kBF16:
            k_c2s_fill<kBF16><<<g, 256, 0, s>>>(c, (const uint16_t *) logits, offsets, n, oc, parent, subidx);
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_c2s_gather(int dtype, const void * x, const int32_t * parent, const int32_t * subidx, void * y,
                             int64_t n_out, int co, hipStream_t s) {
    const int kvec = 16 / (int) dtype_bytes(dtype);
    if (co % kvec == 0 && n_out * (co / kvec) < (int64_t) INT32_MAX - (int64_t) kIlp * 65536 * 256) {
        const int vpr = co / kvec;
        int vshift = -1;
        for (int b = 0; b < 30; ++b) {
            if ((1 << b) == vpr) vshift = b;
        }
        const int gv = blocks_for((n_out * vpr + kIlp - 1) / kIlp, 256, 65536);
        switch (dtype) {
            case kF32:
                k_c2s_gather_vec<kF32><<<gv, 256, 0, s>>>((const float *) x, parent, subidx, (float *) y, (int) n_out,
                                                          co, vpr, vshift);
                break;
            case kF16:
                k_c2s_gather_vec<kF16><<<gv, 256, 0, s>>>((const _Float16 *) x, parent, subidx, (_Float16 *) y,
                                                          (int) n_out, co, vpr, vshift);
                break;
            case kBF16:
                k_c2s_gather_vec<kBF16><<<gv, 256, 0, s>>>((const uint16_t *) x, parent, subidx, (uint16_t *) y,
                                                           (int) n_out, co, vpr, vshift);
                break;
            default: return hipErrorInvalidValue;
        }
        return hipGetLastError();
    }
    const int g = blocks_for(n_out * co / 4 + 1, 256, 32768);
    switch (dtype) {
        case kF32: k_c2s_gather<kF32><<<g, 256, 0, s>>>((const float *) x, parent, subidx, (float *) y, n_out, co); break;
        case kF16:
            k_c2s_gather<kF16><<<g, 256, 0, s>>>((const _Float16 *) x, parent, subidx, (_Float16 *) y, n_out, co);
            break;
        case kBF16:
            k_c2s_gather<kBF16><<<g, 256, 0, s>>>((const uint16_t *) x, parent, subidx, (uint16_t *) y, n_out, co);
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_skip_repeat(int dtype, const void * x, const int32_t * parent, const int32_t * subidx, void * y,
                              int64_t n_out, int ci, int co, hipStream_t s) {
    const int repeat = (8 * co + ci - 1) / ci;
    const int kvec = 16 / (int) dtype_bytes(dtype);
    if (co % kvec == 0 && n_out * (co / kvec) < (int64_t) INT32_MAX - (int64_t) kIlp * 65536 * 256) {
        const int vpr = co / kvec;
        int vshift = -1, rshift = -1;
        for (int b = 0; b < 30; ++b) {
            if ((1 << b) == vpr) vshift = b;
            if ((1 << b) == repeat) rshift = b;
        }
        const int g = blocks_for((n_out * vpr + kIlp - 1) / kIlp, 256, 65536);
        const bool single = repeat % kvec == 0;
#define TSH_SR(DTV, TYPE)                                                                                       \
    do {                                                                                                        \
        if (single) {                                                                                           \
            k_skip_repeat_vec<DTV, true><<<g, 256, 0, s>>>((const TYPE *) x, parent, subidx, (TYPE *) y,         \
                                                           (int) n_out, ci, co, repeat, rshift, vpr, vshift);    \
        } else {                                                                                                \
            k_skip_repeat_vec<DTV, false><<<g, 256, 0, s>>>((const TYPE *) x, parent, subidx, (TYPE *) y,        \
                                                            (int) n_out, ci, co, repeat, rshift, vpr, vshift);   \
        }                                                                                                       \
    } while (0)
        switch (dtype) {
            case kF32: TSH_SR(kF32, float); break;
            case kF16: TSH_SR(kF16, _Float16); break;
            case kBF16: TSH_SR(kBF16, uint16_t); break;
            default: return hipErrorInvalidValue;
        }
#undef TSH_SR
        return hipGetLastError();
    }
    const int g = blocks_for(n_out * co, 256, 32768);
    switch (dtype) {
        case kF32:
            k_skip_repeat<kF32><<<g, 256, 0, s>>>((const float *) x, parent, subidx, (float *) y, n_out, ci, co, repeat);
            break;
        case kF16:
            k_skip_repeat<kF16><<<g, 256, 0, s>>>((const _Float16 *) x, parent, subidx, (_Float16 *) y, n_out, ci, co,
                                                  repeat);
            break;
        case kBF16:
            k_skip_repeat<kBF16><<<g, 256, 0, s>>>((const uint16_t *) x, parent, subidx, (uint16_t *) y, n_out, ci, co,
                                                   repeat);
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace tsh
