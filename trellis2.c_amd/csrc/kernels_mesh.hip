// kernels_mesh.hip - FlexiDualGrid mesh extraction from decoder logits.
//
// Reference semantics (src/ops/mesh/flex_dual_grid.c:166-313): one vertex per
// voxel, vertex = (coord + 2 sigmoid(f[a]) - 0.5) / res - 0.5 per axis a;
// weight softplus(f[6]); for voxel i in row order and axis a = 0, 1, 2 in
// order, when f[3+a] > 0 and the voxels at the quad's corners exist, two
// triangles split along the diagonal with the larger weight product.  Batch
// index 0 only, coordinates in [0, res), logits 0..6 finite, no repeated
// coordinate.
//
// Here the corner voxels come from the kernel map's neighbour table (every
// corner is at offset 0 or +1 per axis, so it is one of the 27 neighbours),
// a count pass and a scan give each voxel's first face, and a fill pass
// writes the faces in the reference's (voxel, axis) order.
#include "tsh_internal.h"

namespace tsh {
namespace {

// Neighbour-table offsets of the quad corners of each axis (k = (dx+1)*9 +
// (dy+1)*3 + (dz+1)); corner 0 is the voxel itself (k = 13).
__constant__ int kQuadK[3][4] = {
    {13, 14, 17, 16},  // x-face: (0,0,0) (0,0,1) (0,1,1) (0,1,0)
    {13, 22, 23, 14},  // y-face: (0,0,0) (1,0,0) (1,0,1) (0,0,1)
    {13, 16, 25, 22},  // z-face: (0,0,0) (0,1,0) (1,1,0) (1,0,0)
};

int grid_for(int64_t count, int block, int cap) {
    int64_t g = (count + block - 1) / block;
    if (g < 1) g = 1;
    if (g > cap) g = cap;
    return (int) g;
}

__device__ inline float fdg_sigmoid(float v) {
    if (v >= 0.0f) return 1.0f / (1.0f + expf(-v));
    const float e = expf(v);
    return e / (1.0f + e);
}

__device__ inline float fdg_softplus(float v) {
    if (v > 20.0f) return v;
    if (v < -20.0f) return expf(v);
    return log1pf(expf(v));
}

// flags[0] = 1 on a rejected row (batch != 0, coordinate outside [0, res),
// non-finite logit in channels 0..6).  Atomics only on that path.
template <int DT>
__global__ void k_fdg_check(const int32_t * __restrict__ coords, const typename Store<DT>::T * __restrict__ f,
                            int64_t n, int channels, int res, int32_t * __restrict__ flags) {
    for (int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t) gridDim.x * blockDim.x) {
        const int4 c = *(const int4 *) (coords + 4 * i);
        bool bad = c.x != 0 || c.y < 0 || c.y >= res || c.z < 0 || c.z >= res || c.w < 0 || c.w >= res;
#pragma unroll
        for (int ch = 0; ch < 7; ++ch) bad |= !isfinite(Store<DT>::ld(f, i * channels + ch));
        if (bad) atomicOr(&flags[0], 1);
    }
}

template <int DT>
__global__ void k_fdg_vertices(const int32_t * __restrict__ coords, const typename Store<DT>::T * __restrict__ f,
                               int64_t n, int channels, float inv_res, float * __restrict__ vert,
                               float * __restrict__ wgt) {
    for (int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t) gridDim.x * blockDim.x) {
        const int4 c = *(const int4 *) (coords + 4 * i);
        const int xyz[3] = {c.y, c.z, c.w};
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            const float local = 2.0f * fdg_sigmoid(Store<DT>::ld(f, i * channels + a)) - 0.5f;
            vert[i * 3 + a] = ((float) xyz[a] + local) * inv_res - 0.5f;
        }
        wgt[i] = fdg_softplus(Store<DT>::ld(f, i * channels + 6));
    }
}

template <int DT>
__device__ inline bool fdg_quad(const typename Store<DT>::T * f, const int32_t * nbr, int64_t i, int channels, int a,
                                int32_t q[4]) {
    if (!(Store<DT>::ld(f, i * channels + 3 + a) > 0.0f)) return false;
    bool ok = true;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        q[j] = nbr[i * 27 + kQuadK[a][j]];
        ok &= q[j] >= 0;
    }
    return ok;
}

template <int DT>
__global__ void k_fdg_count(const typename Store<DT>::T * __restrict__ f, const int32_t * __restrict__ nbr,
                            int64_t n, int channels, int32_t * __restrict__ counts) {
    for (int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t) gridDim.x * blockDim.x) {
        int cnt = 0;
        int32_t q[4];
#pragma unroll
        for (int a = 0; a < 3; ++a) cnt += fdg_quad<DT>(f, nbr, i, channels, a, q) ? 1 : 0;
        counts[i] = cnt;
    }
}

template <int DT>
__global__ void k_fdg_faces(const typename Store<DT>::T * __restrict__ f, const int32_t * __restrict__ nbr,
                            const float * __restrict__ wgt, const int32_t * __restrict__ first, int64_t n,
                            int channels, int32_t * __restrict__ faces) {
    for (int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t) gridDim.x * blockDim.x) {
        int64_t quad = first[i];
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            int32_t q[4];
            if (!fdg_quad<DT>(f, nbr, i, channels, a, q)) continue;
            const float w02 = wgt[q[0]] * wgt[q[2]], w13 = wgt[q[1]] * wgt[q[3]];
            int32_t * o = faces + quad * 6;
            if (w02 > w13) {
                o[0] = q[0]; o[1] = q[1]; o[2] = q[2];
                o[3] = q[0]; o[4] = q[2]; o[5] = q[3];
            } else {
                o[0] = q[0]; o[1] = q[1]; o[2] = q[3];
                o[3] = q[3]; o[4] = q[1]; o[5] = q[2];
            }
            ++quad;
        }
    }
}

template <int DT> struct FdgLaunch {
    using T = typename Store<DT>::T;
    static hipError_t check(const int32_t * coords, const void * f, int64_t n, int channels, int res, int32_t * flags,
                            hipStream_t s) {
        k_fdg_check<DT><<<grid_for(n, 256, 8192), 256, 0, s>>>(coords, (const T *) f, n, channels, res, flags);
        return hipGetLastError();
    }
    static hipError_t vertices(const int32_t * coords, const void * f, int64_t n, int channels, float inv_res,
                               float * vert, float * wgt, hipStream_t s) {
        k_fdg_vertices<DT><<<grid_for(n, 256, 8192), 256, 0, s>>>(coords, (const T *) f, n, channels, inv_res, vert,
                                                                  wgt);
        return hipGetLastError();
    }
    static hipError_t count(const void * f, const int32_t * nbr, int64_t n, int channels, int32_t * counts,
                            hipStream_t s) {
        k_fdg_count<DT><<<grid_for(n, 256, 8192), 256, 0, s>>>((const T *) f, nbr, n, channels, counts);
        return hipGetLastError();
    }
    static hipError_t faces(const void * f, const int32_t * nbr, const float * wgt, const int32_t * first, int64_t n,
                            int channels, int32_t * out, hipStream_t s) {
        k_fdg_faces<DT><<<grid_for(n, 256, 8192), 256, 0, s>>>((const T *) f, nbr, wgt, first, n, channels, out);
        return hipGetLastError();
    }
};

}  // namespace

hipError_t launch_fdg_check(int dtype, const int32_t * coords, const void * feats, int64_t n, int channels, int res,
                            int32_t * flags, hipStream_t s) {
    if (dtype == kF32) return FdgLaunch<kF32>::check(coords, feats, n, channels, res, flags, s);
    if (dtype == kF16) return FdgLaunch<kF16>::check(coords, feats, n, channels, res, flags, s);
    return FdgLaunch<kBF16>::check(coords, feats, n, channels, res, flags, s);
}

hipError_t launch_fdg_vertices(int dtype, const int32_t * coords, const void * feats, int64_t n, int channels, int res,
                               float * vert, float * wgt, hipStream_t s) {
    const float inv_res = 1.0f / (float) res;
    if (dtype == kF32) return FdgLaunch<kF32>::vertices(coords, feats, n, channels, inv_res, vert, wgt, s);
    if (dtype == kF16) return FdgLaunch<kF16>::vertices(coords, feats, n, channels, inv_res, vert, wgt, s);
    return FdgLaunch<kBF16>::vertices(coords, feats, n, channels, inv_res, vert, wgt, s);
}

hipError_t launch_fdg_count(int dtype, const void * feats, const int32_t * nbr, int64_t n, int channels,
                            int32_t * counts, hipStream_t s) {
    if (dtype == kF32) return FdgLaunch<kF32>::count(feats, nbr, n, channels, counts, s);
    if (dtype == kF16) return FdgLaunch<kF16>::count(feats, nbr, n, channels, counts, s);
    return FdgLaunch<kBF16>::count(feats, nbr, n, channels, counts, s);
}

hipError_t launch_fdg_faces(int dtype, const void * feats, const int32_t * nbr, const float * wgt,
                            const int32_t * first, int64_t n, int channels, int32_t * faces, hipStream_t s) {
    if (dtype == kF32) return FdgLaunch<kF32>::faces(feats, nbr, wgt, first, n, channels, faces, s);
    if (dtype == kF16) return FdgLaunch<kF16>::faces(feats, nbr, wgt, first, n, channels, faces, s);
    return FdgLaunch<kBF16>::faces(feats, nbr, wgt, first, n, channels, faces, s);
}

}  // namespace tsh
