// kernels_s2c.hip - the encoder's spatial-to-channel downsample (S2C) on the device.
//
// Reference semantics:
//   S2C map   src/architectures/sparse_unet_encoder/s2c_host.c:33-120: the coarse
//             voxel of fine voxel (b, x, y, z) is (b, x/2, y/2, z/2), its child slot
//             subidx = (x&1) | (y&1)<<1 | (z&1)<<2; the distinct coarse voxels in
//             ascending (b, x, y, z) order; parent[f] = coarse row.  Negative
//             coordinates are rejected; two fine voxels in one child slot are a
//             parse error.
//   pack      sparse_unet_encoder/executor.c:279-286: packed[parent][subidx*pc + c]
//             = x[f][c], pc = co/8, zero where a coarse voxel lacks that child.
//   skip mean executor.c:287-292: skip[parent][(subidx*ci + c)/g] += x[f][c]/g,
//             g = 8ci/co, fp32, channels in ascending order from zero.
//
// The reference sorts on the host (qsort of the n records by coarse voxel,
// then fine row).  Here the order comes from a least-significant-digit radix
// sort of a key holding the coarse voxel in just the bits its coordinates use
// (b highest, then x/2, y/2, z/2, each field as wide as its largest value)
// above the child slot in the lowest 3 bits; at most 127 bits, in two words;
// the fine row is the payload.  The passes cover the coarse-voxel bits only
// (digits from bit 3): the slot bits ride along unsorted, so within one
// coarse voxel the rows keep their input order, as in the reference, and the
// config-3 children's 27-bit key takes 3 passes instead of 4.  Nothing the
// map records depends on that order (parent, subidx and the child table are
// slot-indexed).  A repeated fine voxel (two rows in one child slot) is found
// by each row comparing its whole key with the up to 8 rows before it in its
// coarse voxel: of any 9 rows of one coarse voxel two share a slot, so a
// repeat always lies within 8 rows of another (the reference compares
// neighbours in fine-row order only and misses a repeat with another child of
// the same coarse voxel between them).  Per 8-bit pass: a per-tile digit
// histogram, one exclusive scan over the digit-major [256][tiles] counts, and
// a stable scatter (ranks within a 64-element round from eight ballots,
// running per-digit counters per wavefront in LDS).  Afterwards head flags,
// a scan of them and one pass that writes parent, the coarse voxels and the
// [coarse][8] child table, which makes pack and skip mean plain gathers with
// coalesced stores.
#include "tsh_internal.h"

namespace tsh {
namespace {

constexpr int kSortBlock = 256;                   // threads per sort block (4 wavefronts)
constexpr int kSortPer = 8;                       // items per thread
constexpr int kSortTile = kSortBlock * kSortPer;  // items per tile
constexpr int kWaveItems = 64 * kSortPer;         // contiguous items per wavefront

int grid_for(int64_t count, int block, int cap) {
    int64_t g = (count + block - 1) / block;
    if (g < 1) g = 1;
    if (g > cap) g = cap;
    return (int) g;
}

// ---------------------------------------------------------------------------
// Validation, child slot, per-field maxima: each block writes its
// {negative seen, max b, max x/2, max y/2, max z/2} to part[block][0..4];
// k_s2c_prep_reduce folds them into flags[0..4] (flags[0] bit 0: a negative
// coordinate).  No atomics: thousands of them on five words serialise.
// ---------------------------------------------------------------------------
constexpr int kPrepBlocks = 1024;

__global__ void __launch_bounds__(256) k_s2c_prep(const int32_t * __restrict__ coords, int64_t n,
                                                  int32_t * __restrict__ subidx, int32_t * __restrict__ part) {
    __shared__ int32_t s_red[4][5];
    int32_t mx[4] = {0, 0, 0, 0};
    int bad = 0;
    for (int64_t f = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; f < n; f += (int64_t) gridDim.x * blockDim.x) {
        const int4 c = *(const int4 *) (coords + 4 * f);
        bad |= (c.x | c.y | c.z | c.w) < 0;
        subidx[f] = (c.y & 1) | ((c.z & 1) << 1) | ((c.w & 1) << 2);
        mx[0] = max(mx[0], c.x);
        mx[1] = max(mx[1], c.y >> 1);
        mx[2] = max(mx[2], c.z >> 1);
        mx[3] = max(mx[3], c.w >> 1);
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
#pragma unroll
        for (int a = 0; a < 4; ++a) mx[a] = max(mx[a], __shfl_xor(mx[a], d));
        bad |= __shfl_xor(bad, d);
    }
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        s_red[wave][0] = bad;
#pragma unroll
        for (int a = 0; a < 4; ++a) s_red[wave][1 + a] = mx[a];
    }
    __syncthreads();
    if (threadIdx.x < 5) {
        int32_t v = s_red[0][threadIdx.x];
        for (int w = 1; w < 4; ++w) v = threadIdx.x == 0 ? (v | s_red[w][0]) : max(v, s_red[w][threadIdx.x]);
        part[blockIdx.x * 5 + threadIdx.x] = v;
    }
}

__global__ void __launch_bounds__(256) k_s2c_prep_reduce(const int32_t * __restrict__ part, int blocks,
                                                         int32_t * __restrict__ flags) {
    __shared__ int32_t s_red[4][5];
    int32_t v[5] = {0, 0, 0, 0, 0};
    for (int b = threadIdx.x; b < blocks; b += 256) {
        v[0] |= part[b * 5];
#pragma unroll
        for (int a = 1; a < 5; ++a) v[a] = max(v[a], part[b * 5 + a]);
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        v[0] |= __shfl_xor(v[0], d);
#pragma unroll
        for (int a = 1; a < 5; ++a) v[a] = max(v[a], __shfl_xor(v[a], d));
    }
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
#pragma unroll
        for (int a = 0; a < 5; ++a) s_red[wave][a] = v[a];
    }
    __syncthreads();
    if (threadIdx.x < 5) {
        const int a = threadIdx.x;
        int32_t r = s_red[0][a];
        for (int w = 1; w < 4; ++w) r = a == 0 ? (r | s_red[w][0]) : max(r, s_red[w][a]);
        flags[a] = r;
    }
}

// Key fields from the top: b, x/2, y/2, z/2 (widths from the maxima), then
// the 3-bit child slot at bit 0.
struct KeyShape {
    int sh[4];  // left shift of b, x/2, y/2, z/2 in the 128-bit key
};

__device__ inline void make_key(const int4 c, const KeyShape & ks, uint64_t & lo, uint64_t & hi) {
    const uint32_t v[4] = {(uint32_t) c.x, (uint32_t) c.y >> 1, (uint32_t) c.z >> 1, (uint32_t) c.w >> 1};
    lo = (uint64_t) ((c.y & 1) | ((c.z & 1) << 1) | ((c.w & 1) << 2));
    hi = 0;
#pragma unroll
    for (int a = 0; a < 4; ++a) {
        const int s = ks.sh[a];
        const uint64_t f = v[a];
        if (s < 64) {
            lo |= f << s;
            if (s > 32) hi |= f >> (64 - s);  // the field straddles the word boundary
        } else {
            hi |= f << (s - 64);
        }
    }
}

__global__ void __launch_bounds__(256) k_s2c_keys(const int32_t * __restrict__ coords, int64_t n, KeyShape ks,
                                                  uint64_t * __restrict__ klo, uint64_t * __restrict__ khi,
                                                  int32_t * __restrict__ row) {
    for (int64_t f = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; f < n; f += (int64_t) gridDim.x * blockDim.x) {
        uint64_t lo, hi;
        make_key(*(const int4 *) (coords + 4 * f), ks, lo, hi);
        klo[f] = lo;
        if (khi != nullptr) khi[f] = hi;
        row[f] = (int32_t) f;
    }
}

// The 8-bit digit at bit `shift` of the key (lo, hi); digits start at bit 3,
// so one of them may straddle the two words.
template <bool WIDE> __device__ inline int digit_of(uint64_t lo, uint64_t hi, int shift) {
    if (WIDE && shift >= 64) return (int) ((hi >> (shift - 64)) & 255u);
    if (WIDE && shift > 56) return (int) (((lo >> shift) | (hi << (64 - shift))) & 255u);
    return (int) ((lo >> shift) & 255u);
}

// Digit histogram of one tile -> hist[digit * n_tiles + tile].
template <bool WIDE>
__global__ void __launch_bounds__(kSortBlock) k_radix_count(const uint64_t * __restrict__ klo,
                                                            const uint64_t * __restrict__ khi, int64_t n, int shift,
                                                            int32_t * __restrict__ hist, int n_tiles) {
    __shared__ int32_t s_cnt[256];
    s_cnt[threadIdx.x] = 0;
    __syncthreads();
    const int64_t base = (int64_t) blockIdx.x * kSortTile;
#pragma unroll
    for (int q = 0; q < kSortPer; ++q) {
        const int64_t i = base + q * kSortBlock + threadIdx.x;
        if (i < n) atomicAdd(&s_cnt[digit_of<WIDE>(klo[i], WIDE ? khi[i] : 0, shift)], 1);
    }
    __syncthreads();
    hist[(int64_t) threadIdx.x * n_tiles + blockIdx.x] = s_cnt[threadIdx.x];
}

// Lanes of this wavefront whose digit equals this lane's (valid lanes only).
__device__ inline uint64_t match_digit(int d, bool valid) {
    uint64_t m = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
        const uint64_t set = __ballot((d >> b) & 1);
        m &= ((d >> b) & 1) ? set : ~set;
    }
    return m;
}

// Stable scatter of one tile: wavefront w owns items [w*512, (w+1)*512) of the
// tile in 8 rounds of 64 consecutive items; offs = exclusive scan of hist.
template <bool WIDE>
__global__ void __launch_bounds__(kSortBlock) k_radix_scatter(const uint64_t * __restrict__ klo,
                                                              const uint64_t * __restrict__ khi,
                                                              const int32_t * __restrict__ row, int64_t n, int shift,
                                                              const int32_t * __restrict__ offs, int n_tiles,
                                                              uint64_t * __restrict__ olo, uint64_t * __restrict__ ohi,
                                                              int32_t * __restrict__ orow) {
    __shared__ int32_t s_cnt[kSortBlock / 64][256];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int d = threadIdx.x; d < (kSortBlock / 64) * 256; d += kSortBlock) (&s_cnt[0][0])[d] = 0;
    __syncthreads();
    const int64_t wbase = (int64_t) blockIdx.x * kSortTile + (int64_t) wave * kWaveItems;
    const uint64_t below = (1ull << lane) - 1ull;
    uint64_t lo[kSortPer], hi[kSortPer];
    int32_t rw[kSortPer];
    int dg[kSortPer];
    // Pass 1: this wavefront's count per digit.
#pragma unroll
    for (int q = 0; q < kSortPer; ++q) {
        const int64_t i = wbase + q * 64 + lane;
        const bool valid = i < n;
        lo[q] = valid ? klo[i] : 0;
        hi[q] = (WIDE && valid) ? khi[i] : 0;
        rw[q] = valid ? row[i] : 0;
        dg[q] = digit_of<WIDE>(lo[q], hi[q], shift);
        const uint64_t m = match_digit(dg[q], valid);
        if (valid && (m & below) == 0) s_cnt[wave][dg[q]] += __popcll(m);
    }
    __syncthreads();
    // Exclusive prefix over wavefronts plus the tile's global start, per digit.
    {
        const int d = threadIdx.x;
        int32_t run = offs[(int64_t) d * n_tiles + blockIdx.x];
#pragma unroll
        for (int w = 0; w < kSortBlock / 64; ++w) {
            const int32_t c = s_cnt[w][d];
            s_cnt[w][d] = run;
            run += c;
        }
    }
    __syncthreads();
    // Pass 2: ranks in item order; the lowest lane of each digit group
    // advances the counter after every lane of the group has read it.
#pragma unroll
    for (int q = 0; q < kSortPer; ++q) {
        const int64_t i = wbase + q * 64 + lane;
        const bool valid = i < n;
        const uint64_t m = match_digit(dg[q], valid);
        if (valid) {
            const int32_t dst = s_cnt[wave][dg[q]] + __popcll(m & below);
            olo[dst] = lo[q];
            if (WIDE) ohi[dst] = hi[q];
            orow[dst] = rw[q];
        }
        __builtin_amdgcn_wave_barrier();
        if (valid && (m & below) == 0) s_cnt[wave][dg[q]] += __popcll(m);
        __builtin_amdgcn_wave_barrier();
    }
}

// head[i] = 1 where sorted key i starts a coarse voxel; flags[0] bit 1 when a
// whole key repeats (the same fine voxel twice) within the 8 rows before it
// in its coarse voxel, which finds every repeat (see the top of this file).
template <bool WIDE>
__global__ void __launch_bounds__(256) k_s2c_heads(const uint64_t * __restrict__ klo, const uint64_t * __restrict__ khi,
                                                   int64_t n, int32_t * __restrict__ head, int32_t * __restrict__ flags) {
    for (int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t) gridDim.x * blockDim.x) {
        const uint64_t lo = klo[i];
        const uint64_t hi = WIDE ? khi[i] : 0;
        bool h = true, repeat = false;
#pragma unroll
        for (int j = 1; j <= 8; ++j) {
            if (i - j < 0) break;
            const uint64_t pl = klo[i - j];
            const bool same = (!WIDE || khi[i - j] == hi) && (pl >> 3) == (lo >> 3);
            if (!same) break;
            if (j == 1) h = false;
            repeat = repeat || pl == lo;
        }
        if (repeat) atomicOr(&flags[0], 2);
        head[i] = h ? 1 : 0;
    }
}

// parent, coarse voxels and the child table; excl = exclusive scan of head.
__global__ void __launch_bounds__(256) k_s2c_emit(const int32_t * __restrict__ coords, const int32_t * __restrict__ row,
                                                  const int32_t * __restrict__ subidx,
                                                  const int32_t * __restrict__ head, const int32_t * __restrict__ excl,
                                                  int64_t n, int32_t * __restrict__ parent,
                                                  int32_t * __restrict__ coarse, int32_t * __restrict__ child) {
    for (int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t) gridDim.x * blockDim.x) {
        const int32_t f = row[i];
        const int32_t c = excl[i] + head[i] - 1;
        parent[f] = c;
        child[(int64_t) c * 8 + subidx[f]] = f;
        if (head[i]) {
            const int4 v = *(const int4 *) (coords + 4 * (int64_t) f);
            *(int4 *) (coarse + 4 * (int64_t) c) = int4{v.x, v.y >> 1, v.z >> 1, v.w >> 1};
        }
    }
}

// ---------------------------------------------------------------------------
// Pack and skip mean as gathers over the child table.
// ---------------------------------------------------------------------------
template <int DT>
__global__ void k_s2c_pack(const typename Store<DT>::T * __restrict__ x, const int32_t * __restrict__ child,
                           typename Store<DT>::T * __restrict__ y, int64_t m, int co) {
    const int pc = co / 8;
    const int64_t count = m * co;
    for (int64_t e = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; e < count; e += (int64_t) gridDim.x * blockDim.x) {
        const int64_t c = e / co;
        const int o = (int) (e - c * co);
        const int s = o / pc, j = o - s * pc;
        const int32_t f = child[c * 8 + s];
        y[e] = f >= 0 ? x[(int64_t) f * pc + j] : (typename Store<DT>::T) 0;
    }
}

// 16-byte chunks when a child slot is a whole number of chunks.
__global__ void k_s2c_pack_vec(const int4 * __restrict__ x, const int32_t * __restrict__ child, int4 * __restrict__ y,
                               int64_t m, int vpc) {
    const int64_t count = m * 8 * vpc;
    for (int64_t e = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; e < count; e += (int64_t) gridDim.x * blockDim.x) {
        const int64_t slot = e / vpc;  // coarse * 8 + s
        const int j = (int) (e - slot * vpc);
        const int32_t f = child[slot];
        y[e] = f >= 0 ? x[(int64_t) f * vpc + j] : int4{0, 0, 0, 0};
    }
}

template <int DT>
__global__ void k_s2c_skip_mean(const typename Store<DT>::T * __restrict__ x, const int32_t * __restrict__ child,
                                typename Store<DT>::T * __restrict__ y, int64_t m, int ci, int co) {
    const int pc = co / 8, g = 8 * ci / co;
    const float gf = (float) g;
    const int64_t count = m * co;
    for (int64_t e = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; e < count; e += (int64_t) gridDim.x * blockDim.x) {
        const int64_t c = e / co;
        const int o = (int) (e - c * co);
        const int s = o / pc, j = o - s * pc;
        const int32_t f = child[c * 8 + s];
        float acc = 0.0f;
        if (f >= 0) {
            const typename Store<DT>::T * xr = x + (int64_t) f * ci + (int64_t) j * g;
            for (int t = 0; t < g; ++t) acc += Store<DT>::ld(xr, t) / gf;
        }
        Store<DT>::st(y, e, acc);
    }
}

// Eight consecutive outputs of one child slot per thread (co % 64 == 0,
// g <= 8): their 8g inputs are contiguous, read as 16-byte chunks, summed in
// the same order as above; one 16-byte store.
template <int DT, int G>
__global__ void k_s2c_skip_mean_vec(const typename Store<DT>::T * __restrict__ x, const int32_t * __restrict__ child,
                                    typename Store<DT>::T * __restrict__ y, int64_t m, int ci, int co) {
    using T = typename Store<DT>::T;
    constexpr int CHUNKS = 8 * G * (int) sizeof(T) / 16;
    constexpr int PER = 16 / (int) sizeof(T);  // values per chunk
    const int pc = co / 8, v8 = co / 8;        // v8 = groups of 8 outputs per row
    const float gf = (float) G;
    const int64_t count = m * v8;
    for (int64_t e = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; e < count; e += (int64_t) gridDim.x * blockDim.x) {
        const int64_t c = e / v8;
        const int o0 = (int) (e - c * v8) * 8;  // first output column
        const int s = o0 / pc, j0 = o0 - s * pc;
        const int32_t f = child[c * 8 + s];
        float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (f >= 0) {
            const int4 * src = (const int4 *) (x + (int64_t) f * ci + (int64_t) j0 * G);
            float v[CHUNKS * PER];
#pragma unroll
            for (int q = 0; q < CHUNKS; ++q) unpack_chunk<DT>(src[q], v + q * PER);
#pragma unroll
            for (int t = 0; t < G; ++t)
#pragma unroll
                for (int o = 0; o < 8; ++o) acc[o] += v[o * G + t] / gf;
        }
        *(int4 *) (y + c * co + o0) = pack_chunk<DT>(acc);
    }
}

}  // namespace

int64_t s2c_sort_tiles(int64_t n) { return (n + kSortTile - 1) / kSortTile; }

size_t s2c_sort_tmp_bytes(int64_t n) {
    const size_t a = scan_tmp_bytes(256 * s2c_sort_tiles(n)), b = scan_tmp_bytes(n);
    return a > b ? a : b;
}

size_t s2c_prep_part_bytes() { return (size_t) kPrepBlocks * 5 * sizeof(int32_t); }

hipError_t launch_s2c_prep(const int32_t * coords, int64_t n, int32_t * subidx, int32_t * part, int32_t * flags,
                           hipStream_t s) {
    if (n <= 0) return hipErrorInvalidValue;
    const int g = grid_for(n, 256, kPrepBlocks);
    k_s2c_prep<<<g, 256, 0, s>>>(coords, n, subidx, part);
    k_s2c_prep_reduce<<<1, 256, 0, s>>>(part, g, flags);
    return hipGetLastError();
}

int s2c_key_shape(const int32_t * maxima, int shifts[4]) {
    int w[4];
    for (int a = 0; a < 4; ++a) {
        uint32_t v = (uint32_t) maxima[a];
        w[a] = 0;
        while (v != 0) {
            ++w[a];
            v >>= 1;
        }
    }
    shifts[3] = 3;
    shifts[2] = shifts[3] + w[3];
    shifts[1] = shifts[2] + w[2];
    shifts[0] = shifts[1] + w[1];
    return shifts[0] + w[0];
}

hipError_t launch_s2c_sort(const int32_t * coords, int64_t n, const int shifts[4], int key_bits, uint64_t * klo[2],
                           uint64_t * khi[2], int32_t * row[2], int32_t * hist, int32_t * offs, int32_t * total,
                           void * tmp, int * out_buffer, hipStream_t s) {
    if (n <= 0 || n > 0x7fffffffLL) return hipErrorInvalidValue;
    const bool wide = key_bits > 64;
    KeyShape ks;
    for (int a = 0; a < 4; ++a) ks.sh[a] = shifts[a];
    k_s2c_keys<<<grid_for(n, 256, 8192), 256, 0, s>>>(coords, n, ks, klo[0], wide ? khi[0] : nullptr, row[0]);
    hipError_t err = hipGetLastError();
    const int n_tiles = (int) ((n + kSortTile - 1) / kSortTile);
    int cur = 0;
    for (int shift = 3; shift < key_bits && err == hipSuccess; shift += 8) {
        if (wide) {
            k_radix_count<true><<<n_tiles, kSortBlock, 0, s>>>(klo[cur], khi[cur], n, shift, hist, n_tiles);
        } else {
            k_radix_count<false><<<n_tiles, kSortBlock, 0, s>>>(klo[cur], nullptr, n, shift, hist, n_tiles);
        }
        err = hipGetLastError();
        if (err == hipSuccess) err = launch_scan_exclusive(hist, offs, 256LL * n_tiles, total, tmp, s);
        if (err != hipSuccess) break;
        if (wide) {
            k_radix_scatter<true><<<n_tiles, kSortBlock, 0, s>>>(klo[cur], khi[cur], row[cur], n, shift, offs,
                                                                 n_tiles, klo[cur ^ 1], khi[cur ^ 1], row[cur ^ 1]);
        } else {
            k_radix_scatter<false><<<n_tiles, kSortBlock, 0, s>>>(klo[cur], nullptr, row[cur], n, shift, offs, n_tiles,
                                                                  klo[cur ^ 1], nullptr, row[cur ^ 1]);
        }
        err = hipGetLastError();
        cur ^= 1;
    }
    *out_buffer = cur;
    return err;
}

hipError_t launch_s2c_heads(const uint64_t * klo, const uint64_t * khi, int64_t n, int32_t * head, int32_t * flags,
                            hipStream_t s) {
    if (khi != nullptr) {
        k_s2c_heads<true><<<grid_for(n, 256, 8192), 256, 0, s>>>(klo, khi, n, head, flags);
    } else {
        k_s2c_heads<false><<<grid_for(n, 256, 8192), 256, 0, s>>>(klo, nullptr, n, head, flags);
    }
    return hipGetLastError();
}

hipError_t launch_s2c_emit(const int32_t * coords, const int32_t * row, const int32_t * subidx, const int32_t * head,
                           const int32_t * excl, int64_t n, int32_t * parent, int32_t * coarse, int32_t * child,
                           hipStream_t s) {
    k_s2c_emit<<<grid_for(n, 256, 8192), 256, 0, s>>>(coords, row, subidx, head, excl, n, parent, coarse, child);
    return hipGetLastError();
}

hipError_t launch_s2c_pack(int dtype, const void * x, const int32_t * child, void * y, int64_t m, int co,
                           hipStream_t s) {
    if (m <= 0 || co <= 0 || co % 8 != 0) return hipErrorInvalidValue;
    const size_t es = dtype_bytes(dtype);
    const size_t slot_bytes = (size_t) (co / 8) * es;
    if (slot_bytes % 16 == 0) {
        const int vpc = (int) (slot_bytes / 16);
        const int g = grid_for(m * 8 * vpc, 256, 65536);
        k_s2c_pack_vec<<<g, 256, 0, s>>>((const int4 *) x, child, (int4 *) y, m, vpc);
        return hipGetLastError();
    }
    const int g = grid_for(m * co, 256, 65536);
    switch (dtype) {
        case kF32: k_s2c_pack<kF32><<<g, 256, 0, s>>>((const float *) x, child, (float *) y, m, co); break;
        case kF16: k_s2c_pack<kF16><<<g, 256, 0, s>>>((const _Float16 *) x, child, (_Float16 *) y, m, co); break;
        default: k_s2c_pack<kBF16><<<g, 256, 0, s>>>((const uint16_t *) x, child, (uint16_t *) y, m, co); break;
    }
    return hipGetLastError();
}

hipError_t launch_s2c_skip_mean(int dtype, const void * x, const int32_t * child, void * y, int64_t m, int ci,
                                int co, hipStream_t s) {
    if (m <= 0 || ci <= 0 || co <= 0 || co % 8 != 0 || (8 * ci) % co != 0) return hipErrorInvalidValue;
    const int grp = 8 * ci / co;
    if (dtype != kF32 && co % 64 == 0 && (grp == 2 || grp == 4 || grp == 8)) {
        const int gv = grid_for(m * (co / 8), 256, 65536);
#define TSH_SKIP(DTV, TYPE, GV) \
    k_s2c_skip_mean_vec<DTV, GV><<<gv, 256, 0, s>>>((const TYPE *) x, child, (TYPE *) y, m, ci, co)
        if (dtype == kBF16) {
            if (grp == 2) TSH_SKIP(kBF16, uint16_t, 2);
            else if (grp == 4) TSH_SKIP(kBF16, uint16_t, 4);
            else TSH_SKIP(kBF16, uint16_t, 8);
        } else {
            if (grp == 2) TSH_SKIP(kF16, _Float16, 2);
            else if (grp == 4) TSH_SKIP(kF16, _Float16, 4);
            else TSH_SKIP(kF16, _Float16, 8);
        }
#undef TSH_SKIP
        return hipGetLastError();
    }
    const int g = grid_for(m * co, 256, 65536);
    switch (dtype) {
        case kF32: k_s2c_skip_mean<kF32><<<g, 256, 0, s>>>((const float *) x, child, (float *) y, m, ci, co); break;
        case kF16:
            k_s2c_skip_mean<kF16><<<g, 256, 0, s>>>((const _Float16 *) x, child, (_Float16 *) y, m, ci, co);
            break;
        default:
            k_s2c_skip_mean<kBF16><<<g, 256, 0, s>>>((const uint16_t *) x, child, (uint16_t *) y, m, ci, co);
            break;
    }
    return hipGetLastError();
}

}  // namespace tsh
