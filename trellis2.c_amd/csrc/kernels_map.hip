// kernels_map.hip - GPU voxel hash and 3x3x3 submanifold kernel map for gfx950.
//
// Reference semantics (src/ops/sparse/trellis_sparse_cpu.c):
//   key packing with 16-bit fields  :24-31   (coordinates wrap modulo 2^16)
//   last duplicate wins             :314-318
//   neighbour (b, x+kd-1, y+kh-1, z+kw-1), k = kd*9+kh*3+kw, never across b  :348-358
//
// Layout in HBM (all sized from n, no host synchronisation):
//   brick table  16-byte slots {uint64 key, int32 idx, pad}, slots = nextpow2(2n),
//                so that one load returns a slot's key and brick index.
//                Key = (b:16 | x>>2:14 | y>>2:14 | z>>2:14) + 1, 0 = empty,
//                linear probing from splitmix64(key).
//   voxel pool   int32 [bricks][64]: row of the voxel at cell (z&3)|(y&3)<<2|(x&3)<<4, -1 = empty
//                (z fastest: a 16-byte load returns a voxel's z-row, the three
//                cells of a (kd, kh) stencil column for cells off the z faces).
//   nbr          int32 [n][27]
//   mask         uint32 [n], bit k <=> nbr[i][k] >= 0
//   tile_counts  int32 [n_tiles][27] valid pairs per 256-row tile and offset
//   pairs        tile-major: tile t's lists for offset k start at tile_off[t][k] (tiles ascending,
//                offsets ascending within a tile, dst ascending within an offset); pair_src int32
//                source rows, pair_dst uint8 destination rows within the 256-row tile (one byte
//                instead of four: config 4's map 0.232 -> 0.175 ms without these stores at all).
//
// A voxel's 27 neighbours lie in at most 8 bricks (on average 3.4), so the
// kernel map does a few hash probes per voxel plus 9 z-row reads (16 bytes)
// from 256-byte brick rows that neighbouring lanes share, and 9 single-cell
// reads for voxels on a z face, instead of 27 random probes.  Halving the
// load instructions against one 4-byte read per neighbour cut the map by a
// fifth: the gathers are bound by the cache lines each instruction touches.
#include "tsh_internal.h"

namespace tsh {
namespace {

constexpr int kBlock = 256;

__device__ __forceinline__ uint64_t mix64(uint64_t v) {
    v = (v ^ (v >> 30)) * 0xbf58476d1ce4e5b9ull;
    v = (v ^ (v >> 27)) * 0x94d049bb133111ebull;
    return v ^ (v >> 31);
}

__device__ __forceinline__ uint64_t brick_key(uint32_t b, uint32_t bx, uint32_t by, uint32_t bz) {
    return (((uint64_t) b << 42) | ((uint64_t) bx << 28) | ((uint64_t) by << 14) | (uint64_t) bz) + 1ull;
}

// Slot s of the brick table (two uint64 words per slot: the key, then the
// brick index in the low half of the second word), read with one load.
typedef unsigned long long U64x2 __attribute__((ext_vector_type(2)));
struct Slot {
    uint64_t key;
    int32_t idx;
};
__device__ __forceinline__ Slot slot_load(const uint64_t * __restrict__ table, uint64_t s) {
    const U64x2 e = *(const U64x2 *) (table + 2 * s);
    return {e.x, (int32_t) (uint32_t) e.y};
}

// Linear probe for key from slot s on (the home slot held another key):
// the brick's index, or -1 at an empty slot.
__device__ __forceinline__ int32_t brick_find_from(const uint64_t * __restrict__ table, uint64_t mask, uint64_t key,
                                                   uint64_t s) {
    for (uint64_t step = 1; step <= mask; ++step) {
        const Slot e = slot_load(table, s);
        if (e.key == key) return e.idx;
        if (e.key == 0) return -1;
        s = (s + 1) & mask;
    }
    return -1;
}

__device__ __forceinline__ uint64_t readlane_u64(uint64_t v, int lane) {
    const uint32_t lo = (uint32_t) __builtin_amdgcn_readlane((int) (uint32_t) v, lane);
    const uint32_t hi = (uint32_t) __builtin_amdgcn_readlane((int) (uint32_t) (v >> 32), lane);
    return ((uint64_t) hi << 32) | lo;
}

__device__ __forceinline__ int lane_id() { return (int) __lane_id(); }

// Empties the brick table (keys to 0), clears the build's counters and sets
// the pool's spare row (the empty brick the kernel map reads for a missing
// neighbour brick) to -1, in one launch.
__global__ void k_hash_clear(uint64_t * __restrict__ table, int64_t slots, int32_t * __restrict__ counters,
                             int32_t * __restrict__ empty_row) {
    const int64_t stride = (int64_t) gridDim.x * blockDim.x;
    const int64_t t = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (t < kCounterInts) counters[t] = 0;
    if (t < kBrickCells) empty_row[t] = -1;
    for (int64_t i = t; i < slots; i += stride) *(U64x2 *) (table + 2 * i) = U64x2{0ull, 0ull};
}

__global__ void k_fill_i32(int32_t * __restrict__ p, int64_t count, int32_t value) {
    const int64_t stride = (int64_t) gridDim.x * blockDim.x;
    for (int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; i < count; i += stride) {
        p[i] = value;
    }
}

// One lane per voxel.  Lanes of a wavefront first agree on one representative
// per distinct brick (ballot/readlane, no memory traffic); representatives
// then insert concurrently with a 64-bit CAS.  The lane that claims an empty
// slot numbers the brick, and its wavefront sets the brick's 64 pool cells to
// -1 (one coalesced 256-byte store per new brick).  Block b numbers its new
// bricks from b * 256 (a block has at most one per voxel), so numbering
// needs no global counter and no second round trip; the pool has a row per
// voxel slot, of which the map reads only the rows of existing bricks.
__global__ void __launch_bounds__(kBlock) k_brick_insert(const int4 * __restrict__ coords, int64_t n,
                                                         uint64_t * __restrict__ table, uint64_t mask,
                                                         int32_t * __restrict__ counters, int32_t * __restrict__ pool) {
    const int64_t i = (int64_t) blockIdx.x * kBlock + threadIdx.x;
    const bool active = i < n;
    uint64_t key = 0;
    if (active) {
        const int4 c = coords[i];
        key = brick_key((uint32_t) c.x & 0xffffu, ((uint32_t) c.y & 0xffffu) >> 2, ((uint32_t) c.z & 0xffffu) >> 2,
                        ((uint32_t) c.w & 0xffffu) >> 2);
    }
    const int lane = lane_id();
    bool first = active;
    uint64_t todo = __ballot(active);
    while (todo != 0) {
        const int leader = __builtin_ctzll(todo);
        const uint64_t lk = readlane_u64(key, leader);
        const uint64_t same = __ballot(active && key == lk);
        if (lane != leader && ((same >> lane) & 1ull)) {
            first = false;
        }
        todo &= ~same;
    }
    // Representatives probe; a lane that claims an empty slot owns a new brick.
    // A slot's key only ever changes from 0 to its final value, so a read
    // that returns a key is final: the CAS is issued only for a slot that
    // read empty.  Other wavefronts insert most bricks first (a 4^3 brick
    // spans rows far apart in raster order).
    uint64_t s = 0;
    bool won = false;
    if (first) {
        s = mix64(key) & mask;
        uint64_t step = 0;
        for (; step <= mask; ++step) {
            uint64_t prev = __hip_atomic_load(&table[2 * s], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (prev == 0) prev = atomicCAS((unsigned long long *) &table[2 * s], 0ull, (unsigned long long) key);
            if (prev == 0) {
                won = true;
                break;
            }
            if (prev == key) {
                break;
            }
            s = (s + 1) & mask;
        }
        if (step > mask) {
            atomicOr(&counters[4], 1);  // table full; cannot happen with slots >= 2n
        }
    }
    // Number the new bricks: wave ballots give each winner its rank, LDS gives
    // each wave its offset in the block's range.
    __shared__ int32_t s_wave_new[kBlock / 64];
    const int wave = threadIdx.x >> 6;
    const uint64_t wins = __ballot(won);
    const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    if (lane == 0) {
        s_wave_new[wave] = __popcll(wins);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        // The brick count (statistics only): one add per block, spread over
        // kBrickCounters counters, whose result nothing waits for.
        int32_t total = 0;
        for (int w = 0; w < kBlock / 64; ++w) total += s_wave_new[w];
        if (total > 0) atomicAdd(&counters[kBrickCounter + blockIdx.x % kBrickCounters], total);
    }
    int32_t idx = 0;
    if (won) {
        idx = (int32_t) blockIdx.x * kBlock + __popcll(wins & below);
        for (int w = 0; w < wave; ++w) idx += s_wave_new[w];
        *(int32_t *) (table + 2 * s + 1) = idx;
    }
    // The wavefront's new bricks start empty: lane c clears cell c of each.
    for (uint64_t left = wins; left != 0; left &= left - 1) {
        const int32_t b = __builtin_amdgcn_readlane(idx, __builtin_ctzll(left));
        pool[(int64_t) b * kBrickCells + lane] = -1;
    }
}

// One lane per voxel: record the row in its brick cell.  atomicMax makes the
// highest row (the last duplicate in input order) win deterministically; its
// result is not waited for (the kernel map finds duplicates: a row whose own
// cell holds another row).
__global__ void __launch_bounds__(kBlock) k_voxel_insert(const int4 * __restrict__ coords, int64_t n,
                                                         const uint64_t * __restrict__ table, uint64_t mask,
                                                         int32_t * __restrict__ pool, int32_t * __restrict__ counters) {
    const int64_t i = (int64_t) blockIdx.x * kBlock + threadIdx.x;
    if (i >= n) {
        return;
    }
    const int4 c = coords[i];
    const uint32_t x = (uint32_t) c.y & 0xffffu, y = (uint32_t) c.z & 0xffffu, z = (uint32_t) c.w & 0xffffu;
    // The home slot's key and index in one round trip; only a home slot
    // holding another key continues the probe.
    const uint64_t key = brick_key((uint32_t) c.x & 0xffffu, x >> 2, y >> 2, z >> 2);
    const uint64_t hs = mix64(key) & mask;
    const Slot h = slot_load(table, hs);
    const int32_t b = h.key == key ? h.idx : (h.key == 0ull ? -1 : brick_find_from(table, mask, key, (hs + 1) & mask));
    if (b < 0) {
        atomicOr(&counters[4], 2);  // unreachable: every voxel's brick was inserted
        return;
    }
    const uint32_t cell = (z & 3u) | ((y & 3u) << 2) | ((x & 3u) << 4);
    atomicMax(&pool[(int64_t) b * kBrickCells + cell], (int32_t) i);
}

// Kernel map in one pass.  One block = one 256-row tile:
//  1. each row's 27 neighbour rows are found (a few brick probes per voxel
//     plus 9 z-row pool reads) and kept in its lane's registers, with the row
//     masks; only a launch that also writes the neighbour table (NBR) stages
//     the tile's [256][27] rows in LDS, for a coalesced copy.  Without that
//     28 KB of LDS per block the kernel runs 8 wavefronts per SIMD instead
//     of 5, which is what its dependent probe and pool loads need;
//  2. per-offset pair counts of the tile (wavefront ballots);
//  3. the neighbour table (16-byte vectorised copy of the LDS block), the
//     per-(tile, offset) counts and list starts, and the pair lists,
//     destination ascending within each (tile, offset).
// Tile t owns the fixed region [t * 256 * 27, (t + 1) * 256 * 27) of the
// pair arrays (the most pairs 256 rows can have), so no tile waits for the
// counts of the tiles before it; the lists of a tile are packed from the
// region's start, the centre offset (k = 13) first, then the others in
// order.  Every row has exactly one centre neighbour (itself, or the last
// duplicate of its coordinates), so the centre list holds the tile's rows in
// order, starting at the region's start: a consumer can find it without the
// tile's counts.
// Seven wavefronts per SIMD (at most 72 registers): 4 % faster than six on
// config 3's map, while eight spill.  The launch that also writes the
// neighbour table holds 28 KB of LDS per block, which allows five.
template <bool NBR>
__global__ void __launch_bounds__(kBlock, NBR ? 5 : 7) k_map_tiles(const int4 * __restrict__ coords, int64_t n,
                                                      const uint64_t * __restrict__ table, uint64_t hmask,
                                                      const int32_t * __restrict__ pool, int32_t empty_brick,
                                                      int32_t * __restrict__ nbr,
                                                      uint32_t * __restrict__ mask_out,
                                                      int32_t * __restrict__ tile_counts,
                                                      int32_t * __restrict__ tile_off,
                                                      int32_t * __restrict__ pair_src,
                                                      uint8_t * __restrict__ pair_dst, int32_t * __restrict__ counters) {
    __shared__ __attribute__((aligned(16))) int32_t s_nbr[NBR ? kBlock * 27 : 4];
    __shared__ int32_t s_wave_cnt[27][kBlock / 64];
    __shared__ int32_t s_koff[27];
    const int t = threadIdx.x;
    const int lane = lane_id();
    const int wave = t >> 6;
    const int64_t tile = blockIdx.x;
    const int64_t row0 = tile * kBlock;
    const int64_t i = row0 + t;
    uint32_t m = 0;
    int32_t nb[27];
#pragma unroll
    for (int k = 0; k < 27; ++k) nb[k] = -1;
    if (i < n) {
        const int4 c = coords[i];
        const uint32_t b = (uint32_t) c.x & 0xffffu;
        const uint32_t x = (uint32_t) c.y & 0xffffu, y = (uint32_t) c.z & 0xffffu, z = (uint32_t) c.w & 0xffffu;
        const uint32_t bx = x >> 2, by = y >> 2, bz = z >> 2;
        const int cx = (int) (x & 3u), cy = (int) (y & 3u), cz = (int) (z & 3u);
        // Adjacent brick per axis: -1 when the cell is on the low face, +1 on the high face, 0 otherwise.
        const int sx = cx == 0 ? -1 : (cx == 3 ? 1 : 0);
        const int sy = cy == 0 ? -1 : (cy == 3 ? 1 : 0);
        const int sz = cz == 0 ? -1 : (cz == 3 ? 1 : 0);
        // The (up to) 8 bricks the 27 neighbours lie in.  Every lane loads
        // the home slot's key and index of all 8 at once (a brick it does
        // not need probes a dummy key), so one round trip resolves nearly
        // all of them; only a home slot holding another key continues the
        // linear probe.
        int32_t br[8];
        uint64_t bkey[8], hkey[8];
        int32_t hidx[8];
        uint64_t hs[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const int ax = q & 1, ay = (q >> 1) & 1, az = (q >> 2) & 1;
            const bool need = (ax == 0 || sx != 0) && (ay == 0 || sy != 0) && (az == 0 || sz != 0);
            const uint32_t nbx = (bx + (uint32_t) (ax * sx)) & 0x3fffu;
            const uint32_t nby = (by + (uint32_t) (ay * sy)) & 0x3fffu;
            const uint32_t nbz = (bz + (uint32_t) (az * sz)) & 0x3fffu;
            bkey[q] = need ? brick_key(b, nbx, nby, nbz) : 0ull;
            hs[q] = mix64(bkey[q]) & hmask;
            const Slot e = slot_load(table, hs[q]);
            hkey[q] = e.key;
            hidx[q] = e.idx;
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            br[q] = -1;
            if (bkey[q] != 0ull && hkey[q] != 0ull) {
                br[q] = hkey[q] == bkey[q] ? hidx[q] : brick_find_from(table, hmask, bkey[q], (hs[q] + 1) & hmask);
            }
        }
        // All 9 z-rows and 9 face cells are loaded before any is used (one
        // round trip per voxel); a missing brick (and, for a voxel off the z
        // faces, the face cell) reads the pool's spare row of -1, so no
        // branch guards a load.
        int4 zrow[9];
        int32_t face[9];
#pragma unroll
        for (int kd = 0; kd < 3; ++kd) {
            const int nx = cx + kd - 1;
            const int ix = (nx < 0 || nx > 3) ? 1 : 0;
#pragma unroll
            for (int kh = 0; kh < 3; ++kh) {
                const int ny = cy + kh - 1;
                const int iy = (ny < 0 || ny > 3) ? 1 : 0;
                const int q0 = ix | (iy << 1);
                int32_t brick = br[0], brick_z = br[4];
#pragma unroll
                for (int qq = 1; qq < 4; ++qq) {
                    brick = q0 == qq ? br[qq] : brick;
                    brick_z = q0 == qq ? br[qq + 4] : brick_z;
                }
                // The z-row (nx, ny, 0..3) of the brick, and the one cell of
                // the next brick along z that a face voxel also needs.
                const int row = ((nx & 3) << 4) | ((ny & 3) << 2);
                const int32_t vb = brick >= 0 ? brick : empty_brick;
                const int32_t eb = (sz != 0 && brick_z >= 0) ? brick_z : empty_brick;
                zrow[kd * 3 + kh] = *(const int4 *) (pool + (int64_t) vb * kBrickCells + row);
                face[kd * 3 + kh] = pool[(int64_t) eb * kBrickCells + row + (sz < 0 ? 3 : 0)];
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int c = 0; c < 9; ++c) {
            const int4 v = zrow[c];
            const int32_t e = face[c];
#pragma unroll
            for (int kw = 0; kw < 3; ++kw) {
                const int nz = cz + kw - 1;
                const int32_t r = nz < 0 || nz > 3 ? e : (nz == 0 ? v.x : (nz == 1 ? v.y : (nz == 2 ? v.z : v.w)));
                const int k = c * 3 + kw;
                nb[k] = r;
                if constexpr (NBR) s_nbr[t * 27 + k] = r;
                m |= (r >= 0 ? 1u : 0u) << k;
            }
        }
        mask_out[i] = m;
        // The centre neighbour is the highest row at these coordinates: any
        // other value means duplicate coordinates.
        if (nb[13] != (int32_t) i) atomicOr(&counters[1], 1);
    }
    // Rows of this wavefront with a neighbour at k (the ranks are recomputed
    // from the same ballots when the pairs are written).
    const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
#pragma unroll
    for (int k = 0; k < 27; ++k) {
        const uint64_t bal = __ballot((m >> k) & 1u);
        if (lane == 0) s_wave_cnt[k][wave] = __popcll(bal);
    }
    __syncthreads();
    if (t < 64) {
        // Tile counts per offset and their exclusive scan in packing order:
        // lane 0 takes the centre offset, lanes 1..26 the others in order.
        const int k = t == 0 ? 13 : (t <= 13 ? t - 1 : t);
        int32_t cnt = 0;
        if (t < 27) {
#pragma unroll
            for (int w = 0; w < kBlock / 64; ++w) cnt += s_wave_cnt[k][w];
            tile_counts[tile * 27 + k] = cnt;
        }
        int32_t incl = cnt;
#pragma unroll
        for (int d = 1; d < 32; d <<= 1) {
            const int32_t o = __shfl_up(incl, d);
            if (lane >= d) incl += o;
        }
        if (t < 27) s_koff[k] = incl - cnt;
        // Layout statistics for the convs with 256-column blocks: this
        // tile's offsets with pairs, and with more than half the tile.
        const int with = __popcll(__ballot(cnt > 0));
        const int busy = __popcll(__ballot(cnt > kBlock / 2));
        if (t == 0) {
            const int slot = (int) (blockIdx.x % kLayoutSlots);
            atomicAdd(&counters[kLayoutStats + slot], with);
            atomicAdd(&counters[kLayoutStats + kLayoutSlots + slot], busy);
        }
    }
    __syncthreads();
    const int64_t base = tile * kBlock * 27;
    if (t < 27) tile_off[tile * 27 + t] = (int32_t) (base + s_koff[t]);
    if constexpr (NBR) {
        // Coalesced copy of the tile's neighbour table.
        const int64_t rows = (n - row0) < kBlock ? (n - row0) : kBlock;
        const int64_t words = rows * 27;
        int32_t * dst = nbr + row0 * 27;
        if ((words & 3) == 0) {
            for (int64_t w = (int64_t) t * 4; w < words; w += kBlock * 4) {
                *(int4 *) (dst + w) = *(const int4 *) (s_nbr + w);
            }
        } else {
            for (int64_t w = t; w < words; w += kBlock) {
                dst[w] = s_nbr[w];
            }
        }
    }
    // Every lane takes part in the ballots; rows past n have no neighbours.
#pragma unroll
    for (int k = 0; k < 27; ++k) {
        const uint64_t bal = __ballot((m >> k) & 1u);
        if ((m >> k) & 1u) {
            int64_t pos = base + s_koff[k] + __popcll(bal & lt);
            for (int w = 0; w < wave; ++w) pos += s_wave_cnt[k][w];
            pair_src[pos] = nb[k];
            pair_dst[pos] = (uint8_t) t;
        }
    }
}

int grid_for(int64_t count, int block, int cap = 65536) {
    int64_t g = (count + block - 1) / block;
    if (g < 1) g = 1;
    if (g > cap) g = cap;
    return (int) g;
}

}  // namespace

hipError_t launch_fill_i32(int32_t * p, int64_t count, int32_t value, hipStream_t s) {
    if (count <= 0) return hipSuccess;
    k_fill_i32<<<grid_for(count, 256, 16384), 256, 0, s>>>(p, count, value);
    return hipGetLastError();
}

int64_t pool_empty_brick(int64_t n) { return (n + kBlock - 1) / kBlock * kBlock; }

hipError_t launch_hash_clear(uint64_t * table, int64_t slots, int32_t * counters, int32_t * pool, int64_t n,
                             hipStream_t s) {
    // The grid has at least 256 threads, which covers the counters and the
    // spare pool row.
    static_assert(kCounterInts <= 256 && kBrickCells <= 256, "cleared by the first block");
    k_hash_clear<<<grid_for(slots, 256, 16384), 256, 0, s>>>(table, slots, counters,
                                                             pool + pool_empty_brick(n) * kBrickCells);
    return hipGetLastError();
}

hipError_t launch_brick_insert(const int32_t * coords, int64_t n, uint64_t * table, int64_t slots,
                               int32_t * counters, int32_t * pool, hipStream_t s) {
    const int64_t blocks = (n + kBlock - 1) / kBlock;
    k_brick_insert<<<(unsigned) blocks, kBlock, 0, s>>>((const int4 *) coords, n, table,
                                                        (uint64_t) (slots - 1), counters, pool);
    return hipGetLastError();
}

hipError_t launch_voxel_insert(const int32_t * coords, int64_t n, const uint64_t * table,
                               int64_t slots, int32_t * pool, int32_t * counters, hipStream_t s) {
    const int64_t blocks = (n + kBlock - 1) / kBlock;
    k_voxel_insert<<<(unsigned) blocks, kBlock, 0, s>>>((const int4 *) coords, n, table,
                                                        (uint64_t) (slots - 1), pool, counters);
    return hipGetLastError();
}

hipError_t launch_map_tiles(const int32_t * coords, int64_t n, const uint64_t * table,
                            int64_t slots, const int32_t * pool, int32_t * nbr, uint32_t * mask,
                            int32_t * tile_counts, int32_t * tile_off, int32_t * pair_src, uint8_t * pair_dst,
                            int32_t * counters, hipStream_t s) {
    const int64_t blocks = (n + kBlock - 1) / kBlock;
    const int32_t empty = (int32_t) pool_empty_brick(n);
    if (nbr != nullptr) {
        k_map_tiles<true><<<(unsigned) blocks, kBlock, 0, s>>>((const int4 *) coords, n, table,
                                                               (uint64_t) (slots - 1), pool, empty, nbr, mask,
                                                               tile_counts, tile_off, pair_src, pair_dst, counters);
    } else {
        k_map_tiles<false><<<(unsigned) blocks, kBlock, 0, s>>>((const int4 *) coords, n, table,
                                                                (uint64_t) (slots - 1), pool, empty, nbr, mask,
                                                                tile_counts, tile_off, pair_src, pair_dst, counters);
    }
    return hipGetLastError();
}

}  // namespace tsh
