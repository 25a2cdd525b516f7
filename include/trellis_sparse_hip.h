/*
 * trellis_sparse_hip.h - C ABI of the MI355X (gfx950) sparse-voxel backend.
 *
 * The library is a drop-in backend behind trellis2.c's sparse backend vtable.
 * It plugs in where the CPU and Vulkan backends plug in today:
 *
 *   reference: src/ops/sparse/trellis_sparse_backend.h:24-201  (ops table)
 *              src/ops/sparse/trellis_sparse_backend.h:203-207 (backend object)
 *              src/ops/sparse/trellis_sparse_backend.h:209-210 (factories)
 *
 * The ops table below is ABI-identical to trellis_sparse_backend_ops: the same
 * 27 function pointers in the same order with the same C signatures, so a
 * backend created here can be handed to the reference executors
 * (src/architectures/sparse_unet_{decoder,encoder}/executor.c) unchanged.
 *
 * Include order inside the reference tree: include "trellis.h" and
 * "sparse/trellis_sparse_backend.h" first; this header then reuses their
 * definitions (guarded by their include guards) and only adds the
 * trellis_sparse_hip_* entry points.  Standalone, it defines the shared types
 * itself with the reference's exact enumerator values.
 *
 * Everything is plain C: pointers, sizes, status codes.  No HIP, torch or C++
 * types appear in any signature.
 */
#ifndef TRELLIS_SPARSE_HIP_H
#define TRELLIS_SPARSE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------ */
/* Types shared with the reference (include/trellis.h:30-40, :55-59).        */
/* ------------------------------------------------------------------------ */
#ifndef TRELLIS2_C_TRELLIS_H
typedef enum trellis_status {
    TRELLIS_STATUS_OK = 0,
    TRELLIS_STATUS_ERROR = 1,
    TRELLIS_STATUS_INVALID_ARGUMENT = 2,
    TRELLIS_STATUS_IO_ERROR = 3,
    TRELLIS_STATUS_PARSE_ERROR = 4,
    TRELLIS_STATUS_OUT_OF_MEMORY = 5,
    TRELLIS_STATUS_CUDA_UNAVAILABLE = 6,
    TRELLIS_STATUS_NOT_FOUND = 7,
    TRELLIS_STATUS_NOT_IMPLEMENTED = 8
} trellis_status;

typedef enum trellis_sparse_backend_kind {
    TRELLIS_SPARSE_BACKEND_CUDA = 0,
    TRELLIS_SPARSE_BACKEND_CPU = 1,
    TRELLIS_SPARSE_BACKEND_VULKAN = 2
} trellis_sparse_backend_kind;

/* include/trellis.h:790-796; arrays malloc'd, released with free() (or the
 * reference's trellis_mesh_free). */
typedef struct trellis_mesh_host {
    float * vertices;      /* [n_vertices, 3] */
    float * vertex_colors; /* optional [n_vertices, 3] in linear 0..1 RGB */
    int32_t * faces;       /* [n_faces, 3] */
    int64_t n_vertices;
    int64_t n_faces;
} trellis_mesh_host;
#endif

/* New backend kind value for this library.  A caller selects it through
 * trellis_sparse_unet_vae_{decoder,encoder}_forward_options.backend_kind
 * together with options.sparse_backend (executor.c:619-621 requires
 * backend->kind == options->backend_kind). */
#define TRELLIS_SPARSE_BACKEND_HIP ((trellis_sparse_backend_kind) 3)

/* ------------------------------------------------------------------------ */
/* Sparse backend vtable (src/ops/sparse/trellis_sparse_backend.h:9-207).    */
/* ------------------------------------------------------------------------ */
#ifndef TRELLIS2_C_OPS_SPARSE_BACKEND_H
typedef struct trellis_sparse_buffer trellis_sparse_buffer;
typedef struct trellis_sparse_rulebook trellis_sparse_rulebook;
typedef struct trellis_sparse_c2s_device_map trellis_sparse_c2s_device_map;
typedef struct trellis_sparse_backend trellis_sparse_backend;
struct trellis_pixal_camera;
struct trellis_pixal_naf_attention_desc;

enum {
    TRELLIS_SPARSE_TRIM_FREE_BUFFERS = 1u << 0,
    TRELLIS_SPARSE_TRIM_WEIGHTS = 1u << 1,
    TRELLIS_SPARSE_TRIM_ALL = (1u << 0) | (1u << 1)
};

typedef struct trellis_sparse_backend_ops {
    void (*destroy)(trellis_sparse_backend * backend);

    trellis_status (*alloc_f32)(trellis_sparse_backend * backend, size_t count, trellis_sparse_buffer ** out);
    trellis_status (*upload_f32)(trellis_sparse_backend * backend, const float * src, size_t count, trellis_sparse_buffer ** out);
    trellis_status (*upload_i32)(trellis_sparse_backend * backend, const int32_t * src, size_t count, trellis_sparse_buffer ** out);
    trellis_status (*download_f32)(trellis_sparse_backend * backend, const trellis_sparse_buffer * src, float * dst, size_t count);
    void (*free_buffer)(trellis_sparse_backend * backend, trellis_sparse_buffer * buffer);

    trellis_status (*linear)(trellis_sparse_backend * backend, const trellis_sparse_buffer * x,
                             const float * weight, const float * bias, trellis_sparse_buffer * y,
                             int64_t n, int in_channels, int out_channels);
    trellis_status (*linear_silu)(trellis_sparse_backend * backend, const trellis_sparse_buffer * x,
                                  const float * weight, const float * bias, trellis_sparse_buffer * y,
                                  int64_t n, int in_channels, int out_channels);
    trellis_status (*row_norm)(trellis_sparse_backend * backend, const trellis_sparse_buffer * x,
                               const float * gamma, const float * beta, trellis_sparse_buffer * y,
                               int64_t n, int channels, float eps);
    trellis_status (*row_norm_silu)(trellis_sparse_backend * backend, const trellis_sparse_buffer * x,
                                    const float * gamma, const float * beta, trellis_sparse_buffer * y,
                                    int64_t n, int channels, float eps);
    trellis_status (*silu_inplace)(trellis_sparse_backend * backend, trellis_sparse_buffer * x, size_t count);
    trellis_status (*add)(trellis_sparse_backend * backend, const trellis_sparse_buffer * a,
                          const trellis_sparse_buffer * b, trellis_sparse_buffer * y, size_t count);

    trellis_status (*build_rulebook)(trellis_sparse_backend * backend, const int32_t * coords_bxyz,
                                     int64_t n, trellis_sparse_rulebook ** out);
    trellis_status (*sparse_conv3d)(trellis_sparse_backend * backend, const trellis_sparse_rulebook * rulebook,
                                    const trellis_sparse_buffer * feats, const float * weight, const float * bias,
                                    trellis_sparse_buffer * out, int64_t n, int in_channels, int out_channels);
    void (*free_rulebook)(trellis_sparse_backend * backend, trellis_sparse_rulebook * rulebook);

    trellis_status (*c2s_gather)(trellis_sparse_backend * backend, const trellis_sparse_buffer * x,
                                 const int32_t * parent, const int32_t * subidx, trellis_sparse_buffer * y,
                                 int64_t n_out, int out_channels);
    trellis_status (*skip_repeat)(trellis_sparse_backend * backend, const trellis_sparse_buffer * x,
                                  const int32_t * parent, const int32_t * subidx, trellis_sparse_buffer * y,
                                  int64_t n_out, int in_channels, int out_channels);
    trellis_status (*build_c2s_map)(trellis_sparse_backend * backend, const int32_t * coords_bxyz,
                                    const trellis_sparse_buffer * logits, int64_t n, int32_t ** coords_out,
                                    int32_t ** parent_out, int32_t ** subidx_out, int64_t * n_out);
    trellis_status (*alias_c2s_map)(trellis_sparse_backend * backend, const int32_t * coords_bxyz,
                                    const int32_t * parent, const int32_t * subidx, int64_t n,
                                    const int32_t * alias_coords_bxyz, const int32_t * alias_parent,
                                    const int32_t * alias_subidx);
    trellis_status (*build_c2s_map_device)(trellis_sparse_backend * backend, const int32_t * coords_bxyz,
                                           const trellis_sparse_c2s_device_map * coords_map,
                                           const trellis_sparse_buffer * logits, int64_t n,
                                           trellis_sparse_c2s_device_map ** map_out, int64_t * n_out);
    trellis_status (*build_rulebook_for_c2s_map)(trellis_sparse_backend * backend,
                                                 const trellis_sparse_c2s_device_map * map,
                                                 trellis_sparse_rulebook ** out);
    trellis_status (*c2s_gather_device)(trellis_sparse_backend * backend, const trellis_sparse_buffer * x,
                                        const trellis_sparse_c2s_device_map * map, trellis_sparse_buffer * y,
                                        int64_t n_out, int out_channels);
    trellis_status (*skip_repeat_device)(trellis_sparse_backend * backend, const trellis_sparse_buffer * x,
                                         const trellis_sparse_c2s_device_map * map, trellis_sparse_buffer * y,
                                         int64_t n_out, int in_channels, int out_channels);
    trellis_status (*download_c2s_coords)(trellis_sparse_backend * backend,
                                          const trellis_sparse_c2s_device_map * map,
                                          int32_t * coords_out, int64_t n);
    trellis_status (*download_c2s_map)(trellis_sparse_backend * backend,
                                       const trellis_sparse_c2s_device_map * map, int32_t * coords_out,
                                       int32_t * parent_out, int32_t * subidx_out, int64_t n);
    /* Releases backend caches only. Device-resident C2S maps remain valid. */
    trellis_status (*trim)(trellis_sparse_backend * backend, unsigned flags, size_t * released_bytes);
    trellis_status (*pixal_naf_attention_project_sparse)(
        trellis_sparse_backend * backend, const float * queries, const float * keys, const float * values,
        const int32_t * coords_bxyz, int64_t n_coords, const struct trellis_pixal_camera * cameras,
        const struct trellis_pixal_naf_attention_desc * desc, float * projected_out, size_t projected_count);
} trellis_sparse_backend_ops;

struct trellis_sparse_backend {
    const trellis_sparse_backend_ops * ops;
    trellis_sparse_backend_kind kind;
    int device;
};
#endif /* TRELLIS2_C_OPS_SPARSE_BACKEND_H */

/* ------------------------------------------------------------------------ */
/* Creation-time policy.                                                     */
/* ------------------------------------------------------------------------ */

/* Storage / MFMA input type of every buffer the backend owns.  The vtable
 * edges stay fp32 (upload_f32 rounds to the storage type with
 * round-to-nearest-even, download_f32 widens), and all arithmetic accumulates
 * in fp32.  Mirrors the per-component compute_dtype policy of the reference
 * model package (models/trellis2/model.json:90-107). */
typedef enum trellis_sparse_hip_dtype {
    TRELLIS_SPARSE_HIP_F32 = 0,
    TRELLIS_SPARSE_HIP_F16 = 1,
    TRELLIS_SPARSE_HIP_BF16 = 2
} trellis_sparse_hip_dtype;

/* Convolution schedule.  AUTO picks by channel counts and dtype: COMPACT where
 * it applies, else MASKED, else GENERIC; a schedule that does not apply falls
 * back the same way.  The choice never changes which pairs contribute, only
 * the order of fp32 summation. */
typedef enum trellis_sparse_hip_conv_algo {
    TRELLIS_SPARSE_HIP_CONV_AUTO = 0,
    TRELLIS_SPARSE_HIP_CONV_GENERIC = 1,   /* one lane per output element, any channels and dtype */
    TRELLIS_SPARSE_HIP_CONV_MASKED = 2,    /* MFMA over the neighbour table; F16/BF16, Ci % 32 == 0, Co % 64 == 0 */
    TRELLIS_SPARSE_HIP_CONV_COMPACT = 3    /* MFMA over compacted per-tile pair lists; F16/BF16, Ci == 64 or
                                              Ci % 128 == 0, Co % 64 == 0 */
} trellis_sparse_hip_conv_algo;

/* Which code runs the linear and linear_silu slots in 16-bit storage. */
typedef enum trellis_sparse_hip_linear_algo {
    TRELLIS_SPARSE_HIP_LINEAR_AUTO = 0,    /* Ci >= 256, Co >= 256 and n >= 2048: the platform GEMM library
                                              (hipBLASLt, bias and SiLU in its epilogue, fp32 accumulation);
                                              other shapes: this library's MFMA kernels */
    TRELLIS_SPARSE_HIP_LINEAR_KERNEL = 1   /* always this library's MFMA / VALU kernels */
} trellis_sparse_hip_linear_algo;

typedef struct trellis_sparse_hip_policy {
    uint32_t struct_size;      /* sizeof(trellis_sparse_hip_policy) */
    int32_t compute_dtype;     /* trellis_sparse_hip_dtype */
    int32_t conv_algo;         /* trellis_sparse_hip_conv_algo */
    int32_t cache_weights;     /* 1: keep device copies of host weights keyed by (pointer, count) until
                                  trim(TRELLIS_SPARSE_TRIM_WEIGHTS) or destroy, like the Vulkan backend
                                  (trellis_sparse_vulkan.c:1019-1052). 0: convert on every call. */
    int32_t reject_duplicates; /* 0: duplicate coordinates resolve to the last row, as the CPU backend does
                                  (trellis_sparse_cpu.c:314-318). 1: build_rulebook returns
                                  TRELLIS_STATUS_INVALID_ARGUMENT on a duplicate. */
    int32_t linear_algo;       /* trellis_sparse_hip_linear_algo */
} trellis_sparse_hip_policy;

/* Fills *policy with the defaults: F32, conv AUTO, cache_weights=1, reject_duplicates=0, linear AUTO. */
void trellis_sparse_hip_policy_init(trellis_sparse_hip_policy * policy);

/* ------------------------------------------------------------------------ */
/* Factories.  Replace trellis_sparse_vulkan_backend_create                  */
/* (src/ops/sparse/trellis_sparse_backend.h:210) with the same contract:     */
/* *out is NULL on failure; no usable device -> TRELLIS_STATUS_CUDA_UNAVAILABLE */
/* (the reference's "device absent" code, trellis_sparse_vulkan.c:4017-4019). */
/* ------------------------------------------------------------------------ */
trellis_status trellis_sparse_hip_backend_create(int device, trellis_sparse_backend ** out);
trellis_status trellis_sparse_hip_backend_create_ex(int device, const trellis_sparse_hip_policy * policy,
                                                    trellis_sparse_backend ** out);

/* Number of visible HIP devices (0 when none or when the runtime is absent). */
int trellis_sparse_hip_device_count(void);

/* Message for the last failing call on this backend ("" if none).  Valid until the next call. */
const char * trellis_sparse_hip_last_error(const trellis_sparse_backend * backend);

/* Waits for all work queued by this backend. */
trellis_status trellis_sparse_hip_synchronize(trellis_sparse_backend * backend);

/* Forced allocation failure, for tests of the out-of-memory paths (no
 * counterpart in the reference, whose Vulkan backend only reacts to real
 * failures by trimming and retrying, trellis_sparse_vulkan.c:533-561).
 * From this call on, device allocation attempts number after .. after +
 * count - 1 (counted from 0) fail as if the device were full; after < 0
 * switches the hook off.  Every slot then returns
 * TRELLIS_STATUS_OUT_OF_MEMORY with its outputs NULL / 0, and an allocation
 * that fails while the backend's pool holds free blocks releases the pool and
 * tries once more.  The environment variable TRELLIS_HIP_FAIL_ALLOC_AFTER=N[,K]
 * sets the same hook at creation (K defaults to all later attempts). */
trellis_status trellis_sparse_hip_fail_alloc(trellis_sparse_backend * backend, int64_t after, int64_t count);

/* ------------------------------------------------------------------------ */
/* Inspection (no counterpart in the reference vtable; used by parity tests */
/* and the benchmark).  All downloads are synchronous.                       */
/* ------------------------------------------------------------------------ */

/* Voxel count, valid (in,out) pairs including the centre (downloads the 27
 * per-offset counts, synchronising), hash slots and occupied bricks. */
trellis_status trellis_sparse_hip_rulebook_stats(trellis_sparse_backend * backend,
                                                 const trellis_sparse_rulebook * rulebook, int64_t * n,
                                                 int64_t * pairs, int64_t * table_slots, int64_t * bricks);

/* Neighbour table, int32 [n][27]: nbr[i][k] is the row of the voxel at
 * (b, x+kd-1, y+kh-1, z+kw-1), k = kd*9 + kh*3 + kw, or -1.  Coordinates wrap
 * modulo 2^16 exactly as the reference key packing does
 * (trellis_sparse_cpu.c:24-31). */
trellis_status trellis_sparse_hip_download_neighbors(trellis_sparse_backend * backend,
                                                     const trellis_sparse_rulebook * rulebook,
                                                     int32_t * nbr_out, int64_t n);

/* Per-offset pair lists in canonical order: offset-major, destination row
 * ascending within an offset.  counts_out[27] receives the per-offset counts;
 * src_out/dst_out receive sum(counts) entries (capacity given in entries). */
trellis_status trellis_sparse_hip_download_pairs(trellis_sparse_backend * backend,
                                                 const trellis_sparse_rulebook * rulebook, int64_t * counts_out,
                                                 int32_t * src_out, int32_t * dst_out, int64_t capacity);

/* Storage-type I/O without conversion: count elements of the backend's
 * compute_dtype (4 bytes for F32, 2 bytes for F16/BF16). */
trellis_status trellis_sparse_hip_upload_raw(trellis_sparse_backend * backend, const void * src, size_t count,
                                             trellis_sparse_buffer ** out);
trellis_status trellis_sparse_hip_download_raw(trellis_sparse_backend * backend,
                                               const trellis_sparse_buffer * src, void * dst, size_t count);

/* ------------------------------------------------------------------------ */
/* Device-resident coordinates and C2S map lifetime (no counterpart in the   */
/* reference vtable, whose device maps live until destroy; the Vulkan        */
/* backend keeps uploaded coordinates in a host-pointer cache instead,       */
/* trellis_sparse_vulkan.c:2059-2096).                                       */
/* ------------------------------------------------------------------------ */

/* Uploads coordinates [n][4] into a backend-owned device map without parent /
 * subidx arrays.  The map can be passed as coords_map to build_c2s_map_device
 * and to build_rulebook_for_c2s_map, so a level's coordinates cross PCIe once.
 * c2s_gather_device, skip_repeat_device and download_c2s_map reject it. */
trellis_status trellis_sparse_hip_upload_coords(trellis_sparse_backend * backend, const int32_t * coords_bxyz,
                                                int64_t n, trellis_sparse_c2s_device_map ** map_out);

/* Releases a device map early (otherwise it lives until destroy).  Rulebooks
 * built from the map with build_rulebook_for_c2s_map borrow its coordinates and
 * must be freed first. */
trellis_status trellis_sparse_hip_free_c2s_map(trellis_sparse_backend * backend,
                                               trellis_sparse_c2s_device_map * map);

/* Allocation-free subdivide: build_c2s_map_device's result written into
 * caller-owned buffers.  No counterpart in the reference; it is for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  It calls no hipMalloc,
 * hipFree or other allocating routine: its working memory (per-parent child
 * counts and their scan) is a fixed device array of about 8 MB per GPU,
 * held until the process ends and shared by every call on that GPU.  Calls
 * on one GPU are ordered: a call holds a per-GPU lock for its duration, and
 * its kernels wait (on its backend's stream) for the previous call's fill,
 * so concurrent callers on other threads or streams wait their turn.
 *   coords      int32 buffer (upload_i32) of the n parents' (b, x, y, z)
 *   logits      [n][8] buffer in the backend's compute_dtype; child s of
 *               parent p exists iff logits[p][s] > 0, exactly as in
 *               build_c2s_map_device
 *   coords_out  int32 buffer of >= 4 m entries, parent_out / subidx_out
 *               int32 buffers of >= m entries; children parent-major,
 *               subidx ascending, coordinates (b, 2x+(s&1), 2y+((s>>1)&1),
 *               2z+((s>>2)&1)) - the same arrays download_c2s_map returns
 *   n_out       m, the number of children (set also when the outputs are too
 *               small, so the caller can size them)
 * n > 1048576 -> INVALID_ARGUMENT (the scratch limit); outputs smaller than m
 * -> INVALID_ARGUMENT with *n_out = m and nothing written; no child ->
 * TRELLIS_STATUS_ERROR, as build_c2s_map_device.  The fill is queued on the
 * backend's stream; the child count is read back synchronously. */
trellis_status trellis_sparse_hip_build_c2s_map_into(trellis_sparse_backend * backend,
                                                     const trellis_sparse_buffer * coords,
                                                     const trellis_sparse_buffer * logits, int64_t n,
                                                     trellis_sparse_buffer * coords_out,
                                                     trellis_sparse_buffer * parent_out,
                                                     trellis_sparse_buffer * subidx_out, int64_t * n_out);

/* ------------------------------------------------------------------------ */
/* Spatial-to-channel downsample of the encoder on the device (no vtable     */
/* counterpart: the reference runs it on the host, replacing                 */
/* trellis_sparse_s2c_host_build, sparse_unet_encoder/s2c_host.c:33-120, and  */
/* the download / pack / skip-mean / upload round trip of encoder_s2c_exec,  */
/* sparse_unet_encoder/executor.c:258-300).                                  */
/* ------------------------------------------------------------------------ */

/* Builds the S2C relation of fine_n fine voxels, given as host coordinates
 * [fine_n][4] or as a device map (fine_coords_map, which wins when both are
 * given).  fine_map_out: a device map of the fine level (coords = a copy of
 * the fine coordinates, parent[f] = coarse row, subidx[f] = (x&1) |
 * (y&1)<<1 | (z&1)<<2, n_parent = coarse_n) - the decoder's C2S guide for
 * this level, usable with c2s_gather_device, skip_repeat_device,
 * download_c2s_map and build_rulebook_for_c2s_map.  coarse_map_out: a
 * coordinates-only map of the coarse voxels (b, x/2, y/2, z/2) in ascending
 * (b, x, y, z) order, for build_rulebook_for_c2s_map and download_c2s_coords.
 * Negative coordinates -> INVALID_ARGUMENT; a fine voxel given twice ->
 * PARSE_ERROR (every repeat; the host build catches a repeat only when no
 * other child of its coarse voxel lies between the two rows).  Both maps
 * live until destroy or trellis_sparse_hip_free_c2s_map. */
trellis_status trellis_sparse_hip_s2c_build_device(trellis_sparse_backend * backend, const int32_t * fine_coords_bxyz,
                                                   const trellis_sparse_c2s_device_map * fine_coords_map,
                                                   int64_t fine_n, trellis_sparse_c2s_device_map ** fine_map_out,
                                                   trellis_sparse_c2s_device_map ** coarse_map_out,
                                                   int64_t * coarse_n_out);
/* y[c][s*(co/8) + j] = x[f][j] for the fine row f in child slot s of coarse
 * voxel c, zero for empty slots (executor.c:279-286).  x [fine_n][co/8],
 * y [coarse_n][co]; co % 8 == 0. */
trellis_status trellis_sparse_hip_s2c_pack_device(trellis_sparse_backend * backend, const trellis_sparse_buffer * x,
                                                  const trellis_sparse_c2s_device_map * fine_map,
                                                  trellis_sparse_buffer * y, int co);
/* y[c][s*(co/8) + j] = sum over t < g of x[f][j*g + t] / g in fp32 from zero,
 * g = 8*ci/co, for the fine row f in child slot s of coarse voxel c; zero for
 * empty slots (executor.c:287-292).  x [fine_n][ci], y [coarse_n][co];
 * co % 8 == 0 and (8*ci) % co == 0 (executor.c:172-175). */
trellis_status trellis_sparse_hip_s2c_skip_mean_device(trellis_sparse_backend * backend,
                                                       const trellis_sparse_buffer * x,
                                                       const trellis_sparse_c2s_device_map * fine_map,
                                                       trellis_sparse_buffer * y, int ci, int co);

/* ------------------------------------------------------------------------ */
/* FlexiDualGrid mesh from decoder logits on the device (no vtable          */
/* counterpart: replaces trellis_flexible_dual_grid_mesh_from_decoder_      */
/* logits_host, src/ops/mesh/flex_dual_grid.c:166-313, which the mesh stage */
/* calls on the downloaded decoder output, latent_decode.c:146).            */
/* ------------------------------------------------------------------------ */

/* Same result contract as the reference function, for decoder output still
 * on the device: coordinates as host [n][4] or a device map (coords_map wins),
 * feats a backend buffer [n][channels] (channels >= 7).  One vertex per voxel
 * (vertex_colors NULL), two faces per quad in the reference's (voxel, axis)
 * order.  INVALID_ARGUMENT for NULL pointers, n < 0, channels < 7 or
 * resolution <= 0; PARSE_ERROR for a batch index other than 0, a coordinate
 * outside [0, resolution), a non-finite logit in channels 0..6 or a repeated
 * coordinate; NOT_IMPLEMENTED for resolution > 65535 (the corner lookups use
 * the kernel map's 16-bit keys).  n = 0 gives an empty mesh. */
trellis_status trellis_sparse_hip_flex_dual_grid_mesh(trellis_sparse_backend * backend, const int32_t * coords_bxyz,
                                                     const trellis_sparse_c2s_device_map * coords_map,
                                                     const trellis_sparse_buffer * feats, int64_t n, int channels,
                                                     int resolution, trellis_mesh_host * mesh_out);

/* ------------------------------------------------------------------------ */
/* Raw tensor dumps in trellis2.c's tool formats (no vtable counterpart:    */
/* the readers of tools/debug/trellis_structured_latent.c:237-333 and the   */
/* intermediate-tensor writer of src/ops/sparse/cuda/forward.cu:99-223).    */
/* Host code; the device variants download first.                           */
/* ------------------------------------------------------------------------ */

/* A whole file of little-endian floats; *data_out malloc'd. IO_ERROR when the
 * file cannot be read, PARSE_ERROR when its size is not a whole number of
 * floats. */
trellis_status trellis_sparse_hip_read_f32(const char * path, float ** data_out, size_t * count_out);
/* Coordinates: [N,4] (b, x, y, z) when the int32 count is a multiple of 4 and
 * force_xyz is 0, otherwise [N,3] (x, y, z) returned as [N,4] with b = 0;
 * PARSE_ERROR when neither fits.  *coords_out malloc'd. */
trellis_status trellis_sparse_hip_read_coords_i32(const char * path, int force_xyz, int32_t ** coords_out,
                                                  int64_t * n_out);

/* A dump directory (created if missing) with a manifest file of one line per
 * tensor, "<name>\t<rows>x<cols>\t<f32|i32>\t<file>", files named
 * "<index>_<name>.<f32|i32>" with a 3-digit running index. */
typedef struct trellis_sparse_hip_dump trellis_sparse_hip_dump;
trellis_status trellis_sparse_hip_dump_open(const char * dir, const char * manifest_name,
                                            trellis_sparse_hip_dump ** out);
trellis_status trellis_sparse_hip_dump_close(trellis_sparse_hip_dump * dump);
trellis_status trellis_sparse_hip_dump_host_f32(trellis_sparse_hip_dump * dump, const char * name, const float * data,
                                                int64_t rows, int cols);
trellis_status trellis_sparse_hip_dump_host_i32(trellis_sparse_hip_dump * dump, const char * name,
                                                const int32_t * data, int64_t rows, int cols);
/* A backend buffer's first rows * cols values, downloaded as fp32. */
trellis_status trellis_sparse_hip_dump_buffer(trellis_sparse_hip_dump * dump, trellis_sparse_backend * backend,
                                              const char * name, const trellis_sparse_buffer * buffer, int64_t rows,
                                              int cols);
/* A device map's coordinates, [n][4] int32. */
trellis_status trellis_sparse_hip_dump_map_coords(trellis_sparse_hip_dump * dump, trellis_sparse_backend * backend,
                                                  const char * name, const trellis_sparse_c2s_device_map * map);

/* ------------------------------------------------------------------------ */
/* Fused ConvNeXt MLP tail (no counterpart in the reference vtable: it       */
/* replaces the slot sequence row_norm -> linear_silu -> linear -> add of     */
/* the decoder's ConvNeXt block, sparse_unet_decoder/executor.c:206-241).    */
/* ------------------------------------------------------------------------ */

/* y = residual + mlp2(SiLU(mlp0(row_norm(x, gamma, beta, eps)))), x, residual
 * and y [n][c] in the backend's compute_dtype (y may be residual);
 * mlp0_w fp32 [4c][c], mlp0_b [4c], mlp2_w fp32 [c][4c], mlp2_b [c] (biases,
 * gamma and beta may be NULL).
 *   c = 64, 128, 256: one kernel; each intermediate is rounded to the storage
 * type where the slot sequence stores it, and the 4c-wide hidden rows never
 * leave the chip.
 *   c a multiple of 128 from 512 (the decoder's 512 and 1024 levels, where a
 * 128-row tile's normalised rows alone would take 128 KB of the 160 KB of
 * LDS): row_norm, then mlp0 + SiLU and mlp2 as GEMMs through n x c and
 * n x 4c intermediates, the residual added to mlp2's fp32 sums in the GEMM
 * library's epilogue (one rounding where the slots round mlp2's output and
 * then the sum; with the LINEAR_KERNEL policy, or rows the library does not
 * take, the slots' two roundings).
 * TRELLIS_STATUS_NOT_IMPLEMENTED for other widths or unless compute_dtype is
 * F16 or BF16; callers then run the slot sequence. */
trellis_status trellis_sparse_hip_convnext_mlp(trellis_sparse_backend * backend, const trellis_sparse_buffer * x,
                                               const float * gamma, const float * beta, const float * mlp0_w,
                                               const float * mlp0_b, const float * mlp2_w, const float * mlp2_b,
                                               const trellis_sparse_buffer * residual, trellis_sparse_buffer * y,
                                               int64_t n, int c, float eps);

/* The whole ConvNeXt block (sparse_unet_decoder/executor.c:176-255):
 * out = h + mlp2(SiLU(mlp0(row_norm(sparse_conv3d(h), gamma, beta, eps)))),
 * h and out [n][c] (out must not be h), conv_w fp32 [c][27][c], conv_b [c],
 * the rest as in trellis_sparse_hip_convnext_mlp: the conv into one n x c
 * intermediate, then the tail (roundings as there).
 * TRELLIS_STATUS_NOT_IMPLEMENTED unless compute_dtype is F16 or BF16 and c is
 * 64, 128, 256 or a multiple of 128 from 512. */
trellis_status trellis_sparse_hip_convnext_block(trellis_sparse_backend * backend,
                                                 const trellis_sparse_rulebook * rulebook,
                                                 const trellis_sparse_buffer * h, const float * conv_w,
                                                 const float * conv_b, const float * gamma, const float * beta,
                                                 const float * mlp0_w, const float * mlp0_b, const float * mlp2_w,
                                                 const float * mlp2_b, trellis_sparse_buffer * out, int64_t n, int c,
                                                 float eps);

/* ------------------------------------------------------------------------ */
/* Convs with a fused epilogue (no counterpart in the reference vtable: each */
/* replaces a slot pair of the residual blocks, sparse_unet_decoder/         */
/* executor.c:176-255 and sparse_unet_encoder/executor.c:160-360).           */
/* ------------------------------------------------------------------------ */

/* out = row_norm(_silu)(sparse_conv3d(feats)) with gamma, beta (NULL allowed)
 * and eps as trellis_sparse_backend_ops.row_norm(_silu) take them; the conv
 * output is rounded to the storage type before the norm, as the slot pair
 * stores it, and is not written anywhere.  out must not be feats.
 * TRELLIS_STATUS_NOT_IMPLEMENTED unless compute_dtype is F16 or BF16, the
 * conv policy is AUTO or COMPACT, Ci is 64 or a multiple of 128 and
 * Co == 128; callers then run the slot pair. */
trellis_status trellis_sparse_hip_conv_norm(trellis_sparse_backend * backend, const trellis_sparse_rulebook * rulebook,
                                            const trellis_sparse_buffer * feats, const float * weight,
                                            const float * bias, const float * gamma, const float * beta, float eps,
                                            int silu, trellis_sparse_buffer * out, int64_t n, int ci, int co);

/* out = sparse_conv3d(feats) + residual (the conv output rounded to the
 * storage type first, as the slot pair conv -> add computes it); residual
 * [n][co] may be out itself (each element is read before it is written) or
 * feats, but out must not be feats.  Same conditions as conv_norm, with Co a
 * multiple of 128. */
trellis_status trellis_sparse_hip_conv_add(trellis_sparse_backend * backend, const trellis_sparse_rulebook * rulebook,
                                           const trellis_sparse_buffer * feats, const float * weight,
                                           const float * bias, const trellis_sparse_buffer * residual,
                                           trellis_sparse_buffer * out, int64_t n, int ci, int co);

/* ------------------------------------------------------------------------ */
/* Stage timing with HIP events recorded on the backend's own stream.        */
/* ------------------------------------------------------------------------ */
typedef enum trellis_sparse_hip_stage {
    TRELLIS_SPARSE_HIP_STAGE_HASH = 0,      /* brick table + voxel pool build */
    TRELLIS_SPARSE_HIP_STAGE_MAP = 1,       /* neighbour table + per-offset pair lists */
    TRELLIS_SPARSE_HIP_STAGE_CONV = 2,      /* sparse_conv3d kernels */
    TRELLIS_SPARSE_HIP_STAGE_SUBDIVIDE = 3, /* C2S count/scan/fill */
    TRELLIS_SPARSE_HIP_STAGE_BROADCAST = 4, /* c2s_gather / skip_repeat */
    TRELLIS_SPARSE_HIP_STAGE_ELEMENTWISE = 5, /* norms, SiLU, add, linear */
    TRELLIS_SPARSE_HIP_STAGE_COUNT = 6
} trellis_sparse_hip_stage;

typedef struct trellis_sparse_hip_stage_times {
    double ms[TRELLIS_SPARSE_HIP_STAGE_COUNT];       /* summed event time per stage */
    int64_t launches[TRELLIS_SPARSE_HIP_STAGE_COUNT]; /* timed launches per stage */
} trellis_sparse_hip_stage_times;

/* Turns per-stage event bracketing on or off (off by default). */
trellis_status trellis_sparse_hip_profile_enable(trellis_sparse_backend * backend, int enable);
/* Synchronises, then returns the accumulated stage times; reset != 0 clears them. */
trellis_status trellis_sparse_hip_profile_read(trellis_sparse_backend * backend,
                                               trellis_sparse_hip_stage_times * out, int reset);

/* Records event `slot` (0..15) on the backend stream; elapsed() synchronises on slot b. */
trellis_status trellis_sparse_hip_event_record(trellis_sparse_backend * backend, int slot);
trellis_status trellis_sparse_hip_event_elapsed(trellis_sparse_backend * backend, int slot_a, int slot_b,
                                                float * ms);

#ifdef __cplusplus
}
#endif

#endif /* TRELLIS_SPARSE_HIP_H */
