// dump_io.hip - raw tensor dumps: the files trellis2.c's tools read and write.
//
// Formats (host code only):
//   reading  tools/debug/trellis_structured_latent.c:237-333: a .f32 file is
//            a whole number of little-endian floats; a coordinates .i32 file
//            is [N,4] (b, x, y, z) when its element count is a multiple of 4,
//            otherwise (or when forced) [N,3] (x, y, z) with batch 0.
//   writing  src/ops/sparse/cuda/forward.cu:99-223: files "<index>_<name>.f32"
//            / ".i32" (index %03d, counting from 0 per writer) and one
//            manifest line per tensor, "<name>\t<rows>x<cols>\t<f32|i32>\t<file>".
// Device tensors are downloaded (as fp32 for feature buffers) before writing.
#include <cerrno>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <sys/stat.h>

#include "tsh_internal.h"

struct trellis_sparse_hip_dump {
    std::string dir;
    FILE * manifest = nullptr;
    int next_index = 0;
};

namespace tsh {
namespace {

trellis_status read_whole(const char * path, size_t elem, void ** data_out, size_t * count_out) {
    *data_out = nullptr;
    *count_out = 0;
    struct stat st;
    if (path == nullptr || stat(path, &st) != 0 || !S_ISREG(st.st_mode)) return TRELLIS_STATUS_IO_ERROR;
    const size_t bytes = (size_t) st.st_size;
    if (bytes % elem != 0) return TRELLIS_STATUS_PARSE_ERROR;
    const size_t count = bytes / elem;
    void * data = malloc(bytes > 0 ? bytes : 1);
    if (data == nullptr) return TRELLIS_STATUS_OUT_OF_MEMORY;
    FILE * f = fopen(path, "rb");
    if (f == nullptr) {
        free(data);
        return TRELLIS_STATUS_IO_ERROR;
    }
    const size_t got = count > 0 ? fread(data, elem, count, f) : 0;
    fclose(f);
    if (got != count) {
        free(data);
        return TRELLIS_STATUS_IO_ERROR;
    }
    *data_out = data;
    *count_out = count;
    return TRELLIS_STATUS_OK;
}

trellis_status write_tensor(trellis_sparse_hip_dump * d, const char * name, const void * data, size_t elem,
                            int64_t rows, int cols, const char * dtype) {
    if (d == nullptr || d->manifest == nullptr || name == nullptr || name[0] == '\0' || strchr(name, '/') != nullptr ||
        rows < 0 || cols <= 0 || (rows > 0 && data == nullptr)) {
        return TRELLIS_STATUS_INVALID_ARGUMENT;
    }
    char rel[512];
    const int k = snprintf(rel, sizeof(rel), "%03d_%s.%s", d->next_index, name, dtype);
    if (k < 0 || (size_t) k >= sizeof(rel)) return TRELLIS_STATUS_INVALID_ARGUMENT;
    ++d->next_index;
    const std::string path = d->dir + "/" + rel;
    FILE * f = fopen(path.c_str(), "wb");
    if (f == nullptr) return TRELLIS_STATUS_IO_ERROR;
    const size_t count = (size_t) rows * (size_t) cols;
    const size_t wrote = count > 0 ? fwrite(data, elem, count, f) : 0;
    const int rc = fclose(f);
    if (wrote != count || rc != 0) return TRELLIS_STATUS_IO_ERROR;
    fprintf(d->manifest, "%s\t%lldx%d\t%s\t%s\n", name, (long long) rows, cols, dtype, rel);
    fflush(d->manifest);
    return ferror(d->manifest) ? TRELLIS_STATUS_IO_ERROR : TRELLIS_STATUS_OK;
}

}  // namespace
}  // namespace tsh

extern "C" {

trellis_status trellis_sparse_hip_read_f32(const char * path, float ** data_out, size_t * count_out) {
    if (path == nullptr || data_out == nullptr || count_out == nullptr) return TRELLIS_STATUS_INVALID_ARGUMENT;
    void * p = nullptr;
    const trellis_status st = tsh::read_whole(path, sizeof(float), &p, count_out);
    *data_out = (float *) p;
    return st;
}

trellis_status trellis_sparse_hip_read_coords_i32(const char * path, int force_xyz, int32_t ** coords_out,
                                                  int64_t * n_out) {
    if (path == nullptr || coords_out == nullptr || n_out == nullptr) return TRELLIS_STATUS_INVALID_ARGUMENT;
    *coords_out = nullptr;
    *n_out = 0;
    void * p = nullptr;
    size_t count = 0;
    trellis_status st = tsh::read_whole(path, sizeof(int32_t), &p, &count);
    if (st != TRELLIS_STATUS_OK) return st;
    int32_t * raw = (int32_t *) p;
    if (!force_xyz && count % 4 == 0) {
        *coords_out = raw;
        *n_out = (int64_t) (count / 4);
        return TRELLIS_STATUS_OK;
    }
    if (count % 3 != 0) {
        free(raw);
        return TRELLIS_STATUS_PARSE_ERROR;
    }
    const size_t n = count / 3;
    int32_t * c = (int32_t *) malloc(n > 0 ? n * 16 : 1);
    if (c == nullptr) {
        free(raw);
        return TRELLIS_STATUS_OUT_OF_MEMORY;
    }
    for (size_t i = 0; i < n; ++i) {
        c[4 * i] = 0;
        memcpy(c + 4 * i + 1, raw + 3 * i, 3 * sizeof(int32_t));
    }
    free(raw);
    *coords_out = c;
    *n_out = (int64_t) n;
    return TRELLIS_STATUS_OK;
}

trellis_status trellis_sparse_hip_dump_open(const char * dir, const char * manifest_name,
                                            trellis_sparse_hip_dump ** out) {
    if (dir == nullptr || dir[0] == '\0' || manifest_name == nullptr || manifest_name[0] == '\0' || out == nullptr) {
        return TRELLIS_STATUS_INVALID_ARGUMENT;
    }
    *out = nullptr;
    if (mkdir(dir, 0777) != 0 && errno != EEXIST) return TRELLIS_STATUS_IO_ERROR;
    auto * d = new (std::nothrow) trellis_sparse_hip_dump();
    if (d == nullptr) return TRELLIS_STATUS_OUT_OF_MEMORY;
    d->dir = dir;
    d->manifest = fopen((d->dir + "/" + manifest_name).c_str(), "w");
    if (d->manifest == nullptr) {
        delete d;
        return TRELLIS_STATUS_IO_ERROR;
    }
    *out = d;
    return TRELLIS_STATUS_OK;
}

trellis_status trellis_sparse_hip_dump_close(trellis_sparse_hip_dump * d) {
    if (d == nullptr) return TRELLIS_STATUS_INVALID_ARGUMENT;
    const int rc = d->manifest != nullptr ? fclose(d->manifest) : 0;
    delete d;
    return rc == 0 ? TRELLIS_STATUS_OK : TRELLIS_STATUS_IO_ERROR;
}

trellis_status trellis_sparse_hip_dump_host_f32(trellis_sparse_hip_dump * d, const char * name, const float * data,
                                                int64_t rows, int cols) {
    return tsh::write_tensor(d, name, data, sizeof(float), rows, cols, "f32");
}

trellis_status trellis_sparse_hip_dump_host_i32(trellis_sparse_hip_dump * d, const char * name, const int32_t * data,
                                                int64_t rows, int cols) {
    return tsh::write_tensor(d, name, data, sizeof(int32_t), rows, cols, "i32");
}

trellis_status trellis_sparse_hip_dump_buffer(trellis_sparse_hip_dump * d, trellis_sparse_backend * backend,
                                              const char * name, const trellis_sparse_buffer * buf, int64_t rows,
                                              int cols) {
    if (d == nullptr || backend == nullptr || buf == nullptr || buf->dtype < 0 || rows < 0 || cols <= 0 ||
        (size_t) rows * (size_t) cols > buf->count) {
        return TRELLIS_STATUS_INVALID_ARGUMENT;
    }
    const size_t count = (size_t) rows * (size_t) cols;
    float * host = (float *) malloc(count > 0 ? count * sizeof(float) : 1);
    if (host == nullptr) return TRELLIS_STATUS_OUT_OF_MEMORY;
    trellis_status st = count > 0 ? backend->ops->download_f32(backend, buf, host, count) : TRELLIS_STATUS_OK;
    if (st == TRELLIS_STATUS_OK) st = tsh::write_tensor(d, name, host, sizeof(float), rows, cols, "f32");
    free(host);
    return st;
}

trellis_status trellis_sparse_hip_dump_map_coords(trellis_sparse_hip_dump * d, trellis_sparse_backend * backend,
                                                  const char * name, const trellis_sparse_c2s_device_map * map) {
    if (d == nullptr || backend == nullptr || map == nullptr) return TRELLIS_STATUS_INVALID_ARGUMENT;
    const int64_t n = map->n;
    int32_t * host = (int32_t *) malloc(n > 0 ? (size_t) n * 16 : 1);
    if (host == nullptr) return TRELLIS_STATUS_OUT_OF_MEMORY;
    trellis_status st = backend->ops->download_c2s_coords(backend, map, host, n);
    if (st == TRELLIS_STATUS_OK) st = tsh::write_tensor(d, name, host, sizeof(int32_t), n, 4, "i32");
    free(host);
    return st;
}

}  // extern "C"
