/*
 * BFW container reader (libbfmodel.so).
 *
 * On-disk layout (the format of reference src/model.c:14-51 and the writer
 * tools/export_checkpoint.py:12-17,49-80; kept identical because it is the
 * file interface the reference's exporter produces):
 *   header  64 B : magic "BFW0001\0", u32 version, u32 header_bytes,
 *                  u64 tensor_count, u64 directory_offset, u64 data_offset,
 *                  u64 file_bytes, u32 directory_crc32, u32 flags, 8 B pad
 *   entry  160 B : char name[96], u32 dtype, u32 rank, u32 dims[8],
 *                  u64 offset, u64 nbytes, u32 crc32, u32 flags
 *   payloads     : 64-byte aligned, little-endian, C order.
 *
 * This implementation maps the file read-only and keeps a name-sorted index
 * for binary-search lookup; every entry is bounds-checked at open, tensor
 * CRCs are checked on demand (bf_model_validate_*).
 */
#define _POSIX_C_SOURCE 200809L
#include "bf_model.h"

#include <errno.h>
#include <fcntl.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

enum { kHeaderBytes = 64, kEntryBytes = 160, kAlign = 64 };
static const char kMagic[8] = {'B', 'F', 'W', '0', '0', '0', '1', '\0'};

struct bf_model {
    int fd;
    const unsigned char *base;
    size_t bytes;
    size_t count;
    bf_tensor *tensors;      /* directory order */
    const bf_tensor **index; /* sorted by name */
};

static int report(char *error, size_t cap, const char *fmt, ...) {
    if (error && cap) {
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(error, cap, fmt, ap);
        va_end(ap);
    }
    return 0;
}

/* Little-endian field readers: the container is defined little-endian. */
static uint32_t rd32(const unsigned char *p) {
    return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 |
           (uint32_t)p[3] << 24;
}
static uint64_t rd64(const unsigned char *p) {
    return (uint64_t)rd32(p) | (uint64_t)rd32(p + 4) << 32;
}

/* Reflected CRC-32 (polynomial 0xEDB88320), byte-table driven. */
static uint32_t crc_table[256];
static int crc_ready;
static void crc_init(void) {
    for (uint32_t i = 0; i < 256; ++i) {
        uint32_t c = i;
        for (int k = 0; k < 8; ++k) c = (c & 1u) ? 0xEDB88320u ^ (c >> 1) : c >> 1;
        crc_table[i] = c;
    }
    crc_ready = 1;
}
static uint32_t crc32_of(const void *data, size_t n) {
    if (!crc_ready) crc_init();
    const unsigned char *p = (const unsigned char *)data;
    uint32_t c = 0xFFFFFFFFu;
    for (size_t i = 0; i < n; ++i) c = crc_table[(c ^ p[i]) & 0xFFu] ^ (c >> 8);
    return c ^ 0xFFFFFFFFu;
}

static int by_name(const void *a, const void *b) {
    const bf_tensor *x = *(const bf_tensor *const *)a;
    const bf_tensor *y = *(const bf_tensor *const *)b;
    return strcmp(x->name, y->name);
}

static int parse_entry(const unsigned char *e, uint64_t file_bytes,
                       uint64_t data_offset, bf_tensor *t,
                       char *error, size_t cap) {
    const char *name = (const char *)e;
    if (!memchr(name, '\0', BF_MODEL_NAME_CAP))
        return report(error, cap, "tensor name is not terminated");
    if (!name[0]) return report(error, cap, "empty tensor name");
    uint32_t dtype = rd32(e + 96), rank = rd32(e + 100);
    if (rank > BF_MODEL_MAX_RANK)
        return report(error, cap, "%s: rank %u exceeds limit", name, rank);
    uint64_t item = dtype == BF_DTYPE_F32 ? 4 : dtype == BF_DTYPE_I64 ? 8 : 0;
    if (!item) return report(error, cap, "%s: unsupported dtype %u", name, dtype);
    uint64_t elements = 1;
    for (uint32_t i = 0; i < rank; ++i) {
        uint32_t d = rd32(e + 104 + 4 * i);
        if (!d) return report(error, cap, "%s: zero dimension", name);
        if (elements > UINT64_MAX / d)
            return report(error, cap, "%s: shape overflows", name);
        elements *= d;
        t->dims[i] = d;
    }
    for (uint32_t i = rank; i < BF_MODEL_MAX_RANK; ++i) t->dims[i] = 0;
    uint64_t offset = rd64(e + 136), nbytes = rd64(e + 144);
    if (elements > UINT64_MAX / item || elements * item != nbytes)
        return report(error, cap, "%s: shape byte count mismatch", name);
    if (offset % kAlign)
        return report(error, cap, "%s: data is not 64-byte aligned", name);
    if (offset < data_offset)
        return report(error, cap, "%s: data overlaps model metadata", name);
    if (offset > file_bytes || nbytes > file_bytes - offset)
        return report(error, cap, "%s: data range exceeds file", name);
    t->name = name;
    t->dtype = dtype;
    t->rank = rank;
    t->nbytes = nbytes;
    t->crc32 = rd32(e + 152);
    t->data = NULL; /* set by caller from the mapping base */
    return 1;
}

int bf_model_open(const char *path, bf_model **out, char *error, size_t cap) {
    if (out) *out = NULL;
    if (!path || !out) return report(error, cap, "invalid model arguments");
    int fd = open(path, O_RDONLY);
    if (fd < 0) return report(error, cap, "open %s: %s", path, strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < kHeaderBytes) {
        close(fd);
        return report(error, cap, "%s: truncated model", path);
    }
    size_t bytes = (size_t)st.st_size;
    void *map = mmap(NULL, bytes, PROT_READ, MAP_PRIVATE, fd, 0);
    if (map == MAP_FAILED) {
        close(fd);
        return report(error, cap, "mmap %s: %s", path, strerror(errno));
    }
    const unsigned char *h = (const unsigned char *)map;
    uint64_t count = rd64(h + 16), dir = rd64(h + 24), data = rd64(h + 32);
    int ok = memcmp(h, kMagic, 8) == 0 && rd32(h + 8) == BF_MODEL_VERSION &&
             rd32(h + 12) == kHeaderBytes && dir == kHeaderBytes &&
             rd64(h + 40) == bytes && count > 0 && count <= 1000000u &&
             data % kAlign == 0 && data >= dir && data <= bytes &&
             count * kEntryBytes <= data - dir;
    if (!ok) {
        munmap(map, bytes);
        close(fd);
        return report(error, cap, "%s: invalid BFW header", path);
    }
    if (crc32_of(h + dir, (size_t)(count * kEntryBytes)) != rd32(h + 48)) {
        munmap(map, bytes);
        close(fd);
        return report(error, cap, "%s: directory CRC mismatch", path);
    }
    bf_model *m = (bf_model *)calloc(1, sizeof(*m));
    bf_tensor *ts = (bf_tensor *)calloc((size_t)count, sizeof(*ts));
    const bf_tensor **ix = (const bf_tensor **)calloc((size_t)count, sizeof(*ix));
    if (!m || !ts || !ix) {
        free(m); free(ts); free(ix);
        munmap(map, bytes);
        close(fd);
        return report(error, cap, "tensor index allocation failed");
    }
    m->fd = fd; m->base = h; m->bytes = bytes; m->count = (size_t)count;
    m->tensors = ts; m->index = ix;
    for (size_t i = 0; i < m->count; ++i) {
        const unsigned char *e = h + dir + i * kEntryBytes;
        if (!parse_entry(e, bytes, data, &ts[i], error, cap)) {
            bf_model_close(m);
            return 0;
        }
        ts[i].data = h + rd64(e + 136);
        ix[i] = &ts[i];
    }
    qsort(ix, m->count, sizeof(*ix), by_name);
    for (size_t i = 1; i < m->count; ++i)
        if (strcmp(ix[i - 1]->name, ix[i]->name) == 0) {
            report(error, cap, "duplicate tensor %s", ix[i]->name);
            bf_model_close(m);
            return 0;
        }
    *out = m;
    return 1;
}

void bf_model_close(bf_model *m) {
    if (!m) return;
    if (m->base) munmap((void *)m->base, m->bytes);
    if (m->fd >= 0) close(m->fd);
    free(m->tensors);
    free(m->index);
    free(m);
}

size_t bf_model_tensor_count(const bf_model *m) { return m ? m->count : 0; }
uint64_t bf_model_file_bytes(const bf_model *m) { return m ? m->bytes : 0; }

const bf_tensor *bf_model_tensor_at(const bf_model *m, size_t i) {
    return m && i < m->count ? &m->tensors[i] : NULL;
}

const bf_tensor *bf_model_find(const bf_model *m, const char *name) {
    if (!m || !name) return NULL;
    size_t lo = 0, hi = m->count;
    while (lo < hi) {
        size_t mid = lo + (hi - lo) / 2;
        int c = strcmp(m->index[mid]->name, name);
        if (c == 0) return m->index[mid];
        if (c < 0) lo = mid + 1; else hi = mid;
    }
    return NULL;
}

int bf_model_validate_tensor(const bf_model *m, const bf_tensor *t,
                             char *error, size_t cap) {
    if (!m || !t || t < m->tensors || t >= m->tensors + m->count)
        return report(error, cap, "tensor does not belong to model");
    if (crc32_of(t->data, (size_t)t->nbytes) != t->crc32)
        return report(error, cap, "%s: data CRC mismatch", t->name);
    return 1;
}

int bf_model_validate_all(const bf_model *m, char *error, size_t cap) {
    if (!m) return report(error, cap, "model is null");
    for (size_t i = 0; i < m->count; ++i)
        if (!bf_model_validate_tensor(m, &m->tensors[i], error, cap)) return 0;
    return 1;
}

const char *bf_dtype_name(uint32_t dtype) {
    return dtype == BF_DTYPE_F32 ? "f32" : dtype == BF_DTYPE_I64 ? "i64" : "unknown";
}
