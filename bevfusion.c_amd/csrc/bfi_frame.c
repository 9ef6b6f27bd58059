/* BFI frame reader (drop-in for reference src/frame.c:58-154; layout in
 * include/bf_frame.h).  The file is mapped read-only; every header field,
 * payload offset, the CRC-32 of the payload and the finiteness of every float
 * are checked before a view is handed out. */
#define _POSIX_C_SOURCE 200809L
#include "bf_frame.h"

#include <errno.h>
#include <fcntl.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

enum { kImages = 6 * 3 * 256 * 704, kMatrices = 6 * 16, kFields = 7 };

struct bf_frame_file {
    void *map;
    size_t bytes;
    bf_frame_input view;
};

static int frame_fail(char *error, size_t cap, const char *what) {
    if (error && cap) snprintf(error, cap, "%s", what);
    return 0;
}

static uint64_t le(const unsigned char *p, int bytes) {
    uint64_t v = 0;
    for (int i = bytes - 1; i >= 0; --i) v = v << 8 | p[i];
    return v;
}

/* CRC-32 (IEEE 802.3, reflected polynomial 0xEDB88320, initial and final
 * XOR 0xFFFFFFFF), one table lookup per byte. */
static uint32_t crc32_ieee(const unsigned char *data, size_t bytes) {
    static uint32_t table[256];
    static int ready;
    if (!ready) {
        for (uint32_t n = 0; n < 256; ++n) {
            uint32_t c = n;
            for (int k = 0; k < 8; ++k) c = c & 1u ? 0xedb88320u ^ (c >> 1) : c >> 1;
            table[n] = c;
        }
        ready = 1;
    }
    uint32_t c = 0xffffffffu;
    for (size_t i = 0; i < bytes; ++i) c = table[(c ^ data[i]) & 0xffu] ^ (c >> 8);
    return c ^ 0xffffffffu;
}

static int all_finite(const float *v, size_t n) {
    for (size_t i = 0; i < n; ++i)
        if (!isfinite(v[i])) return 0;
    return 1;
}

int bf_frame_open(const char *path, bf_frame_file **out, char *error, size_t cap) {
    if (out) *out = NULL;
    if (!path || !out) return frame_fail(error, cap, "invalid frame arguments");
    const uint16_t probe = 1;
    if (*(const unsigned char *)&probe != 1)
        return frame_fail(error, cap, "BFI requires a little-endian host");
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) {
        if (error && cap) snprintf(error, cap, "cannot open frame: %s", strerror(errno));
        return 0;
    }
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < (off_t)BF_FRAME_HEADER_BYTES) {
        close(fd);
        return frame_fail(error, cap, "invalid frame file size");
    }
    const size_t bytes = (size_t)st.st_size;
    void *map = mmap(NULL, bytes, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map == MAP_FAILED) return frame_fail(error, cap, "frame mmap failed");
    const unsigned char *p = (const unsigned char *)map;
    const uint64_t points = le(p + 24, 8);
    /* Canonical payload layout for this point count. */
    const uint64_t sizes[kFields] = {(uint64_t)kImages * 4, points * 20, kMatrices * 4,
                                     kMatrices * 4, kMatrices * 4, 16 * 4, kMatrices * 4};
    uint64_t at[kFields], end = BF_FRAME_HEADER_BYTES;
    int ok = memcmp(p, "BFI1", 4) == 0 && le(p + 4, 4) == BF_FRAME_VERSION &&
             le(p + 8, 4) == BF_FRAME_HEADER_BYTES && le(p + 16, 8) == bytes && points > 0 &&
             points <= bytes / 20;
    for (int f = 0; ok && f < kFields; ++f) {
        at[f] = end;
        ok = le(p + 40 + 8 * f, 8) == at[f] && (at[f] & 3u) == 0 && sizes[f] <= bytes - end;
        end += sizes[f];
    }
    ok = ok && end == bytes &&
         crc32_ieee(p + BF_FRAME_HEADER_BYTES, bytes - BF_FRAME_HEADER_BYTES) ==
             (uint32_t)le(p + 32, 4);
    if (!ok) {
        munmap(map, bytes);
        return frame_fail(error, cap, "malformed, non-canonical, or corrupt BFI frame");
    }
    bf_frame_file *file = (bf_frame_file *)calloc(1, sizeof(*file));
    if (!file) {
        munmap(map, bytes);
        return frame_fail(error, cap, "frame handle allocation failed");
    }
    file->map = map;
    file->bytes = bytes;
    const float *field[kFields];
    for (int f = 0; f < kFields; ++f) field[f] = (const float *)(p + at[f]);
    bf_frame_input *v = &file->view;
    v->camera_images = field[0];
    v->points = field[1];
    v->point_count = (size_t)points;
    v->camera_intrinsics_6x16 = field[2];
    v->camera_to_lidar_6x16 = field[3];
    v->image_augmentation_6x16 = field[4];
    v->lidar_augmentation_16 = field[5];
    v->lidar_to_image_6x16 = field[6];
    for (int f = 0; f < kFields; ++f)
        if (!all_finite(field[f], (size_t)(sizes[f] / 4))) {
            bf_frame_close(file);
            return frame_fail(error, cap, "BFI frame contains non-finite values");
        }
    *out = file;
    return 1;
}

void bf_frame_close(bf_frame_file *file) {
    if (!file) return;
    if (file->map) munmap(file->map, file->bytes);
    free(file);
}

const bf_frame_input *bf_frame_input_view(const bf_frame_file *file) {
    return file ? &file->view : NULL;
}

size_t bf_frame_file_bytes(const bf_frame_file *file) { return file ? file->bytes : 0; }
