/*
 * Driver for the host file readers (bevfusion.c_amd/csrc/bfw_model.c and
 * bfi_frame.c) under AddressSanitizer and UndefinedBehaviorSanitizer; built
 * and run by tests/test_sanitize_readers.py with gcc (host code only).
 *
 *   san_readers bfw|bfi FILE...
 *
 * For each file it prints "begin FILE", then opens it.  A file the reader
 * rejects prints "rejected FILE: message".  An opened BFW model has every
 * tensor looked up by name, validated on its own and summed byte by byte,
 * then the whole model validated ("ok" or "invalid FILE: message"); an opened
 * BFI frame has every array of its view summed ("ok FILE points N").  Every
 * handle is closed, so LeakSanitizer also checks that close releases what
 * open acquired.  A sanitizer report ends the process with a non-zero status
 * right after the "begin" line of the file that caused it.
 */
#include "bf_frame.h"
#include "bf_model.h"

#include <stdint.h>
#include <stdio.h>
#include <string.h>

static unsigned long long sum_bytes(const void *data, size_t n) {
    const unsigned char *b = (const unsigned char *)data;
    unsigned long long s = 0;
    for (size_t i = 0; i < n; ++i) s += b[i];
    return s;
}

static int run_bfw(const char *path) {
    char error[256] = {0};
    bf_model *m = NULL;
    if (!bf_model_open(path, &m, error, sizeof(error))) {
        printf("rejected %s: %s\n", path, error);
        return 0;
    }
    const size_t n = bf_model_tensor_count(m);
    unsigned long long s = bf_model_file_bytes(m);
    int each = 1;
    for (size_t k = 0; k < n; ++k) {
        const bf_tensor *t = bf_model_tensor_at(m, k);
        if (!t) return 1;
        if (bf_model_find(m, t->name) == NULL) each = 0;
        s += strlen(t->name) + t->dtype + t->rank + sum_bytes(t->data, (size_t)t->nbytes);
        char e2[256] = {0};
        if (!bf_model_validate_tensor(m, t, e2, sizeof(e2))) each = 0;
        s += strlen(bf_dtype_name(t->dtype));
    }
    const int valid = bf_model_validate_all(m, error, sizeof(error));
    if (valid)
        printf("ok %s tensors %zu each %d sum %llu\n", path, n, each, s);
    else
        printf("invalid %s: %s\n", path, error);
    bf_model_close(m);
    return 0;
}

static int run_bfi(const char *path) {
    char error[256] = {0};
    bf_frame_file *f = NULL;
    if (!bf_frame_open(path, &f, error, sizeof(error))) {
        printf("rejected %s: %s\n", path, error);
        return 0;
    }
    const bf_frame_input *v = bf_frame_input_view(f);
    unsigned long long s = bf_frame_file_bytes(f);
    s += sum_bytes(v->camera_images, (size_t)6 * 3 * 256 * 704 * sizeof(float));
    s += sum_bytes(v->points, v->point_count * 5 * sizeof(float));
    s += sum_bytes(v->camera_intrinsics_6x16, 96 * sizeof(float));
    s += sum_bytes(v->camera_to_lidar_6x16, 96 * sizeof(float));
    s += sum_bytes(v->image_augmentation_6x16, 96 * sizeof(float));
    s += sum_bytes(v->lidar_augmentation_16, 16 * sizeof(float));
    s += sum_bytes(v->lidar_to_image_6x16, 96 * sizeof(float));
    printf("ok %s points %zu sum %llu\n", path, v->point_count, s);
    bf_frame_close(f);
    return 0;
}

int main(int argc, char **argv) {
    if (argc < 3 || (strcmp(argv[1], "bfw") != 0 && strcmp(argv[1], "bfi") != 0)) {
        fprintf(stderr, "usage: %s bfw|bfi FILE...\n", argv[0]);
        return 2;
    }
    const int bfw = strcmp(argv[1], "bfw") == 0;
    for (int i = 2; i < argc; ++i) {
        printf("begin %s\n", argv[i]);
        fflush(stdout);
        if (bfw ? run_bfw(argv[i]) : run_bfi(argv[i])) return 3;
        fflush(stdout);
    }
    return 0;
}
