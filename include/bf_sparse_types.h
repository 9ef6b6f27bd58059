/*
 * Types shared by the sparse LiDAR entry points: bf_coord4 and
 * bf_sparse_conv3d_desc, with the names and layout of the reference's
 * include/bf_kernels.h:34-46.
 *
 * The reference defines them in its CPU operator header, together with the
 * CPU operator declarations (bf_conv2d_f32, bf_linear_f32, ...) that this
 * library does not provide.  This header therefore has its own name and
 * guard: when the reference's bf_kernels.h is on the include path it is
 * included here and its definitions are used; otherwise the two types are
 * defined below.  Either include order then compiles, and nothing of the
 * reference's operator header is shadowed.
 */
#ifndef BFHIP_SPARSE_TYPES_H
#define BFHIP_SPARSE_TYPES_H

#include <stddef.h>
#include <stdint.h>

#if defined(__has_include)
#if __has_include("bf_kernels.h")
#include "bf_kernels.h"
#endif
#endif

#ifndef BF_KERNELS_H
typedef struct {
    int32_t batch, z, y, x;
} bf_coord4;

typedef struct {
    size_t batches, in_depth, in_height, in_width;
    size_t in_channels, out_channels;
    size_t kernel_depth, kernel_height, kernel_width;
    size_t stride_depth, stride_height, stride_width;
    size_t pad_depth, pad_height, pad_width;
    size_t dilation_depth, dilation_height, dilation_width;
    int submanifold;
} bf_sparse_conv3d_desc;
#endif

#endif
