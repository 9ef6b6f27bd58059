/*
 * Types shared by the sparse LiDAR entry points.
 *
 * Same names and layout as the reference's include/bf_kernels.h:34-46
 * (bf_coord4, bf_sparse_conv3d_desc).  The CPU operator functions that header
 * also declares stay in the reference's C library; this repository restates
 * them only as its test oracle (oracle/).
 */
#ifndef BF_KERNELS_H
#define BF_KERNELS_H

#include <stddef.h>
#include <stdint.h>

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
