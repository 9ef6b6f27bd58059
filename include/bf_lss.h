/*
 * Lift-splat-shoot pooling descriptor, shared by the CPU and GPU routes.
 *
 * Same type, field order and meaning as the reference's include/bf_lss.h:6-16
 * (the CPU functions that header also declares stay in the reference's C
 * library; this repository restates them only as its test oracle, oracle/).
 *
 *   batches, cameras        B, N
 *   depth_bins              D (<= 128 on the GPU routes)
 *   feature_height/_width   H, W of the depth/context maps
 *   channels                C of the context map
 *   grid_minimum/step/cells per axis x, y, z of the BEV grid; a point p lands
 *                           in cell trunc((p - minimum) / step) when that is in
 *                           [0, cells) on every axis.
 * The BEV output is [B, C*Z, X, Y] fp32 (OpenPCDet layout before its final
 * x/y permute).
 */
#ifndef BF_LSS_H
#define BF_LSS_H

#include <stddef.h>

typedef struct {
    size_t batches;
    size_t cameras;
    size_t depth_bins;
    size_t feature_height;
    size_t feature_width;
    size_t channels;
    float grid_minimum[3];
    float grid_step[3];
    size_t grid_cells[3];
} bf_lss_desc;

#endif
