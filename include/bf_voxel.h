/*
 * Voxelisation configuration and statistics.
 *
 * Same names and layout as the reference's include/bf_voxel.h:11-28.  The
 * CPU voxeliser itself stays in the reference's C library; this repository
 * restates it only as its test oracle (oracle/).
 */
#ifndef BF_VOXEL_H
#define BF_VOXEL_H

#include "bf_sparse_types.h"

#include <stddef.h>

typedef struct {
    float minimum[3];
    float maximum[3];
    float voxel_size[3];
    size_t point_features;
    size_t max_points_per_voxel;
    size_t max_voxels;
} bf_voxel_config;

typedef struct {
    size_t input_points;
    size_t accepted_points;
    size_t rejected_nonfinite;
    size_t rejected_out_of_range;
    size_t dropped_voxel_capacity;
    size_t dropped_point_capacity;
} bf_voxel_stats;

#endif
