/*
 * Profiling hooks of libbfhip.so.  These have no counterpart in the
 * reference: they exist so a benchmark can time one kernel of the path in
 * isolation with HIP events, at the exact shape and kernel instance the
 * forward uses (the reference instead records CUDA events per stage inside
 * its forward, src/cuda_swin.cu:358-417).
 *
 * Each call enqueues exactly the kernel(s) of one op on `stream`, reading
 * and writing the context's own scratch buffers; it changes context scratch
 * contents, never the weights, and the next forward recomputes everything.
 * Returns 1 on success, 0 with a message in error[0..error_cap).
 */
#ifndef BFHIP_PROFILE_H
#define BFHIP_PROFILE_H

#include "bf_cuda_camera.h"
#include "bf_cuda_swin.h"

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Ops of one Swin block, in forward order; MERGE is the patch merge that
 * follows stage `stage` (0..2; `block` is ignored).  MLP is the fused
 * proj -> residual -> LN2 -> fc1 -> GELU -> fc2 -> residual (+ next block's
 * LN1) kernel of the stages that run it (stage 0); those stages launch LN1
 * only in block 0 and refuse PROJ / LN2 / FC1 / FC2, the other stages refuse
 * MLP. */
enum {
    BFHIP_SWIN_LN1 = 0,
    BFHIP_SWIN_QKV = 1,
    BFHIP_SWIN_ATTENTION = 2,
    BFHIP_SWIN_PROJ = 3,
    BFHIP_SWIN_LN2 = 4,
    BFHIP_SWIN_FC1 = 5,
    BFHIP_SWIN_FC2 = 6,
    BFHIP_SWIN_MERGE = 7,
    BFHIP_SWIN_MLP = 8
};

int bfhip_swin_profile_op(bf_cuda_swin *swin, int stage, int block, int op,
                          void *stream, char *error, size_t error_cap);

/* Camera-neck convolution `layer` in the context's layer table: 0 lateral 1,
 * 1 fpn 1, 2 lateral 0, 3 fpn 0, 5 dtransform.6, 6 depthnet.0, 7 depthnet.3,
 * 9-11 downsample.  Layers 4 (dtransform.3, reads the caller's dense depth)
 * and 8 (depthnet.6, writes the caller's logits/context) are refused. */
int bfhip_camera_profile_layer(bf_cuda_camera_neck *neck, int layer, void *stream,
                               char *error, size_t error_cap);

#ifdef __cplusplus
}
#endif

#endif
