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
 * LN1) kernel of the stages that run it (stage 0), which refuse PROJ / FC1 /
 * FC2; the other stages refuse MLP.  WMSA is the fused QKV projection +
 * window attention of the stages that run it (stage 0), which refuse QKV and
 * ATTENTION; the other stages refuse WMSA.  No stage launches LN1 or LN2 any
 * more (the patch embedding and the fused MLP write stage 0's LN1, and stages
 * 1-3 fold both norms into their QKV and fc1 linears), so both are refused;
 * the ids stay reserved. */
enum {
    BFHIP_SWIN_LN1 = 0,
    BFHIP_SWIN_QKV = 1,
    BFHIP_SWIN_ATTENTION = 2,
    BFHIP_SWIN_PROJ = 3,
    BFHIP_SWIN_LN2 = 4,
    BFHIP_SWIN_FC1 = 5,
    BFHIP_SWIN_FC2 = 6,
    BFHIP_SWIN_MERGE = 7,
    BFHIP_SWIN_MLP = 8,
    BFHIP_SWIN_WMSA = 9
};

int bfhip_swin_profile_op(bf_cuda_swin *swin, int stage, int block, int op,
                          void *stream, char *error, size_t error_cap);

/* The Swin launches outside the blocks, on caller device buffers, at the
 * forward's shape and kernel instance:
 *   BFHIP_SWIN_PATCH_EMBED  the patch embedding (4x4/s4 conv + patch norm +
 *                           block 0's LN1): reads `images` [B,3,H,W];
 *                           `stage` must be 0;
 *   BFHIP_SWIN_OUT_NORM     the output LayerNorm of stage `stage` (1..3),
 *                           alone: writes `out`, the stage's NCHW output
 *                           (the forward runs it alone at stage 3);
 *   BFHIP_SWIN_MERGE_OUT_NORM  the patch merge after stage `stage` (1..2)
 *                           and that stage's output LayerNorm into `out`, in
 *                           one launch, as the forward runs them. */
enum {
    BFHIP_SWIN_PATCH_EMBED = 10,
    BFHIP_SWIN_OUT_NORM = 11,
    BFHIP_SWIN_MERGE_OUT_NORM = 12
};

int bfhip_swin_profile_io(bf_cuda_swin *swin, int stage, int op, const float *images, float *out,
                          void *stream, char *error, size_t error_cap);

/* Camera-neck convolution `layer` in the context's layer table: 0 lateral 1,
 * 1 fpn 1, 2 lateral 0, 3 fpn 0, 5 dtransform.6, 6 depthnet.0, 7 depthnet.3,
 * 9-11 downsample.  The forward runs each lateral as two launches: the
 * upper-level product, and the lower half (which adds the upsampled product)
 * in one launch with a depth-encoder conv.  So layers 0 and 2 here run the
 * upper-level product alone, and layer 5 runs dtransform.6 together with
 * lateral 0's lower half (the forward's launch).  Layers 4 (dtransform.3,
 * reads the caller's dense depth; shares its launch with lateral 1's lower
 * half) and 8 (depthnet.6, writes the caller's logits/context) are refused
 * here; bfhip_camera_profile_layer_io runs them on caller buffers.  Layer 11
 * here stores channels-last into context scratch instead of the transposed
 * caller output (bfhip_camera_profile_layer_io runs the forward's kernel). */
int bfhip_camera_profile_layer(bf_cuda_camera_neck *neck, int layer, void *stream,
                               char *error, size_t error_cap);

/* The layers whose forward launch reads or writes caller buffers, on caller
 * device buffers, at the forward's shape and kernel instance:
 *   4   dtransform.0 fused into dtransform.3: reads `input`, the dense depth
 *       [B,1,8h,8w]; runs in one launch with lateral 1's lower half;
 *   8   depthnet.6: writes `out0` (logits [B,118,h,w]) and `out1` (context
 *       [B,80,h,w]);
 *   11  the last downsample conv: writes `out0`, the x/y-transposed
 *       [1,80,bev_w/2,bev_h/2] output.
 * Unused pointers may be NULL. */
int bfhip_camera_profile_layer_io(bf_cuda_camera_neck *neck, int layer, const float *input,
                                  float *out0, float *out1, void *stream, char *error,
                                  size_t error_cap);

/* The neck's pack of the three Swin levels (NCHW fp32 [B,192,h,w],
 * [B,384,h1,w1], [B,768,h2,w2] -> channels-last fp16), one launch, as the
 * FPN forward runs it. */
int bfhip_camera_profile_pack(bf_cuda_camera_neck *neck, const float *s0, const float *s1,
                              const float *s2, void *stream, char *error, size_t error_cap);

/* Calibration kernels (machine rates for the roofline discussion).  Each
 * enqueues one launch of `grid` workgroups on `stream`:
 *   EMPTY   an empty kernel of 64 threads per workgroup (launch cost);
 *   MFMA16  256 threads, each wave `iters` x 8 independent
 *           v_mfma_f32_16x16x32_bf16 (16384 flops each);
 *   MFMA32  same with v_mfma_f32_32x32x16_bf16 (32768 flops each);
 *   LDS     256 threads, each `iters` (a multiple of 8) conflict-free 16-byte
 *           LDS reads, issued 8 at a time;
 *   COPY    a float4 copy of `bytes` from src to dst (16-byte aligned);
 *   MFMA_LDS         512 threads (8 waves); per iteration each wave reads
 *                    8 KiB of fragments from LDS and issues 32
 *                    v_mfma_f32_16x16x32_f16 on a 64 x 64 tile, operands
 *                    random fp16 values in [-1, 1);
 *   MFMA_LDS_FLAT    the same with constant small-integer operands;
 *   MFMA_LDS_NARROW  the same as MFMA_LDS on 32 x 32 tiles: per iteration
 *                    4 KiB of LDS reads and 8 MFMAs per wave (LDS-heavy);
 *   MFMA_LDS_NARROW_FLAT  MFMA_LDS_NARROW with constant operands.
 * For the compute kinds, dst may receive one float per thread when `bytes`
 * covers grid * threads floats (it keeps the work observable); otherwise
 * nothing is stored. */
enum {
    BFHIP_CALIB_EMPTY = 0,
    BFHIP_CALIB_MFMA16 = 1,
    BFHIP_CALIB_MFMA32 = 2,
    BFHIP_CALIB_LDS = 3,
    BFHIP_CALIB_COPY = 4,
    BFHIP_CALIB_MFMA_LDS = 5,
    BFHIP_CALIB_MFMA_LDS_FLAT = 6,
    BFHIP_CALIB_MFMA_LDS_NARROW = 7,
    BFHIP_CALIB_MFMA_LDS_NARROW_FLAT = 8
};

int bfhip_calibrate(int kind, int grid, int iters, const void *src, void *dst, size_t bytes,
                    void *stream, char *error, size_t error_cap);

#ifdef __cplusplus
}
#endif

#endif
