/*
 * Index-map probes of libbfhip.so.  These have no counterpart in the
 * reference: they let a test compare the integer work of the Swin window path
 * bit for bit against the CPU oracle, on the device code the forward uses.
 *
 *   bfhip_debug_window_map
 *       For every window (n, wy, wx) of a [batches, height, width] token grid
 *       (padded up to multiples of 7, cyclic shift `shift`) and window token
 *       t < 49, writes at [((n*wy_n + wy)*wx_n + wx)*49 + t]:
 *         token[] = the source token row n*H*W + sy*W + sx, or -1 when the
 *                   padded source lies outside the map (a zero row);
 *         label[] = the shifted-window region label 3*ry + rx.
 *       Same device functions as the attention kernel (reference
 *       gather_windows_kernel / mask_region_device, src/cuda_swin.cu:120-134;
 *       cyclic_source / mask_region, src/swin.c:106-117).
 *
 *   bfhip_debug_window_attention
 *       Launches the production window-attention kernel on caller buffers:
 *       qkv fp16 [tokens, 3C] (token-major, tokens = batches*height*width),
 *       qkv_bias fp32 [3C], bias_mat fp32 [heads, 49, 49] (relative-position
 *       bias already gathered), out fp16 [tokens, C].  C = 32 * heads.
 *       qkv, qkv_bias and out must be 16-byte aligned.
 *       (fp16 is the Swin path's operand format.)
 *
 *   bfhip_debug_window_attention_noalloc
 *       The same operation with no allocation: no counterpart in the
 *       reference.  It is for callers that cannot call hipMalloc (code under
 *       HIP graph capture, serving loops that forbid allocation): the score
 *       terms go to a 1 MiB file-scope device array instead of a per-call
 *       buffer, and the call neither allocates nor synchronises.  At most 32
 *       heads (larger counts return 0 with a message); the stream must belong
 *       to the current device.  Every call on a device shares that device's
 *       array, so calls that overlap in time on one device (other streams or
 *       host threads) race; calls queued on one stream do not.  The array's
 *       device address is looked up on every call (a host-side lookup that
 *       allocates nothing), with the stream's device current.
 *
 *   bfhip_debug_camera_gather
 *       Runs the A-operand gather of camera-neck conv `layer` (the layer
 *       numbering of bfhip_camera_profile_layer: 1 fpn_convs.1, 3
 *       fpn_convs.0, 4 dtransform.3, 5 dtransform.6, 6 depthnet.0, 7
 *       depthnet.3, 8 depthnet.6, 9-11 downsample.0/.1/.2), with the tile,
 *       pipeline and loader instance the forward uses and the layer's
 *       geometry in `neck`, over identity weights: out fp32 [M, K] row-major
 *       (M = batch*OH*OW in the GEMM's row order, x-major for layer 11;
 *       K = KH*KW*Ci, k = (ky*KW + kx)*Ci + c) is the gathered operand,
 *       0 where a tap lies outside the map.  src0 is the layer's
 *       channels-last fp16 input [batch, IH, IW, Ci] (for layer 6 the
 *       64-channel depth features, with src1 the 256-channel fpn0 map; the
 *       downsample maps carry a 96-channel row stride), or for layer 4 the
 *       fp32 dense depth [batch, IH, IW], whose 8 channels per tap are
 *       fp16(relu(d * affine[c] + affine[8 + c])).  Reference addressing:
 *       cuda_ops.cu:23-56, cuda_camera.cu:219-271.
 *
 *   bfhip_debug_fpn_upsample
 *       The epilogue of lateral conv `level` (0: lateral_convs.0, upsampling
 *       level 1 to level 0; 1: lateral_convs.1, level 2 to level 1) over a
 *       zero product: out fp16 [batch, H, W, 256] = fp16(relu(bilinear(up)))
 *       with up fp32 [batch, h, w, 256] at the upper level's resolution
 *       (bilinear_channel, align_corners = False; image_fpn.c:123-142).
 *
 *   bfhip_debug_swin_merge_gather
 *       The patch merge after Swin stage `stage` (0-2) with its tile and
 *       gather instance, on caller tokens xh fp16 [batch, H, W, C], over
 *       identity weights put through the create-time column permutation:
 *       out fp32 [batch*H2*W2, 4C] is the reference's unfold matrix,
 *       out[m][c*4 + 2*ky + kx] = xh[n, 2*oy + ky, 2*ox + kx, c], 0 past an
 *       odd edge (swin_backbone.c:278-302).  16-byte aligned buffers.
 *
 *   bfhip_debug_runtime_fail_next
 *       Arms a one-shot failure in the next bf_cuda_runtime_infer of
 *       `runtime`: that call uploads the frame, queues the LSS cell-list
 *       rebuild if the calibration changed, then fails (returns 0) before
 *       the camera graph, draining both streams as any later failure does.
 *       Lets a test check that the calibration cache stays consistent with
 *       the queued cell lists across a failed frame.
 *
 * All pointers are device pointers; stream is a hipStream_t.  Returns 1 on
 * success, 0 with a message in error[0..error_cap).
 */
#ifndef BFHIP_DEBUG_H
#define BFHIP_DEBUG_H

#include "bf_cuda_camera.h"
#include "bf_cuda_runtime.h"
#include "bf_cuda_swin.h"

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

int bfhip_debug_window_map(int batches, int height, int width, int shift,
                           int *token_device, int *label_device, void *stream,
                           char *error, size_t error_cap);

int bfhip_debug_window_attention(const void *qkv_f16_device, const float *qkv_bias_device,
                                 const float *bias_mat_device, void *out_f16_device,
                                 int batches, int height, int width, int channels, int heads,
                                 int shift, void *stream, char *error, size_t error_cap);

int bfhip_debug_window_attention_noalloc(const void *qkv_f16_device,
                                         const float *qkv_bias_device,
                                         const float *bias_mat_device, void *out_f16_device,
                                         int batches, int height, int width, int channels,
                                         int heads, int shift, void *stream, char *error,
                                         size_t error_cap);

int bfhip_debug_runtime_fail_next(bf_cuda_runtime *runtime, char *error, size_t error_cap);

int bfhip_debug_camera_gather(bf_cuda_camera_neck *neck, int layer, const void *src0,
                              const void *src1, const float *affine, float *out, void *stream,
                              char *error, size_t error_cap);

int bfhip_debug_fpn_upsample(bf_cuda_camera_neck *neck, int level, const float *up,
                             void *out_f16, void *stream, char *error, size_t error_cap);

int bfhip_debug_swin_merge_gather(bf_cuda_swin *swin, int stage, const void *xh_f16, float *out,
                                  void *stream, char *error, size_t error_cap);

#ifdef __cplusplus
}
#endif

#endif
