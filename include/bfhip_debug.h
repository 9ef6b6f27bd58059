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
 *       host threads) race; calls queued on one stream do not.
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

#include "bf_cuda_runtime.h"

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

#ifdef __cplusplus
}
#endif

#endif
