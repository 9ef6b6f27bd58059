/*
 * TransFusion decoder context on AMD gfx950, served by libbfhip.so.
 *
 * Drop-in for the reference's include/bf_cuda_transfusion.h:14-39
 * (implemented there by src/cuda_transfusion.cu:283-418): same names,
 * argument meaning and error convention (1 = success, 0 = failure with a
 * message in error[0..error_cap)).
 *
 * create binds the decoder under the checkpoint's names (class encoding,
 * self / cross attention with their position-embedding heads, FFN, three
 * LayerNorms, six prediction heads) for a fixed BEV map of height x width
 * cells and `proposals` queries.  Contract, as the reference: height, width
 * and proposals nonzero, proposals <= BF_MAX_PROPOSALS (200),
 * 10 * height * width <= UINT32_MAX; this build also requires
 * proposals <= 10 * height * width (every query needs a candidate) and
 * 128 * height * width <= INT_MAX.
 *
 * forward: shared [1,128,H,W] and dense heatmap logits [1,10,H,W] fp32, and
 * every pointer inside *outputs_device, are device pointers (the struct
 * itself lives in host memory); stream is a hipStream_t or NULL.  Proposals
 * are the top `proposals` cells of the 3x3-NMS'd sigmoid heatmap ordered by
 * (score descending, flat index class * H * W + y * W + x ascending).
 * Forward allocates nothing and issues no memset or host synchronisation, so
 * it can be captured into a HIP graph; one forward at a time per context.
 *
 * decode_detections: decodes and range-filters one forward's raw outputs on
 * the GPU (box centre = cell * 0.6 - 54 m, keep score > threshold and
 * |x|, |y| <= 61.2, |z| <= 10), then copies one bf_detections to
 * detections_host and synchronises the stream.  Returns 0 for a non-finite
 * threshold or null buffers.
 */
#ifndef BF_CUDA_TRANSFUSION_H
#define BF_CUDA_TRANSFUSION_H

#include "bf_model.h"
#include "bf_transfusion_decoder.h"
#include "bevfusion.h"

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct bf_cuda_transfusion bf_cuda_transfusion;

int bf_cuda_transfusion_create(const bf_model *model,
                               size_t height, size_t width, size_t proposals,
                               bf_cuda_transfusion **out,
                               char *error, size_t error_cap);
void bf_cuda_transfusion_destroy(bf_cuda_transfusion *decoder);

int bf_cuda_transfusion_forward(bf_cuda_transfusion *decoder,
                                const float *shared_b128hw_device,
                                const float *dense_heatmap_b10hw_device,
                                bf_transfusion_raw_outputs *outputs_device,
                                void *stream,
                                char *error, size_t error_cap);

int bf_cuda_transfusion_decode_detections(bf_cuda_transfusion *decoder,
                                          const bf_transfusion_raw_outputs *outputs_device,
                                          float score_threshold,
                                          bf_detections *detections_host,
                                          void *stream,
                                          char *error, size_t error_cap);

size_t bf_cuda_transfusion_resident_bytes(const bf_cuda_transfusion *decoder);

#ifdef __cplusplus
}
#endif

#endif
