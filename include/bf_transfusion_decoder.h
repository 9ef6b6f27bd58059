/*
 * TransFusion decoder output buffers, shared by the CPU and GPU routes.
 *
 * Same type, field order and meaning as the reference's
 * include/bf_transfusion_decoder.h:10-24 (the CPU decoder functions that
 * header also declares stay in the reference's C library; this repository
 * restates them only as its test oracle, oracle/).  Every array is
 * channel-major over the P proposals of batch b:
 *
 *   center_b2p           [B,2,P]  cell-centre-relative x/y + the cell centre
 *   height_b1p           [B,1,P]
 *   dimension_log_b3p    [B,3,P]  log width/length/height
 *   rotation_sincos_b2p  [B,2,P]  sin, cos of yaw
 *   velocity_b2p         [B,2,P]
 *   heatmap_logits_b10p  [B,10,P] refined class logits
 *   query_heatmap_scores_b10p [B,10,P] NMS-suppressed dense scores at each
 *                        proposal's cell
 *   query_labels_bp, query_indices_bp [B,P] int64 class and flat cell index
 *                        (y * W + x) of each proposal
 */
#ifndef BF_TRANSFUSION_DECODER_H
#define BF_TRANSFUSION_DECODER_H

#include <stddef.h>
#include <stdint.h>

#define BF_TRANSFUSION_CLASSES 10u
#define BF_TRANSFUSION_CHANNELS 128u

typedef struct {
    float *center_b2p;
    float *height_b1p;
    float *dimension_log_b3p;
    float *rotation_sincos_b2p;
    float *velocity_b2p;
    float *heatmap_logits_b10p;
    float *query_heatmap_scores_b10p;
    int64_t *query_labels_bp;
    int64_t *query_indices_bp;
} bf_transfusion_raw_outputs;

#endif
