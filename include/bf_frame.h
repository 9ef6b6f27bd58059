/*
 * BFI frame files (host side), served by libbfmodel.so.
 *
 * Drop-in for the reference's include/bf_frame.h:7-25 (implemented there by
 * src/frame.c:58-154); the file layout is the reference's, so frames packed
 * for it open here unchanged.  A BFI file is little-endian: a 128-byte
 * header -- "BFI1", u32 version 1 at byte 4, u32 header size 128 at 8, u64
 * file size at 16, u64 point count (> 0) at 24, u32 CRC-32 (IEEE, reflected
 * 0xEDB88320) of every byte after the header at 32, seven u64 payload
 * offsets at 40 -- followed, densely and in this order, by float32 images
 * [6,3,256,704], points [P,5], intrinsics [6,16], camera-to-lidar [6,16],
 * image augmentation [6,16], lidar augmentation [16] and lidar-to-image
 * [6,16].  open maps the file read-only and rejects any header, offset, size,
 * checksum or non-finite value that differs from that canonical form; the
 * bf_frame_input view points into the mapping and lives until close.
 */
#ifndef BF_FRAME_H
#define BF_FRAME_H

#include "bf_runtime.h"

#include <stddef.h>

#define BF_FRAME_VERSION 1u
#define BF_FRAME_HEADER_BYTES 128u

#ifdef __cplusplus
extern "C" {
#endif

typedef struct bf_frame_file bf_frame_file;

int bf_frame_open(const char *path, bf_frame_file **out,
                  char *error, size_t error_cap);
void bf_frame_close(bf_frame_file *file);
const bf_frame_input *bf_frame_input_view(const bf_frame_file *file);
size_t bf_frame_file_bytes(const bf_frame_file *file);

#ifdef __cplusplus
}
#endif

#endif
