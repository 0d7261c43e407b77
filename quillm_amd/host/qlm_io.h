/* .qlm reading and synthetic-model writing for the HIP host (C11).
 *
 * Format (reference src/qlm_file.h:1-9, little-endian):
 *   "QLMF" | u32 version=1 | u32 n_kv | u32 n_tensors | u64 data_offset
 *   n_kv x      { u32 key_len, key, u32 type (0 u32, 1 f32, 2 str, 3 u32 array), value }
 *   n_tensors x { u32 name_len, name, u32 dtype, u32 ndim, u64 ne[ndim], u64 offset }
 *   zero padding to data_offset (multiple of 64); tensor data at data_offset + offset (64-aligned)
 */
#ifndef QLM_IO_H
#define QLM_IO_H

#include <stddef.h>
#include <stdint.h>

#include "../../include/qmhip.h"

typedef struct {
    char name[64];
    qmh_tensor_view view;
} qlm_tensor;

typedef struct {
    uint8_t *map;
    size_t size;
    uint32_t n_tensors;
    qlm_tensor *tensors;
    qmh_config cfg;
    int have[7]; /* which required u32 keys were present */
} qlm_map;

size_t qlm_row_bytes(int dtype, int64_t n);
/* map + parse with bounds checks (as reference src/qlm_file.c:73-150 validates); 0 or -1 + err */
int qlm_map_open(qlm_map *f, const char *path, char *err, size_t errlen);
void qlm_map_close(qlm_map *f);
const qlm_tensor *qlm_map_find(const qlm_map *f, const char *name);

#endif
