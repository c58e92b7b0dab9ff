/*
 * g2_host.h -- host-only helpers of libg2hip (safetensors reader, file
 * slurp, fp16 widening).  Not part of the public ABI.
 */
#ifndef G2_HOST_H
#define G2_HOST_H

#define _FILE_OFFSET_BITS 64
#include <stdint.h>
#include <stdio.h>

enum { G2H_ST_F32 = 0, G2H_ST_F16 = 1, G2H_ST_BF16 = 2, G2H_ST_OTHER = 3 };

typedef struct {
    char name[256];
    char dtype_name[16];
    int dtype, esize, ndim;
    int64_t shape[8];
    int64_t begin, end, numel;
} g2h_tensor;

typedef struct {
    FILE *fp;
    int64_t data_start;
    int n;
    g2h_tensor *t;
} g2h_st;

char *g2h_slurp(const char *path, size_t *size);
int g2h_st_open(const char *path, g2h_st *st);
void g2h_st_close(g2h_st *st);
const g2h_tensor *g2h_st_find(const g2h_st *st, const char *name);
int g2h_st_read_f32(const g2h_st *st, const g2h_tensor *t, float *dst, int64_t cap);
float g2h_f16_to_f32(uint16_t h);

#endif /* G2_HOST_H */
