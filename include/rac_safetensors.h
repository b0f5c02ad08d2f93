/*
 * rac_safetensors.h — safetensors weight loading for the MI355X library.
 *
 * Replaces bench/safetensors_reader.h:33-96: the same types, struct layout
 * and functions (a caller that reads f->n_tensors or t->shape keeps working),
 * with the element conversion done on the GPU.  Added: device-memory forms
 * that stream a tensor from the mapped file into HBM and convert it there,
 * to fp32 or straight to Q8_0 blocks (the rac_q8_0.h decode format).
 *
 * The file is mapped read-only; tensor pointers stay valid until st_close.
 * st_open validates every tensor's byte range against the file and, for the
 * known dtypes, its size against the shape (the reference does not check).
 */
#ifndef RAC_AMD_SAFETENSORS_H
#define RAC_AMD_SAFETENSORS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ST_MAX_TENSORS 8192
#define ST_MAX_NAME    256
#define ST_MAX_NDIM    8

typedef enum {
    ST_UNKNOWN = 0,
    ST_F32 = 1,
    ST_F16 = 2,
    ST_BF16 = 3,
    ST_F64 = 4,
    ST_I8 = 5,
    ST_U8 = 6,
    ST_I16 = 7,
    ST_I32 = 8,
    ST_I64 = 9,
    ST_BOOL = 10,
} st_dtype;

typedef struct {
    char name[ST_MAX_NAME];
    st_dtype dtype;
    int ndim;
    int64_t shape[ST_MAX_NDIM];
    size_t offset; /* relative to the start of the data segment */
    size_t nbytes;
} st_tensor;

typedef struct st_file {
    int fd;
    void *mmap_base;
    size_t mmap_len;
    size_t data_offset; /* 8 + header length */
    st_tensor *tensors;
    int n_tensors;
    char *header_copy; /* NUL-terminated copy of the header JSON */
    char err[256];
} st_file;

/* bench/safetensors_reader.h:73 — open and parse; NULL on failure with the
 * reason in errout (may be NULL) and rac_last_error(). */
st_file *st_open(const char *path, char errout[256]);

/* :76 — release everything; NULL is allowed. */
void st_close(st_file *f);

/* :79 — tensor by exact name, NULL when absent. */
const st_tensor *st_find(const st_file *f, const char *name);

/* :82 — the tensor's bytes inside the mapping (host memory; do not free). */
const void *st_data(const st_file *f, const st_tensor *t);

/* :87 — tensor as fp32 into `out` (prod(shape) floats; host or device
 * memory), converted on the GPU.  0 on success, -1 for dtypes other than
 * F32 / F16 / BF16 / F64 or on a device error (rac_last_error()). */
int st_to_f32(const st_file *f, const st_tensor *t, float *out);

/* :90 — number of elements (product of the shape). */
size_t st_numel(const st_tensor *t);

/* :93 — "F32", "BF16", ..., "UNKNOWN". */
const char *st_dtype_name(st_dtype d);

/* :96 — list the tensors on stdout. */
void st_dump(const st_file *f);

/* ── device forms (no counterpart in the reader; status codes 0, -1 null
 *    argument, -2 bad shape, -3 allocation, -4 HIP error, -5 dtype) ──── */

#define RAC_ST_ERR_DTYPE (-5)

/* Stream tensor t from the mapped file into device memory `out` as fp32
 * (numel floats), converting on the GPU; ordered on `stream`.  The call
 * returns once every byte has left the mapping (host memory may be unmapped
 * afterwards); the device work completes in stream order. */
int rac_st_to_f32_dev(const st_file *f, const st_tensor *t, float *out, void *stream);

/* Same, quantized to Q8_0 (rac_q8_0.h blocks, 34 bytes per 32 values) as
 * rac_q8_0_quantize_matrix would from the fp32 values: rows = numel / K,
 * K = the last dimension, which must be a multiple of 32. */
int rac_st_to_q8_0_dev(const st_file *f, const st_tensor *t, void *out_blocks, void *stream);

/* Conversions of raw safetensors bytes already in device memory:
 * n elements of `dtype` to fp32, or n_blocks * 32 of them to Q8_0. */
int rac_st_convert_dev(int dtype, const void *src, long n, float *out, void *stream);
int rac_st_quantize_dev(int dtype, const void *src, long n_blocks, void *out_blocks, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* RAC_AMD_SAFETENSORS_H */
