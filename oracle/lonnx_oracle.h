/*
 * lonnx_oracle.h -- TEST INFRASTRUCTURE ONLY: CPU restatement of the
 * Lokad.Onnx C# CPU operators, used as the parity checker and the CPU
 * baseline.  Never linked into the product library.
 */
#ifndef LONNX_ORACLE_H
#define LONNX_ORACLE_H
#include <stdint.h>

#define LXO_MAX_RANK 8

/* TensorElementType codes (Tensor.cs:31-50) */
enum {
    LXO_FLOAT = 1, LXO_UINT8 = 2, LXO_INT8 = 3, LXO_UINT16 = 4, LXO_INT16 = 5,
    LXO_INT32 = 6, LXO_INT64 = 7, LXO_BOOL = 9, LXO_DOUBLE = 11,
    LXO_UINT32 = 12, LXO_UINT64 = 13
};

/* binary ops */
enum { LXO_ADD = 0, LXO_SUB = 1, LXO_MUL = 2, LXO_DIV = 3, LXO_POW = 4 };
/* unary ops */
enum { LXO_SQRT = 0, LXO_ERF = 1, LXO_NEG = 2, LXO_EXP = 3 };
/* reductions */
enum { LXO_RSUM = 0, LXO_RMEAN = 1, LXO_RMAX = 2 };

/* status codes (same numbering as the product C-ABI's lx_status) */
enum {
    LXO_OK = 0,
    LXO_ERR_CANNOT_BROADCAST = 3,
    LXO_ERR_NOT_SUPPORTED = 5,
    LXO_ERR_ATTRIBUTE_NOT_SUPPORTED = 6,
    LXO_ERR_INVALID_ARGUMENT = 8,
    LXO_ERR_DIVIDE_BY_ZERO = 9,
    LXO_ERR_OVERFLOW = 10,
    LXO_ERR_OUT_OF_MEMORY = 11
};

int lxo_elem_size(int dtype);
int lxo_broadcast_shape(int ra, const int64_t *da, int rb, const int64_t *db, int *rout, int64_t *dout);
void lxo_materialize(int esize, int rsrc, const int64_t *dsrc, const void *src, int rout, const int64_t *dout, void *out);
int lxo_binary(int op, int dtype, int64_t n, const void *a, const void *b, void *out, int64_t *err_index);
int lxo_op_binary(int op, int dtype, int ra, const int64_t *da, const void *a, int rb, const int64_t *db,
                  const void *b, void *out, int *ry, int64_t *dy, int64_t *err_index);
float lxo_erf_f32(float x);
double lxo_erf_f64(double x);
float lxo_expf(float x);
float lxo_powf(float x, float y);
int lxo_unary(int op, int dtype, int64_t n, const void *in, void *out);
int lxo_cast(int src_dtype, int dst_dtype, int64_t n, const void *in, void *out);
int lxo_reduce(int op, int dtype, int rank, const int64_t *dims, const void *x, int naxes, const int64_t *axes,
               int keepdims, void *out, int *rout, int64_t *dout);
int lxo_softmax(int dtype, int rank, const int64_t *dims, const void *x, int axis, void *out);
int lxo_matmul2d(int dtype, int64_t M, int64_t N, int64_t K, const void *a, const void *b, void *c);
void lxo_gelu_chain(int64_t n, const float *x, float *y);

#endif
