/*
 * lonnx_oracle.c -- TEST INFRASTRUCTURE ONLY.
 *
 * CPU restatement of the Lokad.Onnx C# CPU path for the elementwise /
 * broadcast / reduction operators (Add, Sub, Mul, Div, Pow, Sqrt, Erf, Cast,
 * ReduceSum, ReduceMean, ReduceMax, Softmax).  It is the checker that the HIP
 * library is compared against, and the "port" CPU baseline timed by bench.py.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it.  The product library never links or calls it.
 *
 * Structure follows the reference's Speed-mode path: broadcast operands are
 * materialised into dense copies, reductions over non-innermost axes transpose
 * first and then fold serially, transcendental functions call the host libm
 * (.NET's MathF.Exp / MathF.Pow / Math.Exp forward to it).
 *
 * Build: gcc -O2 -ffp-contract=off -fno-builtin (no FMA contraction, no
 * constant folding of powf/expf) -- see oracle/Makefile.
 *
 * Pinning of each function (what checks it besides this text) is listed in the
 * header comment of tests/test_oracle.py.  Nothing here is "parity unpinned"
 * except where stated at the function.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "lonnx_oracle.h"

/* ------------------------------------------------------------------------ */
/* element sizes for TensorElementType codes (Tensor.cs:31-50)              */
/* ------------------------------------------------------------------------ */
int lxo_elem_size(int dtype)
{
    switch (dtype) {
    case LXO_FLOAT: return 4;
    case LXO_UINT8: return 1;
    case LXO_INT8: return 1;
    case LXO_UINT16: return 2;
    case LXO_INT16: return 2;
    case LXO_INT32: return 4;
    case LXO_INT64: return 8;
    case LXO_BOOL: return 1;
    case LXO_DOUBLE: return 8;
    case LXO_UINT32: return 4;
    case LXO_UINT64: return 8;
    default: return 0;
    }
}

static int64_t numel(int rank, const int64_t *dims)
{
    int64_t n = 1;
    for (int i = 0; i < rank; i++) n *= dims[i];
    return n;
}

/* ------------------------------------------------------------------------ */
/* Broadcast shape: ITensor.Broadcast (ITensor.cs:64-120).                  */
/* A rank-0 operand takes the other's shape (66-83); otherwise ranks are    */
/* right-aligned, missing leading axes are inserted and broadcast (92-101), */
/* equal axes kept, size-1 axes broadcast (105-112), else failure (113-117).*/
/* Returns 0 on success, -1 when the shapes cannot be broadcast.            */
/* ------------------------------------------------------------------------ */
int lxo_broadcast_shape(int ra, const int64_t *da, int rb, const int64_t *db,
                        int *rout, int64_t *dout)
{
    if (ra == 0 && rb != 0) {
        *rout = rb;
        memcpy(dout, db, sizeof(int64_t) * rb);
        return 0;
    }
    if (rb == 0 && ra != 0) {
        *rout = ra;
        memcpy(dout, da, sizeof(int64_t) * ra);
        return 0;
    }
    int r = ra > rb ? ra : rb;
    for (int i = 0; i < r; i++) {
        int ia = i - r + ra, ib = i - r + rb;
        if (i < r - ra) dout[i] = db[ib];
        else if (i < r - rb) dout[i] = da[ia];
        else if (da[ia] == db[ib]) dout[i] = da[ia];
        else if (da[ia] == 1) dout[i] = db[ib];
        else if (db[ib] == 1) dout[i] = da[ia];
        else return -1;
    }
    *rout = r;
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Materialisation of a broadcast view: Tensor.ToDenseTensor over a         */
/* BroadcastedTensor (Tensor.cs:1605-1613, BroadcastedTensor.cs:24-53):     */
/* dense[index] = source[sum_k effStride_k * index_k] with effStride 0 on   */
/* broadcast axes.  Walks the output with an N-d odometer like              */
/* TensorDimensionsIterator.Next (TensorDimensionsIterator.cs:72-99).       */
/* ------------------------------------------------------------------------ */
void lxo_materialize(int esize, int rsrc, const int64_t *dsrc, const void *src,
                     int rout, const int64_t *dout, void *out)
{
    int64_t n = numel(rout, dout);
    if (n == 0) return;
    if (rsrc == 0) { /* rank-0 expansion loop, ITensor.cs:66-83 */
        for (int64_t i = 0; i < n; i++)
            memcpy((char *)out + i * esize, src, esize);
        return;
    }
    int64_t eff[LXO_MAX_RANK] = {0};
    int64_t idx[LXO_MAX_RANK] = {0};
    /* source strides right-aligned into the output rank */
    int64_t s = 1;
    for (int k = rsrc - 1; k >= 0; k--) {
        int o = k + (rout - rsrc);
        eff[o] = (dsrc[k] == 1 && dout[o] != 1) ? 0 : s;
        s *= dsrc[k];
    }
    int64_t off = 0;
    for (int64_t i = 0; i < n; i++) {
        memcpy((char *)out + i * esize, (const char *)src + off * esize, esize);
        for (int k = rout - 1; k >= 0; k--) {
            idx[k]++;
            off += eff[k];
            if (idx[k] < dout[k]) break;
            off -= eff[k] * idx[k];
            idx[k] = 0;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Elementwise binary kernels over dense operands of equal length           */
/* (VectorizedApply / Apply, TensorOps.cs:68-116; typed ops 235-297).       */
/* Integer semantics are C# unchecked arithmetic: two's-complement wrap,    */
/* division truncating toward zero, x/0 -> DivideByZeroException,           */
/* MIN/-1 -> OverflowException.  The loop stops at the first throwing       */
/* element like the C# loop does; *err_index receives its index.            */
/* byte: (byte)(l op r) after int promotion (TensorOps.cs:235, 253, 271,    */
/* 289).  int64 has no overload in the reference (C# semantics restated).   */
/* Pow: MathF.Pow / Math.Pow -> host powf / pow (TensorOps.cs:307-309).     */
/* ------------------------------------------------------------------------ */
#define BIN_INT_LOOP(T, UT, MINV)                                            \
    do {                                                                     \
        const T *x = (const T *)a; const T *y = (const T *)b; T *z = (T *)out;\
        for (int64_t i = 0; i < n; i++) {                                    \
            T l = x[i], r = y[i];                                            \
            switch (op) {                                                    \
            case LXO_ADD: z[i] = (T)((UT)l + (UT)r); break;                  \
            case LXO_SUB: z[i] = (T)((UT)l - (UT)r); break;                  \
            case LXO_MUL: z[i] = (T)((UT)l * (UT)r); break;                  \
            case LXO_DIV:                                                    \
                if (r == 0) { *err_index = i; return LXO_ERR_DIVIDE_BY_ZERO; }\
                if (l == (MINV) && r == -1) { *err_index = i; return LXO_ERR_OVERFLOW; }\
                z[i] = l / r; break;                                         \
            default: return LXO_ERR_NOT_SUPPORTED;                           \
            }                                                                \
        }                                                                    \
    } while (0)

int lxo_binary(int op, int dtype, int64_t n, const void *a, const void *b,
               void *out, int64_t *err_index)
{
    int64_t dummy;
    if (!err_index) err_index = &dummy;
    *err_index = -1;
    switch (dtype) {
    case LXO_FLOAT: {
        const float *x = (const float *)a, *y = (const float *)b;
        float *z = (float *)out;
        switch (op) {
        case LXO_ADD: for (int64_t i = 0; i < n; i++) z[i] = x[i] + y[i]; break;
        case LXO_SUB: for (int64_t i = 0; i < n; i++) z[i] = x[i] - y[i]; break;
        case LXO_MUL: for (int64_t i = 0; i < n; i++) z[i] = x[i] * y[i]; break;
        case LXO_DIV: for (int64_t i = 0; i < n; i++) z[i] = x[i] / y[i]; break;
        case LXO_POW: for (int64_t i = 0; i < n; i++) z[i] = powf(x[i], y[i]); break;
        default: return LXO_ERR_NOT_SUPPORTED;
        }
        return 0;
    }
    case LXO_DOUBLE: {
        const double *x = (const double *)a, *y = (const double *)b;
        double *z = (double *)out;
        switch (op) {
        case LXO_ADD: for (int64_t i = 0; i < n; i++) z[i] = x[i] + y[i]; break;
        case LXO_SUB: for (int64_t i = 0; i < n; i++) z[i] = x[i] - y[i]; break;
        case LXO_MUL: for (int64_t i = 0; i < n; i++) z[i] = x[i] * y[i]; break;
        case LXO_DIV: for (int64_t i = 0; i < n; i++) z[i] = x[i] / y[i]; break;
        case LXO_POW: for (int64_t i = 0; i < n; i++) z[i] = pow(x[i], y[i]); break;
        default: return LXO_ERR_NOT_SUPPORTED;
        }
        return 0;
    }
    case LXO_UINT8: {
        const uint8_t *x = (const uint8_t *)a, *y = (const uint8_t *)b;
        uint8_t *z = (uint8_t *)out;
        for (int64_t i = 0; i < n; i++) {
            int l = x[i], r = y[i];
            switch (op) {
            case LXO_ADD: z[i] = (uint8_t)(l + r); break;
            case LXO_SUB: z[i] = (uint8_t)(l - r); break;
            case LXO_MUL: z[i] = (uint8_t)(l * r); break;
            case LXO_DIV:
                if (r == 0) { *err_index = i; return LXO_ERR_DIVIDE_BY_ZERO; }
                z[i] = (uint8_t)(l / r); break;
            default: return LXO_ERR_NOT_SUPPORTED;
            }
        }
        return 0;
    }
    case LXO_INT32: BIN_INT_LOOP(int32_t, uint32_t, INT32_MIN); return 0;
    case LXO_INT64: BIN_INT_LOOP(int64_t, uint64_t, INT64_MIN); return 0;
    default: return LXO_ERR_NOT_SUPPORTED;
    }
}

/* ------------------------------------------------------------------------ */
/* Whole binary operator as CPUExecutionProvider.Add/Sub/Mul/Div/Pow runs it */
/* in Speed mode (CPUExecutionProvider.cs:82-236): broadcast shapes,        */
/* materialise both operands (ToDenseTensor), then the dense loop.          */
/* Output shape is written to (*ry, dy).                                    */
/* ------------------------------------------------------------------------ */
int lxo_op_binary(int op, int dtype,
                  int ra, const int64_t *da, const void *a,
                  int rb, const int64_t *db, const void *b,
                  void *out, int *ry, int64_t *dy, int64_t *err_index)
{
    int es = lxo_elem_size(dtype);
    if (!es) return LXO_ERR_NOT_SUPPORTED;
    if (lxo_broadcast_shape(ra, da, rb, db, ry, dy) != 0) return LXO_ERR_CANNOT_BROADCAST;
    int64_t n = numel(*ry, dy);
    void *ma = malloc(n * es + 1), *mb = malloc(n * es + 1);
    if (!ma || !mb) { free(ma); free(mb); return LXO_ERR_OUT_OF_MEMORY; }
    lxo_materialize(es, ra, da, a, *ry, dy, ma);
    lxo_materialize(es, rb, db, b, *ry, dy, mb);
    int st = lxo_binary(op, dtype, n, ma, mb, out, err_index);
    free(ma);
    free(mb);
    return st;
}

/* ------------------------------------------------------------------------ */
/* Erf: MathOps.Erf(float) (MathOps.cs:988-1010), Abramowitz & Stegun       */
/* 7.1.26 evaluated in float32, every operation rounded separately,         */
/* exp = MathF.Exp = host expf.  Double twin MathOps.cs:1012-1034.           */
/* ------------------------------------------------------------------------ */
float lxo_erf_f32(float x)
{
    const float a1 = 0.254829592f;
    const float a2 = -0.284496736f;
    const float a3 = 1.421413741f;
    const float a4 = -1.453152027f;
    const float a5 = 1.061405429f;
    const float p = 0.3275911f;
    int sign = 1;
    if (x < 0) sign = -1;
    x = fabsf(x);
    float t = 1.0f / (1.0f + p * x);
    float poly = ((((a5 * t + a4) * t) + a3) * t + a2) * t + a1;
    float e = expf(-x * x);
    float y = 1.0f - poly * t * e;
    return (float)sign * y;
}

double lxo_erf_f64(double x)
{
    const double a1 = 0.254829592;
    const double a2 = -0.284496736;
    const double a3 = 1.421413741;
    const double a4 = -1.453152027;
    const double a5 = 1.061405429;
    const double p = 0.3275911;
    int sign = 1;
    if (x < 0) sign = -1;
    x = fabs(x);
    double t = 1.0 / (1.0 + p * x);
    double poly = ((((a5 * t + a4) * t) + a3) * t + a2) * t + a1;
    double e = exp(-x * x);
    double y = 1.0 - poly * t * e;
    return (double)sign * y;
}

float lxo_expf(float x) { return expf(x); }
float lxo_powf(float x, float y) { return powf(x, y); }

/* ------------------------------------------------------------------------ */
/* Unary: Sqrt (TensorOps.cs:315-317, MathF.Sqrt / Vector.SquareRoot,       */
/* correctly rounded), Erf (TensorOps.cs:1353-1355), Neg (299-301),         */
/* Exp (the Apply(MathF.Exp) step of Softmax, TensorOps.cs:1323).           */
/* ------------------------------------------------------------------------ */
int lxo_unary(int op, int dtype, int64_t n, const void *in, void *out)
{
    if (dtype == LXO_FLOAT) {
        const float *x = (const float *)in;
        float *y = (float *)out;
        switch (op) {
        case LXO_SQRT: for (int64_t i = 0; i < n; i++) y[i] = sqrtf(x[i]); return 0;
        case LXO_ERF: for (int64_t i = 0; i < n; i++) y[i] = lxo_erf_f32(x[i]); return 0;
        case LXO_NEG: for (int64_t i = 0; i < n; i++) y[i] = -x[i]; return 0;
        case LXO_EXP: for (int64_t i = 0; i < n; i++) y[i] = expf(x[i]); return 0;
        default: return LXO_ERR_NOT_SUPPORTED;
        }
    }
    if (dtype == LXO_DOUBLE) {
        const double *x = (const double *)in;
        double *y = (double *)out;
        switch (op) {
        case LXO_SQRT: for (int64_t i = 0; i < n; i++) y[i] = sqrt(x[i]); return 0;
        case LXO_ERF: for (int64_t i = 0; i < n; i++) y[i] = lxo_erf_f64(x[i]); return 0;
        case LXO_NEG: for (int64_t i = 0; i < n; i++) y[i] = -x[i]; return 0;
        case LXO_EXP: for (int64_t i = 0; i < n; i++) y[i] = exp(x[i]); return 0;
        default: return LXO_ERR_NOT_SUPPORTED;
        }
    }
    return LXO_ERR_NOT_SUPPORTED;
}

/* ------------------------------------------------------------------------ */
/* Cast: ITensor.Cast<U> (ITensor.cs:161-170):                              */
/*   output[i] = (U)Convert.ChangeType(input[i], typeof(U))                 */
/* i.e. .NET System.Convert rules:                                          */
/*  - integer -> integer: value must be representable, else Overflow;       */
/*  - float/double -> Int32, Int16, UInt16, Byte, SByte: round half to even  */
/*    within [-2147483648.5, 2147483647.5) (Convert.ToInt32(double)), then  */
/*    the narrow range check;  -> UInt32: (-0.5, 4294967295.5) round half   */
/*    even;  -> Int64 / UInt64: checked((long)Math.Round(v));  NaN always   */
/*    overflows;                                                             */
/*  - anything -> Bool: value != 0;  Bool -> number: 1 / 0;                  */
/*  - integer -> float/double: one IEEE round-to-nearest-even conversion;    */
/*  - double -> float: (float)v.                                             */
/* The C# loop throws on the first failing element; only the status is      */
/* reported here (OverflowException -> OpResult.Failure).                    */
/* ------------------------------------------------------------------------ */
typedef struct { int kind; int64_t i; uint64_t u; double f; } lxo_val; /* kind 0 int,1 uint,2 float */

static lxo_val load_val(int dt, const void *p, int64_t k)
{
    lxo_val v = {0, 0, 0, 0.0};
    switch (dt) {
    case LXO_BOOL: v.kind = 0; v.i = ((const uint8_t *)p)[k] != 0; break;
    case LXO_UINT8: v.kind = 0; v.i = ((const uint8_t *)p)[k]; break;
    case LXO_INT8: v.kind = 0; v.i = ((const int8_t *)p)[k]; break;
    case LXO_UINT16: v.kind = 0; v.i = ((const uint16_t *)p)[k]; break;
    case LXO_INT16: v.kind = 0; v.i = ((const int16_t *)p)[k]; break;
    case LXO_INT32: v.kind = 0; v.i = ((const int32_t *)p)[k]; break;
    case LXO_UINT32: v.kind = 0; v.i = ((const uint32_t *)p)[k]; break;
    case LXO_INT64: v.kind = 0; v.i = ((const int64_t *)p)[k]; break;
    case LXO_UINT64: v.kind = 1; v.u = ((const uint64_t *)p)[k]; break;
    case LXO_FLOAT: v.kind = 2; v.f = ((const float *)p)[k]; break;
    case LXO_DOUBLE: v.kind = 2; v.f = ((const double *)p)[k]; break;
    }
    return v;
}

/* Convert.ToInt32(double): round half to even inside the allowed window */
static int to_i32_from_double(double d, int64_t *o)
{
    if (!(d >= -2147483648.5 && d < 2147483647.5)) return -1;
    *o = (int64_t)nearbyint(d);
    return 0;
}

static int store_val(int dt, void *p, int64_t k, lxo_val v)
{
    int64_t iv = 0;
    if (dt == LXO_BOOL) {
        uint8_t bv;
        if (v.kind == 2) bv = v.f != 0.0;
        else if (v.kind == 1) bv = v.u != 0;
        else bv = v.i != 0;
        ((uint8_t *)p)[k] = bv;
        return 0;
    }
    if (dt == LXO_FLOAT) {
        float f;
        if (v.kind == 2) f = (float)v.f;      /* float source: exact round trip */
        else if (v.kind == 1) f = (float)v.u;
        else f = (float)v.i;
        ((float *)p)[k] = f;
        return 0;
    }
    if (dt == LXO_DOUBLE) {
        double f;
        if (v.kind == 2) f = v.f;
        else if (v.kind == 1) f = (double)v.u;
        else f = (double)v.i;
        ((double *)p)[k] = f;
        return 0;
    }
    /* integer targets */
    if (dt == LXO_UINT64) {
        uint64_t u;
        if (v.kind == 2) {
            double r = nearbyint(v.f);
            if (!(r > -1.0 && r < 18446744073709551616.0)) return -1;
            u = (uint64_t)(r < 0 ? 0.0 : r);
        } else if (v.kind == 1) u = v.u;
        else { if (v.i < 0) return -1; u = (uint64_t)v.i; }
        ((uint64_t *)p)[k] = u;
        return 0;
    }
    if (dt == LXO_INT64) {
        int64_t s;
        if (v.kind == 2) {
            double r = nearbyint(v.f);
            if (!(r >= -9223372036854775808.0 && r < 9223372036854775808.0)) return -1;
            s = (int64_t)r;
        } else if (v.kind == 1) { if (v.u > (uint64_t)INT64_MAX) return -1; s = (int64_t)v.u; }
        else s = v.i;
        ((int64_t *)p)[k] = s;
        return 0;
    }
    if (dt == LXO_UINT32) {
        if (v.kind == 2) {
            if (!(v.f > -0.5 && v.f < 4294967295.5)) return -1;
            iv = (int64_t)nearbyint(v.f);
        } else if (v.kind == 1) { if (v.u > 0xFFFFFFFFull) return -1; iv = (int64_t)v.u; }
        else iv = v.i;
        if (iv < 0 || iv > 0xFFFFFFFFll) return -1;
        ((uint32_t *)p)[k] = (uint32_t)iv;
        return 0;
    }
    /* Int32, Int16, UInt16, Int8, UInt8: floating sources go through ToInt32 */
    if (v.kind == 2) { if (to_i32_from_double(v.f, &iv)) return -1; }
    else if (v.kind == 1) { if (v.u > (uint64_t)INT64_MAX) return -1; iv = (int64_t)v.u; }
    else iv = v.i;
    switch (dt) {
    case LXO_INT32: if (iv < INT32_MIN || iv > INT32_MAX) return -1; ((int32_t *)p)[k] = (int32_t)iv; return 0;
    case LXO_INT16: if (iv < INT16_MIN || iv > INT16_MAX) return -1; ((int16_t *)p)[k] = (int16_t)iv; return 0;
    case LXO_UINT16: if (iv < 0 || iv > UINT16_MAX) return -1; ((uint16_t *)p)[k] = (uint16_t)iv; return 0;
    case LXO_INT8: if (iv < INT8_MIN || iv > INT8_MAX) return -1; ((int8_t *)p)[k] = (int8_t)iv; return 0;
    case LXO_UINT8: if (iv < 0 || iv > UINT8_MAX) return -1; ((uint8_t *)p)[k] = (uint8_t)iv; return 0;
    }
    return -2;
}

int lxo_cast(int src_dtype, int dst_dtype, int64_t n, const void *in, void *out)
{
    if (!lxo_elem_size(src_dtype)) return LXO_ERR_NOT_SUPPORTED;
    if (!lxo_elem_size(dst_dtype)) return LXO_ERR_ATTRIBUTE_NOT_SUPPORTED;
    for (int64_t i = 0; i < n; i++) {
        lxo_val v = load_val(src_dtype, in, i);
        if (src_dtype == LXO_FLOAT && dst_dtype == LXO_FLOAT) { ((float *)out)[i] = ((const float *)in)[i]; continue; }
        int st = store_val(dst_dtype, out, i, v);
        if (st == -1) return LXO_ERR_OVERFLOW;
        if (st != 0) return LXO_ERR_NOT_SUPPORTED;
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Transpose (TensorOps.cs:1358-1407): r[perm-index] = data[index].          */
/* ------------------------------------------------------------------------ */
static void transpose(int es, int rank, const int64_t *dims, const void *src,
                      const int *perm, void *dst)
{
    int64_t n = numel(rank, dims);
    int64_t rdims[LXO_MAX_RANK], rstr[LXO_MAX_RANK], idx[LXO_MAX_RANK] = {0};
    for (int i = 0; i < rank; i++) rdims[i] = dims[perm[i]];
    int64_t s = 1;
    for (int i = rank - 1; i >= 0; i--) { rstr[i] = s; s *= rdims[i]; }
    /* output stride seen from input axis perm[i] */
    int64_t in_to_out[LXO_MAX_RANK];
    for (int i = 0; i < rank; i++) in_to_out[perm[i]] = rstr[i];
    int64_t off = 0;
    for (int64_t i = 0; i < n; i++) {
        memcpy((char *)dst + off * es, (const char *)src + i * es, es);
        for (int k = rank - 1; k >= 0; k--) {
            idx[k]++;
            off += in_to_out[k];
            if (idx[k] < dims[k]) break;
            off -= in_to_out[k] * idx[k];
            idx[k] = 0;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Reductions: Tensor<T>.ReduceSum / ReduceMean / ReduceMax                 */
/* (TensorOps.cs:1561-1891) with ArrayUtilities helpers (328-394):          */
/*  - axes null/empty => all axes; negative axes normalised;               */
/*  - if the axes are not the innermost ones in order, Transpose with      */
/*    permutation [kept axes..., axes as given] (GetAxesPermutationFor-    */
/*    Reduction) then fold the r = prod(reduced dims) innermost elements;  */
/*  - fold: acc = 0; for j in 0..r-1: acc += x  (float acc for float,      */
/*    wrapping int for int32/int64, double for double);                    */
/*  - ReduceMean float: sum, then out / (float)r (1747-1751);               */
/*    ReduceMean int32 / double: x / r per element first, then sum         */
/*    (1723-1724, 1777-1778);                                               */
/*  - ReduceMax: acc = 0 seed, acc = v if v > acc (1820-1827).              */
/* Output shape: kept dims, plus 1s at the reduced axes when keepdims.      */
/* ------------------------------------------------------------------------ */
static int normalize_axes(int rank, int naxes, const int64_t *axes, int *ax, int *nax)
{
    if (naxes > rank) return LXO_ERR_INVALID_ARGUMENT;
    if (naxes <= 0) {
        for (int i = 0; i < rank; i++) ax[i] = i;
        *nax = rank;
        return 0;
    }
    for (int i = 0; i < naxes; i++) {
        if (axes[i] >= rank) return LXO_ERR_INVALID_ARGUMENT;
        for (int j = 0; j < i; j++)
            if (axes[j] == axes[i]) return LXO_ERR_INVALID_ARGUMENT;
        int64_t a = axes[i] < 0 ? axes[i] + rank : axes[i];
        if (a < 0) return LXO_ERR_INVALID_ARGUMENT;
        ax[i] = (int)a;
    }
    for (int i = 0; i < naxes; i++)
        for (int j = 0; j < i; j++)
            if (ax[i] == ax[j]) return LXO_ERR_INVALID_ARGUMENT;
    *nax = naxes;
    return 0;
}

/* permutation for reduction; returns 0 if the axes are already innermost */
static int reduction_perm(int rank, const int *ax, int nax, int *perm)
{
    int inner = 1;
    for (int i = 0; i < nax; i++)
        if (ax[nax - i - 1] != rank - 1 - i) { inner = 0; break; }
    if (inner) return 0;
    int k = 0;
    for (int d = 0; d < rank; d++) {
        int red = 0;
        for (int i = 0; i < nax; i++) if (ax[i] == d) red = 1;
        if (!red) perm[k++] = d;
    }
    for (int i = 0; i < nax; i++) perm[k++] = ax[i];
    return 1;
}

int lxo_reduce(int op, int dtype, int rank, const int64_t *dims, const void *x,
               int naxes, const int64_t *axes, int keepdims,
               void *out, int *rout, int64_t *dout)
{
    int ax[LXO_MAX_RANK], nax, perm[LXO_MAX_RANK];
    int es = lxo_elem_size(dtype);
    if (op == LXO_RMAX && dtype != LXO_FLOAT && dtype != LXO_DOUBLE) return LXO_ERR_NOT_SUPPORTED;
    if (dtype != LXO_FLOAT && dtype != LXO_DOUBLE && dtype != LXO_INT32 && dtype != LXO_INT64)
        return LXO_ERR_NOT_SUPPORTED;
    int st = normalize_axes(rank, naxes, axes, ax, &nax);
    if (st) return st;
    int64_t n = numel(rank, dims);
    int64_t r = 1;
    for (int i = 0; i < nax; i++) r *= dims[ax[i]];
    int64_t nout = r ? n / r : 0;
    if (r == 0) { /* output has the kept dims */
        nout = 1;
        for (int d = 0; d < rank; d++) {
            int red = 0;
            for (int i = 0; i < nax; i++) if (ax[i] == d) red = 1;
            if (!red) nout *= dims[d];
        }
    }
    /* output shape */
    int ro = 0;
    for (int d = 0; d < rank; d++) {
        int red = 0;
        for (int i = 0; i < nax; i++) if (ax[i] == d) red = 1;
        if (!red) dout[ro++] = dims[d];
        else if (keepdims) dout[ro++] = 1;
    }
    *rout = ro;

    /* ReduceMean for int32/int64/double divides every element first */
    const void *src = x;
    void *pre = NULL;
    if (op == LXO_RMEAN && dtype != LXO_FLOAT) {
        pre = malloc(n * es + 1);
        if (!pre) return LXO_ERR_OUT_OF_MEMORY;
        for (int64_t i = 0; i < n; i++) {
            if (dtype == LXO_DOUBLE) ((double *)pre)[i] = ((const double *)x)[i] / (double)r;
            else if (dtype == LXO_INT32) {
                if (r == 0) { free(pre); return LXO_ERR_DIVIDE_BY_ZERO; }
                int32_t v = ((const int32_t *)x)[i], d = (int32_t)r;
                if (v == INT32_MIN && d == -1) { free(pre); return LXO_ERR_OVERFLOW; }
                ((int32_t *)pre)[i] = v / d;
            } else {
                if (r == 0) { free(pre); return LXO_ERR_DIVIDE_BY_ZERO; }
                ((int64_t *)pre)[i] = ((const int64_t *)x)[i] / r;
            }
        }
        src = pre;
    }
    const void *pdata = src;
    void *tr = NULL;
    if (reduction_perm(rank, ax, nax, perm)) {
        tr = malloc(n * es + 1);
        if (!tr) { free(pre); return LXO_ERR_OUT_OF_MEMORY; }
        transpose(es, rank, dims, src, perm, tr);
        pdata = tr;
    }
    for (int64_t i = 0; i < nout; i++) {
        int64_t o = i * r;
        switch (dtype) {
        case LXO_FLOAT: {
            const float *p = (const float *)pdata;
            float acc = 0.0f;
            if (op == LXO_RMAX) { for (int64_t j = 0; j < r; j++) { float v = p[o + j]; if (v > acc) acc = v; } }
            else { for (int64_t j = 0; j < r; j++) acc += p[o + j]; }
            if (op == LXO_RMEAN) acc = acc / (float)r;
            ((float *)out)[i] = acc;
            break;
        }
        case LXO_DOUBLE: {
            const double *p = (const double *)pdata;
            double acc = 0.0;
            if (op == LXO_RMAX) { for (int64_t j = 0; j < r; j++) { double v = p[o + j]; if (v > acc) acc = v; } }
            else { for (int64_t j = 0; j < r; j++) acc += p[o + j]; }
            ((double *)out)[i] = acc;
            break;
        }
        case LXO_INT32: {
            const int32_t *p = (const int32_t *)pdata;
            uint32_t acc = 0;
            for (int64_t j = 0; j < r; j++) acc += (uint32_t)p[o + j];
            ((int32_t *)out)[i] = (int32_t)acc;
            break;
        }
        case LXO_INT64: {
            const int64_t *p = (const int64_t *)pdata;
            uint64_t acc = 0;
            for (int64_t j = 0; j < r; j++) acc += (uint64_t)p[o + j];
            ((int64_t *)out)[i] = (int64_t)acc;
            break;
        }
        }
    }
    free(tr);
    free(pre);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Softmax: Tensor<float>.Softmax (TensorOps.cs:1312-1330):                  */
/*   m = ReduceMax(x, [axis], keepdims)   (seed 0)                           */
/*   e = MathF.Exp(x - broadcast(m))                                         */
/*   s = ReduceSum(e, [axis], keepdims)   (serial float fold along axis)     */
/*   y = e / broadcast(s)                                                    */
/* ------------------------------------------------------------------------ */
int lxo_softmax(int dtype, int rank, const int64_t *dims, const void *x, int axis, void *out)
{
    if (dtype != LXO_FLOAT && dtype != LXO_DOUBLE) return LXO_ERR_NOT_SUPPORTED;
    if (axis < 0) axis += rank;
    if (axis < 0 || axis >= rank) return LXO_ERR_INVALID_ARGUMENT;
    int es = lxo_elem_size(dtype);
    int64_t n = numel(rank, dims);
    int64_t ax = axis, rdims[LXO_MAX_RANK];
    int rr;
    int64_t mcount = dims[axis] ? n / dims[axis] : 0;
    void *m = malloc((mcount + 1) * es), *s = malloc((mcount + 1) * es);
    void *bm = malloc(n * es + 1), *e = malloc(n * es + 1);
    if (!m || !s || !bm || !e) { free(m); free(s); free(bm); free(e); return LXO_ERR_OUT_OF_MEMORY; }
    int st = lxo_reduce(LXO_RMAX, dtype, rank, dims, x, 1, &ax, 1, m, &rr, rdims);
    if (!st) {
        lxo_materialize(es, rr, rdims, m, rank, dims, bm);
        lxo_binary(LXO_SUB, dtype, n, x, bm, e, NULL);
        lxo_unary(LXO_EXP, dtype, n, e, e);
        st = lxo_reduce(LXO_RSUM, dtype, rank, dims, e, 1, &ax, 1, s, &rr, rdims);
    }
    if (!st) {
        lxo_materialize(es, rr, rdims, s, rank, dims, bm);
        lxo_binary(LXO_DIV, dtype, n, e, bm, out, NULL);
    }
    free(m); free(s); free(bm); free(e);
    return st;
}

/* ------------------------------------------------------------------------ */
/* The BERT GELU subgraph node by node without materialising its scalar     */
/* operands (the values are those of CPUExecutionProvider.Div/Erf/Add/Mul   */
/* run in sequence: every node rounds to float32):                          */
/*   a = x / 1.4142135f; e = Erf(a); b = e + 1f; c = x * b; y = c * 0.5f    */
/* ------------------------------------------------------------------------ */
void lxo_gelu_chain(int64_t n, const float *x, float *y)
{
    const float c2 = 1.41421353816986083984375f;
    for (int64_t i = 0; i < n; i++) {
        float a = x[i] / c2;
        float e = lxo_erf_f32(a);
        float b = e + 1.0f;
        float c = x[i] * b;
        y[i] = c * 0.5f;
    }
}

/* ------------------------------------------------------------------------ */
/* MatMul2D inner loop in the reference's order (MathOps.cs:380-419,         */
/* mm_unsafe_vectorized): C starts at zero; for each row i, for each inner j */
/* in order, C[i][k] += A[i][j] * B[j][k] -- the product rounded, then the   */
/* sum rounded (Vector<T> '+' of '*', no FMA).  x is M x N, y is N x K.      */
/* Int32 wraps (unchecked C#).                                               */
/* ------------------------------------------------------------------------ */
int lxo_matmul2d(int dtype, int64_t M, int64_t N, int64_t K, const void *a, const void *b, void *c)
{
    if (dtype == LXO_FLOAT) {
        const float *A = (const float *)a, *B = (const float *)b;
        float *C = (float *)c;
        for (int64_t i = 0; i < M * K; i++) C[i] = 0.0f;
        for (int64_t i = 0; i < M; i++)
            for (int64_t j = 0; j < N; j++) {
                const float av = A[i * N + j];
                for (int64_t k = 0; k < K; k++) {
                    const float p = av * B[j * K + k];
                    C[i * K + k] = C[i * K + k] + p;
                }
            }
        return LXO_OK;
    }
    if (dtype == LXO_DOUBLE) {
        const double *A = (const double *)a, *B = (const double *)b;
        double *C = (double *)c;
        for (int64_t i = 0; i < M * K; i++) C[i] = 0.0;
        for (int64_t i = 0; i < M; i++)
            for (int64_t j = 0; j < N; j++) {
                const double av = A[i * N + j];
                for (int64_t k = 0; k < K; k++) {
                    const double p = av * B[j * K + k];
                    C[i * K + k] = C[i * K + k] + p;
                }
            }
        return LXO_OK;
    }
    if (dtype == LXO_INT32) {
        const int32_t *A = (const int32_t *)a, *B = (const int32_t *)b;
        uint32_t *C = (uint32_t *)c;
        for (int64_t i = 0; i < M * K; i++) C[i] = 0u;
        for (int64_t i = 0; i < M; i++)
            for (int64_t j = 0; j < N; j++) {
                const uint32_t av = (uint32_t)A[i * N + j];
                for (int64_t k = 0; k < K; k++) C[i * K + k] += av * (uint32_t)B[j * K + k];
            }
        return LXO_OK;
    }
    return LXO_ERR_NOT_SUPPORTED;
}
