/* kansai_oracle.h -- CPU restatement of the reference's int8 path.
 * TEST INFRASTRUCTURE ONLY: the checker, never the thing measured or
 * shipped.  See kansai_oracle.c for the reference citations. */
#ifndef KANSAI_ORACLE_H
#define KANSAI_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KO_OK 0
#define KO_NONFINITE 4

int ko_quantize_tensor(const float* x, int64_t n, int8_t* q, double* scale);
int ko_quantize_rows(const float* x, int64_t rows, int64_t cols, int8_t* q, double* scales);
int ko_quantize_cols_packed(const float* w, int64_t k, int64_t n, int8_t* q_packed, double* scales);
int ko_quantize_tensor_packed(const float* w, int64_t k, int64_t n, int8_t* q_packed, double* scale);
void ko_dequantize_tensor(const int8_t* q, int64_t n, double scale, float* out);
void ko_dequantize_rows(const int8_t* q, int64_t rows, int64_t cols, const double* scales, float* out);
void ko_gemm_i8(const int8_t* a, const int8_t* bt, int64_t M, int64_t N, int64_t K, int32_t* acc);
void ko_epilogue(const int32_t* acc, int64_t M, int64_t N, const double* sa, int64_t sa_n,
                 const double* sb, int64_t sb_n, const float* bias, float* out);
void ko_matmul_f32(const float* a, const float* b, float* out, int64_t M, int64_t K, int64_t N);
void ko_add_bias(const float* x, const float* bias, float* out, int64_t batch, int64_t features);

#ifdef __cplusplus
}
#endif
#endif
