/*
 * oracle.h -- CPU restatement of AIHost's GGUF block dequantization and
 * weight-matmul semantics.  TEST INFRASTRUCTURE ONLY: this code is the checker
 * for the HIP library (tests/, the smoke check and the CPU-baseline leg of the
 * benchmark).  Nothing in the shipped library links or calls it.
 *
 * What each function restates (paths relative to the reference repository):
 *   orc_f16_refcpu      AIHost/AIHost/Compute/ComputeOps.cs:1497-1522 (F16ToF32,
 *                       including its subnormal-exponent defect)
 *   orc_f16_glsl        AIHost/AIHost/Compute/QuantizationFormats.cs:147-152
 *                       (the GLSL decoder that actually runs; IEEE, NaN -> 0x7FC00000)
 *   orc_get_scale_min_k4  QuantizationFormats.cs:157-165, ComputeOps.cs:1653-1666
 *   Q4_K row dequant    ComputeOps.cs:1629-1678
 *   Q6_K row dequant    ComputeOps.cs:1735-1774
 *   Q8_0 / Q4_0         absent from the reference (ComputeOps.cs:743 throws);
 *                       restated from the GGUF/ggml format definition
 *                       (ggml dequantize_row_q8_0 / dequantize_row_q4_0)
 *   orc_matvec          C[m,n] = sum_k A[m*K+k] * W[k + n*K] with W the dequantized
 *                       GGUF tensor (AIHost/AIHost/Compute/ComputeShaders.cs:93-129),
 *                       accumulated sequentially in k in fp32 as the reference's only
 *                       CPU dot product does (AIHost/AIHost/Compute/TransformerBase.cs:454-456)
 *
 * Parity pins (tests/test_oracle_*.py):
 *   f16 decoders        exhaustive over all 65536 halves vs numpy's IEEE float16
 *   get_scale_min_k4    exhaustive over the bytes each index reads vs a bit-level
 *                       statement of the 6-bit packing
 *   element order       single-bit known-answer blocks vs ggml's loop-structured
 *                       statement of each format (written independently in numpy)
 *   arithmetic          hand-computed known-answer blocks
 *   matvec              basis-vector probes (orientation) and fp64 brute force
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off), output oracle/_build/liboracle.so.
 */
#ifndef AIH_ORACLE_H
#define AIH_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids, as AIHost/AIHost/GGUF/GGUFValueType.cs:26-56 */
enum { ORC_F32 = 0, ORC_Q4_0 = 2, ORC_Q8_0 = 8, ORC_Q4_K = 12, ORC_Q6_K = 14 };
/* fp16 decoding modes */
enum { ORC_F16_IEEE = 0, ORC_F16_REFCPU = 1 };

float   orc_f16_refcpu(uint16_t h);
float   orc_f16_glsl(uint16_t h);
/* out[i] = decode(h[i]) for i < n, written to memory (keeps NaN payloads intact) */
void    orc_f16_decode_array(const uint16_t *h, float *out, int64_t n, int mode);
void    orc_get_scale_min_k4(int j, const uint8_t *scales, uint8_t *sc, uint8_t *mn);

int64_t orc_block_elems(int type);
int64_t orc_block_bytes(int type);
/* bytes of a row of k elements, or -1 if k is not a whole number of blocks */
int64_t orc_row_bytes(int type, int64_t k);

/* Dequantize n elements (a whole number of blocks).  Returns 0 or -1. */
int orc_dequantize(int type, const void *src, float *dst, int64_t n, int f16_mode);

/* Y[b*N + n] = sum_k X[b*ldx + k] * W[n, k], sequential fp32 accumulation in k,
 * rows of W dequantized with f16_mode.  nthreads > 1 splits rows over OpenMP
 * threads (same per-output arithmetic).  Returns 0 or -1. */
int orc_matvec(int type, const void *w, int64_t n_rows, int64_t k,
               const float *x, int64_t ldx, int64_t batch, float *y, int64_t ldy,
               int f16_mode, int nthreads);

/* Same product accumulated in double (for error analysis), output double. */
int orc_matvec_f64(int type, const void *w, int64_t n_rows, int64_t k,
                   const float *x, int64_t ldx, int64_t batch, double *y, int64_t ldy,
                   int f16_mode, int nthreads);

#ifdef __cplusplus
}
#endif
#endif
