/*
 * qik_fp8.h -- C ABI of the W8A8 fp8 linear of a Qwen-Image 2.1 DiT layer
 * (replaces the device work of `FP8Linear.forward`, qwen_image_kernel/fp8.py:78-90):
 *
 *   qik_fp8_quantize  per-tensor fp8e4m3fn quantisation of an activation
 *                     (`quantize_tensorwise`, fp8.py:24-53) or of a weight
 *                     (`quantize_weight_tensorwise`, fp8.py:56-60)
 *   qik_fp8_gemm      out = (A_fp8 . W_fp8^T) * (scale_a * scale_b) + bias
 *                     (the `torch._scaled_mm` call, fp8.py:87-88)
 *   qik_fp8_dequant   bf16(fp32(w_fp8) * scale), the weight of the bf16 path
 *                     that layers with fewer than 256 inputs take (fp8.py:79-84)
 *   qik_fp8_quantize_weight_host
 *                     the weight quantiser for a weight in host memory, run on
 *                     the CPU (`quantize_weight_tensorwise` of a CPU tensor)
 *
 * Same conventions as qik_attn.h: plain C, no allocation, device pointers of
 * the current HIP device, `stream` a hipStream_t as void*, asynchronous and
 * stream-ordered launches, return QIK_OK or a negative qik_status.  fp8 data
 * is OCP e4m3fn (bias 7, max 448, 0x7f / 0xff NaN), one byte per element.
 */
#ifndef QIK_FP8_H
#define QIK_FP8_H

#include <stdint.h>

#include "qik_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Element type of a quantiser input (in addition to QIK_DTYPE_BF16 / _FP16). */
#define QIK_DTYPE_FP32 2

/* How qik_fp8_quantize forms the codes once the scale is known. */
enum qik_fp8_mode {
  QIK_FP8_ACTIVATION = 0,  /* code = e4m3_rne(x * (1 / scale))            (fp8.py:28-40) */
  QIK_FP8_WEIGHT = 1       /* code = e4m3_rne(clamp(x / scale, +-448))    (fp8.py:58-59) */
};

/* Per-tensor quantisation of n contiguous elements:
 *   amax  = max |x|                                      (fp32; NaN if any x is NaN)
 *   scale = max(amax * fp32(1/448), fp32(1e-12))          (NaN stays NaN)
 *   out   = codes by `mode`; *scale_out = scale
 * The scale is what torch computes on a HIP device for
 * (x.abs().amax().float() / 448.0).clamp_min(1e-12): a tensor divided by a
 * Python scalar is multiplied by the scalar's fp32 reciprocal there.  The
 * activation form takes the reciprocal of the scale once (IEEE fp32 division)
 * and multiplies, as the reference's cast kernel does; the weight form divides
 * every element (the correctly rounded quotient of an IEEE division) and
 * clamps, as the reference's weight quantiser does.
 * Both round to nearest even.  Finite inputs give codes bit-identical to those
 * torch ops on the device; a non-finite input makes the scale non-finite and
 * the codes NaN or zero, as in the reference ("non-finite inputs poison the
 * output", fp8.py:33-34).
 * x: 16-byte aligned; out: aligned to the bytes one 16-byte vector of x
 * yields (8 for bf16/fp16, 4 for fp32). */
typedef struct qik_fp8_quant_args {
  int32_t abi_version;        /* QIK_ABI_VERSION                                     */
  int32_t dtype;              /* QIK_DTYPE_BF16, QIK_DTYPE_FP16 or QIK_DTYPE_FP32      */
  int32_t mode;               /* enum qik_fp8_mode                                   */
  int32_t reserved0;          /* must be 0                                           */
  const void* x;              /* [n] input                                           */
  void* out;                  /* [n] fp8e4m3fn codes                                 */
  float* scale;               /* [1] fp32, written                                   */
  int64_t n;                  /* elements, 1 <= n < 2^40                             */
} qik_fp8_quant_args;

/* One launch when x fits the registers of the workgroups the device holds at
 * once (about 109 MB of bf16/fp16 on MI355X, half that of fp32): every
 * workgroup reads its share of x once, the workgroups exchange their maxima
 * through the workspace, and each writes its codes.  Larger inputs take two
 * launches: per-block partial maxima into the workspace, then the codes (x
 * read twice).  The workspace (at least qik_fp8_quant_workspace_size bytes,
 * 4-byte aligned) must be zero-filled before its first use; every call leaves
 * it fit for the next call on the same stream (calls that overlap must not
 * share one).  QIK_ERR_WORKSPACE for a missing, misaligned or short
 * workspace.  If a workgroup of a one-pass launch cannot start within tens of
 * milliseconds (the device fully occupied by other work for that long), the
 * launch writes a NaN scale and NaN codes rather than wait without bound. */
int qik_fp8_quant_workspace_size(const qik_fp8_quant_args* args, int64_t* bytes);
int qik_fp8_quantize(const qik_fp8_quant_args* args, void* workspace, int64_t workspace_bytes, void* stream);

/* out[m, n] = round(fp32(sum_k A[m, k] * W[n, k]) * (scale_a * scale_b) + bias[n])
 * with fp32 accumulation of the exact fp8 products, the two scales multiplied
 * once in fp32, the bias (if any) added in fp32 and one round to nearest even
 * into the output dtype: torch._scaled_mm(A, W.t(), scale_a, scale_b, bias,
 * out_dtype) with tensorwise scales.  Both operands are K-contiguous (row
 * strides lda / ldb in bytes, multiples of 16 and >= K); out is N-contiguous
 * with row stride ldc elements.  K and N multiples of 16 (as the _scaled_mm
 * contract requires), M >= 1.  Pointers 16-byte aligned (bias: 8). */
typedef struct qik_fp8_gemm_args {
  int32_t abi_version;        /* QIK_ABI_VERSION                                     */
  int32_t out_dtype;          /* QIK_DTYPE_BF16 or QIK_DTYPE_FP16 (bias has it too)   */
  int32_t reserved0;          /* must be 0                                           */
  int32_t reserved1;          /* must be 0                                           */
  const void* a;              /* [M, K] fp8e4m3fn activations                        */
  const void* w;              /* [N, K] fp8e4m3fn weight                             */
  const float* scale_a;       /* [1] fp32 device scalar                              */
  const float* scale_w;       /* [1] fp32 device scalar                              */
  const void* bias;           /* [N] in out_dtype, or NULL                           */
  void* out;                  /* [M, N] in out_dtype                                 */
  int64_t M, N, K;
  int64_t lda, ldw;           /* row strides of a and w, bytes                       */
  int64_t ldc;                /* row stride of out, elements                         */
} qik_fp8_gemm_args;

int qik_fp8_gemm_validate(const qik_fp8_gemm_args* args);
int qik_fp8_gemm(const qik_fp8_gemm_args* args, void* stream);

/* The same product with a workspace (no counterpart in the reference, whose
 * torch._scaled_mm call, fp8.py:87-88, gets its scratch from hipBLASLt): a
 * launch with few output tiles and a long K (the text stream's 256-token MLP
 * out, 256 x 3072 x 12288) splits K into up to 8 slices whose fp32 sums go
 * into the workspace and are added in slice order by a second launch.  The
 * sums then round differently from the one-pass product (within an fp32
 * accumulation bound; the output differs in the last bit on a small share of
 * elements).  qik_fp8_gemm_workspace_size gives the bytes the call needs: 0
 * when it does not split, and then qik_fp8_gemm_ws is qik_fp8_gemm (the
 * workspace may be NULL).  Otherwise the workspace must be 16-byte aligned and
 * at least that size (QIK_ERR_WORKSPACE); its contents are irrelevant. */
int qik_fp8_gemm_workspace_size(const qik_fp8_gemm_args* args, int64_t* bytes);
int qik_fp8_gemm_ws(const qik_fp8_gemm_args* args, void* workspace, int64_t workspace_bytes, void* stream);

/* The launch qik_fp8_gemm_ws makes for an M x N x K product on a device with
 * `cus` compute units (0: 256), host only, no device involved (no counterpart
 * in the reference; for tests and tooling, as qik_attn_work_map is for the
 * attention launch).  plan[0..5] = big tile rows, big tile columns, small
 * tile rows, small tile columns, 1 when the small tiles' workgroups come
 * first in blockIdx order, the number of K slices (1: no split); *n1 = the
 * output columns [0, n1) the big tiles cover (N for a K split, which runs
 * 128 x 128 tiles only).  QIK_ERR_SHAPE for a shape qik_fp8_gemm_validate
 * refuses (with its strides equal to K, K and N). */
int qik_fp8_gemm_plan(int64_t M, int64_t N, int64_t K, int32_t cus, int32_t* plan, int64_t* n1);

/* out[i] = round(fp32(code[i]) * scale[0]) into out_dtype, for i < n: the
 * dequantised weight of the bf16 path (fp8.py:81: fp8 -> bf16 -> fp32 is
 * exact, one fp32 multiply).  out_dtype QIK_DTYPE_BF16 or QIK_DTYPE_FP16
 * rounds once to nearest even; QIK_DTYPE_FP32 writes the fp32 product itself
 * (the weight an fp32 activation multiplies, fp8.py:81-82).  w 8-byte
 * aligned, out 16. */
int qik_fp8_dequant(const void* w, const float* scale, void* out, int64_t n, int32_t out_dtype, void* stream);

/* Weight quantisation of a weight in HOST memory, on the CPU (no device
 * involved): replaces `quantize_weight_tensorwise` (fp8.py:56-60) when the
 * weight is a CPU tensor, as in the offline conversion on a machine without
 * a GPU (quantize_offline.py:15-25).  Bit-identical to those torch ops run on
 * the CPU, where both divisions are IEEE fp32 divisions:
 *   scale = max(amax / 448, 1e-12)                    (NaN stays NaN)
 *   out   = e4m3fn_rne(clamp(fp32(w) / scale, +-448))
 * (qik_fp8_quantize's QIK_FP8_WEIGHT mode gives what the same ops give on a
 * HIP device, where torch multiplies the amax by the reciprocal of 448.)
 * w: n host elements of `dtype` (QIK_DTYPE_BF16, _FP16 or _FP32); out: n host
 * bytes; *scale written.  `threads` host threads at most (< 1 means 1); the
 * bytes do not depend on it.  Blocking; 1 <= n < 2^40. */
int qik_fp8_quantize_weight_host(const void* w, int32_t dtype, int64_t n, void* out, float* scale,
                                 int32_t threads);

#ifdef __cplusplus
}
#endif

#endif /* QIK_FP8_H */
