/*
 * qik_ops.h -- C ABI of the two device steps on either side of the attention
 * call in a Qwen-Image 2.1 attention layer:
 *
 *   qik_rms_rope    per-head RMSNorm + rotary embedding producing Q and K
 *                   (replaces `fused_rms_norm_rope`, qwen_image_kernel/triton_fused.py:75-105)
 *   qik_slab_store  writes one layer's prefix K/V into the contiguous slab,
 *                   quantising V to fp8e4m3fn per (b, h)
 *                   (replaces `_LayerView.store`, qwen_image_kernel/kv_cache.py:30-45);
 *                   qik_slab_store_ws is the same store in fewer launches with a
 *                   small caller workspace
 *
 * Same conventions as qik_attn.h: plain C, no allocation, device pointers of
 * the current HIP device, `stream` a hipStream_t as void*, asynchronous and
 * stream-ordered launches, return QIK_OK or a negative qik_status.  Strides
 * are in ELEMENTS; the innermost (D) stride is 1.
 */
#ifndef QIK_OPS_H
#define QIK_OPS_H

#include <stdint.h>

#include "qik_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* out[b, s, h, :] = rope(bf16(rmsnorm(x[b, s, h, :]) * weight), s).
 * Per row: ms = sum(x^2) / D, r = 1 / sqrt(ms + eps), n = bf16((x * r) * w)
 * (fp32 math, one bf16 rounding, triton_fused.py:51-58), then each pair
 * (n[2i], n[2i+1]) is rotated by (cos[s, i], sin[s, i]) in fp32 and rounded to
 * the output dtype (:60-69).  x may be a strided view (e.g. the q or k slice of
 * a fused QKV output); out may be the same memory as x only if identical. */
typedef struct qik_rms_rope_args {
  int32_t abi_version;        /* QIK_ABI_VERSION                                     */
  int32_t dtype;              /* enum qik_dtype of x and out                         */
  const void* x;              /* [B, S, H, D]                                        */
  void* out;                  /* [B, S, H, D]                                        */
  const float* weight;        /* [D] fp32 RMSNorm weight                             */
  const float* cos;           /* [S, D/2] fp32, contiguous                           */
  const float* sin;           /* [S, D/2] fp32, contiguous                           */
  int64_t B, S, H, D;         /* D in {32, 64, 128, 256}                             */
  int64_t stride_x[3];        /* b, s, h                                             */
  int64_t stride_out[3];      /* b, s, h                                             */
  float eps;
  int32_t reserved0;          /* must be 0                                           */
} qik_rms_rope_args;

int qik_rms_rope(const qik_rms_rope_args* args, void* stream);

/* One layer's prefix K/V into the slab (layout [B, H, P_max, D] per layer):
 *   k_dst[b, h, p, :] = k[b, p, h, :]
 *   bf16/fp16 V:  v_dst[b, h, p, :] = v[b, p, h, :]
 *   fp8 V (v_fp8 != 0; v bf16 or fp16), per (b, h) over all p < P and d:
 *     amax  = max |fp32(v)|
 *     scale = max(amax * fp32(1/448), fp32(1e-12))
 *     v_dst = e4m3fn_rne(clamp(v / scale, -448, 448))   (IEEE fp32 division)
 *     v_scale[b*H + h] = scale
 *   This is what `store` computes with torch on a HIP device (kv_cache.py:36-42:
 *   torch divides a tensor by the Python scalar 448 as a multiply by the
 *   fp32 reciprocal, and the tensor/tensor division correctly rounded). */
typedef struct qik_slab_store_args {
  int32_t abi_version;        /* QIK_ABI_VERSION                                     */
  int32_t dtype;              /* enum qik_dtype of k, v and k_dst (and v_dst unless fp8) */
  int32_t v_fp8;              /* nonzero: v_dst is fp8e4m3fn and v_scale is written  */
  int32_t reserved0;          /* must be 0                                           */
  const void* k;              /* [B, P, H, D]                                        */
  const void* v;              /* [B, P, H, D]                                        */
  void* k_dst;                /* slab K of the layer                                 */
  void* v_dst;                /* slab V of the layer                                 */
  float* v_scale;             /* [B*H] fp32 (v_fp8 only, else NULL)                  */
  int64_t B, P, H, D;         /* D in {32, 64, 128, 256}                             */
  int64_t stride_k[3];        /* b, p, h of k                                        */
  int64_t stride_v[3];        /* b, p, h of v                                        */
  int64_t stride_k_dst[3];    /* b, h, p of k_dst                                    */
  int64_t stride_v_dst[3];    /* b, h, p of v_dst                                    */
  int64_t* length_dst;        /* optional: the store's first launch also writes P
                                 here (the layer's entry of a device length table,
                                 kv_cache.py:45 sets it after the store); NULL: not
                                 written.  Nothing is launched, and nothing written,
                                 when B*H*P is 0.                                   */
} qik_slab_store_args;

int qik_slab_store(const qik_slab_store_args* args, void* stream);

/* The same store in two launches instead of three, for an fp8 V: the K copy and
 * the scales of the V rows' chunks in one launch, the codes in the second
 * (replaces the body of _LayerView.store, kv_cache.py:30-45, like
 * qik_slab_store; the results are bit-identical to it).  The chunks' scales
 * go to the caller's workspace, at least qik_slab_store_workspace_size bytes,
 * 4-byte aligned, contents irrelevant (every launch writes what it reads), so
 * one workspace serves every later call on its stream.  Without an fp8 V it is
 * qik_slab_store and the workspace may be NULL.  QIK_ERR_WORKSPACE for a
 * missing, misaligned or short one. */
int qik_slab_store_workspace_size(const qik_slab_store_args* args, int64_t* bytes);
int qik_slab_store_ws(const qik_slab_store_args* args, void* workspace, int64_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* QIK_OPS_H */
