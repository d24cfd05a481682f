// W8A8 fp8 linear of a Qwen-Image 2.1 DiT layer on MI355X (gfx950, CDNA4):
// per-tensor quantisation of the activation (qwen_image_kernel/fp8.py:24-53)
// and of a weight (fp8.py:56-60), the fp8 GEMM with tensorwise scales that
// replaces torch._scaled_mm (fp8.py:87-88), and the weight dequantisation of
// the bf16 path for layers with fewer than 256 inputs (fp8.py:79-84).
//
// The quantiser is an HBM-bound byte mover: when the tensor fits the
// registers of the resident workgroups, one launch in which every workgroup
// holds its share, publishes its max |x| and reads everyone else's before it
// writes its codes; otherwise two passes (max |x| per block into a small
// workspace, then every block re-reduces those maxima, forms the scale and
// writes the codes).  Contraction is off in it, so every fp32 multiply and
// division rounds on its own, as torch's elementwise ops do.  Weights in host
// memory are quantised on the host with torch's CPU rounding.
//
// The GEMM runs on the gfx950 fp8 matrix cores: v_mfma_f32_32x32x64_f8f6f4
// (e4m3 x e4m3, fp32 accumulate; 32x32 outputs x 64 k per instruction, twice
// the k of the CDNA3 fp8 MFMA).  One workgroup of 4 or 8 waves computes a
// BM x BN tile of out^T = W . A^T (MFMA A operand = weight rows n, B operand
// = activation rows m), so each lane ends with 4 consecutive n of one row m
// per register quad.  Tiles of A and W reach LDS directly
// (buffer_load_dwordx4 ... lds, no register staging), 64 or 128 k-bytes per
// stage, ahead of their use, with a 16-byte chunk swizzle that makes the
// fragment reads conflict-free; each wave reads the next fragments while its
// MFMAs run on the current ones, and the copies are issued between the MFMAs.
// The outputs go out through LDS as whole rows.  Workgroups map to tiles XCD
// by XCD (the dispatcher deals workgroup b to XCD b % 8), so one XCD's L2
// serves a compact block of tiles.

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>
#include <limits.h>
#include <algorithm>
#include <cmath>
#include <thread>
#include <type_traits>
#include <utility>
#include <vector>

#include "qik_fp8.h"

namespace qik_fp8 {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((__vector_size__(2 * sizeof(__bf16))));
typedef _Float16 f16x2 __attribute__((__vector_size__(2 * sizeof(_Float16))));

inline bool aligned_to(const void* ptr, uintptr_t a) { return (reinterpret_cast<uintptr_t>(ptr) % a) == 0; }

// CUs of the current device (0 if the runtime cannot say), cached per device
int device_cus() {
  static int cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (dev >= 0 && dev < 64) {
    const int c = __atomic_load_n(&cache[dev], __ATOMIC_RELAXED);
    if (c > 0) return c;
  }
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  if (dev >= 0 && dev < 64) __atomic_store_n(&cache[dev], cus, __ATOMIC_RELAXED);
  return cus;
}

// ---------------------------------------------------------------------------
// Quantiser
// ---------------------------------------------------------------------------

constexpr int QT = 256;          // threads per block
constexpr int QU = 4;            // 16-byte vectors per thread in flight
constexpr int MAX_PARTS = 1024;  // blocks of the maximum pass = workspace words

// Workspace of the quantiser (32-bit words): QCTL words of control (word 0:
// the generation of the next one-pass launch), RES_SLOTS 64-bit slots (the
// maximum each workgroup of a one-pass launch publishes, tagged with the
// launch's generation + 1), then MAX_PARTS partial maxima of the two-pass
// form.  Zero-filled once; no launch needs it cleared again.
constexpr int QCTL = 64;
constexpr int RES_SLOTS = 1024;  // most workgroups of a one-pass launch
constexpr int QWS_WORDS = QCTL + 2 * RES_SLOTS + MAX_PARTS;

struct QuantParams {
  const char* x;
  unsigned char* out;
  float* scale;
  unsigned* part;  // [nparts] max |x| of each block's share, as fp32 bit patterns
  unsigned* ctl;   // one-pass launch: control words and slots (zero between launches)
  int64_t n;       // elements
  int64_t nvec;    // whole 16-byte vectors of x
  int nparts;
  int spin;        // one-pass launch: polls of a slot before the launch gives up (scale NaN)
};

template <int DT>
struct Elem;
template <>
struct Elem<QIK_DTYPE_BF16> {
  static constexpr int PER_VEC = 8;
  __device__ static float get(const char* x, int64_t i) {
    return __uint_as_float((unsigned)reinterpret_cast<const unsigned short*>(x)[i] << 16);
  }
  __device__ static void unpack(const u32x4 v, float (&f)[8]) {
    const unsigned w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = __uint_as_float(w[i] << 16);
      f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
};
template <>
struct Elem<QIK_DTYPE_FP16> {
  static constexpr int PER_VEC = 8;
  __device__ static float get(const char* x, int64_t i) { return (float)reinterpret_cast<const _Float16*>(x)[i]; }
  __device__ static void unpack(const u32x4 v, float (&f)[8]) {
    const unsigned w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f16x2 h = __builtin_bit_cast(f16x2, w[i]);
      f[2 * i] = (float)h[0];
      f[2 * i + 1] = (float)h[1];
    }
  }
};
template <>
struct Elem<QIK_DTYPE_FP32> {
  static constexpr int PER_VEC = 4;
  __device__ static float get(const char* x, int64_t i) { return reinterpret_cast<const float*>(x)[i]; }
  __device__ static void unpack(const u32x4 v, float (&f)[4]) {
    f[0] = __uint_as_float(v.x);
    f[1] = __uint_as_float(v.y);
    f[2] = __uint_as_float(v.z);
    f[3] = __uint_as_float(v.w);
  }
};

// |x| as an fp32 bit pattern: unsigned order = |x| order, with every NaN above
// +inf, so an integer max propagates NaN like torch's amax does
__device__ __forceinline__ unsigned abs_bits(float f) { return __float_as_uint(f) & 0x7fffffffu; }

// max over the block of v (valid in thread 0)
__device__ __forceinline__ unsigned block_max(unsigned v) {
  __shared__ unsigned red[QT / 64];
#pragma unroll
  for (int k = 32; k >= 1; k >>= 1) v = max(v, (unsigned)__shfl_xor((int)v, k));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  if (threadIdx.x == 0) {
#pragma unroll
    for (int i = 1; i < QT / 64; ++i) v = max(v, red[i]);
  }
  return v;
}

// Block b: max |x| over vectors [b*nvec/nparts, (b+1)*nvec/nparts); the last
// block also covers the elements past the last whole vector.
template <int DT>
__global__ void __launch_bounds__(QT) amax_kernel(const QuantParams p) {
  using E = Elem<DT>;
  const int64_t v0 = p.nvec * blockIdx.x / p.nparts;
  const int64_t v1 = p.nvec * (blockIdx.x + 1) / p.nparts;
  const u32x4* src = reinterpret_cast<const u32x4*>(p.x);
  unsigned m = 0;
  for (int64_t v = v0 + threadIdx.x; v < v1; v += QT * QU) {
    u32x4 raw[QU];
#pragma unroll
    for (int u = 0; u < QU; ++u) raw[u] = (v + u * QT < v1) ? src[v + u * QT] : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int u = 0; u < QU; ++u) {
      float f[E::PER_VEC];
      E::unpack(raw[u], f);
#pragma unroll
      for (int i = 0; i < E::PER_VEC; ++i) m = max(m, abs_bits(f[i]));
    }
  }
  if (blockIdx.x == gridDim.x - 1) {
    for (int64_t i = p.nvec * E::PER_VEC + threadIdx.x; i < p.n; i += QT) m = max(m, abs_bits(E::get(p.x, i)));
  }
  m = block_max(m);
  if (threadIdx.x == 0) p.part[blockIdx.x] = m;
}

// amax -> scale = max(amax * fp32(1/448), 1e-12) (NaN stays NaN: fmaxf would drop it)
__device__ __forceinline__ float scale_of(unsigned amax_bits) {
#pragma clang fp contract(off)
  const float amax = __uint_as_float(amax_bits);
  if (amax != amax) return amax;
  return fmaxf(amax * (1.0f / 448.0f), 1e-12f);
}

// two fp32 values -> two e4m3fn codes (round to nearest even), as 16 bits
__device__ __forceinline__ unsigned cvt2(float a, float b) {
  return (unsigned)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false) & 0xffffu;
}

// Weights: x / scale rounded to nearest as an IEEE division gives it, from
// inv = RN(1/scale): q = RN(x*inv) is within an ulp of x/scale, r = x -
// q*scale is exact (fma), and RN(q + r*inv) is the correctly rounded quotient
// (Markstein's theorem; no overflow or underflow on the way, since |x| never
// exceeds the amax that set the scale, so |x/scale| <= 448 (1 + 2^-22), and a
// subnormal quotient gives a zero code either way).  The quotient takes x's
// sign, so -0 stays -0.  A non-finite scale (an inf or NaN in the tensor) has
// no exact remainder: the division is kept there (`exact` false).
template <int MODE>
__device__ __forceinline__ float quant_value(float x, float scale, float inv, bool exact) {
#pragma clang fp contract(off)
  if constexpr (MODE == QIK_FP8_ACTIVATION) {
    return x * inv;
  } else {
    float q;
    if (exact) {
      const float q0 = x * inv;
      const float r = __builtin_fmaf(-q0, scale, x);
      q = __builtin_copysignf(__builtin_fmaf(r, inv, q0), x);
    } else {
      q = x / scale;
    }
    return fminf(fmaxf(q, -448.0f), 448.0f);
  }
}

// Every block reduces the partial maxima to the scale (block 0 stores it),
// then writes the codes of vectors [blockIdx*QT*QU, (blockIdx+1)*QT*QU); the
// last block also codes the elements past the last whole vector.
template <int DT, int MODE>
__global__ void __launch_bounds__(QT) cast_kernel(const QuantParams p) {
#pragma clang fp contract(off)
  using E = Elem<DT>;
  constexpr int PV = E::PER_VEC;
  const int64_t vbase = (int64_t)blockIdx.x * QT * QU + threadIdx.x;
  const u32x4* src = reinterpret_cast<const u32x4*>(p.x);
  u32x4 raw[QU];
#pragma unroll
  for (int u = 0; u < QU; ++u) raw[u] = (vbase + u * QT < p.nvec) ? src[vbase + u * QT] : u32x4{0u, 0u, 0u, 0u};

  unsigned m = 0;
  for (int i = threadIdx.x; i < p.nparts; i += QT) m = max(m, p.part[i]);
  m = block_max(m);
  __shared__ float sh_scale;
  if (threadIdx.x == 0) {
    sh_scale = scale_of(m);
    if (blockIdx.x == 0) p.scale[0] = sh_scale;
  }
  __syncthreads();
  const float scale = sh_scale;
  const float inv = 1.0f / scale;  // IEEE division (the reference's cast kernel: 1.0 / scale)
  const bool ex = __builtin_isfinite(scale);

#pragma unroll
  for (int u = 0; u < QU; ++u) {
    const int64_t v = vbase + u * QT;
    if (v >= p.nvec) continue;
    float f[PV];
    E::unpack(raw[u], f);
    if constexpr (PV == 8) {
      u32x2 o;
      o.x = cvt2(quant_value<MODE>(f[0], scale, inv, ex), quant_value<MODE>(f[1], scale, inv, ex)) |
            (cvt2(quant_value<MODE>(f[2], scale, inv, ex), quant_value<MODE>(f[3], scale, inv, ex)) << 16);
      o.y = cvt2(quant_value<MODE>(f[4], scale, inv, ex), quant_value<MODE>(f[5], scale, inv, ex)) |
            (cvt2(quant_value<MODE>(f[6], scale, inv, ex), quant_value<MODE>(f[7], scale, inv, ex)) << 16);
      reinterpret_cast<u32x2*>(p.out)[v] = o;
    } else {
      reinterpret_cast<unsigned*>(p.out)[v] =
          cvt2(quant_value<MODE>(f[0], scale, inv, ex), quant_value<MODE>(f[1], scale, inv, ex)) |
          (cvt2(quant_value<MODE>(f[2], scale, inv, ex), quant_value<MODE>(f[3], scale, inv, ex)) << 16);
    }
  }
  if (blockIdx.x == gridDim.x - 1) {
    for (int64_t i = p.nvec * PV + threadIdx.x; i < p.n; i += QT)
      p.out[i] = (unsigned char)cvt2(quant_value<MODE>(E::get(p.x, i), scale, inv, ex), 0.0f);
  }
}

// ---------------------------------------------------------------------------
// One-pass quantiser
// ---------------------------------------------------------------------------
//
// x is read from HBM once.  Every workgroup of the launch is resident at once
// (the host sizes the grid to the device's occupancy) and keeps its share of x
// in registers, VPT 16-byte vectors per thread.  Each workgroup publishes its
// maximum in a 64-bit slot of its own, tagged with the launch's generation + 1
// (written through to device scope), then reads every slot until all carry
// that tag: no workgroup waits on a shared counter and no atomic is needed.
// Each then forms the scale and writes its codes from the registers.
// Workgroup 0, once it has seen every slot (so every workgroup has read the
// generation), advances the generation for the next launch; stale slots of
// earlier launches carry other tags, so nothing is ever cleared.  A slot that
// stays untagged for `spin` polls (a workgroup that never became resident)
// makes the launch write a NaN scale and NaN codes, never plausible numbers.

__device__ __forceinline__ void store_dev(unsigned* p, unsigned v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned load_dev(unsigned* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_dev64(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t load_dev64(uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int DT, int MODE, int VPT>
__global__ void __launch_bounds__(QT, 2) quant_onepass_kernel(const QuantParams p) {
#pragma clang fp contract(off)
  using E = Elem<DT>;
  constexpr int PV = E::PER_VEC;
  // buffer accesses: one 32-bit lane offset plus a constant per vector, and
  // vectors past the end read as zero / are not written (x of a one-pass
  // launch is far below 4 GiB)
  const uint32_t v0 = blockIdx.x * (uint32_t)(QT * VPT) + threadIdx.x;
  const __amdgpu_buffer_rsrc_t xs = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(p.x), (short)0,
                                                                      (int)(p.nvec * 16), 0x00020000);
  const __amdgpu_buffer_rsrc_t os = __builtin_amdgcn_make_buffer_rsrc(p.out, (short)0, (int)(p.nvec * PV),
                                                                      0x00020000);
  u32x4 raw[VPT];
#pragma unroll
  for (int u = 0; u < VPT; ++u)
    raw[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xs, v0 * 16u, u * QT * 16, 0));
  unsigned m = 0;
#pragma unroll
  for (int u = 0; u < VPT; ++u) {
    float f[PV];
    E::unpack(raw[u], f);
#pragma unroll
    for (int i = 0; i < PV; ++i) m = max(m, abs_bits(f[i]));
  }
  // hold x packed across the exchange: without the empty asm the compiler
  // keeps the unpacked fp32 values of the maximum pass for the codes, twice
  // the registers
#pragma unroll
  for (int u = 0; u < VPT; ++u) asm volatile("" : "+v"(raw[u]));
  const bool last_wg = blockIdx.x == gridDim.x - 1;
  if (last_wg) {
    for (int64_t i = p.nvec * PV + threadIdx.x; i < p.n; i += QT) m = max(m, abs_bits(E::get(p.x, i)));
  }
  __shared__ unsigned sh_gen;
  if (threadIdx.x == 0) sh_gen = load_dev(p.ctl);
  m = block_max(m);  // its barrier also publishes sh_gen
  const uint64_t tag = (uint64_t)(sh_gen + 1u) << 32;
  uint64_t* const slots = reinterpret_cast<uint64_t*>(p.ctl + QCTL);
  if (threadIdx.x == 0) store_dev64(slots + blockIdx.x, tag | m);
  __syncthreads();  // thread 0 has read block_max's words before they are reused

  unsigned mm = 0;
  int missing = 0;
  for (int s = threadIdx.x; s < (int)gridDim.x; s += QT) {
    uint64_t w = load_dev64(slots + s);
    for (int i = 0; i < p.spin && (w & 0xffffffff00000000ull) != tag; ++i) {
      __builtin_amdgcn_s_sleep(1);
      w = load_dev64(slots + s);
    }
    missing |= (w & 0xffffffff00000000ull) == tag ? 0 : 1;
    mm = max(mm, (unsigned)w);
  }
  const int bad = __syncthreads_or(missing);
  mm = block_max(mm);
  __shared__ float sh_scale;
  if (threadIdx.x == 0) {
    const float sc = bad ? __builtin_nanf("") : scale_of(mm);
    sh_scale = sc;
    if (blockIdx.x == 0) {
      p.scale[0] = sc;
      // every workgroup has published, hence read the generation
      store_dev(p.ctl, sh_gen + 1u);
    }
  }
  __syncthreads();
  const float scale = sh_scale;
  const float inv = 1.0f / scale;  // IEEE division (the reference's cast kernel: 1.0 / scale)
  const bool ex = __builtin_isfinite(scale);
#pragma unroll
  for (int u = 0; u < VPT; ++u) {
    float f[PV];
    E::unpack(raw[u], f);
    if constexpr (PV == 8) {
      u32x2 o;
      o.x = cvt2(quant_value<MODE>(f[0], scale, inv, ex), quant_value<MODE>(f[1], scale, inv, ex)) |
            (cvt2(quant_value<MODE>(f[2], scale, inv, ex), quant_value<MODE>(f[3], scale, inv, ex)) << 16);
      o.y = cvt2(quant_value<MODE>(f[4], scale, inv, ex), quant_value<MODE>(f[5], scale, inv, ex)) |
            (cvt2(quant_value<MODE>(f[6], scale, inv, ex), quant_value<MODE>(f[7], scale, inv, ex)) << 16);
      __builtin_amdgcn_raw_buffer_store_b64(o, os, v0 * 8u, u * QT * 8, 0);
    } else {
      __builtin_amdgcn_raw_buffer_store_b32(
          cvt2(quant_value<MODE>(f[0], scale, inv, ex), quant_value<MODE>(f[1], scale, inv, ex)) |
              (cvt2(quant_value<MODE>(f[2], scale, inv, ex), quant_value<MODE>(f[3], scale, inv, ex)) << 16),
          os, v0 * 4u, u * QT * 4, 0);
    }
  }
  if (last_wg) {
    for (int64_t i = p.nvec * PV + threadIdx.x; i < p.n; i += QT)
      p.out[i] = (unsigned char)cvt2(quant_value<MODE>(E::get(p.x, i), scale, inv, ex), 0.0f);
  }
}

// ---------------------------------------------------------------------------
// Dequantiser (the bf16 path's weight)
// ---------------------------------------------------------------------------

template <bool FP16>
__device__ __forceinline__ unsigned pack2(float a, float b) {  // round to nearest even
  if constexpr (FP16) {
    const f16x2 h = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(unsigned, h);
  } else {
    const bf16x2 h = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(unsigned, h);
  }
}

template <bool FP16>
__device__ __forceinline__ void unpack2(unsigned w, float& a, float& b) {
  if constexpr (FP16) {
    const f16x2 h = __builtin_bit_cast(f16x2, w);
    a = (float)h[0];
    b = (float)h[1];
  } else {
    a = __uint_as_float(w << 16);
    b = __uint_as_float(w & 0xffff0000u);
  }
}

// fp32 value of an e4m3fn code pair (bytes 2*hi, 2*hi+1 of w): exact
template <bool HI>
__device__ __forceinline__ f32x2 decode2(unsigned w) {
  return __builtin_amdgcn_cvt_pk_f32_fp8((int)w, HI);
}

// round(fp32(code) * s) in the output type (OUT: QIK_DTYPE_BF16, _FP16 or
// _FP32, the last with no rounding: the exact fp32 product)
template <int OUT>
__device__ __forceinline__ void dequant_store(f32x2 f, float s, char* out, int64_t pair) {
#pragma clang fp contract(off)
  f[0] *= s;
  f[1] *= s;
  // the empty asm keeps the fp32 product from being folded into a
  // mixed-precision fma that rounds once
  asm volatile("" : "+v"(f));
  if constexpr (OUT == QIK_DTYPE_FP32) {
    reinterpret_cast<f32x2*>(out)[pair] = f;
  } else {
    reinterpret_cast<unsigned*>(out)[pair] = pack2<OUT == QIK_DTYPE_FP16>(f[0], f[1]);
  }
}

template <int OUT>
__global__ void __launch_bounds__(QT) dequant_kernel(const unsigned char* w, const float* scale, char* out,
                                                      int64_t n) {
  const float s = scale[0];
  const int64_t v = (int64_t)blockIdx.x * QT + threadIdx.x;  // 8 codes per thread
  const int64_t nvec = n / 8;
  if (v < nvec) {
    const u32x2 c = reinterpret_cast<const u32x2*>(w)[v];
    dequant_store<OUT>(decode2<false>(c.x), s, out, 4 * v + 0);
    dequant_store<OUT>(decode2<true>(c.x), s, out, 4 * v + 1);
    dequant_store<OUT>(decode2<false>(c.y), s, out, 4 * v + 2);
    dequant_store<OUT>(decode2<true>(c.y), s, out, 4 * v + 3);
  }
  if (v == 0) {
    for (int64_t i = nvec * 8; i < n; ++i) {
#pragma clang fp contract(off)
      f32x2 f = decode2<false>((unsigned)w[i]);
      f[0] *= s;
      asm volatile("" : "+v"(f));
      if constexpr (OUT == QIK_DTYPE_FP32) {
        reinterpret_cast<float*>(out)[i] = f[0];
      } else {
        const unsigned h = pack2<OUT == QIK_DTYPE_FP16>(f[0], 0.0f);
        reinterpret_cast<unsigned short*>(out)[i] = (unsigned short)(h & 0xffffu);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// GEMM
// ---------------------------------------------------------------------------

constexpr int KB = 64;   // k bytes per stage (one MFMA k-step)

// A range of output columns computed with one tile shape.
struct GemmRegion {
  const unsigned char* w;  // weight row of the region's first column
  const char* bias;        // its first bias element, or null
  char* out;               // its first output column
  int N;                   // columns in the region
  int ntm, ntn;            // tiles along m and n
  int group_m;             // tile rows per group of the tile order
  int wgs;                 // workgroups: tiles rounded up to a multiple of 8
};

struct GemmParams {
  const unsigned char* a;
  const float* sa;
  const float* sw;
  int M, K;
  int lda, ldw;   // bytes
  int64_t ldc;    // elements
  GemmRegion r[2];  // columns [0, n1) with the larger tile, then [n1, N)
  int small_first;  // 1: region 1's workgroups come first in blockIdx order
  int ksplit;       // split launches: k-slices per tile (region 0 only)
  float* partial;   // split launches: [ksplit][M][N] fp32 sums of each slice
};

template <int BM_, int BN_, int NS_, int WGM_ = 2, int WGN_ = 2>
struct Cfg {
  static constexpr int KB = qik_fp8::KB;
  static constexpr int BM = BM_, BN = BN_, NS = NS_;
  static constexpr int WGM = WGM_, WGN = WGN_;     // waves along m and n
  static constexpr int NW = WGM * WGN, NT = 64 * NW;
  static constexpr int WM = BM / WGM, WN = BN / WGN;  // wave tile
  static constexpr int MI = WM / 32, NJ = WN / 32;
  static constexpr int A_BYTES = BM * KB;          // A tile of one stage
  static constexpr int STAGE = (BM + BN) * KB;
  static constexpr int AI = BM / (16 * NW);        // 1 KiB copies of A per wave per stage
  static constexpr int WI = BN / (16 * NW);
  static constexpr int COPIES = AI + WI;
  static_assert(NW == 4 || NW == 8, "one or two waves per SIMD");
  static_assert(AI * 16 * NW == BM && WI * 16 * NW == BN, "whole copies per wave");
  static_assert(MI * 32 == WM && NJ * 32 == WN, "whole MFMA blocks per wave");
  static_assert(NS >= 3, "copies run at least two stages ahead");
};

// Tiles with 128 k-bytes per stage: two MFMA k-steps per barrier, and each
// copied row a whole 128-byte line (at 64 bytes a row is half a line, fetched
// by two stages).  Two stages: a stage's copies go out one step (two MFMA
// k-steps) before its first fragment reads.
template <int BM_, int BN_, int WGM_ = 2, int WGN_ = 4>
struct CfgK128 {
  static constexpr int KB = 128, NS = 2;
  static constexpr int BM = BM_, BN = BN_;
  static constexpr int WGM = WGM_, WGN = WGN_;
  static constexpr int NW = WGM * WGN, NT = 64 * NW;
  static constexpr int WM = BM / WGM, WN = BN / WGN;
  static constexpr int MI = WM / 32, NJ = WN / 32;
  static constexpr int A_BYTES = BM * KB;
  static constexpr int STAGE = (BM + BN) * KB;
  static constexpr int AI = BM / (8 * NW);  // 1 KiB copies (8 rows) of A per wave per stage
  static constexpr int WI = BN / (8 * NW);
  static constexpr int COPIES = AI + WI;
  static_assert(NW == 4 || NW == 8, "one or two waves per SIMD");
  static_assert(AI * 8 * NW == BM && WI * 8 * NW == BN, "whole copies per wave");
  static_assert(MI * 32 == WM && NJ * 32 == WN, "whole MFMA blocks per wave");
};

typedef __attribute__((address_space(3))) void* lds_ptr_t;

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// 64 lanes x 16 B global -> LDS (buffer_load_dwordx4 ... lds): lane l's 16
// bytes land at LDS byte lds_addr + 16*l.  Asm, so the compiler neither moves
// the fragment reads around it nor waits for it; the main loop waits for the
// copies itself (vmcnt) before the barrier that publishes a stage.
__device__ __forceinline__ void dma16(u32x4 rsrc, uint32_t lds_addr, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :: "s"(lds_addr), "v"(voff), "s"(rsrc) : "m0");
}
#pragma clang diagnostic pop

// Wave-uniform buffer resource over [base, base + bytes): loads at or past
// `bytes` return zeros.
__device__ __forceinline__ u32x4 rsrc_words(const unsigned char* base, uint32_t bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)base;
  return u32x4{(uint32_t)a, (uint32_t)(a >> 32) & 0xffffu, bytes, 0x00020000u};
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt field");
  // vmcnt in bits 3:0 and 15:14, expcnt (7) and lgkmcnt (63) left alone
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0x3f << 8));
}

// Layout of a stage in LDS: A rows [BM][64 B], then W rows [BN][64 B].  The
// 16-byte chunk c of row r sits at physical chunk c ^ ((r >> 2) & 3): a
// fragment read (32 rows, one chunk each per 32 lanes) then touches all 64
// banks once per 16 lanes, and a 1 KiB copy (16 rows x 4 chunks) writes one
// contiguous KiB.
__device__ __forceinline__ int swz(int r) { return (r >> 2) & 3; }

// Origin of the tile of workgroup bx of region rg (bx % 8 is the XCD: every
// region starts at a multiple of 8): XCD x takes a contiguous run of the tile
// order, which walks group_m tile rows at a time.  False for a padding
// workgroup.
template <class C>
__device__ __forceinline__ bool tile_origin(const GemmRegion& rg, const int bx, int& m0, int& n0) {
  const int T = rg.ntm * rg.ntn;
  const int x = bx & 7, s = bx >> 3;
  const int q = T >> 3, r = T & 7;
  if (s >= q + (x < r ? 1 : 0)) return false;
  const int t = x * q + min(x, r) + s;
  const int gsz_full = rg.group_m * rg.ntn;
  const int g = t / gsz_full;
  const int first = g * rg.group_m;
  const int gm = min(rg.group_m, rg.ntm - first);
  const int tr = t - g * gsz_full;
  m0 = (first + tr % gm) * C::BM;
  n0 = (tr / gm) * C::BN;
  return true;
}

template <class C, bool FP16>
__device__ __forceinline__ void store_tile(const GemmParams& p, const GemmRegion& rg, const int m0, const int n0,
                                           const f32x16 (&acc)[C::NJ][C::MI], unsigned char* lds, const int wave,
                                           const int lane);

// One BM x BN output tile of region g; bx counts the region's workgroups.
// SPLIT: the workgroup sums k-steps [kb, ke) of slice `slice` and writes the
// fp32 sums to p.partial instead of the outputs.
template <class C, bool FP16, bool SPLIT = false>
__device__ __forceinline__ void gemm_tile(const GemmParams& p, const GemmRegion& rg, const int bx,
                                          unsigned char* lds, const int slice = 0) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: copy targets go to SGPRs
  const int wm = wave % C::WGM, wn = wave / C::WGM;

  int m0, n0;
  if (!tile_origin<C>(rg, bx, m0, n0)) return;
  const int mrows = min(C::BM, p.M - m0);
  const int nrows = min(C::BN, rg.N - n0);

  // per-lane copy offsets: copy i of this wave fills 16-row group wave + NW i
  // of its tile; lane l writes row l/4 of the group, physical chunk l%4,
  // which holds logical chunk (l%4) ^ swz(row)
  const int crow = wave * 16 + (lane >> 2);
  const int cchunk = ((lane & 3) ^ ((lane >> 4) & 3)) * 16;
  uint32_t aoff[C::AI], woff[C::WI];
#pragma unroll
  for (int i = 0; i < C::AI; ++i) aoff[i] = (uint32_t)((crow + 16 * C::NW * i) * p.lda + cchunk);
#pragma unroll
  for (int i = 0; i < C::WI; ++i) woff[i] = (uint32_t)((crow + 16 * C::NW * i) * p.ldw + cchunk);
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_ptr_t)lds;
  const unsigned char* abase = p.a + (int64_t)m0 * p.lda;
  const unsigned char* wbase = rg.w + (int64_t)n0 * p.ldw;
  const int nkall = (p.K + KB - 1) / KB;
  const int kb = SPLIT ? (int)((int64_t)nkall * slice / p.ksplit) : 0;
  const int nk = SPLIT ? (int)((int64_t)nkall * (slice + 1) / p.ksplit) : nkall;  // end of the k-steps

  // copy state of one k-step: the stage's LDS address and the two buffer
  // resources; past the end of K a lane's chunk would read the next row, so
  // its offset gets the top bit (out of range: it lands as zeros)
  struct StepCopies {
    u32x4 ra, rw;
    uint32_t st;
    uint32_t dead;  // 0, or 0x80000000 for a lane whose chunk lies past K
  };
  // A k-step at or past the end (kt >= nk) gets empty resources: its copies
  // fetch nothing and write zeros into a stage that no later step reads, so
  // every step issues the same copies and the vmcnt waits stay uniform.
  auto prepare = [&](const int kt) __attribute__((always_inline)) {
    StepCopies sc;
    const int koff = kt * KB;
    const int lim = p.K - koff;  // k bytes left in every row
    const int kin = min(KB, lim);
    sc.ra = rsrc_words(abase + koff, kt < nk ? (uint32_t)((mrows - 1) * p.lda + kin) : 0u);
    sc.rw = rsrc_words(wbase + koff, kt < nk ? (uint32_t)((nrows - 1) * p.ldw + kin) : 0u);
    sc.st = lds0 + (uint32_t)((kt % C::NS) * C::STAGE);
    sc.dead = (lim < KB && cchunk >= lim) ? 0x80000000u : 0u;
    return sc;
  };
  // copy i of this wave's list (A copies first, then W)
  auto issue = [&](const StepCopies& sc, const int i) __attribute__((always_inline)) {
    if (i < C::AI) dma16(sc.ra, sc.st + (uint32_t)((wave + C::NW * i) * 1024), aoff[i] | sc.dead);
    else dma16(sc.rw, sc.st + (uint32_t)(C::A_BYTES + (wave + C::NW * (i - C::AI)) * 1024), woff[i - C::AI] | sc.dead);
  };
  auto copy_stage = [&](const int kt) __attribute__((always_inline)) {
    const StepCopies sc = prepare(kt);
#pragma unroll
    for (int i = 0; i < C::COPIES; ++i) issue(sc, i);
  };

  // fragment read offsets: lane l reads row l%32 of a 32-row block, logical
  // chunks 2*(l/32) and 2*(l/32)+1
  const int frow = lane & 31;
  const uint32_t f0 = (uint32_t)(frow * KB + (((lane >> 5) * 2) ^ swz(frow)) * 16);
  const uint32_t f1 = (uint32_t)(frow * KB + (((lane >> 5) * 2 + 1) ^ swz(frow)) * 16);
  // half r % 2 of fragment r / 2 (A fragments first, then W) of stage kt
  constexpr int NRD = 2 * (C::MI + C::NJ);
  auto read_frag = [&](const int kt, const int r, i32x8 (&fa)[C::MI], i32x8 (&fw)[C::NJ])
      __attribute__((always_inline)) {
    const unsigned char* st = lds + (kt % C::NS) * C::STAGE;
    const int f = r >> 1;
    const uint32_t off = (r & 1) ? f1 : f0;
    const unsigned char* b = f < C::MI ? st + (wm * C::WM + f * 32) * KB
                                       : st + C::A_BYTES + (wn * C::WN + (f - C::MI) * 32) * KB;
    const u32x4 v = *reinterpret_cast<const u32x4*>(b + off);
    i32x8& dst = f < C::MI ? fa[f] : fw[f - C::MI];
    const int e = (r & 1) * 4;
    dst[e] = (int)v.x;
    dst[e + 1] = (int)v.y;
    dst[e + 2] = (int)v.z;
    dst[e + 3] = (int)v.w;
  };
  auto read_frags = [&](const int kt, i32x8 (&fa)[C::MI], i32x8 (&fw)[C::NJ]) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < NRD; ++r) read_frag(kt, r, fa, fw);
  };

  f32x16 acc[C::NJ][C::MI];
#pragma unroll
  for (int j = 0; j < C::NJ; ++j)
#pragma unroll
    for (int i = 0; i < C::MI; ++i) acc[j][i] = f32x16{};

  // prologue: stages 0 .. NS-2 in flight, stage 0 published, its fragments read
#pragma unroll
  for (int s0 = 0; s0 < C::NS - 1; ++s0) copy_stage(kb + s0);
  wait_vmcnt<(C::NS - 2) * C::COPIES>();
  __syncthreads();
  i32x8 fa[2][C::MI], fw[2][C::NJ];
  read_frags(kb, fa[0], fw[0]);

  // k-step kt: publish stage kt+1 (its copies done, and every wave past its
  // MFMAs of kt-1, so stage kt-1 = kt+NS-1 is free), then run the MFMAs of kt
  // with the fragment reads of kt+1 between the first half of them and the
  // copies of kt+NS-1 between the second half.  Issued as one burst, the 16
  // reads of a 256 x 256 tile held the wave at its second MFMA while the
  // matrix core idled.  sched_barrier(0) pins the order: the compiler would
  // otherwise hoist the wait and barrier of the next step above this step's
  // MFMAs and bunch the reads and copies together.  The reads of the step
  // after the last (a stage whose contents are not used) are issued too, so
  // the step stays one basic block.
  auto step = [&](const int kt, const int cur) __attribute__((always_inline)) {
    constexpr int NMF = C::NJ * C::MI;
    // reads after MFMAs [0, H), copies after MFMAs [CB, NMF); a wave with a
    // single MFMA per step (64 x 64 tiles) issues both after it
    constexpr int H = NMF >= 2 ? NMF / 2 : 1;
    constexpr int CB = NMF >= 2 ? H : 0;
    constexpr int CN = NMF - CB;
    __builtin_amdgcn_sched_barrier(0);
    wait_vmcnt<(C::NS - 3) * C::COPIES>();
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    const StepCopies sc = prepare(kt + C::NS - 1);
#pragma unroll
    for (int idx = 0; idx < NMF; ++idx) {
      const int j = idx / C::MI, i = idx % C::MI;
      acc[j][i] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fw[cur][j], fa[cur][i], acc[j][i], 0, 0, 0, 0,
                                                                   0, 0);
      __builtin_amdgcn_sched_barrier(0);
      if (idx < H) {
#pragma unroll
        for (int r = idx * NRD / H; r < (idx + 1) * NRD / H; ++r) read_frag(kt + 1, r, fa[cur ^ 1], fw[cur ^ 1]);
      }
      if (idx >= CB) {
#pragma unroll
        for (int c = (idx - CB) * C::COPIES / CN; c < (idx - CB + 1) * C::COPIES / CN; ++c) issue(sc, c);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  int kt = kb;
  for (; kt + 1 < nk; kt += 2) {
    step(kt, 0);
    step(kt + 1, 1);
  }
  if (kt < nk) step(kt, 0);

  wait_vmcnt<0>();  // the copies of the steps past the end still land in their stages
  if constexpr (SPLIT) {
    // the slice's fp32 sums, 4 columns of one row per lane and register quad
    float* dst = p.partial + (int64_t)slice * p.M * rg.N;
#pragma unroll
    for (int j = 0; j < C::NJ; ++j) {
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        const int n = n0 + wn * C::WN + j * 32 + qd * 8 + (lane >> 5) * 4;
#pragma unroll
        for (int i = 0; i < C::MI; ++i) {
          const int m = m0 + wm * C::WM + i * 32 + (lane & 31);
          if (m < p.M && n < rg.N) {
            const f32x4 v = {acc[j][i][qd * 4], acc[j][i][qd * 4 + 1], acc[j][i][qd * 4 + 2], acc[j][i][qd * 4 + 3]};
            *reinterpret_cast<f32x4*>(dst + (int64_t)m * rg.N + n) = v;
          }
        }
      }
    }
    return;
  }
  store_tile<C, FP16>(p, rg, m0, n0, acc, lds, wave, lane);
}

// The tile's outputs: out[m][n..n+3] = round(acc * (sa * sw) + bias[n..n+3]),
// staged through LDS (the stage memory, once every copy has landed): a
// lane's results are 4 columns of one row, so stored straight from the
// accumulators every store instruction would touch 32 rows; from LDS each one
// writes whole rows of the tile (64 lanes x 16 B).  Staged row ml keeps its
// 16-byte chunk c at physical chunk c ^ (ml % CPR), which spreads a
// fragment's 32 rows over the banks.
template <class C, bool FP16>
__device__ __forceinline__ void store_tile(const GemmParams& p, const GemmRegion& rg, const int m0, const int n0,
                                           const f32x16 (&acc)[C::NJ][C::MI], unsigned char* lds, const int wave,
                                           const int lane) {
  const int wm = wave % C::WGM, wn = wave / C::WGM;
  constexpr int RB = C::BN * 2;   // bytes of a staged row
  constexpr int CPR = RB / 16;    // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;   // rows per store instruction
  static_assert(C::BM * RB <= C::NS * C::STAGE, "the output tile fits the stages");
  __syncthreads();  // and every wave is done with the last stage's fragments
  {
#pragma clang fp contract(off)
    const float ab = p.sa[0] * p.sw[0];
#pragma unroll
    for (int j = 0; j < C::NJ; ++j) {
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        const int nl = wn * C::WN + j * 32 + qd * 8 + (lane >> 5) * 4;
        const int n = n0 + nl;
        float bv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (rg.bias != nullptr && n < rg.N) {
          const u32x2 braw = *reinterpret_cast<const u32x2*>(rg.bias + (int64_t)n * 2);
          unpack2<FP16>(braw.x, bv[0], bv[1]);
          unpack2<FP16>(braw.y, bv[2], bv[3]);
        }
#pragma unroll
        for (int i = 0; i < C::MI; ++i) {
          const int ml = wm * C::WM + i * 32 + (lane & 31);
          float y[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            y[e] = acc[j][i][qd * 4 + e] * ab;
            y[e] = y[e] + bv[e];
          }
          const u32x2 o = {pack2<FP16>(y[0], y[1]), pack2<FP16>(y[2], y[3])};
          const int phys = (nl >> 3) ^ (ml & (CPR - 1));
          *reinterpret_cast<u32x2*>(lds + ml * RB + phys * 16 + (lane >> 5) * 8) = o;
        }
      }
    }
  }
  __syncthreads();
  const int c = lane % CPR;
  const int n = n0 + c * 8;
#pragma unroll 4
  for (int r0 = wave * RPI; r0 < C::BM; r0 += C::NW * RPI) {
    const int ml = r0 + lane / CPR;
    const u32x4 v = *reinterpret_cast<const u32x4*>(lds + ml * RB + ((c ^ (ml & (CPR - 1))) * 16));
    const int m = m0 + ml;
    if (m < p.M && n < rg.N) *reinterpret_cast<u32x4*>(rg.out + ((int64_t)m * p.ldc + n) * 2) = v;
  }
}

// One BM x BN output tile with 128 k-bytes per stage (CfgK128).  Layout of a
// stage in LDS: A rows [BM][128 B], then W rows [BN][128 B]; the 16-byte chunk
// c of row r sits at physical chunk c ^ swz8(r), swz8(r) = (r >> 1) & 7: a
// fragment read (16 lanes on 16 consecutive rows, one chunk each) then
// touches all 64 banks once, and a 1 KiB copy (8 rows x 8 chunks) writes one
// contiguous KiB.  Each step of 128 k-bytes runs two MFMA k-steps:
//   A: the MFMAs of the stage's first half, with the reads of its second half
//      between the first half of them;
//   B: the MFMAs of the second half: the first two, then the wait for the
//      next stage's copies and one barrier, which publishes the next stage
//      and releases this one (every wave has read both of its halves; the
//      barrier's LDS fence waits for those reads), then the rest, with the
//      reads of the next stage's first half and the copies of the stage after
//      next (into this stage's memory) spread between them.
// Interleaved on one box against the 64-byte form (4 stages, a barrier per
// MFMA k-step): 4352 x 9216 x 3072 103.8 against 110.0 us, 4352 x 12288 x 3072
// 137.2 / 146.0, 4352 x 3072 x 12288 120.8 / 127.7, 4096 x 4096 x 12288
// 137.1 / 151.1; with B's copies after its second half of MFMAs only (as the
// 64-byte form places them) the gain was 0-5%, and spreading them in the
// 64-byte form changed nothing.  Two of B's MFMAs ahead of the barrier: 0.7-5%
// faster again (1536 x 4096 x 12288 77.5 against 81.5 us, 4352 x 3072 x 12288
// 119.8 / 121.8), one or four: no better.
template <class C, bool FP16>
__device__ __forceinline__ void gemm_tile_k128(const GemmParams& p, const GemmRegion& rg, const int bx,
                                               unsigned char* lds) {
  static_assert(C::KB == 128 && C::NS == 2, "two stages of 128 k-bytes");
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: copy targets go to SGPRs
  const int wm = wave % C::WGM, wn = wave / C::WGM;

  int m0, n0;
  if (!tile_origin<C>(rg, bx, m0, n0)) return;
  const int mrows = min(C::BM, p.M - m0);
  const int nrows = min(C::BN, rg.N - n0);

  // per-lane copy offsets: copy i of this wave fills 8-row group wave + NW i
  // of its tile; lane l writes row l/8 of the group, physical chunk l%8, which
  // holds logical chunk (l%8) ^ swz8(row).  NW is even, so the groups of one
  // wave share swz8 and one chunk offset serves all of its copies.
  const int crow = wave * 8 + (lane >> 3);
  const int cchunk = ((lane & 7) ^ ((crow >> 1) & 7)) * 16;
  uint32_t aoff[C::AI], woff[C::WI];
#pragma unroll
  for (int i = 0; i < C::AI; ++i) aoff[i] = (uint32_t)((crow + 8 * C::NW * i) * p.lda + cchunk);
#pragma unroll
  for (int i = 0; i < C::WI; ++i) woff[i] = (uint32_t)((crow + 8 * C::NW * i) * p.ldw + cchunk);
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_ptr_t)lds;
  const unsigned char* abase = p.a + (int64_t)m0 * p.lda;
  const unsigned char* wbase = rg.w + (int64_t)n0 * p.ldw;
  const int nk = (p.K + C::KB - 1) / C::KB;

  // copy state of one step, as in gemm_tile: past the end of K a lane's chunk
  // gets the top offset bit (it lands as zeros), and a step at or past the
  // end gets empty resources, so every step issues the same copies
  struct StepCopies {
    u32x4 ra, rw;
    uint32_t st;
    uint32_t dead;
  };
  auto prepare = [&](const int kt) __attribute__((always_inline)) {
    StepCopies sc;
    const int koff = kt * C::KB;
    const int lim = p.K - koff;
    const int kin = min(C::KB, lim);
    sc.ra = rsrc_words(abase + koff, kt < nk ? (uint32_t)((mrows - 1) * p.lda + kin) : 0u);
    sc.rw = rsrc_words(wbase + koff, kt < nk ? (uint32_t)((nrows - 1) * p.ldw + kin) : 0u);
    sc.st = lds0 + (uint32_t)((kt & 1) * C::STAGE);
    sc.dead = (lim < C::KB && cchunk >= lim) ? 0x80000000u : 0u;
    return sc;
  };
  auto issue = [&](const StepCopies& sc, const int i) __attribute__((always_inline)) {
    if (i < C::AI) dma16(sc.ra, sc.st + (uint32_t)((wave + C::NW * i) * 1024), aoff[i] | sc.dead);
    else dma16(sc.rw, sc.st + (uint32_t)(C::A_BYTES + (wave + C::NW * (i - C::AI)) * 1024), woff[i - C::AI] | sc.dead);
  };

  // fragment reads: lane l reads row l%32 of a 32-row block, logical chunks
  // 4h + 2(l/32) and 4h + 2(l/32) + 1 of k-half h; blocks start at multiples
  // of 32 rows, so swz8 of the row is swz8(l%32)
  const int frow = lane & 31;
  uint32_t fo[2][2];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int e = 0; e < 2; ++e)
      fo[h][e] = (uint32_t)(frow * C::KB + ((4 * h + 2 * (lane >> 5) + e) ^ ((frow >> 1) & 7)) * 16);
  constexpr int NRD = 2 * (C::MI + C::NJ);
  // half r % 2 of fragment r / 2 (A fragments first, then W), k-half h of stage kt
  auto read_frag = [&](const int kt, const int h, const int r, i32x8 (&fa)[C::MI], i32x8 (&fw)[C::NJ])
      __attribute__((always_inline)) {
    const unsigned char* st = lds + (kt & 1) * C::STAGE;
    const int f = r >> 1;
    const unsigned char* b = f < C::MI ? st + (wm * C::WM + f * 32) * C::KB
                                       : st + C::A_BYTES + (wn * C::WN + (f - C::MI) * 32) * C::KB;
    const u32x4 v = *reinterpret_cast<const u32x4*>(b + fo[h][r & 1]);
    i32x8& dst = f < C::MI ? fa[f] : fw[f - C::MI];
    const int e = (r & 1) * 4;
    dst[e] = (int)v.x;
    dst[e + 1] = (int)v.y;
    dst[e + 2] = (int)v.z;
    dst[e + 3] = (int)v.w;
  };

  f32x16 acc[C::NJ][C::MI];
#pragma unroll
  for (int j = 0; j < C::NJ; ++j)
#pragma unroll
    for (int i = 0; i < C::MI; ++i) acc[j][i] = f32x16{};

  // prologue: both stages in flight, stage 0 published, its first half read
  {
    const StepCopies s0 = prepare(0);
#pragma unroll
    for (int c = 0; c < C::COPIES; ++c) issue(s0, c);
    const StepCopies s1 = prepare(1);
#pragma unroll
    for (int c = 0; c < C::COPIES; ++c) issue(s1, c);
  }
  wait_vmcnt<C::COPIES>();
  __syncthreads();
  i32x8 fa[2][C::MI], fw[2][C::NJ];
#pragma unroll
  for (int r = 0; r < NRD; ++r) read_frag(0, 0, r, fa[0], fw[0]);

  // One MFMA k-step on fragments `cur`, with the reads of (stage rkt, half rh)
  // into the other fragments between its MFMAs.  The second k-step (COPY)
  // issues its first PRE MFMAs (their fragments are in registers) before the
  // wait for the next stage's copies and the barrier, so the matrix core has
  // work while the wave waits there; its reads and the copies of sc follow,
  // spread over the remaining MFMAs.
  constexpr int NMF = C::NJ * C::MI;
  constexpr int PRE = 2 < NMF ? 2 : NMF - 1;
  auto kstep = [&](auto copy_tag, const int cur, const int rkt, const int rh, const StepCopies& sc)
      __attribute__((always_inline)) {
    constexpr bool COPY = decltype(copy_tag)::value;
    constexpr int R0 = COPY ? PRE : 0;  // reads (and copies) after MFMAs [R0, R0 + H)
    constexpr int H = COPY ? NMF - PRE : (NMF >= 2 ? NMF / 2 : 1);
#pragma unroll
    for (int idx = 0; idx < NMF; ++idx) {
      const int j = idx / C::MI, i = idx % C::MI;
      acc[j][i] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fw[cur][j], fa[cur][i], acc[j][i], 0, 0, 0, 0,
                                                                   0, 0);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (COPY) {
        if (idx == PRE - 1) {
          wait_vmcnt<0>();  // the next stage's copies (issued one step ago) have landed
          __syncthreads();
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      if (idx >= R0 && idx < R0 + H) {
#pragma unroll
        for (int r = (idx - R0) * NRD / H; r < (idx - R0 + 1) * NRD / H; ++r)
          read_frag(rkt, rh, r, fa[cur ^ 1], fw[cur ^ 1]);
        if constexpr (COPY) {
#pragma unroll
          for (int c = (idx - R0) * C::COPIES / H; c < (idx - R0 + 1) * C::COPIES / H; ++c) issue(sc, c);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  for (int kt = 0; kt < nk; ++kt) {
    const StepCopies none = {};
    kstep(std::false_type{}, 0, kt, 1, none);
    __builtin_amdgcn_sched_barrier(0);
    const StepCopies sc = prepare(kt + 2);
    kstep(std::true_type{}, 1, kt + 1, 0, sc);
  }

  wait_vmcnt<0>();  // the copies of the steps past the end still land in their stages
  store_tile<C, FP16>(p, rg, m0, n0, acc, lds, wave, lane);
}

// A tile of either form.
template <class C, bool FP16>
__device__ __forceinline__ void run_tile(const GemmParams& p, const GemmRegion& rg, const int bx, unsigned char* lds) {
  if constexpr (C::KB == 128) gemm_tile_k128<C, FP16>(p, rg, bx, lds);
  else gemm_tile<C, FP16>(p, rg, bx, lds);
}

// Region 0 (C1 tiles) and region 1 (C2 tiles), one after the other in
// blockIdx order; the dispatcher starts workgroups in that order.  Region 0
// first: region 1's smaller tiles fill the CUs that region 0's last round
// leaves free.  Region 1 first (small_first, when the host's makespan
// estimate is no worse): the CUs that took a small tile start their big ones
// part of a tile later than the others, so the tiles' output stores do not
// all fall at once beside the next round's copies.
template <class C1, class C2, bool FP16>
__global__ void __launch_bounds__(C1::NT) __attribute__((amdgpu_waves_per_eu(C1::NW / 4, C1::NW / 4)))
fp8_gemm_kernel(const GemmParams p) {
  static_assert(C1::NT == C2::NT, "one workgroup size per launch");
  constexpr int LDS1 = C1::NS * C1::STAGE, LDS2 = C2::NS * C2::STAGE;
  __shared__ __attribute__((aligned(1024))) unsigned char lds[LDS1 > LDS2 ? LDS1 : LDS2];
  const int bx = blockIdx.x;
  const int off0 = p.small_first ? p.r[1].wgs : 0;  // first workgroup of each region
  const int off1 = p.small_first ? 0 : p.r[0].wgs;
  if (bx >= off0 && bx < off0 + p.r[0].wgs) run_tile<C1, FP16>(p, p.r[0], bx - off0, lds);
  else run_tile<C2, FP16>(p, p.r[1], bx - off1, lds);
}

// Split launch: workgroup b sums k-slice b / wgs of tile b % wgs of region 0
// (wgs a multiple of 8, so a tile's slices all run on one XCD).
template <class C, bool FP16>
__global__ void __launch_bounds__(C::NT) __attribute__((amdgpu_waves_per_eu(C::NW / 4, C::NW / 4)))
fp8_gemm_split_kernel(const GemmParams p) {
  __shared__ __attribute__((aligned(1024))) unsigned char lds[C::NS * C::STAGE];
  const int wgs = p.r[0].wgs;
  const int bx = blockIdx.x;
  gemm_tile<C, FP16, true>(p, p.r[0], bx % wgs, lds, bx / wgs);
}

// out[m][n..n+7] = round((sum over the slices, in slice order) * (sa * sw)
// + bias[n..n+7]), 8 outputs per thread.
template <bool FP16>
__global__ void __launch_bounds__(256) splitk_reduce_kernel(const GemmParams p) {
#pragma clang fp contract(off)
  const GemmRegion& rg = p.r[0];
  const int per_row = rg.N / 8;
  const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (g >= (int64_t)p.M * per_row) return;
  const int m = (int)(g / per_row);
  const int n = (int)(g - (int64_t)m * per_row) * 8;
  const int64_t slice_elems = (int64_t)p.M * rg.N;
  const float* src = p.partial + (int64_t)m * rg.N + n;
  f32x4 lo = *reinterpret_cast<const f32x4*>(src);
  f32x4 hi = *reinterpret_cast<const f32x4*>(src + 4);
  for (int sl = 1; sl < p.ksplit; ++sl) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(src + sl * slice_elems);
    const f32x4 b = *reinterpret_cast<const f32x4*>(src + sl * slice_elems + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      lo[e] = lo[e] + a[e];
      hi[e] = hi[e] + b[e];
    }
  }
  const float ab = p.sa[0] * p.sw[0];
  float bv[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  if (rg.bias != nullptr) {  // the bias is 8-byte aligned
    const u32x2 b0 = *reinterpret_cast<const u32x2*>(rg.bias + (int64_t)n * 2);
    const u32x2 b1 = *reinterpret_cast<const u32x2*>(rg.bias + (int64_t)n * 2 + 8);
    unpack2<FP16>(b0.x, bv[0], bv[1]);
    unpack2<FP16>(b0.y, bv[2], bv[3]);
    unpack2<FP16>(b1.x, bv[4], bv[5]);
    unpack2<FP16>(b1.y, bv[6], bv[7]);
  }
  float y[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    y[e] = lo[e] * ab;
    y[e] = y[e] + bv[e];
    y[e + 4] = hi[e] * ab;
    y[e + 4] = y[e + 4] + bv[e + 4];
  }
  const u32x4 o = {pack2<FP16>(y[0], y[1]), pack2<FP16>(y[2], y[3]), pack2<FP16>(y[4], y[5]), pack2<FP16>(y[6], y[7])};
  *reinterpret_cast<u32x4*>(rg.out + ((int64_t)m * p.ldc + n) * 2) = o;
}

}  // namespace qik_fp8

namespace qik_fp8 {

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

int validate_quant(const qik_fp8_quant_args* a) {
  if (a == nullptr) return QIK_ERR_NULL_ARG;
  if (a->abi_version != QIK_ABI_VERSION || a->reserved0 != 0) return QIK_ERR_ABI_VERSION;
  if (a->dtype != QIK_DTYPE_BF16 && a->dtype != QIK_DTYPE_FP16 && a->dtype != QIK_DTYPE_FP32) return QIK_ERR_DTYPE;
  if (a->mode != QIK_FP8_ACTIVATION && a->mode != QIK_FP8_WEIGHT) return QIK_ERR_DTYPE;
  if (a->n < 1 || a->n >= ((int64_t)1 << 40)) return QIK_ERR_SHAPE;
  if (a->x == nullptr || a->out == nullptr || a->scale == nullptr) return QIK_ERR_NULL_ARG;
  const int per_vec = a->dtype == QIK_DTYPE_FP32 ? 4 : 8;
  if (!aligned_to(a->x, 16) || !aligned_to(a->out, per_vec) || !aligned_to(a->scale, 4)) return QIK_ERR_ALIGN;
  return QIK_OK;
}

// blocks of the maximum pass: about 8 vectors per thread, at most MAX_PARTS
int quant_parts(const qik_fp8_quant_args* a) {
  const int per_vec = a->dtype == QIK_DTYPE_FP32 ? 4 : 8;
  const int64_t nvec = a->n / per_vec;
  const int64_t parts = (nvec + QT * 8 - 1) / (QT * 8);
  return (int)std::max<int64_t>(1, std::min<int64_t>(parts, MAX_PARTS));
}

// Vectors per thread of the one-pass launches, smallest first: dense enough
// that most inputs find a size whose grid nearly fills the CUs with one
// workgroup each (measured at [4352, 3072] bf16 on MI355X: 252 workgroups of
// 26 vectors 10.7 us, 204 of 32 12.0 us, 272 of 24 13.2 us).
constexpr int ONEPASS_N = 10;
constexpr int ONEPASS_VPT[ONEPASS_N] = {4, 8, 12, 16, 20, 24, 26, 32, 40, 52};
constexpr int ONEPASS_DEFAULT_SPIN = 1 << 16;  // polls of one device-scope round trip each: tens of ms

template <int DT, int MODE, int VPT>
const void* onepass_fn() {
  return (const void*)quant_onepass_kernel<DT, MODE, VPT>;
}

// Workgroups of one one-pass variant that the current device holds at once
// (occupancy x CUs, at most RES_SLOTS), cached per device; 0 if unknown.
int onepass_capacity(const void* fn, int which) {
  static int cache[64][3 * 2 * ONEPASS_N];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int c = __atomic_load_n(&cache[dev][which], __ATOMIC_RELAXED);
  if (c > 0) return c;
  const int cus = device_cus();
  int occ = 0;
  if (cus <= 0 || hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, fn, QT, 0) != hipSuccess || occ <= 0) return 0;
  c = std::min(occ * cus, RES_SLOTS);
  __atomic_store_n(&cache[dev][which], c, __ATOMIC_RELAXED);
  return c;
}

template <int DT, int MODE, int... I>
const void* onepass_pick_seq(int i, std::integer_sequence<int, I...>) {
  const void* fns[] = {onepass_fn<DT, MODE, ONEPASS_VPT[I]>()...};
  return fns[i];
}
template <int DT, int MODE>
const void* onepass_pick(int i) {
  return onepass_pick_seq<DT, MODE>(i, std::make_integer_sequence<int, ONEPASS_N>{});
}

// The one-pass launch for n elements: kernel and grid, or fn = NULL when x
// does not fit the registers of the resident workgroups (the two-pass form).
struct OnePass {
  const void* fn;
  int64_t grid;
};

// The fewest workgroups win: every workgroup reads every slot, so the exchange
// grows with the square of the grid.  The smallest VPT that needs at most one
// workgroup per CU, else the smallest that fits the resident workgroups.
template <int DT>
OnePass plan_onepass(const qik_fp8_quant_args* a) {
  constexpr int PV = Elem<DT>::PER_VEC;
  const int64_t nvec = std::max<int64_t>(1, a->n / PV);
  if (nvec * 16 >= (int64_t)INT_MAX) return OnePass{nullptr, 0};  // 32-bit buffer offsets
  const int cus = device_cus();
  OnePass fit{nullptr, 0};
  for (int i = 0; i < ONEPASS_N; ++i) {
    const int64_t grid = (nvec + (int64_t)QT * ONEPASS_VPT[i] - 1) / ((int64_t)QT * ONEPASS_VPT[i]);
    const void* fn = a->mode == QIK_FP8_ACTIVATION ? onepass_pick<DT, QIK_FP8_ACTIVATION>(i)
                                                   : onepass_pick<DT, QIK_FP8_WEIGHT>(i);
    const int dt_i = DT == QIK_DTYPE_BF16 ? 0 : DT == QIK_DTYPE_FP16 ? 1 : 2;
    const int cap = onepass_capacity(fn, (dt_i * 2 + a->mode) * ONEPASS_N + i);
    if (cap <= 0 || grid > cap) continue;
    if (grid <= cus) return OnePass{fn, grid};
    if (fit.fn == nullptr) fit = OnePass{fn, grid};
  }
  return fit;
}

template <int DT>
int launch_quant(const qik_fp8_quant_args* a, unsigned* ws, hipStream_t s) {
  constexpr int PV = Elem<DT>::PER_VEC;
  QuantParams p;
  memset(&p, 0, sizeof(p));
  p.x = static_cast<const char*>(a->x);
  p.out = static_cast<unsigned char*>(a->out);
  p.scale = a->scale;
  p.ctl = ws;
  p.part = ws + QCTL + 2 * RES_SLOTS;
  p.n = a->n;
  p.nvec = a->n / PV;
  p.nparts = quant_parts(a);
  p.spin = ONEPASS_DEFAULT_SPIN;
  void* args[] = {&p};
  const OnePass op = plan_onepass<DT>(a);
  if (op.fn != nullptr)
    return hipLaunchKernel(op.fn, dim3((unsigned)op.grid), dim3(QT), args, 0, s) == hipSuccess ? QIK_OK
                                                                                                 : QIK_ERR_LAUNCH;
  if (hipLaunchKernel((const void*)amax_kernel<DT>, dim3((unsigned)p.nparts), dim3(QT), args, 0, s) != hipSuccess)
    return QIK_ERR_LAUNCH;
  const int64_t grid = std::max<int64_t>(1, (p.nvec + QT * QU - 1) / (QT * QU));
  if (grid > (int64_t)INT_MAX) return QIK_ERR_SHAPE;
  const void* fn = a->mode == QIK_FP8_ACTIVATION ? (const void*)cast_kernel<DT, QIK_FP8_ACTIVATION>
                                                 : (const void*)cast_kernel<DT, QIK_FP8_WEIGHT>;
  return hipLaunchKernel(fn, dim3((unsigned)grid), dim3(QT), args, 0, s) == hipSuccess ? QIK_OK : QIK_ERR_LAUNCH;
}

// GEMM tile shapes, largest first
// The 256-row pair: 128 k-bytes per stage (CfgK128) and 8 waves, two per
// SIMD (2 x 4 waves, 128 x 64 wave tiles, 128 accumulators and 240 registers
// per wave).  With 64 k-bytes per stage, 8 waves against 4 of 128 x 128:
// 4352 x 9216 x 3072 109.4 against 113.1 us, 4352 x 12288 x 3072 145.8 /
// 150.6, 4352 x 3072 x 12288 128.7 / 129.3 (interleaved on one box); with 128,
// 4 waves were within 2% of 8 either way.
typedef CfgK128<256, 256, 2, 4> Cfg256x256;
typedef CfgK128<256, 128, 2, 4> Cfg256x128w8;
typedef Cfg<256, 128, 4> Cfg256x128;
// The smaller tiles' k-steps are short (four and one MFMAs per wave), so they
// keep more stages in flight to cover the copies' latency: at 256 x 3072 x
// 12288 (64 x 64 tiles) 8 stages took 27.9 us against 45.5 with 4 (16: 28.9);
// at 256 x 9216 x 3072 (128 x 128) 6 stages 17.0 against 18.8 with 4.
typedef Cfg<128, 128, 6> Cfg128x128;
typedef Cfg<64, 64, 8> Cfg64x64;
// The 192-row pair (the reference test's 1536 x 4096 x 4096 takes 256 of its
// tiles) at 128 k-bytes per stage, 4 waves: 1536 x 4096 x 4096 30.2-31.9
// against 31.2-33.8 us, 1536 x 4096 x 12288 82.4 / 86.0, interleaved on one
// box.  The 256 x 128 / 128 x 128 pair stays at 64 k-bytes: at 128 (4 waves,
// eight MFMAs per step) 768 x 3072 x 12288 took 67.7 against 54.4 us.
typedef CfgK128<192, 128, 2, 2> Cfg192x128k;
typedef CfgK128<128, 128, 2, 2> Cfg128x128k;

// Time of a tile of each shape relative to a 256 x 256 tile: area / rate,
// the rates measured on MI355X with each shape forced over whole launches
// (1536x4096x4096 50.0 / 35.1 / 45.8 us, 4352x9216x3072 146.7 / 153.1 /
// 201.1 us, 4352x3072x12288 141.4 / 188.0 / 265.1 us for 256x256 / 256x128 /
// 128x128).  A 256 x 128 tile moves 24 KiB into LDS per 512 MFMA cycles,
// close to what the copy path sustains, so it runs at about 0.8 of the big
// tile's rate per output, and 128 x 128 at about 0.6.  The 64 x 64 tile (one
// MFMA per wave and step) is for launches with few tiles: at 256 x 3072 x
// 12288 its 192 tiles took 45.7 us against 65.5 for 48 tiles of 128 x 128;
// 0.3 is the rate that keeps it out of the 512- and 1024-row shapes (0.45
// chose it there, 16-25% slower).  The 192 x 128 tile makes 256 tiles of
// 1536 x 4096 (one per CU): 33.0 us against 35.6 for 192 tiles of 256 x 128,
// a rate of about 0.65.
struct TileShape {
  int bm, bn;
  double t;
};
static const TileShape kShapes[5] = {
    {256, 256, 1.0}, {256, 128, 0.5 / 0.8}, {128, 128, 0.25 / 0.6}, {64, 64, 0.0625 / 0.3}, {192, 128, 0.375 / 0.65}};
// the (big, small) shape pairs a launch can take, as indices into kShapes
static const int kPairs[4][2] = {{0, 1}, {1, 2}, {4, 2}, {2, 3}};

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Finish time of one XCD whose P CUs run t1 tiles of time d1 and then t2
// tiles of time d2, one workgroup per CU (a 256-thread workgroup of these
// tiles holds a CU's four SIMDs), each started on the CU that frees first.
double xcd_makespan(int64_t t1, double d1, int64_t t2, double d2, int64_t P) {
  const int64_t full = t1 / P, rem = t1 % P;
  const double a = (double)full * d1, b = a + d1;  // CUs free after t1: P - rem at a, rem at b
  const int64_t na = P - rem, nb = rem;
  const double end1 = nb > 0 ? b : a;
  if (t2 == 0) return end1;
  // the j-th tile of t2 starts at the j-th smallest of {a + k d2} (na times
  // each) and {b + k d2} (nb times each)
  int64_t ka = 0, kb = 0, placed = 0;
  double last = a;
  while (placed < t2) {
    const double ta = a + (double)ka * d2, tb = nb > 0 ? b + (double)kb * d2 : 1e300;
    if (ta <= tb) {
      last = ta;
      placed += na;
      ++ka;
    } else {
      last = tb;
      placed += nb;
      ++kb;
    }
  }
  return std::max(end1, last + d2);
}

// Columns [0, n1) with tile shape `big`, [n1, N) with shape big + 1.
struct GemmPlan {
  int pair;  // index into kPairs
  int64_t n1;
  double t;  // estimated makespan, in 256 x 256 tile times
  bool small_first;  // launch the small tiles' region first (fp8_gemm_kernel)
};

// The split with the shortest estimated makespan on `cus` CUs.  Workgroups go
// to the XCDs in turn, so the XCD that finishes last holds ceil(tiles / 8) of
// each region.  The split points are whole big-tile columns; n1 = N is one
// region of the big shape, n1 = 0 one of the small shape.  A later candidate
// replaces an earlier one only if it is estimated 3% faster (the rates above
// are good to a few percent); the first candidate is 256 x 256 tiles.
GemmPlan choose_plan(int64_t M, int64_t N, int cus) {
  const int64_t P = std::max(1, (cus > 0 ? cus : 256) / 8);
  GemmPlan best = {0, N, 0.0};
  double best_t = 1e300;
  for (int pr = 0; pr < 4; ++pr) {
    const TileShape& s1 = kShapes[kPairs[pr][0]];
    const TileShape& s2 = kShapes[kPairs[pr][1]];
    for (int64_t k = cdiv(N, s1.bn); k >= 0; --k) {
      const int64_t n1 = std::min(k * s1.bn, N);
      const int64_t t1 = cdiv(M, s1.bm) * cdiv(n1, s1.bn);
      const int64_t t2 = cdiv(M, s2.bm) * cdiv(N - n1, s2.bn);
      const double t = xcd_makespan(cdiv(t1, 8), s1.t, cdiv(t2, 8), s2.t, P);
      if (t < best_t * 0.97) {
        best_t = t;
        best = {pr, n1, t, false};
      }
    }
  }
  best.t = best_t;
  // the small tiles first when that is estimated no slower (measured: 1-2%
  // faster at 4352 x 9216 x 3072 and 4352 x 12288 x 3072, whose makespans are
  // equal either way; 12% slower at 1543 x 9232 x 1104, whose is not)
  const TileShape& s1 = kShapes[kPairs[best.pair][0]];
  const TileShape& s2 = kShapes[kPairs[best.pair][1]];
  const int64_t t1 = cdiv(M, s1.bm) * cdiv(best.n1, s1.bn);
  const int64_t t2 = cdiv(M, s2.bm) * cdiv(N - best.n1, s2.bn);
  if (t1 > 0 && t2 > 0)
    best.small_first = xcd_makespan(cdiv(t2, 8), s2.t, cdiv(t1, 8), s1.t, P) <= best_t * 1.0001;
  return best;
}

// K-split of a launch with few tiles and many k-steps: S slices of 128 x 128
// tiles, each summing nk / S k-steps into fp32 partials that a second launch
// adds in slice order.  Only when it is estimated well ahead of the unsplit
// plan (the partials, the second launch and the shorter pipelines cost
// something): at least 96 k-steps, at most half the CUs' worth of tiles.
// 1 means no split.
int choose_ksplit(int64_t M, int64_t N, int64_t K, int cus) {
  if (cus <= 0) cus = 256;
  const int64_t nk = cdiv(K, KB);
  if (nk < 96) return 1;
  const int64_t t128 = cdiv(M, 128) * cdiv(N, 128);
  if (t128 * 2 > cus) return 1;
  const int S = (int)std::min<int64_t>({cus / t128, 8, nk / 16});
  if (S < 2) return 1;
  const int64_t P = std::max(1, cus / 8);
  const double t_split = xcd_makespan(cdiv(t128 * S, 8), kShapes[2].t / S, 0, 0.0, P);
  return t_split < 0.6 * choose_plan(M, N, cus).t ? S : 1;
}

// tile rows per group of the tile order: the group size that minimises the
// bytes one XCD's run of tiles reads (its distinct A row blocks + W row blocks)
int choose_group_m(int ntm, int ntn, int bm, int bn) {
  const int64_t T = (int64_t)ntm * ntn;
  const int64_t per_xcd = std::max<int64_t>(1, (T + 7) / 8);
  int best = 1;
  double best_bytes = 1e300;
  for (int gm = 1; gm <= std::min(ntm, 16); ++gm) {
    const int64_t rows = std::min<int64_t>(gm, per_xcd);
    const int64_t cols = std::min<int64_t>(ntn, (per_xcd + gm - 1) / gm);
    const double bytes = (double)rows * bm + (double)cols * bn;
    if (bytes < best_bytes) {
      best_bytes = bytes;
      best = gm;
    }
  }
  return best;
}

// Region of columns [c0, c1) of the call with tile shape C.
template <class C>
int set_region(GemmRegion& rg, const qik_fp8_gemm_args* a, int64_t c0, int64_t c1) {
  rg.w = static_cast<const unsigned char*>(a->w) + c0 * a->ldw;
  rg.bias = a->bias != nullptr ? static_cast<const char*>(a->bias) + c0 * 2 : nullptr;
  rg.out = static_cast<char*>(a->out) + c0 * 2;
  rg.N = (int)(c1 - c0);
  rg.ntm = (int)cdiv(a->M, C::BM);
  rg.ntn = (int)cdiv(c1 - c0, C::BN);
  rg.group_m = choose_group_m(rg.ntm, rg.ntn, C::BM, C::BN);
  const int64_t wgs = cdiv((int64_t)rg.ntm * rg.ntn, 8) * 8;
  if (wgs > (int64_t)INT_MAX / 2) return QIK_ERR_SHAPE;
  rg.wgs = (int)wgs;
  return QIK_OK;
}

template <class C1, class C2>
int launch_gemm(GemmParams& p, const qik_fp8_gemm_args* a, int64_t n1, bool fp16, hipStream_t s) {
  int st = set_region<C1>(p.r[0], a, 0, n1);
  if (st == QIK_OK) st = set_region<C2>(p.r[1], a, n1, a->N);
  if (st != QIK_OK) return st;
  const unsigned grid = (unsigned)p.r[0].wgs + (unsigned)p.r[1].wgs;
  void* args[] = {&p};
  const void* fn = fp16 ? (const void*)fp8_gemm_kernel<C1, C2, true> : (const void*)fp8_gemm_kernel<C1, C2, false>;
  return hipLaunchKernel(fn, dim3(grid), dim3(C1::NT), args, 0, s) == hipSuccess ? QIK_OK : QIK_ERR_LAUNCH;
}

// ---------------------------------------------------------------------------
// Weight quantiser for weights in host memory (no device involved)
// ---------------------------------------------------------------------------
//
// What torch's CPU ops compute for (w.abs().amax().float() / 448).clamp_min(1e-12)
// and (w.float() / scale).clamp(-448, 448).to(float8_e4m3fn) (fp8.py:56-60):
// on the CPU both divisions are IEEE fp32 divisions (on a HIP device torch
// multiplies by the fp32 reciprocal of 448 instead, which is what the device
// quantiser reproduces).  Elementwise, so any thread split gives the same
// bytes.

// exact fp32 value of element i of a bf16 / fp16 / fp32 host array
inline float host_elem(const void* w, int32_t dtype, int64_t i) {
  if (dtype == QIK_DTYPE_FP32) return static_cast<const float*>(w)[i];
  const uint16_t h = static_cast<const uint16_t*>(w)[i];
  uint32_t bits;
  if (dtype == QIK_DTYPE_BF16) {
    bits = (uint32_t)h << 16;
  } else {
    // binary16: 1 sign, 5 exponent bits (bias 15), 10 mantissa bits
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0x1f) {
      bits = sign | 0x7f800000u | (m << 13);
    } else if (e != 0) {
      bits = sign | ((e + 112u) << 23) | (m << 13);
    } else {
      // zero or subnormal: m * 2^-24, exact in fp32
      const float f = (float)m * 5.9604644775390625e-8f;
      memcpy(&bits, &f, 4);
      bits |= sign;
    }
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

// e4m3fn code of q (|q| <= 448 or NaN), round to nearest even; NaN keeps its
// sign bit (0x7f / 0xff), and a magnitude that rounds past 448 is NaN (the
// format has no infinity)
inline unsigned char host_e4m3fn(float q) {
  uint32_t u;
  memcpy(&u, &q, 4);
  const unsigned char sign = (unsigned char)((u >> 24) & 0x80u);
  const uint32_t a = u & 0x7fffffffu;
  if (a >= 0x43e80000u) return sign | 0x7f;  // NaN, or |q| >= 464 (= 448 + half a step)
  if (a < 0x3c800000u) {
    // below 2^-6: subnormal codes m * 2^-9, m = round_even(|q| * 512) (exact scaling)
    float fa;
    memcpy(&fa, &a, 4);
    return sign | (unsigned char)std::nearbyint(fa * 512.0f);
  }
  // normal: keep 3 mantissa bits with round-to-nearest-even at bit 20, then
  // move the exponent from bias 127 to bias 7
  const uint32_t r = a + 0x7ffffu + ((a >> 20) & 1u);
  return sign | (unsigned char)((r >> 20) - (120u << 3));
}

int host_quantize_weight(const void* w, int32_t dtype, int64_t n, unsigned char* out, float* scale_out,
                         int32_t threads) {
  const int nt = (int)std::max<int64_t>(1, std::min<int64_t>(std::max(threads, 1), (n + 65535) / 65536));
  auto chunk = [&](int t, int64_t& i0, int64_t& i1) {
    i0 = n * t / nt;
    i1 = n * (t + 1) / nt;
  };
  // amax as fp32 bit patterns of |x|: unsigned order is |x| order with NaN
  // above +inf, so a NaN anywhere gives a NaN amax, as torch's amax does
  std::vector<uint32_t> part(nt, 0u);
  auto amax_part = [&](int t) {
    int64_t i0, i1;
    chunk(t, i0, i1);
    uint32_t m = 0;
    for (int64_t i = i0; i < i1; ++i) {
      uint32_t b;
      const float f = host_elem(w, dtype, i);
      memcpy(&b, &f, 4);
      m = std::max(m, b & 0x7fffffffu);
    }
    part[t] = m;
  };
  std::vector<std::thread> pool;
  for (int t = 1; t < nt; ++t) pool.emplace_back(amax_part, t);
  amax_part(0);
  for (auto& th : pool) th.join();
  pool.clear();
  uint32_t mb = 0;
  for (uint32_t v : part) mb = std::max(mb, v);
  float amax;
  memcpy(&amax, &mb, 4);
  volatile float d448 = 448.0f;  // a division, not a multiply by a folded reciprocal
  float scale = amax / d448;
  if (!(scale != scale)) scale = std::max(scale, 1e-12f);
  *scale_out = scale;
  auto codes = [&](int t) {
    int64_t i0, i1;
    chunk(t, i0, i1);
    for (int64_t i = i0; i < i1; ++i) {
      float q = host_elem(w, dtype, i) / scale;
      if (q == q) q = std::min(std::max(q, -448.0f), 448.0f);
      out[i] = host_e4m3fn(q);
    }
  };
  for (int t = 1; t < nt; ++t) pool.emplace_back(codes, t);
  codes(0);
  for (auto& th : pool) th.join();
  return QIK_OK;
}

}  // namespace qik_fp8

extern "C" {

int qik_fp8_quant_workspace_size(const qik_fp8_quant_args* a, int64_t* bytes) {
  if (bytes == nullptr) return QIK_ERR_NULL_ARG;
  *bytes = 0;
  const int st = qik_fp8::validate_quant(a);
  if (st != QIK_OK) return st;
  *bytes = (int64_t)qik_fp8::QWS_WORDS * (int64_t)sizeof(unsigned);
  return QIK_OK;
}

int qik_fp8_quantize(const qik_fp8_quant_args* a, void* workspace, int64_t workspace_bytes, void* stream) {
  using namespace qik_fp8;
  const int st = validate_quant(a);
  if (st != QIK_OK) return st;
  const int64_t need = (int64_t)QWS_WORDS * (int64_t)sizeof(unsigned);
  if (workspace == nullptr || workspace_bytes < need || !aligned_to(workspace, 4)) return QIK_ERR_WORKSPACE;
  unsigned* part = static_cast<unsigned*>(workspace);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  switch (a->dtype) {
    case QIK_DTYPE_BF16: return launch_quant<QIK_DTYPE_BF16>(a, part, s);
    case QIK_DTYPE_FP16: return launch_quant<QIK_DTYPE_FP16>(a, part, s);
    default: return launch_quant<QIK_DTYPE_FP32>(a, part, s);
  }
}

int qik_fp8_gemm_validate(const qik_fp8_gemm_args* a) {
  using namespace qik_fp8;
  if (a == nullptr) return QIK_ERR_NULL_ARG;
  if (a->abi_version != QIK_ABI_VERSION || a->reserved0 != 0 || a->reserved1 != 0) return QIK_ERR_ABI_VERSION;
  if (a->out_dtype != QIK_DTYPE_BF16 && a->out_dtype != QIK_DTYPE_FP16) return QIK_ERR_DTYPE;
  if (a->M < 1 || a->N < 16 || a->K < 16 || a->N % 16 != 0 || a->K % 16 != 0) return QIK_ERR_SHAPE;
  if (a->M > (int64_t)INT_MAX || a->N > (int64_t)INT_MAX || a->K > (int64_t)INT_MAX) return QIK_ERR_SHAPE;
  if (a->lda < a->K || a->ldw < a->K || a->ldc < a->N) return QIK_ERR_SHAPE;
  // a tile's rows must be addressable by a 31-bit buffer offset
  if (a->lda > (int64_t)(INT_MAX / 256) || a->ldw > (int64_t)(INT_MAX / 256)) return QIK_ERR_SHAPE;
  if (a->a == nullptr || a->w == nullptr || a->scale_a == nullptr || a->scale_w == nullptr || a->out == nullptr)
    return QIK_ERR_NULL_ARG;
  if (a->lda % 16 != 0 || a->ldw % 16 != 0 || a->ldc % 8 != 0) return QIK_ERR_ALIGN;
  if (!aligned_to(a->a, 16) || !aligned_to(a->w, 16) || !aligned_to(a->out, 16) || !aligned_to(a->scale_a, 4) ||
      !aligned_to(a->scale_w, 4))
    return QIK_ERR_ALIGN;
  if (a->bias != nullptr && !aligned_to(a->bias, 8)) return QIK_ERR_ALIGN;
  return QIK_OK;
}

int qik_fp8_gemm(const qik_fp8_gemm_args* a, void* stream) {
  using namespace qik_fp8;
  const int st = qik_fp8_gemm_validate(a);
  if (st != QIK_OK) return st;
  GemmParams p;
  memset(&p, 0, sizeof(p));
  p.a = static_cast<const unsigned char*>(a->a);
  p.sa = a->scale_a;
  p.sw = a->scale_w;
  p.M = (int)a->M;
  p.K = (int)a->K;
  p.lda = (int)a->lda;
  p.ldw = (int)a->ldw;
  p.ldc = a->ldc;
  const bool fp16 = a->out_dtype == QIK_DTYPE_FP16;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const GemmPlan plan = choose_plan(a->M, a->N, device_cus());
  p.small_first = plan.small_first ? 1 : 0;
  switch (plan.pair) {
    case 0: return launch_gemm<Cfg256x256, Cfg256x128w8>(p, a, plan.n1, fp16, s);
    case 1: return launch_gemm<Cfg256x128, Cfg128x128>(p, a, plan.n1, fp16, s);
    case 2: return launch_gemm<Cfg192x128k, Cfg128x128k>(p, a, plan.n1, fp16, s);
    default: return launch_gemm<Cfg128x128, Cfg64x64>(p, a, plan.n1, fp16, s);
  }
}

int qik_fp8_gemm_workspace_size(const qik_fp8_gemm_args* a, int64_t* bytes) {
  using namespace qik_fp8;
  if (bytes == nullptr) return QIK_ERR_NULL_ARG;
  *bytes = 0;
  const int st = qik_fp8_gemm_validate(a);
  if (st != QIK_OK) return st;
  const int S = choose_ksplit(a->M, a->N, a->K, device_cus());
  if (S > 1) *bytes = (int64_t)S * a->M * a->N * (int64_t)sizeof(float);
  return QIK_OK;
}

int qik_fp8_gemm_ws(const qik_fp8_gemm_args* a, void* workspace, int64_t workspace_bytes, void* stream) {
  using namespace qik_fp8;
  const int st = qik_fp8_gemm_validate(a);
  if (st != QIK_OK) return st;
  const int S = choose_ksplit(a->M, a->N, a->K, device_cus());
  if (S <= 1) return qik_fp8_gemm(a, stream);
  const int64_t need = (int64_t)S * a->M * a->N * (int64_t)sizeof(float);
  if (workspace == nullptr || workspace_bytes < need || !aligned_to(workspace, 16)) return QIK_ERR_WORKSPACE;
  GemmParams p;
  memset(&p, 0, sizeof(p));
  p.a = static_cast<const unsigned char*>(a->a);
  p.sa = a->scale_a;
  p.sw = a->scale_w;
  p.M = (int)a->M;
  p.K = (int)a->K;
  p.lda = (int)a->lda;
  p.ldw = (int)a->ldw;
  p.ldc = a->ldc;
  p.ksplit = S;
  p.partial = static_cast<float*>(workspace);
  if (set_region<Cfg128x128>(p.r[0], a, 0, a->N) != QIK_OK) return QIK_ERR_SHAPE;
  const int64_t grid = (int64_t)p.r[0].wgs * S;
  const int64_t rgrid = (a->M * (a->N / 8) + 255) / 256;
  if (grid > (int64_t)INT_MAX || rgrid > (int64_t)INT_MAX) return QIK_ERR_SHAPE;
  const bool fp16 = a->out_dtype == QIK_DTYPE_FP16;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  void* args[] = {&p};
  const void* fk = fp16 ? (const void*)fp8_gemm_split_kernel<Cfg128x128, true>
                        : (const void*)fp8_gemm_split_kernel<Cfg128x128, false>;
  if (hipLaunchKernel(fk, dim3((unsigned)grid), dim3(Cfg128x128::NT), args, 0, s) != hipSuccess)
    return QIK_ERR_LAUNCH;
  const void* fr = fp16 ? (const void*)splitk_reduce_kernel<true> : (const void*)splitk_reduce_kernel<false>;
  return hipLaunchKernel(fr, dim3((unsigned)rgrid), dim3(256), args, 0, s) == hipSuccess ? QIK_OK : QIK_ERR_LAUNCH;
}

int qik_fp8_gemm_plan(int64_t M, int64_t N, int64_t K, int32_t cus, int32_t* plan, int64_t* n1) {
  using namespace qik_fp8;
  if (plan == nullptr || n1 == nullptr) return QIK_ERR_NULL_ARG;
  if (M < 1 || N < 16 || K < 16 || N % 16 != 0 || K % 16 != 0) return QIK_ERR_SHAPE;
  if (M > (int64_t)INT_MAX || N > (int64_t)INT_MAX || K > (int64_t)(INT_MAX / 256)) return QIK_ERR_SHAPE;
  if (cus <= 0) cus = 256;
  const int S = choose_ksplit(M, N, K, cus);
  if (S > 1) {
    const int32_t v[6] = {128, 128, 128, 128, 0, S};
    memcpy(plan, v, sizeof(v));
    *n1 = N;
    return QIK_OK;
  }
  const GemmPlan g = choose_plan(M, N, cus);
  const TileShape& s1 = kShapes[kPairs[g.pair][0]];
  const TileShape& s2 = kShapes[kPairs[g.pair][1]];
  const int32_t v[6] = {s1.bm, s1.bn, s2.bm, s2.bn, g.small_first ? 1 : 0, 1};
  memcpy(plan, v, sizeof(v));
  *n1 = g.n1;
  return QIK_OK;
}

int qik_fp8_dequant(const void* w, const float* scale, void* out, int64_t n, int32_t out_dtype, void* stream) {
  using namespace qik_fp8;
  if (out_dtype != QIK_DTYPE_BF16 && out_dtype != QIK_DTYPE_FP16 && out_dtype != QIK_DTYPE_FP32)
    return QIK_ERR_DTYPE;
  if (n < 0 || n / 8 >= (int64_t)INT_MAX * QT) return QIK_ERR_SHAPE;
  if (n == 0) return QIK_OK;
  if (w == nullptr || scale == nullptr || out == nullptr) return QIK_ERR_NULL_ARG;
  if (!aligned_to(w, 8) || !aligned_to(out, 16) || !aligned_to(scale, 4)) return QIK_ERR_ALIGN;
  const int64_t grid = std::max<int64_t>(1, (n / 8 + QT - 1) / QT);
  const unsigned char* wp = static_cast<const unsigned char*>(w);
  char* op = static_cast<char*>(out);
  void* args[] = {&wp, &scale, &op, &n};
  const void* fn = out_dtype == QIK_DTYPE_FP16   ? (const void*)dequant_kernel<QIK_DTYPE_FP16>
                   : out_dtype == QIK_DTYPE_FP32 ? (const void*)dequant_kernel<QIK_DTYPE_FP32>
                                                 : (const void*)dequant_kernel<QIK_DTYPE_BF16>;
  return hipLaunchKernel(fn, dim3((unsigned)grid), dim3(QT), args, 0, static_cast<hipStream_t>(stream)) ==
                 hipSuccess
             ? QIK_OK
             : QIK_ERR_LAUNCH;
}

int qik_fp8_quantize_weight_host(const void* w, int32_t dtype, int64_t n, void* out, float* scale,
                                 int32_t threads) {
  using namespace qik_fp8;
  if (dtype != QIK_DTYPE_BF16 && dtype != QIK_DTYPE_FP16 && dtype != QIK_DTYPE_FP32) return QIK_ERR_DTYPE;
  if (n < 1 || n >= ((int64_t)1 << 40)) return QIK_ERR_SHAPE;
  if (w == nullptr || out == nullptr || scale == nullptr) return QIK_ERR_NULL_ARG;
  return host_quantize_weight(w, dtype, n, static_cast<unsigned char*>(out), scale, threads);
}

}  // extern "C"
