// Device steps beside the attention call of a Qwen-Image 2.1 layer on MI355X:
// the per-head RMSNorm + RoPE that produces Q and K
// (qwen_image_kernel/triton_fused.py:28-105) and the prefix-KV slab store with
// per-(b, h) fp8 quantisation of V (qwen_image_kernel/kv_cache.py:30-45).
//
// Both are HBM-bound byte movers: every thread moves one 16-byte chunk of a
// row (8 elements) per step, rows are read and written whole, and no MFMA is
// involved.  Floating-point contraction is off in these kernels, so every fp32
// multiply and add rounds on its own and a plain fp32 restatement reproduces
// every bit.

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>
#include <limits.h>
#include <algorithm>

#include "qik_ops.h"

namespace qik_ops {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((__vector_size__(2 * sizeof(__bf16))));
typedef _Float16 f16x2 __attribute__((__vector_size__(2 * sizeof(_Float16))));

constexpr int NTHREADS = 256;

// two packed 16-bit values <-> fp32
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
// fp32 -> nearest value of the element type -> fp32.  The empty asm pins x as
// an fp32 value: otherwise the fp16 conversion of a product is folded into
// v_fma_mixlo_f16, which rounds the exact product once instead of the fp32
// product (a different result on about one element in 10^4).
template <bool FP16>
__device__ __forceinline__ float round_elem(float x) {
  if constexpr (FP16) {
    asm volatile("" : "+v"(x));
    return (float)(_Float16)x;
  } else {
    return (float)(__bf16)x;
  }
}

// ---------------------------------------------------------------------------
// RMSNorm + RoPE.  D/8 threads per row, 256/(D/8) rows per workgroup.
struct RmsRopeParams {
  const char* x;
  char* out;
  const float* w;
  const float* cos;
  const float* sin;
  int rows;      // B*S*H (< 2^31, checked on the host)
  int S, H;
  int64_t sx[3], so[3];
  float eps;
};

// One row's chunk t: 8 elements of x in fp32, and their sum of squares over the
// row.  The squares of 16-bit inputs are exact in fp32, so only the additions
// round: in thread left to right, then a butterfly over the row's TPR lanes
// (lane t adds lane t^k for k = TPR/2 .. 1).
template <int D, bool FP16>
__device__ __forceinline__ float row_sumsq(const u32x4 raw, float (&x)[8]) {
#pragma clang fp contract(off)
  constexpr int TPR = D / 8;
  unpack2<FP16>(raw.x, x[0], x[1]);
  unpack2<FP16>(raw.y, x[2], x[3]);
  unpack2<FP16>(raw.z, x[4], x[5]);
  unpack2<FP16>(raw.w, x[6], x[7]);
  float ss = x[0] * x[0];
#pragma unroll
  for (int i = 1; i < 8; ++i) ss = ss + x[i] * x[i];
#pragma unroll
  for (int k = TPR / 2; k >= 1; k >>= 1) ss = ss + __shfl_xor(ss, k);
  return ss;
}

// r = 1 / sqrt(sum / D + eps): the mean is exact (D a power of two), the sum
// with eps rounds in fp32, the square root and the reciprocal are taken in fp64
// (both correctly rounded) and rounded once to fp32.
template <int D>
__device__ __forceinline__ float row_rsqrt(const float ss, const float eps) {
#pragma clang fp contract(off)
  const float ms = ss * (1.0f / (float)D);
  return (float)(1.0 / sqrt((double)(ms + eps)));
}

// The row's chunk t normalised, weighted, rounded to the element type and
// rotated -> 16 output bytes.
template <int D, bool FP16>
__device__ __forceinline__ u32x4 rope_chunk(const float (&x)[8], const float r, const float (&wv)[8],
                                            const float4 c4, const float4 s4) {
#pragma clang fp contract(off)
  // n = round((x * r) * w) to the element type, back in fp32 (triton_fused.py:57-58)
  float n[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) n[i] = round_elem<FP16>((x[i] * r) * wv[i]);

  // pairs (n[2i], n[2i+1]) use frequency 4t + i of the row's position (:60-66)
  const float cs[4] = {c4.x, c4.y, c4.z, c4.w};
  const float sn[4] = {s4.x, s4.y, s4.z, s4.w};
  unsigned o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float e = n[2 * i], od = n[2 * i + 1];
    const float re = e * cs[i] - od * sn[i];
    const float im = e * sn[i] + od * cs[i];
    o[i] = pack2<FP16>(re, im);
  }
  return u32x4{o[0], o[1], o[2], o[3]};
}

// RR rows per thread, their loads issued before any arithmetic; RPB rows per
// workgroup pass, RR passes per workgroup.
constexpr int RR = 4;

template <int D, bool FP16>
__global__ void __launch_bounds__(NTHREADS) rms_rope_kernel(const RmsRopeParams p) {
  constexpr int TPR = D / 8;             // threads per row
  constexpr int RPB = NTHREADS / TPR;    // rows per pass
  constexpr int HALF = D / 2;
  const int t = threadIdx.x % TPR;       // 16-byte chunk of the row: elements 8t .. 8t+7
  const int row0 = blockIdx.x * (RPB * RR) + threadIdx.x / TPR;

  const float4 w0 = *reinterpret_cast<const float4*>(p.w + 8 * t);
  const float4 w1 = *reinterpret_cast<const float4*>(p.w + 8 * t + 4);
  const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};

  u32x4 raw[RR];
  float4 c4[RR], s4[RR];
  int64_t ooff[RR];
  bool live[RR];
  // (b, s, h) of the first row by division, then stepped by RPB rows with
  // additions only: the element offsets move by RPB*h-stride, and by the
  // position (and batch) carries when h (and s) wrap.  64-bit multiplies and
  // divisions per row made this kernel VALU-bound.
  int h, s, b;
  {
    const int row = min(row0, p.rows - 1);
    const unsigned bs = (unsigned)row / (unsigned)p.H;
    h = row - (int)bs * p.H;
    b = (int)(bs / (unsigned)p.S);
    s = (int)bs - b * p.S;
  }
  int64_t xo = b * p.sx[0] + s * p.sx[1] + h * p.sx[2];
  int64_t oo = b * p.so[0] + s * p.so[1] + h * p.so[2];
  const int64_t xh = (int64_t)RPB * p.sx[2], oh = (int64_t)RPB * p.so[2];   // RPB heads on
  const int64_t xs = p.sx[1] - p.H * p.sx[2], os = p.so[1] - p.H * p.so[2]; // h wraps: next position
  const int64_t xb = p.sx[0] - p.S * p.sx[1], ob = p.so[0] - p.S * p.so[1]; // s wraps: next batch
#pragma unroll
  for (int u = 0; u < RR; ++u) {
    live[u] = row0 + u * RPB < p.rows;
    raw[u] = u32x4{0u, 0u, 0u, 0u};
    if (live[u]) raw[u] = *reinterpret_cast<const u32x4*>(p.x + xo * 2 + t * 16);
    c4[u] = *reinterpret_cast<const float4*>(p.cos + s * HALF + 4 * t);
    s4[u] = *reinterpret_cast<const float4*>(p.sin + s * HALF + 4 * t);
    ooff[u] = oo * 2 + t * 16;
    if (u + 1 < RR) {
      h += RPB;
      xo += xh;
      oo += oh;
      while (h >= p.H) {
        h -= p.H;
        xo += xs;
        oo += os;
        if (++s == p.S) {
          s = 0;
          xo += xb;
          oo += ob;
        }
      }
    }
  }
  // the RR rows' sums of squares; then one fp64 reciprocal square root per
  // lane instead of RR: lane t < RR of a row group takes pass t's row, and
  // every lane fetches its rows' results back from those lanes
  float x[RR][8], ss[RR];
#pragma unroll
  for (int u = 0; u < RR; ++u) ss[u] = row_sumsq<D, FP16>(raw[u], x[u]);
  static_assert(RR <= TPR, "a row group has a lane per pass");
  float mine = ss[0];
#pragma unroll
  for (int u = 1; u < RR; ++u) mine = (t == u) ? ss[u] : mine;
  const float rl = row_rsqrt<D>(mine, p.eps);
  const int g0 = (int)(threadIdx.x % 64) - t;   // first lane of this row group
#pragma unroll
  for (int u = 0; u < RR; ++u) {
    const float r = __shfl(rl, g0 + u);
    const u32x4 o = rope_chunk<D, FP16>(x[u], r, wv, c4[u], s4[u]);
    if (live[u]) *reinterpret_cast<u32x4*>(p.out + ooff[u]) = o;
  }
}

// ---------------------------------------------------------------------------
// Slab store.  Row copy [B, P, H, D] -> [B, H, P_max, D] (K, and V unless
// fp8): threads walk destination rows in order, so each head's block of the
// slab is written densely; blockIdx.y picks K (0) or V (1).
struct CopyParams {
  const char* src[2];
  char* dst[2];
  float* zero;       // fp8 V: the [B*H] scales, zeroed for the atomic max that follows (else NULL)
  int64_t nzero;
  int64_t ss[2][3];  // source b, p, h (elements)
  int64_t sd[2][3];  // destination b, h, p (elements)
  int64_t rows;      // B*H*P
  int64_t P, H;
  int row_bytes;     // D * element size
  int64_t* len_dst;  // NULL, or where the first launch writes P
};

// One 16-byte chunk g of the copy of tensor `which` (0 = K, 1 = V).
__device__ __forceinline__ void copy_chunk(const CopyParams& p, const int which, const int64_t g) {
  const int tpr = p.row_bytes / 16;
  const int64_t row = g / tpr;
  const int t = (int)(g % tpr);
  if (row >= p.rows) return;
  const int64_t pp = row % p.P;  // destination row order: b, h, p
  const int64_t bh = row / p.P;
  const int64_t h = bh % p.H;
  const int64_t b = bh / p.H;
  const u32x4 v = *reinterpret_cast<const u32x4*>(
      p.src[which] + (b * p.ss[which][0] + pp * p.ss[which][1] + h * p.ss[which][2]) * 2 + t * 16);
  *reinterpret_cast<u32x4*>(p.dst[which] + (b * p.sd[which][0] + h * p.sd[which][1] + pp * p.sd[which][2]) * 2 +
                            t * 16) = v;
}

__global__ void __launch_bounds__(NTHREADS) slab_copy_kernel(const CopyParams p) {
  const int which = blockIdx.y;
  const int64_t g = (int64_t)blockIdx.x * NTHREADS + threadIdx.x;
  if (p.zero != nullptr && which == 0 && g < p.nzero) p.zero[g] = 0.0f;
  if (p.len_dst != nullptr && which == 0 && g == 0) *p.len_dst = p.P;
  copy_chunk(p, which, g);
}

// fp8 V over `chunks` workgroups per (b, h), workgroup c owning rows
// [c*P/chunks, (c+1)*P/chunks) of the head.  The scale of a chunk's rows is
// max(amax * fp32(1/448), 1e-12); the map amax -> scale is monotone (fp32
// rounding included), so the largest chunk scale is the scale of the head's
// amax.  Two forms:
//   qik_slab_store: slab_scale_fp8_kernel maxes each chunk's scale atomically
//     into scale[b*H + h] (zeroed by the copy launch before), then
//     slab_quant_fp8_kernel writes the codes (three launches with the copy);
//   qik_slab_store_ws: slab_copy_scale_kernel copies K and writes each chunk's
//     scale into the workspace, then slab_quant_fp8_kernel takes the largest of
//     its head's and writes the codes and the scale (two launches).
struct QuantParams {
  const char* v;     // bf16 or fp16 [B, P, H, D]
  char* dst;         // fp8 slab V of the layer
  float* scale;      // [B*H]
  float* partial;    // workspace launches: [B*H*chunks] scales of each chunk's rows (else NULL)
  int64_t sv[3];     // b, p, h (elements)
  int64_t sd[3];     // b, h, p (elements = bytes)
  int P, H, chunks;
};

constexpr int QTHREADS = 512;
constexpr int MAX_SCALE_CHUNKS = 64;   // scale chunks per head at most: the workspace holds this many per head

// max(amax * fp32(1/448), 1e-12) of the rows of chunk bx = bh * chunks + c,
// valid in thread 0 (a block of QTHREADS threads); FP16: the rows are fp16, else bf16
template <int D, bool FP16>
__device__ __forceinline__ float chunk_scale(const QuantParams& p, const int bx) {
  constexpr int TPR = D / 8;             // threads per row
  constexpr int RPS = QTHREADS / TPR;    // rows per step
  constexpr int U = 4;                   // steps in flight per thread
  __shared__ float red[QTHREADS / 64];
  const int bh = bx / p.chunks;
  const int c = bx - bh * p.chunks;
  const int h = bh % p.H;
  const int b = bh / p.H;
  const int t = threadIdx.x % TPR;
  const int r0 = threadIdx.x / TPR;
  const char* src = p.v + (b * p.sv[0] + h * p.sv[2]) * 2 + t * 16;
  const int64_t rs = p.sv[1] * 2;        // source row stride, bytes
  const int p0 = (int)((int64_t)p.P * c / p.chunks);
  const int p1 = (int)((int64_t)p.P * (c + 1) / p.chunks);

  float amax = 0.0f;
  auto absmax8 = [&](const u32x4 raw) __attribute__((always_inline)) {
    const unsigned w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float lo, hi;
      unpack2<FP16>(w[i], lo, hi);
      amax = fmaxf(amax, fabsf(lo));
      amax = fmaxf(amax, fabsf(hi));
    }
  };
  // U rows per batch, all loads issued before the first is used; rows past
  // the chunk are skipped (a chunk is a few batches, so a batch is never
  // broken into one-row steps that would each wait for their load)
  for (int pp = p0 + r0; pp < p1; pp += U * RPS) {
    u32x4 raw[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      raw[u] = u32x4{0u, 0u, 0u, 0u};
      if (pp + u * RPS < p1) raw[u] = *reinterpret_cast<const u32x4*>(src + (pp + u * RPS) * rs);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) absmax8(raw[u]);
  }
#pragma unroll
  for (int k = 32; k >= 1; k >>= 1) amax = fmaxf(amax, __shfl_xor(amax, k));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  float sc = 0.0f;
  if (threadIdx.x == 0) {
    for (int i = 1; i < QTHREADS / 64; ++i) amax = fmaxf(amax, red[i]);
    amax = fmaxf(amax, red[0]);
    // torch: amax / 448.0 multiplies by the fp32 reciprocal; clamp_min(1e-12)
    sc = fmaxf(amax * (1.0f / 448.0f), 1e-12f);
  }
  return sc;
}

template <int D, bool FP16>
__global__ void __launch_bounds__(QTHREADS) slab_scale_fp8_kernel(const QuantParams p) {
  const float sc = chunk_scale<D, FP16>(p, blockIdx.x);
  // non-negative fp32 values order like their bit patterns
  if (threadIdx.x == 0) atomicMax(reinterpret_cast<unsigned*>(p.scale) + blockIdx.x / p.chunks, __float_as_uint(sc));
}

// Workspace form, first launch: blocks [0, ncopy) copy K (QTHREADS 16-byte
// chunks each), the others write their chunk's scale into p.partial.  Every
// partial is written, so the workspace needs no clearing.
template <int D, bool FP16>
__global__ void __launch_bounds__(QTHREADS) slab_copy_scale_kernel(const CopyParams cp, const QuantParams p,
                                                                   const int ncopy) {
  if ((int)blockIdx.x < ncopy) {
    const int64_t g = (int64_t)blockIdx.x * QTHREADS + threadIdx.x;
    if (cp.len_dst != nullptr && g == 0) *cp.len_dst = cp.P;
    copy_chunk(cp, 0, g);
    return;
  }
  const int bx = (int)blockIdx.x - ncopy;
  const float sc = chunk_scale<D, FP16>(p, bx);
  if (threadIdx.x == 0) p.partial[bx] = sc;
}

template <int D, bool FP16>
__global__ void __launch_bounds__(QTHREADS) slab_quant_fp8_kernel(const QuantParams p) {
#pragma clang fp contract(off)
  constexpr int TPR = D / 8;             // threads per row
  constexpr int RPS = QTHREADS / TPR;    // rows per step
  const int bh = blockIdx.x / p.chunks;
  const int c = blockIdx.x - bh * p.chunks;
  const int h = bh % p.H;
  const int b = bh / p.H;
  const int t = threadIdx.x % TPR;
  const int r0 = threadIdx.x / TPR;
  const char* src = p.v + (b * p.sv[0] + h * p.sv[2]) * 2 + t * 16;
  const int64_t rs = p.sv[1] * 2;
  const int p0 = (int)((int64_t)p.P * c / p.chunks);
  const int p1 = (int)((int64_t)p.P * (c + 1) / p.chunks);
  // U rows per batch, all loads issued before the first is used; the first
  // batch is in flight while the head's scale is formed
  constexpr int U = 4;
  u32x4 raw[U];
  auto load_batch = [&](const int q0) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      raw[u] = u32x4{0u, 0u, 0u, 0u};
      if (q0 + u * RPS < p1) raw[u] = *reinterpret_cast<const u32x4*>(src + (q0 + u * RPS) * rs);
    }
  };
  int q0 = p0 + r0;
  load_batch(q0);
  float scale;
  if (p.partial != nullptr) {
    // the head's scale is the largest of its chunks' (amax -> scale is
    // monotone, rounding included); chunk 0 also stores it
    scale = 0.0f;
    for (int i = 0; i < p.chunks; ++i) scale = fmaxf(scale, p.partial[bh * p.chunks + i]);
    if (c == 0 && threadIdx.x == 0) p.scale[bh] = scale;
  } else {
    scale = p.scale[bh];
  }
  char* dst = p.dst + b * p.sd[0] + h * p.sd[1] + t * 8;
  // v / scale rounded to nearest, as an IEEE division gives it, from the
  // correctly rounded reciprocal y of the scale and one correction:
  // q = RN(v*y) is within an ulp of v/scale, r = v - q*scale is exact (fma),
  // and RN(q + r*y) is the correctly rounded quotient (Markstein's theorem,
  // which needs no overflow or underflow on the way: every |v| is at most the
  // amax its scale came from, so |v/scale| <= 448 (1 + 2^-22), and a quotient
  // that is subnormal rounds to a zero code either way).  The quotient takes
  // v's sign, which keeps -0 for v = -0.  A non-finite scale (an inf in the
  // head) has no exact remainder; the division is kept there.
  const float rcp = 1.0f / scale;
  const bool fast = __builtin_isfinite(scale);
  auto quot = [&](const float x) __attribute__((always_inline)) {
    if (!fast) return x / scale;
    const float q = x * rcp;
    const float r = __builtin_fmaf(-q, scale, x);
    return __builtin_copysignf(__builtin_fmaf(r, rcp, q), x);
  };
  for (;;) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (q0 + u * RPS >= p1) continue;
      const unsigned w[4] = {raw[u].x, raw[u].y, raw[u].z, raw[u].w};
      // v / scale (correctly rounded, above), clamped to the e4m3fn range,
      // rounded to nearest even by the hardware conversion; byte k of the 8 =
      // element 8t+k
      float q[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float lo, hi;
        unpack2<FP16>(w[i], lo, hi);
        q[2 * i] = fminf(fmaxf(quot(lo), -448.0f), 448.0f);
        q[2 * i + 1] = fminf(fmaxf(quot(hi), -448.0f), 448.0f);
      }
      int lo = __builtin_amdgcn_cvt_pk_fp8_f32(q[0], q[1], 0, false);
      lo = __builtin_amdgcn_cvt_pk_fp8_f32(q[2], q[3], lo, true);
      int hi = __builtin_amdgcn_cvt_pk_fp8_f32(q[4], q[5], 0, false);
      hi = __builtin_amdgcn_cvt_pk_fp8_f32(q[6], q[7], hi, true);
      *reinterpret_cast<u32x2*>(dst + (q0 + u * RPS) * p.sd[2]) = u32x2{(unsigned)lo, (unsigned)hi};
    }
    q0 += U * RPS;
    if (q0 >= p1) break;
    load_batch(q0);
  }
}

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

inline bool aligned_to(const void* ptr, uintptr_t a) { return (reinterpret_cast<uintptr_t>(ptr) % a) == 0; }

inline bool strides_ok(const int64_t st[3], int64_t mult) {
  return st[0] % mult == 0 && st[1] % mult == 0 && st[2] % mult == 0;
}

// Head dims of these kernels: 32, 64, 128, 256 (the attention kernel's).
inline bool head_dim_ok(int64_t D) { return D == 32 || D == 64 || D == 128 || D == 256; }
inline int head_dim_index(int64_t D) { return D == 32 ? 0 : D == 64 ? 1 : D == 128 ? 2 : 3; }

inline bool sizes_ok(int64_t a, int64_t b, int64_t c, int64_t d) {
  if (a < 0 || b < 0 || c < 0 || d < 0) return false;
  const int64_t lim = (int64_t)INT_MAX;
  return a <= lim && b <= lim && c <= lim && (a == 0 || b == 0 || c == 0 || a * b * c <= lim * 64);
}

}  // namespace qik_ops

extern "C" {

int qik_rms_rope(const qik_rms_rope_args* a, void* stream) {
  using namespace qik_ops;
  if (a == nullptr) return QIK_ERR_NULL_ARG;
  if (a->abi_version != QIK_ABI_VERSION || a->reserved0 != 0) return QIK_ERR_ABI_VERSION;
  if (a->dtype != QIK_DTYPE_BF16 && a->dtype != QIK_DTYPE_FP16) return QIK_ERR_DTYPE;
  if (!head_dim_ok(a->D)) return QIK_ERR_HEAD_DIM;
  if (!sizes_ok(a->B, a->S, a->H, a->D)) return QIK_ERR_SHAPE;
  const int64_t rows = a->B * a->S * a->H;
  if (rows == 0) return QIK_OK;
  if (rows >= (int64_t)INT_MAX) return QIK_ERR_SHAPE;
  if (a->x == nullptr || a->out == nullptr || a->weight == nullptr || a->cos == nullptr || a->sin == nullptr)
    return QIK_ERR_NULL_ARG;
  if (!aligned_to(a->x, 16) || !aligned_to(a->out, 16) || !aligned_to(a->weight, 16) || !aligned_to(a->cos, 16) ||
      !aligned_to(a->sin, 16))
    return QIK_ERR_ALIGN;
  if (!strides_ok(a->stride_x, 8) || !strides_ok(a->stride_out, 8)) return QIK_ERR_ALIGN;

  RmsRopeParams p;
  memset(&p, 0, sizeof(p));
  p.x = static_cast<const char*>(a->x);
  p.out = static_cast<char*>(a->out);
  p.w = a->weight;
  p.cos = a->cos;
  p.sin = a->sin;
  p.rows = (int)rows;
  p.S = (int)a->S;
  p.H = (int)a->H;
  for (int i = 0; i < 3; ++i) {
    p.sx[i] = a->stride_x[i];
    p.so[i] = a->stride_out[i];
  }
  p.eps = a->eps;
  const bool fp16 = a->dtype == QIK_DTYPE_FP16;
  const int rpb = NTHREADS / (int)(a->D / 8) * RR;
  const int64_t grid = (rows + rpb - 1) / rpb;
  if (grid > (int64_t)UINT_MAX) return QIK_ERR_SHAPE;
  const void* const fns[4][2] = {
      {(const void*)rms_rope_kernel<32, false>, (const void*)rms_rope_kernel<32, true>},
      {(const void*)rms_rope_kernel<64, false>, (const void*)rms_rope_kernel<64, true>},
      {(const void*)rms_rope_kernel<128, false>, (const void*)rms_rope_kernel<128, true>},
      {(const void*)rms_rope_kernel<256, false>, (const void*)rms_rope_kernel<256, true>}};
  const void* fn = fns[head_dim_index(a->D)][fp16 ? 1 : 0];
  void* kargs[] = {&p};
  const hipError_t e =
      hipLaunchKernel(fn, dim3((unsigned)grid), dim3(NTHREADS), kargs, 0, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? QIK_OK : QIK_ERR_LAUNCH;
}

}  // extern "C"

namespace qik_ops {

// Checks of qik_slab_store's arguments; rows = B*H*P on success.
int validate_store(const qik_slab_store_args* a, int64_t* rows) {
  if (a == nullptr) return QIK_ERR_NULL_ARG;
  if (a->abi_version != QIK_ABI_VERSION || a->reserved0 != 0) return QIK_ERR_ABI_VERSION;
  if (a->dtype != QIK_DTYPE_BF16 && a->dtype != QIK_DTYPE_FP16) return QIK_ERR_DTYPE;
  const bool fp8 = a->v_fp8 != 0;
  if (fp8 != (a->v_scale != nullptr)) return QIK_ERR_FP8_SCALE;
  if (!head_dim_ok(a->D)) return QIK_ERR_HEAD_DIM;
  if (!sizes_ok(a->B, a->P, a->H, a->D)) return QIK_ERR_SHAPE;
  *rows = a->B * a->H * a->P;
  if (*rows == 0) return QIK_OK;
  if (a->k == nullptr || a->v == nullptr || a->k_dst == nullptr || a->v_dst == nullptr) return QIK_ERR_NULL_ARG;
  if (!aligned_to(a->k, 16) || !aligned_to(a->v, 16) || !aligned_to(a->k_dst, 16)) return QIK_ERR_ALIGN;
  if (!aligned_to(a->v_dst, fp8 ? 8 : 16)) return QIK_ERR_ALIGN;
  if (a->length_dst != nullptr && !aligned_to(a->length_dst, 8)) return QIK_ERR_ALIGN;
  if (!strides_ok(a->stride_k, 8) || !strides_ok(a->stride_v, 8) || !strides_ok(a->stride_k_dst, 8) ||
      !strides_ok(a->stride_v_dst, 8))
    return QIK_ERR_ALIGN;
  if (a->B * a->H > (int64_t)(UINT_MAX / MAX_SCALE_CHUNKS)) return QIK_ERR_SHAPE;
  return QIK_OK;
}

// The store; `partial` (B*H*MAX_SCALE_CHUNKS floats or more) selects the
// two-launch form for an fp8 V, NULL the three-launch one.
int store(const qik_slab_store_args* a, float* partial, hipStream_t s) {
  int64_t rows = 0;
  const int st = validate_store(a, &rows);
  if (st != QIK_OK || rows == 0) return st;
  const bool fp8 = a->v_fp8 != 0;

  CopyParams cp;
  memset(&cp, 0, sizeof(cp));
  cp.src[0] = static_cast<const char*>(a->k);
  cp.dst[0] = static_cast<char*>(a->k_dst);
  cp.src[1] = static_cast<const char*>(a->v);
  cp.dst[1] = static_cast<char*>(a->v_dst);
  for (int i = 0; i < 3; ++i) {
    cp.ss[0][i] = a->stride_k[i];
    cp.sd[0][i] = a->stride_k_dst[i];
    cp.ss[1][i] = a->stride_v[i];
    cp.sd[1][i] = a->stride_v_dst[i];
  }
  cp.rows = rows;
  cp.P = a->P;
  cp.H = a->H;
  cp.row_bytes = (int)(a->D * 2);
  cp.len_dst = a->length_dst;
  cp.zero = (fp8 && partial == nullptr) ? a->v_scale : nullptr;
  cp.nzero = a->B * a->H;
  const int64_t threads = rows * (a->D * 2 / 16);
  const int64_t grid = (threads + NTHREADS - 1) / NTHREADS;
  if (grid > (int64_t)UINT_MAX) return QIK_ERR_SHAPE;

  QuantParams qp;
  memset(&qp, 0, sizeof(qp));
  qp.v = static_cast<const char*>(a->v);
  qp.dst = static_cast<char*>(a->v_dst);
  qp.scale = a->v_scale;
  qp.partial = partial;
  for (int i = 0; i < 3; ++i) {
    qp.sv[i] = a->stride_v[i];
    qp.sd[i] = a->stride_v_dst[i];
  }
  qp.P = (int)a->P;
  qp.H = (int)a->H;
  // spread the heads over the device: about two workgroups per CU in total,
  // at least 32 rows per workgroup, at most MAX_SCALE_CHUNKS per head
  const int64_t heads = a->B * a->H;
  const int cus = device_cus();
  int64_t chunks = cus > 0 ? 2 * cus / heads : 1;
  chunks = std::max<int64_t>(1, std::min<int64_t>({chunks, (int64_t)MAX_SCALE_CHUNKS, a->P / 32}));
  qp.chunks = (int)chunks;
  void* qargs[] = {&qp};
  // the fp8 kernels per head size and source type (bf16 or fp16 V)
  const bool f16 = a->dtype == QIK_DTYPE_FP16;
  const int kix = 2 * head_dim_index(a->D) + (f16 ? 1 : 0);
  const void* const quant_fns[8] = {
      (const void*)slab_quant_fp8_kernel<32, false>,  (const void*)slab_quant_fp8_kernel<32, true>,
      (const void*)slab_quant_fp8_kernel<64, false>,  (const void*)slab_quant_fp8_kernel<64, true>,
      (const void*)slab_quant_fp8_kernel<128, false>, (const void*)slab_quant_fp8_kernel<128, true>,
      (const void*)slab_quant_fp8_kernel<256, false>, (const void*)slab_quant_fp8_kernel<256, true>};
  const void* fq = quant_fns[kix];

  if (fp8 && partial != nullptr) {
    // K copy and the chunks' scales in one launch, then the codes.  The copy
    // blocks are rounded up to a multiple of 8 (the extra ones find no row and
    // return), so chunk c runs on XCD c % 8 in both launches (the dispatcher
    // deals block b to XCD b % 8): the codes launch re-reads its V rows from
    // the L2 that the scale launch read them through.
    const int64_t ncopy = ((threads + QTHREADS - 1) / QTHREADS + 7) / 8 * 8;
    if (ncopy + heads * chunks > (int64_t)INT_MAX) return QIK_ERR_SHAPE;
    int nc = (int)ncopy;
    void* args2[] = {&cp, &qp, &nc};
    const void* const copy_scale_fns[8] = {
        (const void*)slab_copy_scale_kernel<32, false>,  (const void*)slab_copy_scale_kernel<32, true>,
        (const void*)slab_copy_scale_kernel<64, false>,  (const void*)slab_copy_scale_kernel<64, true>,
        (const void*)slab_copy_scale_kernel<128, false>, (const void*)slab_copy_scale_kernel<128, true>,
        (const void*)slab_copy_scale_kernel<256, false>, (const void*)slab_copy_scale_kernel<256, true>};
    const void* fc = copy_scale_fns[kix];
    if (hipLaunchKernel(fc, dim3((unsigned)(ncopy + heads * chunks)), dim3(QTHREADS), args2, 0, s) != hipSuccess)
      return QIK_ERR_LAUNCH;
    return hipLaunchKernel(fq, dim3((unsigned)(heads * chunks)), dim3(QTHREADS), qargs, 0, s) == hipSuccess
               ? QIK_OK : QIK_ERR_LAUNCH;
  }

  void* cargs[] = {&cp};
  hipError_t e = hipLaunchKernel(reinterpret_cast<const void*>(slab_copy_kernel), dim3((unsigned)grid, fp8 ? 1 : 2),
                                 dim3(NTHREADS), cargs, 0, s);
  if (e != hipSuccess) return QIK_ERR_LAUNCH;
  if (!fp8) return QIK_OK;
  const void* const scale_fns[8] = {
      (const void*)slab_scale_fp8_kernel<32, false>,  (const void*)slab_scale_fp8_kernel<32, true>,
      (const void*)slab_scale_fp8_kernel<64, false>,  (const void*)slab_scale_fp8_kernel<64, true>,
      (const void*)slab_scale_fp8_kernel<128, false>, (const void*)slab_scale_fp8_kernel<128, true>,
      (const void*)slab_scale_fp8_kernel<256, false>, (const void*)slab_scale_fp8_kernel<256, true>};
  const void* fs = scale_fns[kix];
  e = hipLaunchKernel(fs, dim3((unsigned)(heads * chunks)), dim3(QTHREADS), qargs, 0, s);
  if (e != hipSuccess) return QIK_ERR_LAUNCH;
  e = hipLaunchKernel(fq, dim3((unsigned)(heads * chunks)), dim3(QTHREADS), qargs, 0, s);
  return e == hipSuccess ? QIK_OK : QIK_ERR_LAUNCH;
}

}  // namespace qik_ops

extern "C" {

int qik_slab_store(const qik_slab_store_args* a, void* stream) {
  return qik_ops::store(a, nullptr, static_cast<hipStream_t>(stream));
}

int qik_slab_store_workspace_size(const qik_slab_store_args* a, int64_t* bytes) {
  if (bytes == nullptr) return QIK_ERR_NULL_ARG;
  *bytes = 0;
  int64_t rows = 0;
  const int st = qik_ops::validate_store(a, &rows);
  if (st != QIK_OK) return st;
  if (a->v_fp8 != 0) *bytes = a->B * a->H * qik_ops::MAX_SCALE_CHUNKS * (int64_t)sizeof(float);
  return QIK_OK;
}

int qik_slab_store_ws(const qik_slab_store_args* a, void* workspace, int64_t workspace_bytes, void* stream) {
  int64_t rows = 0;
  const int st = qik_ops::validate_store(a, &rows);
  if (st != QIK_OK || rows == 0) return st;
  if (a->v_fp8 == 0) return qik_ops::store(a, nullptr, static_cast<hipStream_t>(stream));
  const int64_t need = a->B * a->H * qik_ops::MAX_SCALE_CHUNKS * (int64_t)sizeof(float);
  if (workspace == nullptr || workspace_bytes < need || !qik_ops::aligned_to(workspace, 4)) return QIK_ERR_WORKSPACE;
  return qik_ops::store(a, static_cast<float*>(workspace), static_cast<hipStream_t>(stream));
}

}  // extern "C"
