// Block-causal flash attention for Qwen-Image 2.1 on MI355X (gfx950, CDNA4).
//
// Semantics follow `_qwen21_attn_fwd` (qwen_image_kernel/triton_attention.py:35-168):
// row q attends key kv iff kv <= L[q] (inclusive; L = -1 attends nothing), the
// keys are the virtual concatenation [slab prefix (P keys), fresh keys (SN)],
// an optional key_valid byte mask gates keys, and the slab V may be fp8e4m3fn
// with one fp32 scale per (b, h).  Rounding points kept from the reference:
//   S      = fp32 MFMA accumulation of bf16 Q.K, scaled by qk_scale = sm_scale*log2(e)
//   p      = exp2(S - m)  in fp32;  l = l*alpha + sum(p) uses the fp32 p
//   P      = bf16(p) (RNE) feeds the PV MFMA
//   V_slab = bf16(fp32(v_fp8) * v_scale[b,h])   (fp32 multiply, RNE to bf16)
//   out    = l > 0 ? acc / l : 0, stored RNE in the output dtype
//
// Work decomposition (one workgroup = BM=128 query rows of one (b, h)):
//   * 4 waves x 32 rows.  Each wave computes S^T = K.Q^T with the MFMA
//     v_mfma_f32_32x32x16_{bf16,f16}, so every lane owns ONE query row
//     (m = lane%32) and 16 keys per 32-key block: the row max / row sum are
//     lane-local plus one v_permlane32_swap between the two lane halves.
//   * O^T = V^T.P^T: P^T is already in the B-operand layout (no shuffles), and
//     the V^T A-operand comes straight from the row-major V tile in LDS through
//     ds_read_b64_tr_b16 (the gfx950 LDS transpose read).
//   * K and V tiles (BN=64 keys) are double-buffered in LDS with a 16-byte
//     chunk swizzle (swz below); the fp8 slab V is dequantised to bf16 once per workgroup
//     while it is written to LDS.
//   * Whole KV tiles past the row block's largest L are never visited; tiles
//     that are entirely allowed for a wave skip the mask arithmetic.
//   * blockIdx is remapped so that one (b, h)'s row blocks share an XCD (and
//     its L2), heaviest row blocks first.

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>
#include <limits.h>
#include <algorithm>

#include "qik_attn.h"

namespace qik {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((__vector_size__(16 * sizeof(float))));
typedef float f32x2 __attribute__((__vector_size__(2 * sizeof(float))));
typedef __bf16 bf16x8 __attribute__((__vector_size__(8 * sizeof(__bf16))));
typedef _Float16 f16x8 __attribute__((__vector_size__(8 * sizeof(_Float16))));
typedef __bf16 bf16x2 __attribute__((__vector_size__(2 * sizeof(__bf16))));
typedef _Float16 f16x2 __attribute__((__vector_size__(2 * sizeof(_Float16))));
typedef short i16x4 __attribute__((__vector_size__(4 * sizeof(short))));

constexpr int BM = 128;        // query rows per workgroup
constexpr int BN = 64;         // keys per KV tile
constexpr int NWAVES = 4;      // 32 query rows per wave
constexpr int NTHREADS = NWAVES * 64;

struct Params {
  const char* q;
  const char* k_new;
  const char* v_new;
  const char* k_cache;
  const char* v_cache;
  const float* v_scale;
  const int32_t* L;
  const uint8_t* key_valid;
  char* out;
  int32_t* debug_tiles;
  int64_t sq[3], skn[3], svn[3], skc[3], svc[3], so[3];  // b, s, h strides in elements
  int64_t svalid_b;
  int SQ, SN, P, H, KV;
  int n_row_blocks;
  int has_cache, has_key_valid, uniform;
  float qk_scale;
};

__device__ __forceinline__ int cdiv_i(int a, int b) { return (a + b - 1) / b; }

template <bool FP16>
__device__ __forceinline__ unsigned pack2(float a, float b) {
  if constexpr (FP16) {
    f16x2 r = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(unsigned, r);
  } else {
    bf16x2 r = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(unsigned, r);
  }
}

template <bool FP16>
__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (FP16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                   __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                    __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
}

// x[lane] (+|max) x[lane ^ 32]: v_permlane32_swap(x, x) hands each lane the
// pair {x[l], x[l+32]} (lower half) or {x[l-32], x[l]} (upper half).
__device__ __forceinline__ float pair_max(float x) {
  unsigned u = __float_as_uint(x);
  auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
  unsigned u = __float_as_uint(x);
  auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// 8 fp8e4m3fn codes (little-endian in w0, w1) -> 8 bf16 = bf16(fp32(code) * s).
__device__ __forceinline__ u32x4 dequant_fp8x8(unsigned w0, unsigned w1, float s) {
  f32x2 a = __builtin_amdgcn_cvt_pk_f32_fp8(w0, false);
  f32x2 b = __builtin_amdgcn_cvt_pk_f32_fp8(w0, true);
  f32x2 c = __builtin_amdgcn_cvt_pk_f32_fp8(w1, false);
  f32x2 d = __builtin_amdgcn_cvt_pk_f32_fp8(w1, true);
  u32x4 r;
  r.x = pack2<false>(a[0] * s, a[1] * s);
  r.y = pack2<false>(b[0] * s, b[1] * s);
  r.z = pack2<false>(c[0] * s, c[1] * s);
  r.w = pack2<false>(d[0] * s, d[1] * s);
  return r;
}

// LDS tiles are row-major [key][d] with the 16-byte chunks of row r XOR-permuted
// by swz(r) = ((r & 3) << 2) | ((r >> 2) & 3) (for 16 chunks per row; 8 chunks
// use the low 3 bits).  Sixteen consecutive rows get distinct values (the K
// operand reads one chunk of 16 rows), and four consecutive rows differ in bits
// 2-3 (the V transpose read takes an aligned group of 4 chunks from 4 rows), so
// both reads touch 16 distinct chunks, i.e. all 64 banks once.
template <int CH>
__device__ __forceinline__ int swz(int r) {
  return (((r & 3) << 2) | ((r >> 2) & 3)) & (CH - 1);
}

__device__ __forceinline__ i16x4 lds_read_tr16(const char* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) i16x4*)(p));
}

template <int D, bool FP16, bool V_FP8>
__global__ void __launch_bounds__(NTHREADS, 2) attn_fwd_kernel(const Params p) {
  constexpr int CH = D / 8;              // 16-byte chunks per row (8 elements)
  constexpr int ROWB = D * 2;            // bytes per row of a K/V tile in LDS
  constexpr int KSTEPS = D / 16;         // k-steps of S^T = K.Q^T
  constexpr int DBLK = D / 32;           // 32-row blocks of O^T
  constexpr int NBLK = BN / 32;          // 32-key blocks of S^T
  constexpr int SLABS = BN / 16;         // k-slabs of O^T = V^T.P^T
  constexpr int LOADS = BN * CH / NTHREADS;
  constexpr int TILE_BYTES = BN * ROWB;
  static_assert(LOADS * NTHREADS == BN * CH, "tile must split evenly over the workgroup");

  __shared__ u32x4 smem[2 * 2 * TILE_BYTES / 16];  // [stage][K, V][BN x D]
  __shared__ int sred[2 * NWAVES];
  char* const sbase = reinterpret_cast<char*>(smem);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int hf = lane >> 5;   // lane half: keys 4*hf.. of each 8-key group
  const int l32 = lane & 31;

  // ---- work item: XCD-aware remap, then (b,h)-major with row blocks heaviest-first
  const int G = gridDim.x;
  const int bid = blockIdx.x;
  const int xcd = bid & 7, loc = bid >> 3;
  const int per = G >> 3, rem = G & 7;
  const int vid = (xcd < rem) ? xcd * (per + 1) + loc : rem * (per + 1) + (xcd - rem) * per + loc;
  const int nmb = p.n_row_blocks;
  const int bh = vid / nmb;
  const int mb = nmb - 1 - (vid - bh * nmb);
  const int b = bh / p.H;
  const int h = bh - b * p.H;

  const int m = mb * BM + wave * 32 + l32;  // this lane's query row
  const bool live = m < p.SQ;

  // ---- causal lengths: this row's L, the block's max (dead rows count as -1,
  // triton_attention.py:82-83) and the wave's min over live rows.
  int Lrow = p.KV - 1;
  if (!p.uniform) Lrow = live ? p.L[m] : -1;
  int lmax = live ? Lrow : -1;
  int lmin = live ? Lrow : INT_MAX;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    lmax = max(lmax, __shfl_xor(lmax, off));
    lmin = min(lmin, __shfl_xor(lmin, off));
  }
  if (lane == 0) sred[wave] = lmax;
  __syncthreads();
  int Lmax = sred[0];
#pragma unroll
  for (int w = 1; w < NWAVES; ++w) Lmax = max(Lmax, sred[w]);
  const int wave_minL = lmin;

  // ---- KV-tile schedule: tile t of a segment starting at absolute key s0 is
  // visited iff s0 + t*BN <= Lmax (segment-local tiles, triton_attention.py:97-124).
  const int s1 = p.has_cache ? p.P : 0;
  int run0 = 0;
  if (p.has_cache && Lmax >= 0) run0 = min(cdiv_i(p.P, BN), Lmax / BN + 1);
  int run1 = 0;
  if (Lmax >= s1) run1 = min(cdiv_i(p.SN, BN), (Lmax - s1) / BN + 1);
  const int T = run0 + run1;

  // ---- per-(b,h) bases
  constexpr int VC_ES = V_FP8 ? 1 : 2;
  const char* const qb = p.q + (b * p.sq[0] + h * p.sq[2]) * 2;
  const char* const knb = p.k_new + (b * p.skn[0] + h * p.skn[2]) * 2;
  const char* const vnb = p.v_new + (b * p.svn[0] + h * p.svn[2]) * 2;
  const char* kcb = nullptr;
  const char* vcb = nullptr;
  float vsc = 1.0f;
  if (p.has_cache) {
    kcb = p.k_cache + (b * p.skc[0] + h * p.skc[2]) * 2;
    vcb = p.v_cache + (b * p.svc[0] + h * p.svc[2]) * VC_ES;
    if constexpr (V_FP8) vsc = p.v_scale[b * p.H + h];
  }
  const int64_t kns = p.skn[1] * 2, vns = p.svn[1] * 2;
  const int64_t kcs = p.skc[1] * 2, vcs = p.svc[1] * VC_ES;
  const float qk_scale = p.qk_scale;

  // ---- Q as the B operand of S^T = K.Q^T: lane holds Q[m, 16j + 8hf .. +8]
  u32x4 qreg[KSTEPS];
  {
    const char* qr = qb + (int64_t)m * p.sq[1] * 2;
#pragma unroll
    for (int j = 0; j < KSTEPS; ++j) {
      qreg[j] = live ? *reinterpret_cast<const u32x4*>(qr + (16 * j + 8 * hf) * 2)
                     : u32x4{0u, 0u, 0u, 0u};
    }
  }

  // ---- global -> register staging of one KV tile, register -> LDS store
  u32x4 kst[LOADS], vst[LOADS];
  auto load_tile = [&](int g) {
    const bool seg0 = g < run0;
    const int t = seg0 ? g : g - run0;
    const int seg_len = seg0 ? p.P : p.SN;
    const char* kbase = seg0 ? kcb : knb;
    const char* vbase = seg0 ? vcb : vnb;
    const int64_t ks = seg0 ? kcs : kns;
    const int64_t vs = seg0 ? vcs : vns;
#pragma unroll
    for (int r = 0; r < LOADS; ++r) {
      const int qd = r * NTHREADS + tid;
      const int n = qd / CH, c = qd % CH;
      const int nl = t * BN + n;
      if (nl < seg_len) {
        kst[r] = *reinterpret_cast<const u32x4*>(kbase + (int64_t)nl * ks + c * 16);
        if (V_FP8 && seg0) {
          const u32x2 w = *reinterpret_cast<const u32x2*>(vbase + (int64_t)nl * vs + c * 8);
          vst[r] = u32x4{w.x, w.y, 0u, 0u};
        } else {
          vst[r] = *reinterpret_cast<const u32x4*>(vbase + (int64_t)nl * vs + c * 16);
        }
      } else {
        kst[r] = u32x4{0u, 0u, 0u, 0u};
        vst[r] = u32x4{0u, 0u, 0u, 0u};
      }
    }
  };
  auto store_tile = [&](int g, int stage) {
    const bool fp8 = V_FP8 && (g < run0);
    char* kd = sbase + stage * 2 * TILE_BYTES;
    char* vd = kd + TILE_BYTES;
#pragma unroll
    for (int r = 0; r < LOADS; ++r) {
      const int qd = r * NTHREADS + tid;
      const int n = qd / CH, c = qd % CH;
      const int off = n * ROWB + ((c ^ swz<CH>(n)) << 4);
      *reinterpret_cast<u32x4*>(kd + off) = kst[r];
      u32x4 vv = vst[r];
      if (fp8) vv = dequant_fp8x8(vv.x, vv.y, vsc);  // zero codes stay zero
      *reinterpret_cast<u32x4*>(vd + off) = vv;
    }
  };

  float m_run = -INFINITY;  // running row max, exp2 domain (scaled)
  float l_run = 0.0f;       // this lane half's share of the running row sum
  f32x16 oacc[DBLK];
#pragma unroll
  for (int db = 0; db < DBLK; ++db) oacc[db] = f32x16{};

  if (T > 0) {
    load_tile(0);
    store_tile(0, 0);
  }
  __syncthreads();

  for (int g = 0; g < T; ++g) {
    const bool has_next = g + 1 < T;
    if (has_next) load_tile(g + 1);

    const char* kS = sbase + (g & 1) * 2 * TILE_BYTES;
    const char* vS = kS + TILE_BYTES;

    // S^T[n, m] = sum_d K[n, d] Q[m, d]; lane holds m = l32, n = 8(i/4) + 4hf + i%4
    f32x16 sacc[NBLK];
#pragma unroll
    for (int nb = 0; nb < NBLK; ++nb) {
      sacc[nb] = f32x16{};
      const int n = nb * 32 + l32;
      const char* krow = kS + n * ROWB;
#pragma unroll
      for (int j = 0; j < KSTEPS; ++j) {
        const int c = 2 * j + hf;
        const u32x4 a = *reinterpret_cast<const u32x4*>(krow + ((c ^ swz<CH>(n)) << 4));
        sacc[nb] = mfma32<FP16>(a, qreg[j], sacc[nb]);
      }
    }

    // mask: segment tail, kv <= L[row], key_valid (triton_attention.py:126-144)
    const bool seg0 = g < run0;
    const int t = seg0 ? g : g - run0;
    const int n_in = (seg0 ? p.P : p.SN) - t * BN;  // keys of this tile inside its segment
    const int kv0 = (seg0 ? 0 : s1) + t * BN;        // absolute index of the tile's first key
    const bool full = (n_in >= BN) && (kv0 + BN - 1 <= wave_minL) && !p.has_key_valid;
    if (!full) {
      const uint8_t* kvrow = p.has_key_valid ? p.key_valid + (int64_t)b * p.svalid_b : nullptr;
#pragma unroll
      for (int nb = 0; nb < NBLK; ++nb) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int n = nb * 32 + 8 * (i >> 2) + 4 * hf + (i & 3);
          const int kv = kv0 + n;
          bool ok = (n < n_in) && (kv <= Lrow);
          if (kvrow != nullptr && ok) ok = kvrow[kv] != 0;
          if (!ok) sacc[nb][i] = -INFINITY;
        }
      }
    }

    // online softmax, exp2 domain (triton_attention.py:146-152)
    float mx = -INFINITY;
#pragma unroll
    for (int nb = 0; nb < NBLK; ++nb)
#pragma unroll
      for (int i = 0; i < 16; ++i) mx = fmaxf(mx, sacc[nb][i]);
    mx = pair_max(mx);
    const float m_new = fmaxf(m_run, mx * qk_scale);
    const float m_safe = (m_new == -INFINITY) ? 0.0f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_safe);
    float rs = 0.0f;
#pragma unroll
    for (int nb = 0; nb < NBLK; ++nb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[nb][i], qk_scale, -m_safe));
        sacc[nb][i] = e;
        rs += e;
      }
    l_run = l_run * alpha + rs;
    m_run = m_new;

    // P^T as the B operand: slab s uses registers 8*(s%2).. of block s/2
    u32x4 pb[SLABS];
#pragma unroll
    for (int s = 0; s < SLABS; ++s) {
      const int nb = s >> 1, i0 = (s & 1) * 8;
      pb[s].x = pack2<FP16>(sacc[nb][i0 + 0], sacc[nb][i0 + 1]);
      pb[s].y = pack2<FP16>(sacc[nb][i0 + 2], sacc[nb][i0 + 3]);
      pb[s].z = pack2<FP16>(sacc[nb][i0 + 4], sacc[nb][i0 + 5]);
      pb[s].w = pack2<FP16>(sacc[nb][i0 + 6], sacc[nb][i0 + 7]);
    }

    // acc *= alpha, skipped when every row of the wave keeps its max (alpha == 1 exactly)
    if (__any(alpha != 1.0f)) {
#pragma unroll
      for (int db = 0; db < DBLK; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) oacc[db][i] *= alpha;
    }

    // O^T[d, m] += sum_n V[n, d] P[m, n]; V^T operand via the LDS transpose read:
    // source lane j of each 16-lane group reads row base + j/4, columns d0 + 4(j%4)..+3
    {
      const int j16 = lane & 15;
      const int colq = 16 * ((lane >> 4) & 1) + 4 * (j16 & 3);
#pragma unroll
      for (int db = 0; db < DBLK; ++db) {
        const int col = db * 32 + colq;
#pragma unroll
        for (int s = 0; s < SLABS; ++s) {
          const int r0 = (s >> 1) * 32 + 16 * (s & 1) + 4 * hf + (j16 >> 2);
          const int r1 = r0 + 8;
          const char* a0 = vS + r0 * ROWB + (((col >> 3) ^ swz<CH>(r0)) << 4) + ((col & 7) << 1);
          const char* a1 = vS + r1 * ROWB + (((col >> 3) ^ swz<CH>(r1)) << 4) + ((col & 7) << 1);
          const i16x4 x0 = lds_read_tr16(a0);
          const i16x4 x1 = lds_read_tr16(a1);
          const u32x2 w0 = __builtin_bit_cast(u32x2, x0);
          const u32x2 w1 = __builtin_bit_cast(u32x2, x1);
          const u32x4 a = u32x4{w0.x, w0.y, w1.x, w1.y};
          oacc[db] = mfma32<FP16>(a, pb[s], oacc[db]);
        }
      }
    }

    if (has_next) store_tile(g + 1, (g + 1) & 1);
    __syncthreads();
  }

  // ---- epilogue: out = l > 0 ? acc / l : 0 (triton_attention.py:166-168)
  const float l_tot = pair_sum(l_run);
  const float inv = (l_tot > 0.0f) ? 1.0f / l_tot : 0.0f;
  if (live) {
    char* orow = p.out + (b * p.so[0] + (int64_t)m * p.so[1] + h * p.so[2]) * 2;
#pragma unroll
    for (int db = 0; db < DBLK; ++db)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int d = db * 32 + 8 * q4 + 4 * hf;
        u32x2 w;
        w.x = pack2<FP16>(oacc[db][4 * q4 + 0] * inv, oacc[db][4 * q4 + 1] * inv);
        w.y = pack2<FP16>(oacc[db][4 * q4 + 2] * inv, oacc[db][4 * q4 + 3] * inv);
        *reinterpret_cast<u32x2*>(orow + d * 2) = w;
      }
  }
  if (p.debug_tiles != nullptr && tid == 0) p.debug_tiles[bh * nmb + mb] = T;
}

// ---------------------------------------------------------------------------
// Causal-length builder (processors.py:22-36), one thread per row.
constexpr int MAX_SEG_PER_LAUNCH = 64;
struct SegList {
  int n;
  int start[MAX_SEG_PER_LAUNCH];
  int end[MAX_SEG_PER_LAUNCH];
};

__global__ void build_lengths_kernel(const SegList segs, int init, int apply_prefix, int prefix_end,
                                     int seq_len, int32_t* L) {
  const int q = blockIdx.x * blockDim.x + threadIdx.x;
  if (q >= seq_len) return;
  int v = init ? q : L[q];
  for (int i = 0; i < segs.n; ++i)
    if (q >= segs.start[i] && q < segs.end[i]) v = segs.end[i] - 1;
  if (apply_prefix && q >= prefix_end) v = seq_len - 1;
  L[q] = v;
}

// ---------------------------------------------------------------------------
// host side

typedef void (*kernel_fn)(Params);

template <int D>
kernel_fn pick_kernel(bool fp16, bool vfp8) {
  if (fp16) return attn_fwd_kernel<D, true, false>;
  if (vfp8) return attn_fwd_kernel<D, false, true>;
  return attn_fwd_kernel<D, false, false>;
}

inline bool aligned_to(const void* ptr, uintptr_t a) { return (reinterpret_cast<uintptr_t>(ptr) % a) == 0; }

// A stride only matters along a dim of size > 1.
inline bool stride_ok(const int64_t st[3], int64_t nb, int64_t ns, int64_t nh, int64_t mult) {
  if (nb > 1 && st[0] % mult != 0) return false;
  if (ns > 1 && st[1] % mult != 0) return false;
  if (nh > 1 && st[2] % mult != 0) return false;
  return true;
}

inline int64_t cdiv64(int64_t a, int64_t b) { return (a + b - 1) / b; }

int schedule_one(int64_t Lmax, int64_t P, int64_t SN, bool has_cache) {
  int64_t run0 = 0, run1 = 0;
  const int64_t s1 = has_cache ? P : 0;
  if (has_cache && Lmax >= 0) run0 = std::min(cdiv64(P, BN), Lmax / BN + 1);
  if (Lmax >= s1) run1 = std::min(cdiv64(SN, BN), (Lmax - s1) / BN + 1);
  return (int)(run0 + run1);
}

}  // namespace qik

extern "C" {

int qik_abi_version(void) { return QIK_ABI_VERSION; }

const char* qik_strerror(int status) {
  switch (status) {
    case QIK_OK: return "ok";
    case QIK_ERR_NULL_ARG: return "a required pointer is NULL";
    case QIK_ERR_ABI_VERSION: return "qik_attn_args.abi_version does not match the library";
    case QIK_ERR_DTYPE: return "fp16/bf16 only";
    case QIK_ERR_HEAD_DIM: return "head_dim must be 64 or 128";
    case QIK_ERR_SHAPE: return "negative or oversized B/SQ/SN/P/H";
    case QIK_ERR_CACHE: return "cache flag, P and cache pointers are inconsistent";
    case QIK_ERR_FP8_SCALE: return "fp8 cache V needs the cache, a v_scale pointer and bf16 q/k/v";
    case QIK_ERR_ALIGN: return "pointers and b/s/h strides must be multiples of 8 elements (16 B rows chunks)";
    case QIK_ERR_LAUNCH: return "HIP kernel launch failed";
    case QIK_ERR_SEGMENTS: return "segments need 0 <= start <= end, and 0 <= prefix_end <= seq_len";
    case QIK_ERR_DEVICE: return "HIP device query failed";
    default: return "unknown qik status";
  }
}

int qik_attn_block_shape(int32_t* block_m, int32_t* block_n) {
  if (block_m == nullptr || block_n == nullptr) return QIK_ERR_NULL_ARG;
  *block_m = qik::BM;
  *block_n = qik::BN;
  return QIK_OK;
}

int qik_attn_validate(const qik_attn_args* a) {
  if (a == nullptr) return QIK_ERR_NULL_ARG;
  if (a->abi_version != QIK_ABI_VERSION || a->reserved0 != 0 || a->reserved1 != 0) return QIK_ERR_ABI_VERSION;
  if (a->dtype != QIK_DTYPE_BF16 && a->dtype != QIK_DTYPE_FP16) return QIK_ERR_DTYPE;
  if (a->D != 64 && a->D != 128) return QIK_ERR_HEAD_DIM;
  const int64_t lim = (int64_t)INT_MAX;
  if (a->B < 0 || a->SQ < 0 || a->SN < 0 || a->P < 0 || a->H < 0) return QIK_ERR_SHAPE;
  if (a->SQ > lim || a->SN > lim || a->P > lim || a->H > lim || a->P + a->SN > lim) return QIK_ERR_SHAPE;
  const int64_t nmb = qik::cdiv64(a->SQ, qik::BM);
  if (a->B > 0 && a->H > 0 && nmb > 0 && a->B * a->H > lim / nmb) return QIK_ERR_SHAPE;
  if ((a->flags & ~(QIK_HAS_CACHE | QIK_HAS_KEY_VALID | QIK_UNIFORM_L | QIK_V_CACHE_FP8)) != 0)
    return QIK_ERR_SHAPE;

  const bool has_cache = (a->flags & QIK_HAS_CACHE) != 0;
  const bool vfp8 = (a->flags & QIK_V_CACHE_FP8) != 0;
  const bool has_kv = (a->flags & QIK_HAS_KEY_VALID) != 0;
  const bool uniform = (a->flags & QIK_UNIFORM_L) != 0;
  if (has_cache != (a->P > 0)) return QIK_ERR_CACHE;
  if (has_cache && (a->k_cache == nullptr || a->v_cache == nullptr)) return QIK_ERR_CACHE;
  if (vfp8 && (!has_cache || a->v_scale == nullptr || a->dtype != QIK_DTYPE_BF16)) return QIK_ERR_FP8_SCALE;
  if (!vfp8 && a->v_scale != nullptr) return QIK_ERR_FP8_SCALE;
  if (has_kv != (a->key_valid != nullptr)) return QIK_ERR_NULL_ARG;

  const bool work = a->B > 0 && a->H > 0 && a->SQ > 0;
  if (!work) return QIK_OK;
  if (a->q == nullptr || a->out == nullptr) return QIK_ERR_NULL_ARG;
  if (a->SN > 0 && (a->k_new == nullptr || a->v_new == nullptr)) return QIK_ERR_NULL_ARG;
  if (!uniform && a->prefix_lengths == nullptr) return QIK_ERR_NULL_ARG;

  // 16-byte chunks of 8 elements: bases 16-B aligned, strides multiples of 8 elements
  if (!qik::aligned_to(a->q, 16) || !qik::aligned_to(a->out, 16)) return QIK_ERR_ALIGN;
  if (!qik::stride_ok(a->stride_q, a->B, a->SQ, a->H, 8)) return QIK_ERR_ALIGN;
  if (!qik::stride_ok(a->stride_out, a->B, a->SQ, a->H, 8)) return QIK_ERR_ALIGN;
  if (a->SN > 0) {
    if (!qik::aligned_to(a->k_new, 16) || !qik::aligned_to(a->v_new, 16)) return QIK_ERR_ALIGN;
    if (!qik::stride_ok(a->stride_k_new, a->B, a->SN, a->H, 8)) return QIK_ERR_ALIGN;
    if (!qik::stride_ok(a->stride_v_new, a->B, a->SN, a->H, 8)) return QIK_ERR_ALIGN;
  }
  if (has_cache) {
    if (!qik::aligned_to(a->k_cache, 16)) return QIK_ERR_ALIGN;
    if (!qik::aligned_to(a->v_cache, vfp8 ? 8 : 16)) return QIK_ERR_ALIGN;
    if (!qik::stride_ok(a->stride_k_cache, a->B, a->P, a->H, 8)) return QIK_ERR_ALIGN;
    if (!qik::stride_ok(a->stride_v_cache, a->B, a->P, a->H, 8)) return QIK_ERR_ALIGN;
  }
  return QIK_OK;
}

int qik_attn_fwd(const qik_attn_args* a, void* stream) {
  const int st = qik_attn_validate(a);
  if (st != QIK_OK) return st;
  const int64_t nmb = qik::cdiv64(a->SQ, qik::BM);
  const int64_t grid = a->B * a->H * nmb;
  if (grid == 0) return QIK_OK;

  qik::Params p;
  memset(&p, 0, sizeof(p));
  p.q = static_cast<const char*>(a->q);
  p.k_new = static_cast<const char*>(a->k_new);
  p.v_new = static_cast<const char*>(a->v_new);
  p.k_cache = static_cast<const char*>(a->k_cache);
  p.v_cache = static_cast<const char*>(a->v_cache);
  p.v_scale = a->v_scale;
  p.L = a->prefix_lengths;
  p.key_valid = a->key_valid;
  p.out = static_cast<char*>(a->out);
  p.debug_tiles = a->debug_tiles;
  for (int i = 0; i < 3; ++i) {
    p.sq[i] = a->stride_q[i];
    p.skn[i] = a->stride_k_new[i];
    p.svn[i] = a->stride_v_new[i];
    p.skc[i] = a->stride_k_cache[i];
    p.svc[i] = a->stride_v_cache[i];
    p.so[i] = a->stride_out[i];
  }
  p.svalid_b = a->stride_valid_b;
  p.SQ = (int)a->SQ;
  p.SN = (int)a->SN;
  p.P = (int)a->P;
  p.H = (int)a->H;
  p.KV = (int)(a->P + a->SN);
  p.n_row_blocks = (int)nmb;
  p.has_cache = (a->flags & QIK_HAS_CACHE) ? 1 : 0;
  p.has_key_valid = (a->flags & QIK_HAS_KEY_VALID) ? 1 : 0;
  p.uniform = (a->flags & QIK_UNIFORM_L) ? 1 : 0;
  // qk_scale = sm_scale * log2(e), both fp32, as triton_attention.py:93 computes it
  p.qk_scale = a->sm_scale * 1.44269504088896340736f;

  const bool fp16 = a->dtype == QIK_DTYPE_FP16;
  const bool vfp8 = (a->flags & QIK_V_CACHE_FP8) != 0;
  qik::kernel_fn fn = (a->D == 128) ? qik::pick_kernel<128>(fp16, vfp8) : qik::pick_kernel<64>(fp16, vfp8);
  void* kargs[] = {&p};
  const hipError_t e = hipLaunchKernel(reinterpret_cast<const void*>(fn), dim3((unsigned)grid),
                                       dim3(qik::NTHREADS), kargs, 0, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? QIK_OK : QIK_ERR_LAUNCH;
}

int qik_attn_tile_schedule(int64_t SQ, int64_t P, int64_t SN, int32_t flags, const int32_t* L, int32_t* out) {
  if (out == nullptr) return QIK_ERR_NULL_ARG;
  if (SQ < 0 || P < 0 || SN < 0) return QIK_ERR_SHAPE;
  const bool has_cache = (flags & QIK_HAS_CACHE) != 0;
  const bool uniform = (flags & QIK_UNIFORM_L) != 0;
  if (has_cache != (P > 0)) return QIK_ERR_CACHE;
  if (!uniform && SQ > 0 && L == nullptr) return QIK_ERR_NULL_ARG;
  const int64_t nmb = qik::cdiv64(SQ, qik::BM);
  for (int64_t mb = 0; mb < nmb; ++mb) {
    int64_t Lmax;
    if (uniform) {
      Lmax = P + SN - 1;
    } else {
      Lmax = -1;
      const int64_t r1 = std::min(SQ, (mb + 1) * qik::BM);
      for (int64_t r = mb * qik::BM; r < r1; ++r) Lmax = std::max<int64_t>(Lmax, L[r]);
    }
    out[mb] = qik::schedule_one(Lmax, P, SN, has_cache);
  }
  return QIK_OK;
}

int qik_build_prefix_lengths(const int32_t* segments, int32_t nseg, int64_t prefix_end, int64_t seq_len,
                             int32_t* L, void* stream) {
  if (nseg < 0 || seq_len < 0 || seq_len > INT_MAX) return QIK_ERR_SEGMENTS;
  if (prefix_end < 0 || prefix_end > seq_len) return QIK_ERR_SEGMENTS;
  if (nseg > 0 && segments == nullptr) return QIK_ERR_NULL_ARG;
  for (int i = 0; i < nseg; ++i) {
    const int32_t s = segments[3 * i], e = segments[3 * i + 1];
    if (s < 0 || e < s) return QIK_ERR_SEGMENTS;
  }
  if (seq_len == 0) return QIK_OK;
  if (L == nullptr) return QIK_ERR_NULL_ARG;
  const int threads = 256;
  const unsigned blocks = (unsigned)((seq_len + threads - 1) / threads);
  hipStream_t s = static_cast<hipStream_t>(stream);
  // non-text segments in order, MAX_SEG_PER_LAUNCH per launch; later launches see earlier writes
  int i = 0;
  bool first = true;
  do {
    qik::SegList segs;
    memset(&segs, 0, sizeof(segs));
    while (i < nseg && segs.n < qik::MAX_SEG_PER_LAUNCH) {
      if (segments[3 * i + 2] == 0) {
        segs.start[segs.n] = segments[3 * i];
        segs.end[segs.n] = segments[3 * i + 1];
        ++segs.n;
      }
      ++i;
    }
    int last = (i >= nseg) ? 1 : 0;
    int init = first ? 1 : 0, pe = (int)prefix_end, sl = (int)seq_len;
    void* kargs[] = {&segs, &init, &last, &pe, &sl, &L};
    if (hipLaunchKernel(reinterpret_cast<const void*>(qik::build_lengths_kernel), dim3(blocks), dim3(threads),
                        kargs, 0, s) != hipSuccess)
      return QIK_ERR_LAUNCH;
    first = false;
  } while (i < nseg);
  return QIK_OK;
}

}  // extern "C"
