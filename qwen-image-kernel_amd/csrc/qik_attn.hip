// Block-causal flash attention for Qwen-Image 2.1 on MI355X (gfx950, CDNA4).
//
// Semantics follow `_qwen21_attn_fwd` (qwen_image_kernel/triton_attention.py:35-168):
// row q attends key kv iff kv <= L[q] (inclusive; L = -1 attends nothing), the
// keys are the virtual concatenation [slab prefix (P keys), fresh keys (SN)],
// an optional key_valid byte mask gates keys, and the slab V may be fp8e4m3fn
// with one fp32 scale per (b, h).  Rounding points kept from the reference:
//   S      = fp32 MFMA accumulation of bf16 Q.K, scaled by qk_scale = sm_scale*log2(e)
//   p      = exp2(S*qk_scale - m) in fp32; l = l*alpha + sum(p) uses the fp32 p
//   P      = bf16(p) (RNE) feeds the PV MFMA
//   V_slab = bf16(fp32(v_fp8) * v_scale[b,h])   (fp32 multiply, RNE to bf16)
//   out    = l > 0 ? acc * (1/l) : 0, stored RNE in the output dtype
// Deviations from the reference's arithmetic, all at fp32 rounding level:
//   * the exp2 reference point m is lazy: it moves only when a row's max grows
//     by more than TAU = 8 (log2 units), so p <= 2^8 and the O rescale is
//     skipped on almost every tile (the reference moves m to every new max);
//   * the epilogue multiplies by one reciprocal of l per row instead of
//     dividing every element;
//   * exp2 is the hardware v_exp_f32.
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
//     chunk swizzle (swz below), copied global -> LDS directly (buffer_load
//     ... lds, issued as asm); the fp8 slab V goes through registers and is
//     dequantised to bf16 once per workgroup while it is written to LDS.
//   * Whole KV tiles past the row block's largest L are never visited; tiles
//     that are entirely allowed for a wave (and, with key_valid, whose keys
//     are all valid) skip the mask arithmetic.
//   * Row blocks reach workgroups through per-XCD queues (qik_plan.h): one
//     (b, h)'s row blocks share an XCD and its L2, heaviest first, and with a
//     workspace the last partial round runs as two pieces per row block.
//   * A launch of at most one row block per CU runs the two-group kernel
//     (KSPLIT = 2): 8-wave workgroups whose two 4-wave groups split a row
//     block's KV tiles and merge in LDS; with at most half a row block per CU,
//     every row block is also cut in two pieces on two CUs, merged through the
//     workspace.

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>
#include <limits.h>
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "qik_attn.h"
#include "qik_plan.h"

namespace qik {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((__vector_size__(16 * sizeof(float))));
typedef float f32x2 __attribute__((__vector_size__(2 * sizeof(float))));
typedef float f32x4 __attribute__((__vector_size__(4 * sizeof(float))));
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
  char* ws_slots;                  // split items: plan.ns partial-state slots per group
  unsigned* ctl;                   // NULL: one workgroup per unit; else the control words
                                   // (QIK_ATTN_WS_CTL_BYTES, zero between launches):
                                   // [0, nx) queue heads, [NXCD_MAX, NXCD_MAX + nx)
                                   // exits, [2 NXCD_MAX, ...) arrivals per group
  int64_t sq[3], skn[3], svn[3], skc[3], svc[3], so[3];  // b, s, h strides in elements
  int64_t svalid_b;
  int SQ, SN, P, H, KV;
  int has_cache, has_key_valid, uniform;
  float qk_scale;
  WorkPlan plan;
};

// A split item with fewer than SPLIT_MIN_TILES KV tiles runs whole (its
// second piece is skipped).  Otherwise piece 0 takes its first
// (7 T + 5) / 10 tiles (half of them, (T + 1) / 2, when the plan says `even`)
// and piece 1 the rest.
constexpr int SPLIT_MIN_TILES = 16;

// Partial softmax state of one thread of a split piece: its DBLK x 16 fp32
// O^T accumulators (relative to its row's reference point m) and (m, l share).
template <int D>
constexpr int slot_oacc_bytes() { return (D / 32) * 16 * 4 * NTHREADS; }
template <int D>
constexpr int slot_bytes() { return slot_oacc_bytes<D>() + 8 * NTHREADS; }

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

// Wave-uniform buffer resource over [base, base + bytes); loads at or past
// `bytes` return zeros (this zero-fills the rows past a segment's end).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const char* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base), (short)0, max(bytes, 0), 0x00020000);
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// 64 lanes x 16 B, global -> LDS without passing through registers
// (buffer_load_dwordx4 ... lds, LDS address in M0): lane l's 16 bytes land at
// lds_dst + 16*l.  Written as asm, so the compiler neither schedules the tile's
// LDS reads around it nor inserts waits for it: the tile loop waits for it
// (vmcnt(0)) before each barrier that hands a stage to the other waves.  With
// the compiler builtin the same copies made the 1024px launch 2% slower.
// M0 is a reserved register, so the compiler warns (once per inlined copy)
// that it does not preserve it across the asm; the clobber only tells it that
// M0 changes.  No other code of these kernels keeps a value in M0.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(u32x4 rsrc, char* lds_dst, uint32_t voff) {
  const uint32_t m0 = (uint32_t)(uintptr_t)(lds_ptr_t)lds_dst;
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :: "s"(m0), "v"(voff), "s"(rsrc) : "m0");
}
#pragma clang diagnostic pop

// The buffer resource of make_rsrc as four dwords, for the asm copy.
__device__ __forceinline__ u32x4 rsrc_words(const char* base, int bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)base;
  return u32x4{(uint32_t)a, (uint32_t)(a >> 32) & 0xffffu, (uint32_t)max(bytes, 0), 0x00020000u};
}

// vmcnt(0) (expcnt and lgkmcnt left alone): every copy of this wave has landed
__device__ __forceinline__ void wait_copies() { __builtin_amdgcn_s_waitcnt(0x0F70); }

__device__ __forceinline__ u32x4 lds128(const char* p) { return *reinterpret_cast<const u32x4*>(p); }

// Global-memory accesses through address-space-1 pointers.  Through a generic
// pointer the compiler emits flat instructions, which count in lgkmcnt as well
// as vmcnt: every later LDS or scalar-load wait (the causal-length reduction,
// the kernel-argument loads of the next unit) then also waits for them, i.e.
// for the Q rows from HBM or for the output stores to be acknowledged.
typedef __attribute__((address_space(1))) unsigned gu32;
__device__ __forceinline__ u32x4 gload16(const char* p) {
  return *(const __attribute__((address_space(1))) u32x4*)p;
}
__device__ __forceinline__ int gload_i32(const int32_t* p) { return *(const __attribute__((address_space(1))) int32_t*)p; }
__device__ __forceinline__ float gload_f32(const float* p) { return *(const __attribute__((address_space(1))) float*)p; }
__device__ __forceinline__ void gstore8(char* p, u32x2 v) { *(__attribute__((address_space(1))) u32x2*)p = v; }
__device__ __forceinline__ void gstore16(char* p, u32x4 v) { *(__attribute__((address_space(1))) u32x4*)p = v; }
__device__ __forceinline__ unsigned g_fetch_add(unsigned* p, unsigned v) {
  return __hip_atomic_fetch_add((gu32*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned g_load(unsigned* p) {
  return __hip_atomic_load((gu32*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void g_store(unsigned* p, unsigned v) {
  __hip_atomic_store((gu32*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Barrier of one group of 4 waves of the two-group kernel (s_barrier would
// hold both groups): an arrival counter in LDS that only grows, the group's
// k-th barrier waiting for 4k arrivals.  The caller has waited for its tile
// copies; the release fence waits for its LDS writes.  The spin is bounded
// (2^18 polls of at least 64 cycles, milliseconds beyond any real wait), so no
// mistake can hold the device; it returns false when the bound ran out, and
// the kernel then writes NaN into the row block's output (the tiles read
// after such a barrier may be half-written), so a tripped bound shows as an
// error, never as plausible numbers.
__device__ __forceinline__ bool group_sync(int* ctr, int& target, int lane) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  if (lane == 0) __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  target += 4;
  bool reached = false;
  for (int i = 0; i < (1 << 18); ++i) {
    const int seen = __builtin_amdgcn_readfirstlane(__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
    if (seen >= target) {
      reached = true;
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  return reached;
}

// Wave-wide min or max of an int, returned as a wave-uniform value: four DPP
// steps inside each 16-lane row (quad_perm 1,0,3,2; quad_perm 2,3,0,1;
// row_half_mirror; row_mirror), after which every lane of a row holds the
// row's result, then the four rows' lane 0 read as scalars.  No LDS round trip
// (a __shfl_xor ladder is six ds_bpermute waits).
template <bool MAX>
__device__ __forceinline__ int wave_reduce_i32(int x) {
  auto op = [](int a, int b) { return MAX ? max(a, b) : min(a, b); };
  x = op(x, __builtin_amdgcn_update_dpp(x, x, 0xB1, 0xF, 0xF, false));
  x = op(x, __builtin_amdgcn_update_dpp(x, x, 0x4E, 0xF, 0xF, false));
  x = op(x, __builtin_amdgcn_update_dpp(x, x, 0x141, 0xF, 0xF, false));
  x = op(x, __builtin_amdgcn_update_dpp(x, x, 0x140, 0xF, 0xF, false));
  const int r0 = __builtin_amdgcn_readlane(x, 0), r1 = __builtin_amdgcn_readlane(x, 16);
  const int r2 = __builtin_amdgcn_readlane(x, 32), r3 = __builtin_amdgcn_readlane(x, 48);
  return op(op(r0, r1), op(r2, r3));
}

// Per-lane source offset (from the tile's first row) of the direct-to-LDS tile
// copy.  Instruction r of wave w of a group fills LDS bytes [R0*ROWB, R0*ROWB +
// 1024) with R0 = (1024/ROWB)*(NWAVES*r + w): lane l writes row R0 + l/CH,
// physical chunk l%CH, which must hold logical chunk (l%CH) ^ swz(row).
// swz() only looks at row bits 0-3 and R0 changes by multiples of 16 between
// instructions, so instruction r adds r * (1024/ROWB)*NWAVES rows to the offset
// returned here (the one of r = 0).
template <int D>
__device__ __forceinline__ uint32_t dma_lane_offset_at(int lane, int R0, int row_stride) {
  constexpr int CH = D / 8;
  const int row = R0 + lane / CH;
  const int c = (lane % CH) ^ swz<CH>(row);
  return (uint32_t)(row * row_stride + c * 16);
}
template <int D>
__device__ __forceinline__ uint32_t dma_lane_offset(int lane, int wave, int row_stride) {
  return dma_lane_offset_at<D>(lane, (1024 / (D * 2)) * wave, row_stride);
}

// Bytes of a tile's rows [0, min(n_in, BN)) when rows are `row_stride` apart
// and `row_bytes` long: a buffer resource of that size zero-fills the rows past
// a segment's end.  Fits in 31 bits (checked on the host: BN * row_stride < 2^31).
__device__ __forceinline__ int tile_bytes(int n_in, int row_stride, int row_bytes) {
  const int rows = min(n_in, BN);
  return rows > 0 ? (rows - 1) * row_stride + row_bytes : 0;
}

// One KV tile of K (or bf16 V) starting at `tile` (its first row), rows
// `row_stride` bytes apart; rows >= n_in are zero-filled.  One buffer resource
// per tile; the instructions differ only in their VGPR offset and LDS target.
// With D = 256 an instruction covers 2 rows and R0 moves by 8 rows, which
// changes swz(): there every instruction's offset is formed afresh.
template <int D>
__device__ __forceinline__ void dma_tile(const char* tile, int row_stride, int n_in, char* lds_tile, int wave,
                                         int lane, uint32_t lane_off) {
  constexpr int ROWB = D * 2;
  constexpr int ROWS_PER_KB = 1024 / ROWB;
  constexpr int PER_WAVE = BN * ROWB / (NWAVES * 1024);
  constexpr bool SAME_SWZ = (ROWS_PER_KB * NWAVES) % 16 == 0;
  const u32x4 rs = rsrc_words(tile, tile_bytes(n_in, row_stride, ROWB));
  const uint32_t step = (uint32_t)(ROWS_PER_KB * NWAVES * row_stride);
#pragma unroll
  for (int r = 0; r < PER_WAVE; ++r) {
    const int R0 = ROWS_PER_KB * (NWAVES * r + wave);
    dma16(rs, lds_tile + R0 * ROWB, SAME_SWZ ? lane_off + r * step : dma_lane_offset_at<D>(lane, R0, row_stride));
  }
}

// The kernel arguments, read again from the kernel-argument segment (where
// the one argument, Params, sits at offset 0).  The empty asm hides that the
// segment never changes, so every call loads afresh: a value the kernel
// needs early and late is then not held in an SGPR in between.
__device__ __forceinline__ Params reread_args() {
  typedef const __attribute__((address_space(4))) uint32_t* karg_ptr;
  karg_ptr pk = (karg_ptr)__builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" : "+s"(pk));
  Params p;
#pragma unroll
  for (int i = 0; i < (int)(sizeof(Params) / 4); ++i) reinterpret_cast<uint32_t*>(&p)[i] = pk[i];
  return p;
}

// KSPLIT = 1: a workgroup of 4 waves runs one unit at a time (two workgroups
// per CU).  KSPLIT = 2: a workgroup of two such groups of 4 waves, one per CU,
// runs one row block: group 0 takes the first half of its KV tiles, group 1
// the second, both through the same code with their own LDS stages, and
// group 1 hands its partial state to group 0 through LDS at the end (the
// launch for row blocks that fit the CUs once; no workspace, no queue).
// D = 256 holds 128 accumulator registers per lane and runs one workgroup per
// CU (one wave per SIMD); the other head dims run two.
template <int D, bool FP16, bool V_FP8, bool KV, int KSPLIT>
__global__ void __launch_bounds__(NTHREADS * KSPLIT, (KSPLIT == 1 && D <= 128) ? 2 : 1)
    attn_fwd_kernel(const Params args) {
  constexpr int CH = D / 8;              // 16-byte chunks per row (8 elements)
  constexpr int ROWB = D * 2;            // bytes per row of a K/V tile in LDS
  constexpr int KSTEPS = D / 16;         // k-steps of S^T = K.Q^T
  constexpr int DBLK = D / 32;           // 32-row blocks of O^T
  constexpr int NBLK = BN / 32;          // 32-key blocks of S^T
  constexpr int SLABS = BN / 16;         // k-slabs of O^T = V^T.P^T
  constexpr int TILE_BYTES = BN * ROWB;
  constexpr int CH8 = D / 16;            // 16-byte chunks per fp8 row
  constexpr int F8_CHUNKS = BN * CH8;     // 16-byte chunks of an fp8 V tile
  // 16-byte fp8 loads per thread (D = 32: half the threads load one chunk each)
  constexpr int F8_LOADS = (F8_CHUNKS + NTHREADS - 1) / NTHREADS;
  constexpr float TAU = 8.0f;            // rescale only when a row max grows by more than 2^8
  static_assert(NBLK == 2, "the S^T code below holds two 32-key blocks");
  static_assert(D == 32 || D == 64 || D == 128 || D == 256, "head dims 32, 64, 128, 256");
  static_assert(F8_LOADS * NTHREADS == F8_CHUNKS || F8_CHUNKS < NTHREADS, "fp8 tile split");
  static_assert(BN == 64, "one key_valid byte per lane of wave 0");

  static_assert(KSPLIT == 1 || KSPLIT == 2, "one or two groups of waves");
  // per group: K stage 0, K stage 1, V stage 0, V stage 1 (one contiguous block)
  __shared__ u32x4 stg[4 * KSPLIT][TILE_BYTES / 16];
  __shared__ uint32_t skv[KSPLIT][2][BN / 4];   // key_valid bytes of each stage's tile (4 per word)
  __shared__ int skvall[KSPLIT][2];             // 1 when every key of the stage's tile is valid
  __shared__ int sred[KSPLIT][NWAVES];
  __shared__ int snext;                         // queue position handed out to this workgroup
  __shared__ f32x2 sml[KSPLIT == 2 ? NTHREADS : 1];  // group 1's (m, l) at the merge
  __shared__ int gctr[KSPLIT];                  // group barrier arrivals (two-group kernel)

  // wave-uniform values go through readfirstlane so that the compiler keeps
  // them (and the buffer resources built from them) in SGPRs
  const int grp = KSPLIT == 1 ? 0 : __builtin_amdgcn_readfirstlane((int)(threadIdx.x / NTHREADS));
  char* const kst[2] = {reinterpret_cast<char*>(stg[4 * grp + 0]), reinterpret_cast<char*>(stg[4 * grp + 1])};
  char* const vst[2] = {reinterpret_cast<char*>(stg[4 * grp + 2]), reinterpret_cast<char*>(stg[4 * grp + 3])};

  const int tid = (int)threadIdx.x & (NTHREADS - 1);  // thread of the group
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  if (KSPLIT == 2 && tid == 0) gctr[grp] = 0;  // read only after the first full barrier
  int gtarget = 0;
  bool synced = true;  // two-group kernel: every group barrier of this unit completed
  // the barrier between tiles: the workgroup's, or the group's own in the
  // two-group kernel (the groups then run free, as two workgroups would)
  auto tile_sync = [&]() {
    if constexpr (KSPLIT == 1) {
      __syncthreads();
    } else {
      synced = group_sync(&gctr[grp], gtarget, lane) && synced;
    }
  };
  const int hf = lane >> 5;   // lane half: keys 4*hf.. of each 8-key group
  const int l32 = lane & 31;

  // ---- units: without a workspace this workgroup's one unit; with one, the
  // units of this XCD's queue until it runs dry (qik_plan.h).  Nothing waits
  // on another workgroup: a workgroup that is not resident yet simply starts
  // later and finds the queue further on.  The gx workgroups of an XCD take
  // positions 0 .. gx-1 in blockIdx order (all of them drawing from the one
  // counter at the start of the launch queued behind each other); later
  // positions come from the counter, drawn at the end of a unit's tile loop so
  // that the atomic's round trip overlaps the unit's merge and store.
  // (the two-group kernel runs one unit per workgroup; a workspace there holds
  // only the merge of split row blocks)
  const bool pulled = KSPLIT == 1 && args.ctl != nullptr;
  const int nx = args.plan.nx;
  const int xcd = (int)(blockIdx.x % nx);
  const int gx = (int)(gridDim.x / nx);
  // A position drawn at the end of a unit's tile loop (thread 0's `pend`) is
  // written to snext just before that unit's output stores (or before it
  // leaves the item to its other piece): its round trip overlaps the merge and
  // the epilogue, and the next unit's head does not wait on it (loads and
  // stores complete in issue order, so a wait there would also wait for the
  // output stores to be acknowledged).
  unsigned pend = 0;
  bool drawn = false;
  for (int first = 1;; first = 0) {
    int bidv = (int)blockIdx.x;
    if (pulled) {
      if (tid == 0 && !drawn) snext = first ? (int)(blockIdx.x / nx) : gx + (int)g_fetch_add(args.ctl + xcd, 1u);
      drawn = false;
      __syncthreads();
      const int loc = snext;
      __syncthreads();  // every thread has read snext before the next unit's head rewrites it
      if (loc >= args.plan.wpx) break;
      bidv = loc * nx + xcd;
    } else if (!first) {
      break;
    }
    // the arguments are re-read from the kernel-argument segment for every
    // unit: kept live across the unit loop instead, they crowd the SGPRs and
    // the scheduler then serialises the tile loop's LDS reads
    const Params p = reread_args();
    Work wk = plan_work(p.plan, bidv);
    if (wk.item < 0) continue;
    // the lead thread of the workgroup (of group 0 in the two-group kernel,
    // whose groups split the unit's tiles between them: wk.piece is the
    // workgroup's piece of a row block split over two workgroups)
    const bool lead = tid == 0 && grp == 0;
    const int vid = wk.item;
    const int nmb = p.plan.nmb;
    const int bh = vid / nmb;
    const int mb = nmb - 1 - (vid - bh * nmb);
    const int b = bh / p.H;
    const int h = bh - b * p.H;

    const int m = mb * BM + wave * 32 + l32;  // this lane's query row
    const bool live = m < p.SQ;

    // ---- the unit's memory reads go out first, in this order: the row's
    // causal length, Q, then the first tile's copies when the unit's first
    // tile is known before the lengths are reduced.  Loads complete in issue
    // order, so the wait for L then covers Q as well but not the copies.
    // Dead rows of the last row block read row SQ-1 instead: the loads need
    // no branch around them (the compiler then counts them and waits for L
    // alone); a dead row's L is -1 below and its results are never stored.
    const int mrd = live ? m : p.SQ - 1;
    // (with uniform lengths there is no L: the load reads a Q word instead and
    // its value is never used; an unconditional load keeps the compiler from
    // ordering a wait before it)
    const int Lraw = gload_i32(p.uniform ? reinterpret_cast<const int32_t*>(p.q) : p.L + mrd);

    // ---- per-(b,h) segment bases (bytes) and row strides
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
      if constexpr (V_FP8) vsc = gload_f32(p.v_scale + b * p.H + h);
    }
    const int kns = (int)(p.skn[1] * 2), vns = (int)(p.svn[1] * 2);
    const int kcs = (int)(p.skc[1] * 2), vcs = (int)(p.svc[1] * VC_ES);
    const float qk_scale = p.qk_scale;

    // ---- Q as the B operand of S^T = K.Q^T: lane holds Q[m, 16j + 8hf .. +8]
    u32x4 qreg[KSTEPS];
    {
      const char* qr = qb + (int64_t)mrd * p.sq[1] * 2;
#pragma unroll
      for (int j = 0; j < KSTEPS; ++j) qreg[j] = gload16(qr + (16 * j + 8 * hf) * 2);
    }

    // lane offsets of the tile copies, per segment and tensor
    const uint32_t koff_new = dma_lane_offset<D>(lane, wave, kns);
    const uint32_t voff_new = dma_lane_offset<D>(lane, wave, vns);
    uint32_t koff_c = 0, voff_c = 0;
    if (p.has_cache) {
      koff_c = dma_lane_offset<D>(lane, wave, kcs);
      if constexpr (!V_FP8) voff_c = dma_lane_offset<D>(lane, wave, vcs);
    }
    const int s1 = p.has_cache ? p.P : 0;  // absolute index of the first fresh key

    // fp8 slab V goes through registers: two 16-fp8 chunks per thread per tile
    u32x4 f8reg[F8_LOADS];
    uint32_t kvbyte = 0;

    // copies of tile t of the slab (seg0) or of the fresh keys into `stage`
    auto issue_seg = [&](bool seg0, int t, int stage) {
      const int row0 = t * BN;
      const int n_in = (seg0 ? p.P : p.SN) - row0;
      char* kd = kst[stage];
      char* vdst = vst[stage];
      if (seg0) {
        dma_tile<D>(kcb + (int64_t)row0 * kcs, kcs, n_in, kd, wave, lane, koff_c);
        if constexpr (V_FP8) {
          const char* tb = vcb + (int64_t)row0 * vcs;
          const auto rs = make_rsrc(tb, tile_bytes(n_in, vcs, D));
#pragma unroll
          for (int i = 0; i < F8_LOADS; ++i) {
            const int qd = i * NTHREADS + tid;
            const int row = qd / CH8, c16 = qd % CH8;
            if (F8_CHUNKS >= NTHREADS || qd < F8_CHUNKS)
              f8reg[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                        rs, (uint32_t)(row * vcs + c16 * 16), 0, 0));
          }
        } else {
          dma_tile<D>(vcb + (int64_t)row0 * vcs, vcs, n_in, vdst, wave, lane, voff_c);
        }
      } else {
        dma_tile<D>(knb + (int64_t)row0 * kns, kns, n_in, kd, wave, lane, koff_new);
        dma_tile<D>(vnb + (int64_t)row0 * vns, vns, n_in, vdst, wave, lane, voff_new);
      }
      if constexpr (KV) {
        // one byte per thread so that bytes past the segment end read as 0
        // (invalid).  The resource is built before the tid < BN branch and its
        // size goes through readfirstlane: built inside the branch, the
        // compiler computes it in VGPRs and loops over the lanes to form it,
        // with a wait for every load in flight (the tile copies included).
        const int kv0 = (seg0 ? 0 : s1) + row0;
        const auto rs = make_rsrc(reinterpret_cast<const char*>(p.key_valid) + b * p.svalid_b + kv0,
                                  __builtin_amdgcn_readfirstlane(min(n_in, BN)));
        if (tid < BN) kvbyte = __builtin_amdgcn_raw_buffer_load_b8(rs, (uint32_t)tid, 0, 0);
      }
    };

    // ---- causal lengths: the block max (dead rows count as -1,
    // triton_attention.py:82-83); the wave's min and max over live rows.
    // With uniform lengths every live row has L = KV - 1 and nothing is read.
    const bool wave_live = mb * BM + wave * 32 < p.SQ;
    int Lrow = p.KV - 1;  // this row's causal length
    int Lmax = p.KV - 1;
    int wave_minL = wave_live ? p.KV - 1 : INT_MAX;
    int wave_maxL = wave_live ? p.KV - 1 : -1;
    // A first piece starts at tile 0 whatever the lengths are (the slab's
    // first tile with a cache, else the fresh keys' first): its copies go out
    // before the lengths are reduced.  With uniform lengths every unit's
    // tiles are known here.
    const bool early = p.uniform || (wk.piece == 0 && grp == 0);
    int run0 = 0, run1 = 0;
    auto schedule = [&]() {
      // KV-tile schedule: tile t of a segment starting at absolute key s0 is
      // visited iff s0 + t*BN <= Lmax (segment-local tiles, triton_attention.py:97-124)
      run0 = (p.has_cache && Lmax >= 0) ? min(cdiv_i(p.P, BN), Lmax / BN + 1) : 0;
      run1 = (Lmax >= s1) ? min(cdiv_i(p.SN, BN), (Lmax - s1) / BN + 1) : 0;
    };
    bool gsplit_on = false;  // two-group kernel: the unit's tiles are split between the groups
    auto piece_tiles = [&](int T, int& g0, int& g1) {
      // this unit's tiles [g0, g1): all of them, or one of the item's two
      // pieces (T, and so the split, is the same for both pieces of the item)
      const bool split = wk.group >= 0 && T >= SPLIT_MIN_TILES;
      if constexpr (KSPLIT == 1) {
        const int gsplit = p.plan.even ? (T + 1) / 2 : (7 * T + 5) / 10;
        g0 = (split && wk.piece) ? gsplit : 0;
        g1 = (split && !wk.piece) ? gsplit : T;
      } else {
        // the workgroup's part of the row block (all of it, or one of two equal
        // halves), split between the groups; group 0's waves are the older ones
        // on every SIMD and win issue arbitration (measured: 9 tiles in 13.4 us
        // against group 1's 17.0 us), so group 0 takes 9/16 of the tiles, and a
        // second group with nothing to do gets an empty range
        const int h = (T + 1) / 2;
        const int a = (split && wk.piece) ? h : 0;
        const int e = (split && !wk.piece) ? h : T;
        gsplit_on = e - a >= SPLIT_MIN_TILES;
        const int mid = a + (9 * (e - a) + 8) / 16;
        g0 = (gsplit_on && grp) ? mid : a;
        g1 = (gsplit_on && !grp) ? mid : e;
        if (!gsplit_on && grp) g0 = e;
      }
      return split;
    };
    if (p.uniform) {
      schedule();
      int e0, e1;
      piece_tiles(run0 + run1, e0, e1);
      if (e0 < e1) {
        const bool seg0 = e0 < run0;
        issue_seg(seg0, seg0 ? e0 : e0 - run0, 0);
      }
    } else {
      if (early) issue_seg(p.has_cache != 0, 0, 0);
      Lrow = live ? Lraw : -1;
      const int lmax = wave_reduce_i32<true>(live ? Lrow : -1);
      wave_minL = wave_reduce_i32<false>(live ? Lrow : INT_MAX);
      wave_maxL = lmax;
      if (lane == 0) sred[grp][wave] = lmax;
      __syncthreads();
      Lmax = sred[grp][0];
#pragma unroll
      for (int w = 1; w < NWAVES; ++w) Lmax = max(Lmax, sred[grp][w]);
      Lmax = __builtin_amdgcn_readfirstlane(Lmax);
      schedule();
    }
    const int T = run0 + run1;

    if (p.debug_tiles != nullptr && lead && wk.piece == 0) p.debug_tiles[bh * nmb + mb] = T;

    int g0, g1;
    const bool split = piece_tiles(T, g0, g1);
    if (wk.piece > 0 && !split) continue;

    // ---- LDS operand offsets inside a stage (lane constants)
    const int swk = swz<CH>(l32);  // rows l32 and l32 + 32 share it
    int koffs[KSTEPS];
#pragma unroll
    for (int j = 0; j < KSTEPS; ++j) koffs[j] = l32 * ROWB + (((2 * j + hf) ^ swk) << 4);
    const int j16 = lane & 15;
    const int rq = 4 * hf + (j16 >> 2);   // V^T read rows: 32*(s>>1) + 16*(s&1) + rq (+8)
    const int colq = 16 * ((lane >> 4) & 1) + 4 * (j16 & 3);
    int voffs[2][DBLK];
#pragma unroll
    for (int db = 0; db < DBLK; ++db) {
      const int col = db * 32 + colq;
      voffs[0][db] = rq * ROWB + (((col >> 3) ^ swz<CH>(rq)) << 4) + ((col & 7) << 1);
      voffs[1][db] = (rq + 8) * ROWB + (((col >> 3) ^ swz<CH>(rq + 8)) << 4) + ((col & 7) << 1);
    }

    auto issue_tile = [&](int g, int stage) {
      const bool seg0 = g < run0;
      issue_seg(seg0, seg0 ? g : g - run0, stage);
    };
    // register-staged parts of a tile: fp8 V dequantised to bf16, key_valid bytes
    auto finish_tile = [&](int g, int stage) {
      char* vd = vst[stage];
      if constexpr (V_FP8) {
        if (g < run0) {
#pragma unroll
          for (int i = 0; i < F8_LOADS; ++i) {
            const int qd = i * NTHREADS + tid;
            const int row = qd / CH8, c16 = qd % CH8;
            if (F8_CHUNKS < NTHREADS && qd >= F8_CHUNKS) continue;
            const u32x4 w = f8reg[i];
            const u32x4 lo = dequant_fp8x8(w.x, w.y, vsc);  // elements 16*c16 .. +7
            const u32x4 hi = dequant_fp8x8(w.z, w.w, vsc);  // elements 16*c16+8 .. +15
            *reinterpret_cast<u32x4*>(vd + row * ROWB + (((2 * c16) ^ swz<CH>(row)) << 4)) = lo;
            *reinterpret_cast<u32x4*>(vd + row * ROWB + (((2 * c16 + 1) ^ swz<CH>(row)) << 4)) = hi;
          }
        }
      }
      if (KV && tid < BN) {
        // wave 0 holds the tile's BN bytes, one per lane
        reinterpret_cast<uint8_t*>(skv[grp][stage])[tid] = (uint8_t)kvbyte;
        const int allv = __all(kvbyte != 0u);
        if (tid == 0) skvall[grp][stage] = allv;
      }
    };

    float m_run = -INFINITY;  // exp2 reference point of each row (scaled units)
    float l_run = 0.0f;       // this lane half's share of the running row sum
    f32x16 oacc[DBLK];
#pragma unroll
    for (int db = 0; db < DBLK; ++db) oacc[db] = f32x16{};

    auto compute_tile = [&](int g, int stage) {
      const char* kS = kst[stage];
      const char* vS = vst[stage];
      const bool seg0 = g < run0;
      const int t = seg0 ? g : g - run0;
      const int n_in = (seg0 ? p.P : p.SN) - t * BN;  // keys of this tile inside its segment
      const int kv0 = (seg0 ? 0 : s1) + t * BN;        // absolute index of the tile's first key
      if (kv0 > wave_maxL) return;                     // no row of this wave sees the tile

      // S^T[n, m] = sum_d K[n, d] Q[m, d]; lane holds m = l32, n = 8(i/4) + 4hf + i%4 (+32)
      f32x16 sa = f32x16{}, sb = f32x16{};
      {
        u32x4 ka0 = lds128(kS + koffs[0]);
        u32x4 kb0 = lds128(kS + koffs[0] + 32 * ROWB);
#pragma unroll
        for (int j = 0; j < KSTEPS; ++j) {
          u32x4 ka1, kb1;
          if (j + 1 < KSTEPS) {
            ka1 = lds128(kS + koffs[j + 1]);
            kb1 = lds128(kS + koffs[j + 1] + 32 * ROWB);
          }
          sa = mfma32<FP16>(ka0, qreg[j], sa);
          sb = mfma32<FP16>(kb0, qreg[j], sb);
          if (j + 1 < KSTEPS) {
            ka0 = ka1;
            kb0 = kb1;
          }
        }
      }

      // mask: segment tail, kv <= L[row], key_valid (triton_attention.py:126-144)
      // a tile whose keys are all valid needs no key_valid term (tail tiles are
      // never all valid: bytes past the segment end read as 0)
      const bool kv_mask = KV && __builtin_amdgcn_readfirstlane(skvall[grp][stage]) == 0;
      const bool full = (n_in >= BN) && (kv0 + BN - 1 <= wave_minL) && !kv_mask;
      if (!full) {
        const int lim = min(Lrow - kv0, n_in - 1) - 4 * hf;  // allowed: n_local - 4hf <= lim
        uint32_t kvw[8];
        if (kv_mask) {
#pragma unroll
          for (int q = 0; q < 8; ++q) kvw[q] = skv[grp][stage][q * 2 + hf];  // bytes of keys 8q + 4hf .. +3
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int na = 8 * (i >> 2) + (i & 3);
          bool oka = na <= lim, okb = na + 32 <= lim;
          if (kv_mask) {
            oka = oka && ((kvw[i >> 2] >> (8 * (i & 3))) & 0xffu) != 0;
            okb = okb && ((kvw[4 + (i >> 2)] >> (8 * (i & 3))) & 0xffu) != 0;
          }
          sa[i] = oka ? sa[i] : -INFINITY;
          sb[i] = okb ? sb[i] : -INFINITY;
        }
      }

      // online softmax in the exp2 domain (triton_attention.py:146-152); the
      // reference point moves only when a row max grows by more than TAU, so
      // p <= 2^TAU and the acc rescale is skipped on most tiles
      float mx = fmaxf(sa[0], sb[0]);
#pragma unroll
      for (int i = 1; i < 16; ++i) mx = fmaxf(fmaxf(mx, sa[i]), sb[i]);
      mx = pair_max(mx) * qk_scale;
      if (__any(mx > m_run + TAU)) {
        const float m_new = fmaxf(m_run, mx);
        const float alpha = (m_new == -INFINITY) ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < DBLK; ++db)
#pragma unroll
          for (int i = 0; i < 16; ++i) oacc[db][i] *= alpha;
        m_run = m_new;
      }
      const float m_safe = (m_run == -INFINITY) ? 0.0f : m_run;
      float rs = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        sa[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(sa[i], qk_scale, -m_safe));
        sb[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(sb[i], qk_scale, -m_safe));
        rs += sa[i];
        rs += sb[i];
      }
      l_run += rs;

      // P^T as the B operand: slab s uses registers 8*(s%2).. of block s/2
      u32x4 pb[SLABS];
#pragma unroll
      for (int s = 0; s < SLABS; ++s) {
        const f32x16& src = (s >> 1) ? sb : sa;
        const int i0 = (s & 1) * 8;
        pb[s].x = pack2<FP16>(src[i0 + 0], src[i0 + 1]);
        pb[s].y = pack2<FP16>(src[i0 + 2], src[i0 + 3]);
        pb[s].z = pack2<FP16>(src[i0 + 4], src[i0 + 5]);
        pb[s].w = pack2<FP16>(src[i0 + 6], src[i0 + 7]);
      }

      // O^T[d, m] += sum_n V[n, d] P[m, n]; the V^T operand comes from the LDS
      // transpose read: source lane j of each 16-lane group reads row base + j/4,
      // columns d0 + 4(j%4)..+3, and receives column d0 + j of rows base..base+3
#pragma unroll
      for (int s = 0; s < SLABS; ++s) {
        const int soff = ((s >> 1) * 32 + 16 * (s & 1)) * ROWB;
#pragma unroll
        for (int db = 0; db < DBLK; ++db) {
          const i16x4 x0 = lds_read_tr16(vS + voffs[0][db] + soff);
          const i16x4 x1 = lds_read_tr16(vS + voffs[1][db] + soff);
          const u32x2 w0 = __builtin_bit_cast(u32x2, x0);
          const u32x2 w1 = __builtin_bit_cast(u32x2, x1);
          oacc[db] = mfma32<FP16>(u32x4{w0.x, w0.y, w1.x, w1.y}, pb[s], oacc[db]);
        }
      }
    };

    if (g0 < g1) {
      if (!early) issue_tile(g0, 0);
      finish_tile(g0, 0);
    }
    wait_copies();
    __syncthreads();

    for (int g = g0; g < g1; g += 2) {
      // tiles g0, g0 + 2, ... from stage 0, the others from stage 1 (constant LDS offsets)
      if (g + 1 < g1) issue_tile(g + 1, 1);
      compute_tile(g, 0);
      if (g + 1 < g1) finish_tile(g + 1, 1);
      wait_copies();
      tile_sync();
      if (g + 1 < g1) {
        if (g + 2 < g1) issue_tile(g + 2, 0);
        compute_tile(g + 1, 1);
        if (g + 2 < g1) finish_tile(g + 2, 0);
        wait_copies();
        tile_sync();
      }
    }


    // ---- split item: both pieces publish their partial state; the second to
    // arrive combines the two in piece order (so the result does not depend
    // on which piece that is) and writes the output.  Nothing waits on another
    // workgroup.  Ordering, at agent (device) scope:
    //   * a piece that publishes writes its slot with device-scope stores (sc1: written
    //     through past the XCD's L2), then waits for all of them to complete
    //     (vmcnt(0)) before its barrier and its arrival atomic, so the slot
    //     is visible device-wide before the arrival count moves (a release
    //     made of the completion wait; the atomic itself is agent-scope);
    //   * the piece that sees the count at 1 (before publishing, or as the
    //     value its own increment returned) reads the other slot with
    //     device-scope loads (sc1: served from the coherence point, not from a
    //     CU or XCD cache), issued only after that atomic returned (barrier in
    //     between), so they observe those stores whichever CU or XCD either
    //     piece ran on.  Both pieces may publish (each sees 0 first); then the
    //     second increment merges, as before.
    // There is no agent-scope fence: on gfx950 one is an L2 writeback plus an
    // L2 invalidate of the whole XCD, which throws away the other workgroups'
    // K/V lines (measured: the first version was 30% slower with it).
    const Params pe = reread_args();
    if (pulled && tid == 0) pend = g_fetch_add(pe.ctl + xcd, 1u);
    drawn = pulled;
    if constexpr (KSPLIT == 2) {
      if (gsplit_on) {
        // group 1 hands its O^T accumulators and (m, l) to group 0 through
        // its own stage block (free: the tile loop ended with a barrier), and
        // group 0 combines the two in piece order, the arithmetic of the
        // merge through the workspace below
        f32x4* const xs = reinterpret_cast<f32x4*>(stg[4]);
        if (grp == 1) {
#pragma unroll
          for (int db = 0; db < DBLK; ++db)
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4)
              xs[(db * 4 + q4) * NTHREADS + tid] =
                  f32x4{oacc[db][4 * q4 + 0], oacc[db][4 * q4 + 1], oacc[db][4 * q4 + 2], oacc[db][4 * q4 + 3]};
          // a timed-out group barrier poisons the merged row sums
          sml[tid] = f32x2{m_run, synced ? l_run : __builtin_nanf("")};
        }
        __syncthreads();
        if (grp == 0) {
          const f32x2 mlo = sml[tid];
          const float m0 = m_run, m1 = mlo[0];
          const float mm = fmaxf(m0, m1);
          const float a0 = (m0 == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m0 - mm);
          const float a1 = (m1 == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m1 - mm);
          l_run = l_run * a0 + mlo[1] * a1;
          m_run = mm;
#pragma unroll
          for (int db = 0; db < DBLK; ++db)
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
              const f32x4 v = xs[(db * 4 + q4) * NTHREADS + tid];
#pragma unroll
              for (int e = 0; e < 4; ++e) oacc[db][4 * q4 + e] = oacc[db][4 * q4 + e] * a0 + v[e] * a1;
            }
        }
      }
      // a timed-out group barrier poisons the row sums (before any merge
      // through the workspace, which carries them on)
      if (!synced) l_run = __builtin_nanf("");
    }
    float l_part = l_run;
    if (split) {
      constexpr int OB = slot_oacc_bytes<D>();
      constexpr int SB = slot_bytes<D>();
      constexpr int SC1 = 16;  // cache policy: device scope
      char* const gslots = pe.ws_slots + (int64_t)wk.group * pe.plan.ns * SB;
      unsigned* const word = pe.ctl + 2 * NXCD_MAX + wk.group;
      // arrival count of the group (0 between launches: whoever merges puts
      // it back).  A piece that finds the other one already arrived merges
      // at once and never writes its own slot; otherwise it publishes its
      // slot and arrives, and the second to arrive merges.
      if (lead) sred[0][0] = g_load(word) == 1u ? 1 : 0;
      __syncthreads();
      const bool other_first = sred[0][0] != 0;
      __syncthreads();  // every thread has read the flag before it is reused
      if (other_first) {
        if (lead) g_store(word, 0u);
      } else {
        const auto mine = make_rsrc(gslots + wk.piece * SB, SB);
        if (grp == 0) {
#pragma unroll
          for (int db = 0; db < DBLK; ++db)
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
              const f32x4 v = {oacc[db][4 * q4 + 0], oacc[db][4 * q4 + 1], oacc[db][4 * q4 + 2], oacc[db][4 * q4 + 3]};
              __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), mine,
                                                     (uint32_t)(((db * 4 + q4) * NTHREADS + tid) * 16), 0, SC1);
            }
          __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, f32x2{m_run, l_run}), mine,
                                                (uint32_t)(OB + tid * 8), 0, SC1);
        }
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the slot has reached device scope
        __syncthreads();
        if (lead) {
          const unsigned before = g_fetch_add(word, 1u);
          const bool last = before == 1u;
          if (last) g_store(word, 0u);
          sred[0][0] = last ? 1 : 0;
        }
        if (pulled && tid == 0) snext = gx + (int)pend;
        __syncthreads();
        if (sred[0][0] == 0) continue;  // not the last piece: the last one finishes the item
      }

      // the other piece's state; the two combine in piece order, the same
      // arithmetic whichever of them arrived last (in the two-group kernel
      // group 0 holds the workgroup's state and stores the rows)
      if (KSPLIT == 1 || grp == 0) {
        const auto other = make_rsrc(gslots + (wk.piece ^ 1) * SB, SB);
        const f32x2 mlo = __builtin_bit_cast(
            f32x2, __builtin_amdgcn_raw_buffer_load_b64(other, (uint32_t)(OB + tid * 8), 0, SC1));
        const bool p1 = wk.piece != 0;
        const float m0 = p1 ? mlo[0] : m_run, m1 = p1 ? m_run : mlo[0];
        const float l0 = p1 ? mlo[1] : l_run, l1 = p1 ? l_run : mlo[1];
        const float mm = fmaxf(m0, m1);
        const float a0 = (m0 == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m0 - mm);
        const float a1 = (m1 == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m1 - mm);
        l_part = l0 * a0 + l1 * a1;
#pragma unroll
        for (int db = 0; db < DBLK; ++db)
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4) {
            const f32x4 v = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                          other, (uint32_t)(((db * 4 + q4) * NTHREADS + tid) * 16), 0, SC1));
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float o0 = p1 ? v[e] : oacc[db][4 * q4 + e];
              const float o1 = p1 ? oacc[db][4 * q4 + e] : v[e];
              oacc[db][4 * q4 + e] = o0 * a0 + o1 * a1;
            }
          }
      }
    }

    // ---- epilogue: out = l > 0 ? acc / l : 0 (triton_attention.py:166-168).
    // A lane holds half of one row's D values; the wave's 32 rows go out
    // through its own 32 x ROWB bytes of LDS (in K stages 0-1: free after the
    // tile loop's last barrier, and written by the next unit's copies only
    // behind the draw's barriers), read back as whole rows, so that a store
    // instruction writes 1 KiB of whole rows instead of 16 B into each of 32
    // rows (which took ~2 us per unit, measured).  Rows past SQ are not stored.
    if constexpr (KSPLIT == 2) {
      if (!synced) l_part = __builtin_nanf("");
    }
    const float l_tot = pair_sum(l_part);
    // a NaN row sum (non-finite inputs, or a timed-out group barrier) gives NaN rows
    // (written as selects around one division, so that no branch is formed:
    // 1/l for l > 0, 1 * (l - l) otherwise, which is 0 for l = 0 and NaN for NaN)
    const bool pos = l_tot > 0.0f;
    const float inv = (1.0f / (pos ? l_tot : 1.0f)) * (pos ? 1.0f : l_tot - l_tot);
    if (pulled && tid == 0) snext = gx + (int)pend;
    if constexpr (V_FP8 || KV) {
      // kernels that write LDS inside the tile loop (the fp8 V dequantisation,
      // the key_valid bytes) store straight from the registers: with the LDS
      // staging below the compiler serialises their PV block's LDS reads
      // (48-64 full waits in the tile loop instead of 18-34)
      if (live && grp == 0) {
        char* orow = pe.out + (b * pe.so[0] + (int64_t)m * pe.so[1] + h * pe.so[2]) * 2;
#pragma unroll
        for (int db = 0; db < DBLK; ++db)
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4) {
            const int d = db * 32 + 8 * q4 + 4 * hf;
            u32x2 w;
            w.x = pack2<FP16>(oacc[db][4 * q4 + 0] * inv, oacc[db][4 * q4 + 1] * inv);
            w.y = pack2<FP16>(oacc[db][4 * q4 + 2] * inv, oacc[db][4 * q4 + 3] * inv);
            gstore8(orow + d * 2, w);
          }
      }
    } else {
      if (grp == 0) {
        // the lane index goes through an empty asm here: the offsets below are the
        // same for every unit, and hoisted out of the unit loop they would hold
        // ~24 registers through the tile loop
        int ln = lane;
        asm volatile("" : "+v"(ln));
        const int r32 = ln & 31, half = ln >> 5;
        char* const ow = kst[0] + wave * (32 * ROWB);
#pragma unroll
        for (int db = 0; db < DBLK; ++db)
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4) {
            // 16-byte chunk c of row r32 holds d = 8c .. 8c + 7; this lane's four are 4half ..
            const int c = db * 4 + q4;
            u32x2 w;
            w.x = pack2<FP16>(oacc[db][4 * q4 + 0] * inv, oacc[db][4 * q4 + 1] * inv);
            w.y = pack2<FP16>(oacc[db][4 * q4 + 2] * inv, oacc[db][4 * q4 + 3] * inv);
            *reinterpret_cast<u32x2*>(ow + r32 * ROWB + ((c ^ swz<CH>(r32)) << 4) + 8 * half) = w;
          }
        constexpr int RPI = 64 / CH;  // rows per store instruction
        const int rr = ln / CH, cc = ln % CH;
        const int row0 = mb * BM + wave * 32;
        char* const obase = pe.out + (b * pe.so[0] + h * pe.so[2]) * 2;
#pragma unroll
        for (int i = 0; i < 32 / RPI; ++i) {
          const int r = i * RPI + rr;
          const u32x4 v = lds128(ow + r * ROWB + ((cc ^ swz<CH>(r)) << 4));
          if (row0 + r < pe.SQ) gstore16(obase + (int64_t)(row0 + r) * pe.so[1] * 2 + cc * 16, v);
        }
      }
    }
  }  // units

  // ---- the last workgroup of the XCD to leave puts its queue words back to 0
  // (every workgroup of the XCD has drawn its last position by then)
  if (pulled && tid == 0) {
    const unsigned g = gridDim.x / nx;
    const unsigned before = g_fetch_add(args.ctl + NXCD_MAX + xcd, 1u);
    if (before == g - 1) {
      g_store(args.ctl + xcd, 0u);
      g_store(args.ctl + NXCD_MAX + xcd, 0u);
    }
  }
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
// The workspace of qik_attn_fwd_noalloc: one array per device, never
// allocated by the library.  Host code uses its device address from
// hipGetSymbolAddress (scratch_ptr below), never the name.
static __device__ __align__(256) unsigned char scratch[QIK_ATTN_SCRATCH_BYTES];

// Zero `n16` 16-byte words (the scratch's control words) with vector stores;
// a fill kernel rather than hipMemsetAsync, so that a captured graph replays it.
__global__ void zero16_kernel(u32x4* p, int n16) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n16) p[i] = u32x4{0u, 0u, 0u, 0u};
}

// ---------------------------------------------------------------------------
// host side

typedef void (*kernel_fn)(Params);

template <int D, bool KV, int KS>
kernel_fn pick_kernel(bool fp16, bool vfp8) {
  if (fp16) return attn_fwd_kernel<D, true, false, KV, KS>;
  if (vfp8) return attn_fwd_kernel<D, false, true, KV, KS>;
  return attn_fwd_kernel<D, false, false, KV, KS>;
}

// key_valid is a template parameter: without a mask the kernel carries none
// of its code (the tile loop is then the same as with no mask support at all)
template <int D>
kernel_fn pick_kernel(bool fp16, bool vfp8, bool kv, bool two_groups) {
  if constexpr (D <= 128) {
    if (two_groups) return kv ? pick_kernel<D, true, 2>(fp16, vfp8) : pick_kernel<D, false, 2>(fp16, vfp8);
  }
  return kv ? pick_kernel<D, true, 1>(fp16, vfp8) : pick_kernel<D, false, 1>(fp16, vfp8);
}

// The two-group form needs two groups' LDS stages in one workgroup (256 KiB
// at D = 256, more than a CU holds): not at D = 256.
inline bool two_group_dim(int64_t D) { return D <= 128; }

kernel_fn pick_kernel_d(int64_t D, bool fp16, bool vfp8, bool kv, bool two_groups) {
  switch (D) {
    case 32: return pick_kernel<32>(fp16, vfp8, kv, two_groups);
    case 64: return pick_kernel<64>(fp16, vfp8, kv, two_groups);
    case 128: return pick_kernel<128>(fp16, vfp8, kv, two_groups);
    default: return pick_kernel<256>(fp16, vfp8, kv, false);
  }
}

int slot_bytes_d(int64_t D) {
  switch (D) {
    case 32: return slot_bytes<32>();
    case 64: return slot_bytes<64>();
    case 128: return slot_bytes<128>();
    default: return slot_bytes<256>();
  }
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

// Workgroups one XCD of the current device holds at once for kernel `which`
// (0..23, see pick_index): occupancy per CU x CUs / XCDs, cached per device.
constexpr int MAX_DEVICES = 64;
std::atomic<int> g_slots[MAX_DEVICES][24];
std::atomic<int> g_xcds[MAX_DEVICES];
std::atomic<int> g_cus[MAX_DEVICES];

// Compute units of the current device, cached per device (0 if unknown).
int device_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (dev >= 0 && dev < MAX_DEVICES) {
    const int c = g_cus[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) return 0;
  if (dev >= 0 && dev < MAX_DEVICES) g_cus[dev].store(cus, std::memory_order_relaxed);
  return cus;
}

// XCDs of the current device (hipDeviceAttributeNumberOfXccs; NXCD if the
// runtime cannot say), clamped to [1, NXCD_MAX], cached per device.
int device_xcds() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return NXCD;
  if (dev >= 0 && dev < MAX_DEVICES) {
    const int c = g_xcds[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int nx = 0;
  if (hipDeviceGetAttribute(&nx, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess || nx <= 0) nx = NXCD;
  nx = std::min(std::max(nx, 1), NXCD_MAX);
  if (dev >= 0 && dev < MAX_DEVICES) g_xcds[dev].store(nx, std::memory_order_relaxed);
  return nx;
}

int pick_index(int D, bool fp16, bool vfp8, bool kv) {
  const int di = D == 32 ? 0 : D == 64 ? 1 : D == 128 ? 2 : 3;
  return 2 * (3 * di + (fp16 ? 1 : (vfp8 ? 2 : 0))) + (kv ? 1 : 0);
}

int slots_per_xcd(kernel_fn fn, int which, int* out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return QIK_ERR_DEVICE;
  if (dev >= 0 && dev < MAX_DEVICES) {
    const int c = g_slots[dev][which].load(std::memory_order_relaxed);
    if (c > 0) {
      *out = c;
      return QIK_OK;
    }
  }
  int cus = 0, occ = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    return QIK_ERR_DEVICE;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, reinterpret_cast<const void*>(fn), NTHREADS, 0) !=
          hipSuccess ||
      occ <= 0)
    return QIK_ERR_DEVICE;
  const int sx = std::max(1, occ * cus / device_xcds());
  if (dev >= 0 && dev < MAX_DEVICES) g_slots[dev][which].store(sx, std::memory_order_relaxed);
  *out = sx;
  return QIK_OK;
}

// Launch geometry of one call.  Without `split`: one workgroup per unit, no
// workspace.  With it: the last partial round's row blocks split into pieces
// (qik_plan.h), sx workgroups per XCD pulling units from the XCD's queue, and
// a workspace of control words (zero between launches) and partial-state
// slots.
struct Launch {
  kernel_fn fn;
  WorkPlan plan;
  int64_t grid;
  int threads;         // per workgroup: NTHREADS, or 2 * NTHREADS for the two-group kernel
  int64_t ws_bytes;    // 0: no workspace
  int64_t ctl_bytes;   // control words at the start of the workspace
  int slot;
};

int plan_launch(const qik_attn_args* a, bool split, Launch* L) {
  const int64_t nmb = cdiv64(a->SQ, BM);
  const int64_t n = a->B * a->H * nmb;  // <= INT_MAX (qik_attn_validate)
  const bool fp16 = a->dtype == QIK_DTYPE_FP16;
  const bool vfp8 = (a->flags & QIK_V_CACHE_FP8) != 0;
  const bool kv = (a->flags & QIK_HAS_KEY_VALID) != 0;
  L->fn = pick_kernel_d(a->D, fp16, vfp8, kv, false);
  L->slot = slot_bytes_d(a->D);
  L->ws_bytes = 0;
  L->ctl_bytes = 0;
  L->grid = 0;
  L->threads = NTHREADS;
  memset(&L->plan, 0, sizeof(L->plan));
  if (n == 0) return QIK_OK;
  const int nx = device_xcds();
  int sx = 1;
  const int cus = device_cus();
  if (split && two_group_dim(a->D) && n <= cus) {
    // row blocks fit the CUs once: one two-group workgroup per row block, its
    // KV tiles split between the groups and merged in LDS (no workspace) ...
    L->fn = pick_kernel_d(a->D, fp16, vfp8, kv, true);
    L->threads = 2 * NTHREADS;
    if (2 * n <= cus && cus >= nx) {
      // ... or, with at most half the CUs' worth of row blocks (one GPU's share
      // of the heads), each row block split into two equal pieces on two CUs,
      // every piece split between the groups, the pieces merged through the
      // workspace as the split launch below merges them
      L->plan = make_plan((int)n, (int)nmb, cus / nx, 1, (a->flags & QIK_UNIFORM_L) ? 0 : 1, nx);
      if (L->plan.ns == 2 && L->plan.wpx <= cus / nx && 2 * NXCD_MAX + L->plan.ngroups <= QIK_ATTN_WS_CTL_BYTES / 4) {
        L->grid = (int64_t)nx * L->plan.wpx;
        L->ctl_bytes = QIK_ATTN_WS_CTL_BYTES;
        L->ws_bytes = L->ctl_bytes + (int64_t)L->plan.ngroups * L->plan.ns * L->slot;
        return QIK_OK;
      }
    }
    L->plan = make_plan((int)n, (int)nmb, 1, 0, 1, nx);
    L->grid = (int64_t)nx * L->plan.wpx;
    return QIK_OK;
  }
  if (split) {
    const int st = slots_per_xcd(L->fn, pick_index((int)a->D, fp16, vfp8, kv), &sx);
    if (st != QIK_OK) return st;
    L->plan = make_plan((int)n, (int)nmb, sx, 1, (a->flags & QIK_UNIFORM_L) ? 0 : 1, nx);
    // queue positions are mapped through loc * nx + x, which must fit an
    // int, and the arrival words must fit the fixed control region (the same
    // for every shape, so that no launch leaves slot data where another
    // launch keeps its control words)
    if ((int64_t)nx * L->plan.wpx <= INT_MAX && 2 * NXCD_MAX + L->plan.ngroups <= QIK_ATTN_WS_CTL_BYTES / 4) {
      L->grid = (int64_t)nx * std::min(sx, L->plan.wpx);
      L->ctl_bytes = QIK_ATTN_WS_CTL_BYTES;
      L->ws_bytes = L->ctl_bytes + (int64_t)L->plan.ngroups * L->plan.ns * L->slot;
      return QIK_OK;
    }
  }
  L->plan = make_plan((int)n, (int)nmb, sx, 0, 1, nx);
  L->grid = (int64_t)nx * L->plan.wpx;
  return QIK_OK;
}

// Device address of `scratch` on the current device, resolved once per device.
std::atomic<void*> g_scratch[MAX_DEVICES];

int scratch_ptr(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return QIK_ERR_DEVICE;
  void* p = g_scratch[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) return QIK_ERR_DEVICE;
    g_scratch[dev].store(p, std::memory_order_release);
  }
  *out = p;
  return QIK_OK;
}

int launch(const qik_attn_args* a, bool split, void* ws, int64_t ws_bytes, void* stream) {
  const int st = qik_attn_validate(a);
  if (st != QIK_OK) return st;
  Launch L;
  const int pst = plan_launch(a, split, &L);
  if (pst != QIK_OK) return pst;
  if (L.grid == 0) return QIK_OK;
  if (L.ws_bytes > 0 && (ws == nullptr || !aligned_to(ws, 256) || ws_bytes < L.ws_bytes)) return QIK_ERR_WORKSPACE;

  Params p;
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
  if (L.ws_bytes > 0) {
    p.ctl = static_cast<unsigned*>(ws);
    p.ws_slots = static_cast<char*>(ws) + L.ctl_bytes;
  }
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
  p.has_cache = (a->flags & QIK_HAS_CACHE) ? 1 : 0;
  p.has_key_valid = (a->flags & QIK_HAS_KEY_VALID) ? 1 : 0;
  p.uniform = (a->flags & QIK_UNIFORM_L) ? 1 : 0;
  // qk_scale = sm_scale * log2(e), both fp32, as triton_attention.py:93 computes it
  p.qk_scale = a->sm_scale * 1.44269504088896340736f;
  p.plan = L.plan;

  void* kargs[] = {&p};
  const hipError_t e = hipLaunchKernel(reinterpret_cast<const void*>(L.fn), dim3((unsigned)L.grid),
                                       dim3((unsigned)L.threads), kargs, 0, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? QIK_OK : QIK_ERR_LAUNCH;
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
    case QIK_ERR_HEAD_DIM: return "head_dim must be 32, 64, 128 or 256";
    case QIK_ERR_SHAPE: return "negative or oversized B/SQ/SN/P/H";
    case QIK_ERR_CACHE: return "cache flag, P and cache pointers are inconsistent";
    case QIK_ERR_FP8_SCALE: return "fp8 cache V needs the cache, a v_scale pointer and bf16 q/k/v";
    case QIK_ERR_ALIGN: return "pointers and b/s/h strides must be multiples of 8 elements, and K/V row strides at least D";
    case QIK_ERR_LAUNCH: return "HIP kernel launch failed";
    case QIK_ERR_SEGMENTS: return "segments need 0 <= start <= end, and 0 <= prefix_end <= seq_len";
    case QIK_ERR_DEVICE: return "HIP device query failed";
    case QIK_ERR_WORKSPACE: return "workspace NULL, not 256-byte aligned, or smaller than qik_attn_workspace_size";
    case QIK_ERR_SCRATCH: return "the call needs more workspace than QIK_ATTN_SCRATCH_BYTES";
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
  if (a->D != 32 && a->D != 64 && a->D != 128 && a->D != 256) return QIK_ERR_HEAD_DIM;
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
  // a KV tile's byte offsets must fit in 31 bits (the tile copies use 32-bit
  // buffer offsets): BN * row stride < 2^31
  const int64_t tile_lim = ((int64_t)1 << 31) / qik::BN;
  if (a->stride_k_new[1] * 2 >= tile_lim || a->stride_v_new[1] * 2 >= tile_lim) return QIK_ERR_SHAPE;
  if (has_cache && (a->stride_k_cache[1] * 2 >= tile_lim || a->stride_v_cache[1] * 2 >= tile_lim)) return QIK_ERR_SHAPE;
  // K/V rows must not overlap (the tile copies zero-fill a segment tail through
  // buffer bounds that assume row_stride >= D)
  if (a->SN > 1 && (a->stride_k_new[1] < a->D || a->stride_v_new[1] < a->D)) return QIK_ERR_ALIGN;
  if (has_cache && a->P > 1 && (a->stride_k_cache[1] < a->D || a->stride_v_cache[1] < a->D)) return QIK_ERR_ALIGN;
  if (has_cache) {
    if (!qik::aligned_to(a->k_cache, 16)) return QIK_ERR_ALIGN;
    if (!qik::aligned_to(a->v_cache, vfp8 ? 8 : 16)) return QIK_ERR_ALIGN;
    if (!qik::stride_ok(a->stride_k_cache, a->B, a->P, a->H, 8)) return QIK_ERR_ALIGN;
    if (!qik::stride_ok(a->stride_v_cache, a->B, a->P, a->H, 8)) return QIK_ERR_ALIGN;
  }
  return QIK_OK;
}

int qik_attn_fwd(const qik_attn_args* a, void* stream) { return qik::launch(a, false, nullptr, 0, stream); }

int qik_attn_workspace_size(const qik_attn_args* a, int64_t* bytes) {
  if (bytes == nullptr) return QIK_ERR_NULL_ARG;
  *bytes = 0;
  const int st = qik_attn_validate(a);
  if (st != QIK_OK) return st;
  qik::Launch L;
  const int pst = qik::plan_launch(a, true, &L);
  if (pst != QIK_OK) return pst;
  *bytes = L.ws_bytes;
  return QIK_OK;
}

int qik_attn_fwd_ws(const qik_attn_args* a, void* workspace, int64_t workspace_bytes, void* stream) {
  return qik::launch(a, true, workspace, workspace_bytes, stream);
}

int qik_attn_fwd_noalloc(const qik_attn_args* a, void* stream) {
  const int st = qik_attn_validate(a);
  if (st != QIK_OK) return st;
  qik::Launch L;
  const int pst = qik::plan_launch(a, true, &L);
  if (pst != QIK_OK) return pst;
  if (L.grid == 0) return QIK_OK;
  if (L.ws_bytes > (int64_t)QIK_ATTN_SCRATCH_BYTES) return QIK_ERR_SCRATCH;
  void* ws = nullptr;
  if (L.ws_bytes > 0) {
    const int sst = qik::scratch_ptr(&ws);
    if (sst != QIK_OK) return sst;
    // the control words must be zero when the attention launch starts
    const int n16 = (int)(L.ctl_bytes / 16);
    void* kargs[] = {&ws, (void*)&n16};
    if (hipLaunchKernel(reinterpret_cast<const void*>(qik::zero16_kernel), dim3((unsigned)((n16 + 255) / 256)),
                        dim3(256), kargs, 0, static_cast<hipStream_t>(stream)) != hipSuccess)
      return QIK_ERR_LAUNCH;
  }
  return qik::launch(a, true, ws, (int64_t)QIK_ATTN_SCRATCH_BYTES, stream);
}

int qik_attn_work_map(int64_t n_items, int32_t n_row_blocks, int32_t slots_per_xcd, int32_t split,
                      int32_t* item, int32_t* piece, int32_t* group, int64_t cap, int64_t* grid,
                      int64_t* ngroups, int32_t* pieces) {
  return qik_attn_work_map_xcds(n_items, n_row_blocks, slots_per_xcd, split, qik::NXCD, item, piece, group, cap,
                                grid, ngroups, pieces);
}

int qik_attn_work_map_xcds(int64_t n_items, int32_t n_row_blocks, int32_t slots_per_xcd, int32_t split,
                           int32_t n_xcds, int32_t* item, int32_t* piece, int32_t* group, int64_t cap,
                           int64_t* grid, int64_t* ngroups, int32_t* pieces) {
  if (grid == nullptr || ngroups == nullptr) return QIK_ERR_NULL_ARG;
  if (n_items < 0 || n_items > INT_MAX || n_row_blocks < 1 || slots_per_xcd < 1) return QIK_ERR_SHAPE;
  if (n_xcds < 1 || n_xcds > qik::NXCD_MAX) return QIK_ERR_SHAPE;
  const qik::WorkPlan pl = qik::make_plan((int)n_items, n_row_blocks, slots_per_xcd, split ? 1 : 0, 1, n_xcds);
  if ((int64_t)pl.nx * pl.wpx > INT_MAX) return QIK_ERR_SHAPE;
  *grid = (int64_t)pl.nx * pl.wpx;
  *ngroups = pl.ngroups;
  if (pieces != nullptr) *pieces = pl.ns;
  if (item == nullptr && piece == nullptr && group == nullptr) return QIK_OK;
  if (item == nullptr || piece == nullptr || group == nullptr) return QIK_ERR_NULL_ARG;
  if (cap < *grid) return QIK_ERR_SHAPE;
  for (int64_t b = 0; b < *grid; ++b) {
    const qik::Work w = qik::plan_work(pl, (int)b);
    item[b] = w.item;
    piece[b] = w.piece;
    group[b] = w.group;
  }
  return QIK_OK;
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
