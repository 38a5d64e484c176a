// loopback_read.hip -- MI355X (gfx950, CDNA4) kernels of the Loopback depth-attention read.
//
// One read at destination s has n = s + 1 sources v_i (bf16, fp16 or fp32 updates, one row of d elements per token)
// and per-token fp32 RMS scales r_i. Every kernel here is HBM-bound streaming over token rows; the design rules are:
//   * a row of d elements is d/8 eight-element vectors (16 bytes in bf16 and fp16, 32 in fp32), covered by `tpr`
//     lanes holding `vpt` vectors each (ldr_row_layout); 256-lane workgroups hold 256/tpr rows side by side, so any
//     d that is a multiple of 8 runs without padding the row to a power of two;
//   * per-(token, source) scalars (scores, probabilities, weights) are staged through LDS per tile of tokens with
//     coalesced loads, then broadcast to the lanes of a row;
//   * row reductions are 64-wide wavefront butterflies, plus one LDS exchange when a row spans several waves;
//   * every sum is fp32 in a fixed order (no atomics): results are deterministic run to run.
// Sources are reached through per-source addresses passed by value in the kernel arguments, so the stacked
// layout (slices of one tensor) and the list layout (one tensor per source) share the kernels.

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>
#include <math.h>

#include <atomic>
#include <type_traits>

#include "loopback_read.h"

// Launch-shape tunables (compile-time; the defaults are the measured choice on MI355X).
#ifndef LDR_RF_UNROLL
#define LDR_RF_UNROLL 8      // read forward: sources loaded per batch
#endif
#ifndef LDR_RF_STAGE
#define LDR_RF_STAGE 65536   // read forward: LDS bytes for a tile's output rows (0: rows stored as they finish)
#endif
#ifndef LDR_RF_TT
#define LDR_RF_TT 16         // read forward: tokens per tile (more when a workgroup holds more rows side by side)
#endif
#ifndef LDR_RF_BIG
#define LDR_RF_BIG 1         // read forward: 512-lane workgroups with 32-token tiles, their output staged in 128 KiB of
#endif                       // LDS and written as one burst, one workgroup per CU (when the tile's rows fit)
#ifndef LDR_RF_BIG_MIN_ROW_BYTES
#define LDR_RF_BIG_MIN_ROW_BYTES 28672   // read forward: fewest bytes read and written per token ((n + 2) rows) for the
#endif                                   // 512-lane launch, whose fixed cost is higher (7 rows of 2048 bf16)
#ifndef LDR_RF_BIG_GRID
#define LDR_RF_BIG_GRID 256  // read forward, 512-lane workgroups: one per CU, each takes tiles in turn
#endif
#ifndef LDR_RF_HALF_TT
#define LDR_RF_HALF_TT 1     // read forward: 8-token tiles for rows whose 16-token tile does not fit the staging space
#endif
#ifndef LDR_RF_STAGE_U
#define LDR_RF_STAGE_U 6     // read forward with staged output: sources loaded per batch (the registers of 8 leave
#endif                       // one wave per SIMD beside the staging code)
#ifndef LDR_RF_U_F32
#define LDR_RF_U_F32 4       // read forward, fp32 updates: sources loaded per batch (fp32 vectors take twice the
#endif                       // registers: 6 or 8 spilled to scratch)
#ifndef LDR_RF_MAX_VPT
#define LDR_RF_MAX_VPT 4     // read forward: most 16-byte vectors per lane in a row
#endif
#ifndef LDR_AS_RB
#define LDR_AS_RB 4          // update gradient: token rows per lane (each query load serves all of them)
#endif
#ifndef LDR_AS_JB
#define LDR_AS_JB 1          // update gradient: reads whose rows are loaded together
#endif
#ifndef LDR_AS_STORES
#define LDR_AS_STORES 0      // update gradient: bit 0 stores dv through the caches, bit 1 dv_neg (else non-temporal)
#endif
#ifndef LDR_AS_MAX_VPT
#define LDR_AS_MAX_VPT 3
#endif
#ifndef LDR_AS_MAX_VPT_F32
#define LDR_AS_MAX_VPT_F32 4   // update gradient, fp32 updates: one wave per row of 2048 (bf16 and fp16: two)
#endif
#ifndef LDR_AS_RB_F32
#define LDR_AS_RB_F32 2        // update gradient, fp32 rows of 3-4 vectors per lane: token rows per lane
#endif
#ifndef LDR_AS_JB_F32
#define LDR_AS_JB_F32 2        // update gradient, fp32 updates: reads whose rows are loaded together
#endif
#ifndef LDR_B1_MAX_VPT
#define LDR_B1_MAX_VPT 4     // backward pass 1 (holds g and two accumulators per element)
#endif
#ifndef LDR_B1_C
#define LDR_B1_C 0           // backward pass 1: sources per chunk (0 = by vectors per lane)
#endif
#ifndef LDR_B1_WAVE_ROWS
#define LDR_B1_WAVE_ROWS 1   // backward pass 1: prefer rows inside one wave (no LDS in the row reductions)
#endif
#ifndef LDR_F32_NT
#define LDR_F32_NT 1         // the reads' fp32 sources streamed non-temporally, as 16-bit ones
#endif
#ifndef LDR_B1_KEEP_LAST
#define LDR_B1_KEEP_LAST 1   // backward pass 1: the newest source loaded through the caches (the update gradient re-reads it)
#endif
#ifndef LDR_B1_GD64
#define LDR_B1_GD64 1        // backward pass 1 with fp32 updates: g . v_i and the scalars formed from it in fp64
#endif
#ifndef LDR_WRITE_VALU
#define LDR_WRITE_VALU 0     // write: the scores on the vector units (k_write_dots) instead of the matrix cores, every
#endif                       // dtype; a comparison build (the scale kernels then follow k_write_dots' summation order)
#ifndef LDR_WM_ROWS
#define LDR_WM_ROWS 1        // write: rows streamed whole (d a multiple of 256), else in the matrix cores' layout
#endif
#ifndef LDR_W32_ROWS
#define LDR_W32_ROWS 1       // fp32 write: rows streamed whole (d a multiple of 256), else in the matrix cores' layout
#endif
#ifndef LDR_NT
#define LDR_NT 1             // non-temporal loads for the streamed sources
#endif
#ifndef LDR_AS_GRID
#define LDR_AS_GRID 65535    // update gradient: most workgroups
#endif
#ifndef LDR_RF_GRID
#define LDR_RF_GRID 512      // read forward: workgroups (2 per CU: all resident, each takes token tiles in turn)
#endif
#ifndef LDR_ON_PD_VPT4
#define LDR_ON_PD_VPT4 1     // one-pass online read at 4 vectors per lane: sources in flight per row (2 spilled 36-120
#endif                       // bytes to scratch: c4 online read bf16 7.38 -> 7.05 ms, fp32 15.88 -> 15.08 ms per pass)
#ifndef LDR_ON_GRID
#define LDR_ON_GRID 512      // one-pass online read: workgroups (2 per CU: all resident, each takes rows in turn)
#endif
#ifndef LDR_ON_WAVES
#define LDR_ON_WAVES 2       // one-pass online read: waves per SIMD the registers must allow
#endif
#ifndef LDR_ON_PD
#define LDR_ON_PD 2          // one-pass online read: sources in flight per row at 3-4 vectors per lane
#endif
#ifndef LDR_B1_GRID
#define LDR_B1_GRID 512      // backward pass 1: workgroups (each takes token tiles in turn)
#endif
#ifndef LDR_RF_VPT
#define LDR_RF_VPT 0         // fixed vectors per lane (0 = chosen from d) for the read forward,
#endif
#ifndef LDR_AS_VPT
#define LDR_AS_VPT 0         // the update gradient
#endif
#ifndef LDR_B1_VPT
#define LDR_B1_VPT 0         // and backward pass 1
#endif

namespace {

constexpr int RF_STAGE_BYTES = LDR_RF_STAGE;
constexpr int WG = 256;                 // lanes per workgroup (4 wave64s)
constexpr int MAXS = LDR_MAX_SOURCES;
constexpr int TT_MAX = 32;              // tokens per tile in the tiled kernels
constexpr int SP = MAXS + 1;            // padded LDS row of per-source scalars
constexpr int PRO_K = 4;                 // tile prologues: scalar entries per lane whose loads go out together

// The launch settings a build may change, and the ranges the kernels are written for (a value outside them would
// overflow a tile in LDS, leave rows unwritten or loop without advancing: the build refuses it).
static_assert(LDR_RF_U_F32 >= 1 && LDR_RF_U_F32 <= 8, "read forward: 1..8 fp32 sources per batch");
static_assert(LDR_RF_UNROLL >= 1 && LDR_RF_STAGE_U >= 1 && LDR_RF_UNROLL <= 8 && LDR_RF_STAGE_U <= 8,
              "read forward: 1..8 sources per batch");
static_assert(LDR_RF_STAGE >= 0, "read forward: staging bytes must be >= 0");
static_assert(LDR_RF_TT >= 1 && LDR_RF_TT <= TT_MAX, "read forward: 1..32 tokens per tile (the LDS planes' rows)");
static_assert(LDR_RF_BIG == 0 || LDR_RF_BIG == 1, "read forward: LDR_RF_BIG is 0 or 1");
static_assert(LDR_RF_BIG_MIN_ROW_BYTES >= 0, "read forward: LDR_RF_BIG_MIN_ROW_BYTES >= 0");
static_assert(LDR_RF_MAX_VPT >= 1 && LDR_RF_MAX_VPT <= 4 && LDR_AS_MAX_VPT >= 1 && LDR_AS_MAX_VPT <= 4 &&
              LDR_B1_MAX_VPT >= 1 && LDR_B1_MAX_VPT <= 4, "vectors per lane: 1..4 (the kernels' instantiations)");
static_assert(LDR_RF_VPT >= 0 && LDR_RF_VPT <= 4 && LDR_AS_VPT >= 0 && LDR_AS_VPT <= 4 && LDR_B1_VPT >= 0 &&
              LDR_B1_VPT <= 4, "fixed vectors per lane: 0 (chosen from d) or 1..4");
static_assert(LDR_AS_STORES >= 0 && LDR_AS_STORES <= 3, "update gradient: LDR_AS_STORES is 0..3");
static_assert(LDR_AS_RB >= 1 && LDR_AS_JB >= 1 && LDR_AS_JB_F32 >= 1,
              "update gradient: at least one row per lane and one read per batch");
static_assert(LDR_AS_MAX_VPT_F32 >= 1 && LDR_AS_MAX_VPT_F32 <= 4, "vectors per lane: 1..4");
static_assert(LDR_B1_C >= 0 && LDR_B1_C <= 8, "backward pass 1: 0 (by vectors per lane) or 1..8 sources per chunk");
static_assert(LDR_B1_GD64 == 0 || LDR_B1_GD64 == 1, "backward pass 1: LDR_B1_GD64 is 0 or 1");
static_assert(LDR_B1_KEEP_LAST == 0 || LDR_B1_KEEP_LAST == 1, "backward pass 1: LDR_B1_KEEP_LAST is 0 or 1");
static_assert(LDR_ON_PD >= 1 && LDR_ON_PD_VPT4 >= 1 && LDR_ON_WAVES >= 1, "online read: at least one source in flight, one wave per SIMD");
static_assert(LDR_AS_GRID >= 1 && LDR_RF_GRID >= 1 && LDR_ON_GRID >= 1 && LDR_B1_GRID >= 1 && LDR_RF_BIG_GRID >= 1,
              "grids: >= 1 workgroup");

typedef uint16_t bf16_t;                // bf16 storage (raw bits)
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

struct SrcTab { const void* v[MAXS]; const float* r[MAXS]; };
struct PtrTab { void* p[MAXS]; };
struct AsmTab { const void* g[MAXS]; const float* wz[MAXS]; const float* q[MAXS]; };

// ---------------------------------------------------------------------------------------------------------------
// element I/O: 8 elements (one 16-byte bf16 or fp16 vector, or two fp32 float4) <-> 8 fp32 registers
// ---------------------------------------------------------------------------------------------------------------
template <typename T> struct IO;

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// bf16 <-> fp32: the upper 16 bits of the fp32 pattern; v_cvt_pk_bf16_f32 rounds to nearest even, NaN stays NaN
struct Bf16Cvt {
  static __device__ __forceinline__ void unpack2(uint32_t w, float& a, float& b) {
    a = __uint_as_float(w << 16);
    b = __uint_as_float(w & 0xffff0000u);
  }
  static __device__ __forceinline__ uint32_t pack2(float a, float b) {
    bf16x2_t v = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, v);
  }
  static __device__ __forceinline__ float round(float x) { return (float)(__bf16)x; }
};
__device__ __forceinline__ uint32_t pack2(float a, float b) { return Bf16Cvt::pack2(a, b); }

// fp32 -> fp16 of the fp32 value: v_cvt_f16_f32 (round to nearest even; subnormals kept, overflow to inf). The empty
// asm holds x as an fp32 register value, so the compiler cannot fold the conversion into the operation that produced
// x (a v_fma_mixlo_f16 rounds the exact product or sum once, straight to fp16, which differs from rounding the fp32
// result in rare cases): every fp16 result is the fp32 result rounded, as torch's conversions round it.
__device__ __forceinline__ _Float16 to_f16(float x) {
  asm("" : "+v"(x));
  return (_Float16)x;
}

// fp16 <-> fp32: v_cvt_f32_f16 (exact) and to_f16
struct F16Cvt {
  static __device__ __forceinline__ void unpack2(uint32_t w, float& a, float& b) {
    a = (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
    b = (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
  }
  static __device__ __forceinline__ uint32_t pack2(float a, float b) {
    return (uint32_t)__builtin_bit_cast(uint16_t, to_f16(a)) |
           ((uint32_t)__builtin_bit_cast(uint16_t, to_f16(b)) << 16);
  }
  static __device__ __forceinline__ float round(float x) { return (float)to_f16(x); }
};

// 16-bit elements (bf16, fp16): one 16-byte vector of 8 elements; the sign is bit 15 of each half-word in both
template <typename T, typename Cvt> struct IO16 {
  struct Raw { uint4 u; };
  static __device__ __forceinline__ Raw raw(const T* p) { Raw r; r.u = *reinterpret_cast<const uint4*>(p); return r; }
  // non-temporal: for data read once per kernel and not again soon (the update stack, the output gradient)
  static __device__ __forceinline__ Raw raw_nt(const T* p) {
    Raw r;
#if LDR_NT
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    r.u = make_uint4(v.x, v.y, v.z, v.w);
#else
    r.u = *reinterpret_cast<const uint4*>(p);
#endif
    return r;
  }
  static __device__ __forceinline__ Raw raw_str(const T* p) { return raw_nt(p); }   // the reads' source stream
  static __device__ __forceinline__ Raw zero() { Raw r; r.u = make_uint4(0u, 0u, 0u, 0u); return r; }
  static __device__ __forceinline__ void unpack(const Raw& r, float (&o)[8]) {
    Cvt::unpack2(r.u.x, o[0], o[1]); Cvt::unpack2(r.u.y, o[2], o[3]);
    Cvt::unpack2(r.u.z, o[4], o[5]); Cvt::unpack2(r.u.w, o[6], o[7]);
  }
  static __device__ __forceinline__ void load(const T* p, float (&o)[8]) { unpack(raw(p), o); }
  static __device__ __forceinline__ void store(T* p, const float (&o)[8]) {
    uint4 u;
    u.x = Cvt::pack2(o[0], o[1]); u.y = Cvt::pack2(o[2], o[3]);
    u.z = Cvt::pack2(o[4], o[5]); u.w = Cvt::pack2(o[6], o[7]);
    *reinterpret_cast<uint4*>(p) = u;
  }
  // non-temporal stores, for results not read again soon (the update gradients): they stream to HBM instead of
  // displacing the rows the next launches re-read from the caches
  static __device__ __forceinline__ void store_nt(T* p, const float (&o)[8]) {
    const u32x4 u{Cvt::pack2(o[0], o[1]), Cvt::pack2(o[2], o[3]), Cvt::pack2(o[4], o[5]), Cvt::pack2(o[6], o[7])};
    __builtin_nontemporal_store(u, reinterpret_cast<u32x4*>(p));
  }
  // stores -o (rounded): the sign bits of the rounded values flipped, exact (cached, and non-temporal)
  static __device__ __forceinline__ void store_neg(T* p, const float (&o)[8]) {
    uint4 u;
    u.x = Cvt::pack2(o[0], o[1]) ^ 0x80008000u; u.y = Cvt::pack2(o[2], o[3]) ^ 0x80008000u;
    u.z = Cvt::pack2(o[4], o[5]) ^ 0x80008000u; u.w = Cvt::pack2(o[6], o[7]) ^ 0x80008000u;
    *reinterpret_cast<uint4*>(p) = u;
  }
  static __device__ __forceinline__ void store_neg_nt(T* p, const float (&o)[8]) {
    const u32x4 u{Cvt::pack2(o[0], o[1]) ^ 0x80008000u, Cvt::pack2(o[2], o[3]) ^ 0x80008000u,
                  Cvt::pack2(o[4], o[5]) ^ 0x80008000u, Cvt::pack2(o[6], o[7]) ^ 0x80008000u};
    __builtin_nontemporal_store(u, reinterpret_cast<u32x4*>(p));
  }
  static __device__ __forceinline__ float round(float x) { return Cvt::round(x); }
};

template <> struct IO<bf16_t> : IO16<bf16_t, Bf16Cvt> {};
template <> struct IO<_Float16> : IO16<_Float16, F16Cvt> {};

template <> struct IO<float> {
  struct Raw { float4 a, b; };
  static __device__ __forceinline__ Raw raw(const float* p) {
    Raw r; r.a = reinterpret_cast<const float4*>(p)[0]; r.b = reinterpret_cast<const float4*>(p)[1]; return r;
  }
  static __device__ __forceinline__ Raw raw_nt(const float* p) { return raw(p); }
  // the reads' source stream: non-temporal (LDR_F32_NT; for the other kernels' fp32 rows the caches measured faster:
  // c4 fp32 read forward 15.5 -> 15.1 ms per pass, backward pass 1 and the update gradient 0.6-0.7 ms slower)
  static __device__ __forceinline__ Raw raw_str(const float* p) {
#if LDR_NT && LDR_F32_NT
    const u32x4 a = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    const u32x4 b = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p) + 1);
    Raw r;
    r.a = make_float4(__uint_as_float(a.x), __uint_as_float(a.y), __uint_as_float(a.z), __uint_as_float(a.w));
    r.b = make_float4(__uint_as_float(b.x), __uint_as_float(b.y), __uint_as_float(b.z), __uint_as_float(b.w));
    return r;
#else
    return raw(p);
#endif
  }
  static __device__ __forceinline__ Raw zero() { Raw r; r.a = make_float4(0.f, 0.f, 0.f, 0.f); r.b = r.a; return r; }
  static __device__ __forceinline__ void unpack(const Raw& r, float (&o)[8]) {
    o[0] = r.a.x; o[1] = r.a.y; o[2] = r.a.z; o[3] = r.a.w; o[4] = r.b.x; o[5] = r.b.y; o[6] = r.b.z; o[7] = r.b.w;
  }
  static __device__ __forceinline__ void load(const float* p, float (&o)[8]) { unpack(raw(p), o); }
  static __device__ __forceinline__ void store(float* p, const float (&o)[8]) {
    reinterpret_cast<float4*>(p)[0] = make_float4(o[0], o[1], o[2], o[3]);
    reinterpret_cast<float4*>(p)[1] = make_float4(o[4], o[5], o[6], o[7]);
  }
  static __device__ __forceinline__ void store_nt(float* p, const float (&o)[8]) {
    __builtin_nontemporal_store(u32x4{__float_as_uint(o[0]), __float_as_uint(o[1]), __float_as_uint(o[2]),
                                      __float_as_uint(o[3])}, reinterpret_cast<u32x4*>(p));
    __builtin_nontemporal_store(u32x4{__float_as_uint(o[4]), __float_as_uint(o[5]), __float_as_uint(o[6]),
                                      __float_as_uint(o[7])}, reinterpret_cast<u32x4*>(p) + 1);
  }
  static __device__ __forceinline__ void store_neg(float* p, const float (&o)[8]) {
    reinterpret_cast<float4*>(p)[0] = make_float4(-o[0], -o[1], -o[2], -o[3]);
    reinterpret_cast<float4*>(p)[1] = make_float4(-o[4], -o[5], -o[6], -o[7]);
  }
  static __device__ __forceinline__ void store_neg_nt(float* p, const float (&o)[8]) {
    __builtin_nontemporal_store(u32x4{__float_as_uint(o[0]) ^ 0x80000000u, __float_as_uint(o[1]) ^ 0x80000000u,
                                      __float_as_uint(o[2]) ^ 0x80000000u, __float_as_uint(o[3]) ^ 0x80000000u},
                                reinterpret_cast<u32x4*>(p));
    __builtin_nontemporal_store(u32x4{__float_as_uint(o[4]) ^ 0x80000000u, __float_as_uint(o[5]) ^ 0x80000000u,
                                      __float_as_uint(o[6]) ^ 0x80000000u, __float_as_uint(o[7]) ^ 0x80000000u},
                                reinterpret_cast<u32x4*>(p) + 1);
  }
  static __device__ __forceinline__ float round(float x) { return x; }
};

__device__ __forceinline__ void load_f32x8(const float* p, float (&o)[8]) { IO<float>::load(p, o); }

// ---------------------------------------------------------------------------------------------------------------
// row geometry and reductions
// ---------------------------------------------------------------------------------------------------------------
struct Rows {
  int d8, tpr, rpw, rs, lr;
  __device__ __forceinline__ Rows(int d, int tpr_, int block = WG)
      : d8(d >> 3), tpr(tpr_), rpw(block / tpr_), rs((int)threadIdx.x / tpr_), lr((int)threadIdx.x % tpr_) {}
  __device__ __forceinline__ int c8(int v) const { return lr + v * tpr; }
  __device__ __forceinline__ bool act(int v) const { return c8(v) < d8; }
  // element offset of vector v inside a row, clamped to the row for lanes past its end: loads stay unconditional
  // (a branch around a load makes the compiler wait for it before the next one), only stores test act(v)
  __device__ __forceinline__ int off(int v) const { const int c = c8(v); return (c < d8 ? c : d8 - 1) * 8; }
};

// Reduction over an aligned group of g lanes of a wave (g a power of two <= 64) in registers, without the LDS
// crossbar: DPP (xor 1 and xor 2 inside quads, the 8- and 16-lane mirrors) and gfx950's row swaps
// (v_permlane16_swap, v_permlane32_swap), the smallest level first. At each level both operands already hold equal
// values across their halves, so every lane of the group ends with the same bits. All lanes of the wave must be
// active.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xf, 0xf, false));
}
template <typename Op>
__device__ __forceinline__ float lanes_reduce(float x, int g, Op op) {
  if (g >= 2) x = op(x, dpp_f<0xB1>(x));    // quad_perm [1, 0, 3, 2]
  if (g >= 4) x = op(x, dpp_f<0x4E>(x));    // quad_perm [2, 3, 0, 1]
  if (g >= 8) x = op(x, dpp_f<0x141>(x));   // row_half_mirror
  if (g >= 16) x = op(x, dpp_f<0x140>(x));  // row_mirror
  if (g >= 32) {
    const unsigned u = __builtin_bit_cast(unsigned, x);
    const auto sw = __builtin_amdgcn_permlane16_swap(u, u, false, false);   // rows (0, 0, 2, 2) and (1, 1, 3, 3)
    x = op(__builtin_bit_cast(float, (unsigned)sw[0]), __builtin_bit_cast(float, (unsigned)sw[1]));
  }
  if (g >= 64) {
    const unsigned u = __builtin_bit_cast(unsigned, x);
    const auto sw = __builtin_amdgcn_permlane32_swap(u, u, false, false);   // lower half twice, upper half twice
    x = op(__builtin_bit_cast(float, (unsigned)sw[0]), __builtin_bit_cast(float, (unsigned)sw[1]));
  }
  return x;
}
struct AddOp { __device__ __forceinline__ float operator()(float a, float b) const { return a + b; } };
struct MaxOp { __device__ __forceinline__ float operator()(float a, float b) const { return fmaxf(a, b); } };

// The same lane-group sum for fp64 values: each level moves the two 32-bit halves with the same DPP or row swap
// (the halves of one value travel together), and adds in fp64.
template <int CTRL>
__device__ __forceinline__ double dpp_d(double x) {
  const uint64_t u = __builtin_bit_cast(uint64_t, x);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, 0xf, 0xf, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, 0xf, 0xf, false);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ double join_d(unsigned lo, unsigned hi) {
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | (uint64_t)lo);
}
__device__ __forceinline__ double lanes_sum_d(double x, int g) {
  if (g >= 2) x += dpp_d<0xB1>(x);
  if (g >= 4) x += dpp_d<0x4E>(x);
  if (g >= 8) x += dpp_d<0x141>(x);
  if (g >= 16) x += dpp_d<0x140>(x);
  if (g >= 32) {
    const uint64_t u = __builtin_bit_cast(uint64_t, x);
    const unsigned lo = (unsigned)u, hi = (unsigned)(u >> 32);
    const auto sl = __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
    const auto sh = __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
    x = join_d((unsigned)sl[0], (unsigned)sh[0]) + join_d((unsigned)sl[1], (unsigned)sh[1]);
  }
  if (g >= 64) {
    const uint64_t u = __builtin_bit_cast(uint64_t, x);
    const unsigned lo = (unsigned)u, hi = (unsigned)(u >> 32);
    const auto sl = __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
    const auto sh = __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
    x = join_d((unsigned)sl[0], (unsigned)sh[0]) + join_d((unsigned)sl[1], (unsigned)sh[1]);
  }
  return x;
}

// Sum NV values over the tpr lanes of a row (tpr a power of two); every lane of the row ends with the totals,
// bitwise equal on all of them. tpr <= 64: the row is an aligned lane group of one wave. tpr > 64: the row spans
// tpr/64 waves and the wave totals meet in `red` (4 * NV floats of LDS); the whole workgroup must then call
// together (barriers inside).
template <int NV>
__device__ __forceinline__ void row_sum(float (&x)[NV], int tpr, float* red) {
  const int w = tpr < 64 ? tpr : 64;
#pragma unroll
  for (int j = 0; j < NV; ++j) x[j] = lanes_reduce(x[j], w, AddOp());
  if (tpr > 64) {
    const int wave = (int)threadIdx.x >> 6, lane = (int)threadIdx.x & 63;
    __syncthreads();
    if (lane == 0) {
#pragma unroll
      for (int j = 0; j < NV; ++j) red[wave * NV + j] = x[j];
    }
    __syncthreads();
    const int nw = tpr >> 6, first = (wave / nw) * nw;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      float s = 0.f;
      for (int k = 0; k < nw; ++k) s += red[(first + k) * NV + j];
      x[j] = s;
    }
  }
}

// row_sum in fp64 (the wave totals meet in `red`, 4 * NV doubles of LDS, when the row spans several waves)
template <int NV>
__device__ __forceinline__ void row_sum_d(double (&x)[NV], int tpr, double* red) {
  const int w = tpr < 64 ? tpr : 64;
#pragma unroll
  for (int j = 0; j < NV; ++j) x[j] = lanes_sum_d(x[j], w);
  if (tpr > 64) {
    const int wave = (int)threadIdx.x >> 6, lane = (int)threadIdx.x & 63;
    __syncthreads();
    if (lane == 0) {
#pragma unroll
      for (int j = 0; j < NV; ++j) red[wave * NV + j] = x[j];
    }
    __syncthreads();
    const int nw = tpr >> 6, first = (wave / nw) * nw;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      double s = 0.0;
      for (int k = 0; k < nw; ++k) s += red[(first + k) * NV + j];
      x[j] = s;
    }
  }
}

// Softmax over a token's logits spread over lpt aligned lanes (slot m of lane j holds logit j + m lpt; -inf past n),
// in place: p = exp(l - max) / sum. Only the first ns = ceil(n / lpt) slots can hold logits; the others are left 0
// without work. The division form (not exp(l - logsumexp)) keeps p within a few ulp, as torch's softmax computes
// it. One code path for the scored and the prior-only logits, so equal inputs give bitwise equal results (the
// zero-query identity tc == c0, out == base).
__device__ __forceinline__ void softmax_lanes(float (&l)[8], int lpt, int ns) {
  float mx = l[0];
#pragma unroll
  for (int m = 1; m < 8; ++m)
    if (m < ns) mx = fmaxf(mx, l[m]);
  mx = lanes_reduce(mx, lpt, MaxOp());
  float s = 0.f;
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    if (m < ns) {
      l[m] = (l[m] == -INFINITY) ? 0.f : expf(l[m] - mx);
      s += l[m];
    }
  }
  s = lanes_reduce(s, lpt, AddOp());
#pragma unroll
  for (int m = 0; m < 8; ++m) l[m] = m < ns ? l[m] / s : 0.f;
}

// The coefficient inputs of a read. Either as the read takes them (cbar [tok][n], c0 [n], lam = 1), or -- fused
// with the caller's bookkeeping -- as the previous read left them: coeffs [tok][n-1] and prior [n-1], the newest
// source's entries implied, cbar = lam * [coeffs, 1] and c0 = lam * [prior, 1] (lam = 1 - beta at an iteration end,
// else 1). x * 1.0f == x, so the plain form is exact.
struct Coef {
  const float* cbar;
  int cbar_cols;   // n, or n - 1 (the newest column implied)
  const float* c0;
  int c0_cols;     // n, or n - 1
  float lam;
};

__device__ __forceinline__ float coef_cbar(const Coef& c, int64_t tok, int i) {
#pragma clang fp contract(off)   // the product is rounded on its own, as the caller's scaling is (never fused into a use)
  return i < c.cbar_cols ? c.lam * c.cbar[tok * c.cbar_cols + i] : c.lam;
}

// coef_cbar in two halves, for the tile prologues, which issue all their loads before the first is used: the load,
// always issued at an in-bounds address (its column clamped; `spare`, any readable float, when there is no cbar
// column), and the value formed from it. A load under a per-lane condition is waited for where the two paths meet
// (the other path writes its register), one memory round trip per call.
__device__ __forceinline__ float cbar_load(const Coef& c, int64_t tok, int i, const float* spare) {
  const float* p = c.cbar_cols > 0 ? c.cbar + (tok * c.cbar_cols + min(i, c.cbar_cols - 1)) : spare;
  return *p;
}
// a scale row's address kept in LDS, as a global-memory pointer: loaded from LDS, a plain pointer is generic and
// its loads flat ones, which the compiler waits for with the LDS reads
typedef const __attribute__((address_space(1))) float* gptr_f32;
typedef __attribute__((address_space(1))) float* gptr_f32w;
__device__ __forceinline__ gptr_f32 as_global(const float* p) { return (gptr_f32)p; }
__device__ __forceinline__ gptr_f32w as_global(float* p) { return (gptr_f32w)p; }

__device__ __forceinline__ float cbar_value(const Coef& c, float loaded, int i) {
#pragma clang fp contract(off)   // as coef_cbar
  return i < c.cbar_cols ? c.lam * loaded : c.lam;
}

// x, as a value the compiler cannot see through: index math formed from it inside a tile loop is formed again in
// each pass instead of hoisted out of the loop, where its registers would stay live through the row stream
__device__ __forceinline__ int opaque(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

// per-read constants from the prior: c0, lc = log(max(c0, 1e-8)), M = sum c0 (in source order); and the sources'
// scale-row addresses into s_rp as global-memory pointers (a lane's scale loads read them from LDS). The prior's
// entry (at a clamped address; `spare`, any readable float, when there is no prior column) and the address are
// requested together, before either is used: one memory round trip.
__device__ __forceinline__ void load_prior(const Coef& c, int n, float* s_c0, float* s_lc, float* s_M,
                                           const SrcTab& src, gptr_f32* s_rp, const float* spare,
                                           const PtrTab* drt = nullptr, gptr_f32w* s_drp = nullptr) {
  const int t = (int)threadIdx.x;
  if (t < n) {
    const float* p = c.c0_cols > 0 ? c.c0 + min(t, c.c0_cols - 1) : spare;
    const float raw = *p;
    const float* rp = src.r[t];
    if (drt) s_drp[t] = as_global(static_cast<float*>(drt->p[t]));   // (backward pass 1: the dr rows too)
    float v;
    {
#pragma clang fp contract(off)   // the product rounded on its own, as the caller's scaling is
      v = t < c.c0_cols ? c.lam * raw : c.lam;
    }
    s_c0[t] = v;
    s_lc[t] = logf(fmaxf(v, 1e-8f));
    s_rp[t] = as_global(rp);
  }
  __syncthreads();
  if (t == 0) {
    float m = 0.f;
    for (int i = 0; i < n; ++i) m += s_c0[i];
    *s_M = m;
  }
  __syncthreads();
}

// ---------------------------------------------------------------------------------------------------------------
// rstd forward / backward (list layout, and the stacked layout's scale when the write did not store it)
// ---------------------------------------------------------------------------------------------------------------
// the fp32 write's tile: 32 tokens, d in chunks of 128 columns (k_write_dots)
constexpr int WR_TT = 32, WR_KC = 128, WR_KP = WR_KC + 4, WR_MQ = 8;

// The scale of a stored update is formed in one summation order wherever it is formed -- by the write kernels
// (which store it beside the update) or by these kernels (the list layout's rstd, the stacked layout when the write
// did not store it) -- so both layouts read with bitwise equal scales, and so bitwise equal outputs.
//
// Every dtype: the order of the matrix-core writes (k_write_mfma, k_write_rows, k_write_mfma32, k_write_rows32).
// Columns go in 64-column chunks, chunk c to slot w = c mod 4; inside a chunk, quad q takes columns [8q, 8q + 8)
// and [32 + 8q, 40 + 8q). Partial (w, q) is the fused multiply-add sum over its chunks in order, its two column groups
// in order, and their elements in order. Then W_w = (p_w0 + p_w1) + (p_w2 + p_w3), and
// sum = ((W_0 + W_1) + W_2) + W_3.
// Here a row takes 16 lanes (lane 4 w + q holds partial (w, q)), 4 rows per wave.
template <typename T>
__global__ __launch_bounds__(WG) void k_rstd_chunks(const T* __restrict__ x, float* __restrict__ r, int64_t n_tok,
                                                    int d, float eps) {
  const int tid = (int)threadIdx.x, lane = tid & 63, j = lane & 15, w = j >> 2, quad = j & 3;
  const int nchunks = (d + 63) >> 6;
  for (int64_t t0 = (int64_t)blockIdx.x * (WG / 16); t0 < n_tok; t0 += (int64_t)gridDim.x * (WG / 16)) {
    const int64_t tok = t0 + (tid >> 4);
    const T* row = x + (tok < n_tok ? tok : n_tok - 1) * (int64_t)d;
    float ss = 0.f;
#pragma unroll 4
    for (int c = w; c < nchunks; c += 4) {
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int col = c * 64 + quad * 8 + 32 * hf;
        if (col < d) {   // d is a multiple of 8: a column group is whole or past the row
          float e[8];
          IO<T>::load(row + col, e);
#pragma unroll
          for (int k = 0; k < 8; ++k) ss = __builtin_fmaf(e[k], e[k], ss);
        }
      }
    }
    ss += __shfl_xor(ss, 1, 64);   // (p_w0 + p_w1), (p_w2 + p_w3)
    ss += __shfl_xor(ss, 2, 64);   // W_w
    const int g0 = lane & ~15;
    const float w0 = __shfl(ss, g0, 64), w1 = __shfl(ss, g0 + 4, 64), w2 = __shfl(ss, g0 + 8, 64),
                w3 = __shfl(ss, g0 + 12, 64);
    const float tot = ((w0 + w1) + w2) + w3;
    if (tok < n_tok && j == 0) r[tok] = rsqrtf(tot / (float)d + eps);
  }
}

// The order of k_write_dots (the vector-unit write of a LDR_WRITE_VALU build). Lane m of a row's 16 takes columns
// [c0 + 8m, c0 + 8m + 8) for c0 = 0, 128, 256, ... (fused multiply-adds, chunks then elements in order); the 16
// partials meet in the butterfly xor 8, 4, 2, 1.
template <typename T>
__global__ __launch_bounds__(WG) void k_rstd_valu(const T* __restrict__ x, float* __restrict__ r, int64_t n_tok,
                                                  int d, float eps) {
  const int tid = (int)threadIdx.x, m = tid & 15;
  for (int64_t t0 = (int64_t)blockIdx.x * (WG / 16); t0 < n_tok; t0 += (int64_t)gridDim.x * (WG / 16)) {
    const int64_t tok = t0 + (tid >> 4);
    const T* row = x + (tok < n_tok ? tok : n_tok - 1) * (int64_t)d;
    float ss = 0.f;
#pragma unroll 4
    for (int c0 = 0; c0 < d; c0 += WR_KC) {
      const int col = c0 + 8 * m;
      if (col < d) {
        float e[8];
        IO<T>::load(row + col, e);
#pragma unroll
        for (int k = 0; k < 8; ++k) ss = __builtin_fmaf(e[k], e[k], ss);
      }
    }
    for (int off = 8; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
    if (tok < n_tok && m == 0) r[tok] = rsqrtf(ss / (float)d + eps);
  }
}

template <typename T, int VPT>
__global__ __launch_bounds__(WG) void k_rstd_bwd(const T* __restrict__ x, const float* __restrict__ r,
                                                 const float* __restrict__ gr, T* __restrict__ gx, int64_t n_tok,
                                                 int d, int tpr) {
  const Rows R(d, tpr);
  const int64_t groups = (n_tok + R.rpw - 1) / R.rpw;
  for (int64_t gi = blockIdx.x; gi < groups; gi += gridDim.x) {
    const int64_t tok = gi * R.rpw + R.rs;
    if (tok >= n_tok) continue;
    const float rv = r[tok];
    const float c = gr[tok] * (-rv * rv * rv) / (float)d;
    float e[VPT][8];
#pragma unroll
    for (int v = 0; v < VPT; ++v) IO<T>::load(x + tok * (int64_t)d + R.off(v), e[v]);
#pragma unroll
    for (int v = 0; v < VPT; ++v) {
#pragma unroll
      for (int k = 0; k < 8; ++k) e[v][k] = c * e[v][k];
      if (R.act(v)) IO<T>::store(gx + tok * (int64_t)d + R.c8(v) * 8, e[v]);
    }
  }
}

// Rows of any width and alignment (those the vector layout does not take: d not a multiple of 8, above the widest
// row, or not 16-byte aligned): one wave per row, its lanes striding the row with scalar loads (64 consecutive
// elements per step, coalesced), the sum reduced in registers.
__device__ __forceinline__ float ld1(const bf16_t* p) { return __uint_as_float((uint32_t)*p << 16); }
__device__ __forceinline__ float ld1(const float* p) { return *p; }
__device__ __forceinline__ float ld1(const _Float16* p) { return (float)*p; }
__device__ __forceinline__ void st1(bf16_t* p, float v) { *p = __builtin_bit_cast(bf16_t, (__bf16)v); }
__device__ __forceinline__ void st1(float* p, float v) { *p = v; }
__device__ __forceinline__ void st1(_Float16* p, float v) { *p = to_f16(v); }

template <typename T>
__global__ __launch_bounds__(WG) void k_rstd_fwd_any(const T* __restrict__ x, float* __restrict__ r, int64_t n_tok,
                                                     int64_t d, float eps) {
  const int lane = (int)threadIdx.x & 63, w = (int)threadIdx.x >> 6;
  for (int64_t tok = (int64_t)blockIdx.x * (WG / 64) + w; tok < n_tok; tok += (int64_t)gridDim.x * (WG / 64)) {
    const T* row = x + tok * d;
    float ss = 0.f;
    for (int64_t k = lane; k < d; k += 64) {
      const float e = ld1(row + k);
      ss += e * e;
    }
    ss = lanes_reduce(ss, 64, AddOp());   // every lane of the wave is here: the row loop is wave-uniform
    if (lane == 0) r[tok] = rsqrtf(ss / (float)d + eps);
  }
}

template <typename T>
__global__ __launch_bounds__(WG) void k_rstd_bwd_any(const T* __restrict__ x, const float* __restrict__ r,
                                                     const float* __restrict__ gr, T* __restrict__ gx, int64_t n_tok,
                                                     int64_t d) {
  const int lane = (int)threadIdx.x & 63, w = (int)threadIdx.x >> 6;
  for (int64_t tok = (int64_t)blockIdx.x * (WG / 64) + w; tok < n_tok; tok += (int64_t)gridDim.x * (WG / 64)) {
    const float rv = r[tok];
    const float c = gr[tok] * (-rv * rv * rv) / (float)d;
    for (int64_t k = lane; k < d; k += 64) st1(gx + tok * d + k, c * ld1(x + tok * d + k));
  }
}

// ---------------------------------------------------------------------------------------------------------------
// write step: V[s] = round(h - x), R[s] from the rounded update, scores against the later read queries.
// A tile of 32 tokens streams d in chunks of 128 columns: the chunk of the update goes to LDS (fp32) next to the
// chunk of up to 64 query rows, and 256 lanes form the 32 x nq dot products (lane = token + 32 * query group).
// ---------------------------------------------------------------------------------------------------------------

// The write kernels load h -- the block's output the caller has just written, which the read that follows takes
// as its base -- non-temporally: the read forward after it runs 6.62 -> 6.40 ms per pass at config 4 and the write
// itself 1.28 -> 1.24; fp32: the read forward 14.22 -> 13.80 ms (x loaded so too made the write slower and the read
// no faster)
__device__ __forceinline__ uint4 ld_nt16(const void* p) {
  const u32x4 t = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(t[0], t[1], t[2], t[3]);
}

template <typename T>
__global__ __launch_bounds__(WG) void k_write_dots(const T* __restrict__ h, const T* __restrict__ x,
                                                   T* __restrict__ v, float* __restrict__ r,
                                                   const float* __restrict__ q, float* __restrict__ dots,
                                                   int64_t n_tok, int d, int nq, int64_t dots_jstride, float eps) {
  __shared__ float sv[WR_TT * WR_KP];
  __shared__ float sq[LDR_MAX_QUERIES * WR_KP];
  const int tid = (int)threadIdx.x;
  const int64_t t0 = (int64_t)blockIdx.x * WR_TT;
  const int tc = tid & 31, jg = tid >> 5;
  const int mq = (nq + 7) >> 3;
  float acc[WR_MQ];
#pragma unroll
  for (int m = 0; m < WR_MQ; ++m) acc[m] = 0.f;
  float ss[2] = {0.f, 0.f};
  // A chunk's update rows (two vectors of h and x per lane) and query values (up to QV float4 per lane) arrive in
  // registers; once they are in LDS the next chunk's are requested, before the current chunk is summed, so a
  // chunk's loads wait behind the previous chunk's products instead of after them.
  using Raw = typename IO<T>::Raw;
  constexpr int QV = LDR_MAX_QUERIES * (WR_KC / 4) / WG;
  static_assert(QV * WG == LDR_MAX_QUERIES * (WR_KC / 4), "write: whole query chunks per lane");
  Raw hn[2], xn[2];
  float4 qn[QV];
  auto fetch = [&](int c0) {
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int u = tid + WG * e, row = u >> 4, col = c0 + (u & 15) * 8;
      const int64_t tok = t0 + row;
      hn[e] = IO<T>::zero();
      xn[e] = IO<T>::zero();
      if (tok < n_tok && col < d) {
        hn[e] = IO<T>::raw(h + tok * (int64_t)d + col);
        xn[e] = IO<T>::raw(x + tok * (int64_t)d + col);
      }
    }
#pragma unroll
    for (int m = 0; m < QV; ++m) {
      const int idx = tid + WG * m, jj = idx >> 5, col = c0 + (idx & 31) * 4;
      qn[m] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (idx < nq * (WR_KC / 4) && col < d) qn[m] = *reinterpret_cast<const float4*>(q + (int64_t)jj * d + col);
    }
  };
  fetch(0);
  for (int c0 = 0; c0 < d; c0 += WR_KC) {
    // the update chunk: 32 rows x 16 vectors, two vectors per lane
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int u = tid + WG * e, row = u >> 4, col = c0 + (u & 15) * 8;
      const int64_t tok = t0 + row;
      float vv[8];
      if (tok < n_tok && col < d) {
        float hv[8], xv[8];
        IO<T>::unpack(hn[e], hv);
        IO<T>::unpack(xn[e], xv);
#pragma unroll
        for (int k = 0; k < 8; ++k) vv[k] = IO<T>::round(hv[k] - xv[k]);
        // non-temporal: the read that follows streams V[s] with its other sources
        IO<T>::store_nt(v + tok * (int64_t)d + col, vv);
#pragma unroll
        for (int k = 0; k < 8; ++k) ss[e] = __builtin_fmaf(vv[k], vv[k], ss[e]);   // the scale's order: k_rstd_valu
      } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) vv[k] = 0.f;
      }
      float4* dst = reinterpret_cast<float4*>(&sv[row * WR_KP + (u & 15) * 8]);
      dst[0] = make_float4(vv[0], vv[1], vv[2], vv[3]);
      dst[1] = make_float4(vv[4], vv[5], vv[6], vv[7]);
    }
    // the query chunk: nq rows x 32 float4
#pragma unroll
    for (int m = 0; m < QV; ++m) {
      const int idx = tid + WG * m;
      if (idx < nq * (WR_KC / 4)) *reinterpret_cast<float4*>(&sq[(idx >> 5) * WR_KP + (idx & 31) * 4]) = qn[m];
    }
    if (c0 + WR_KC < d) fetch(c0 + WR_KC);   // uniform branch
    __syncthreads();
    if (nq > 0) {
      const int kend = (d - c0) < WR_KC ? (d - c0) : WR_KC;
      for (int k = 0; k < kend; k += 4) {
        const float4 a = *reinterpret_cast<const float4*>(&sv[tc * WR_KP + k]);
#pragma unroll
        for (int m = 0; m < WR_MQ; ++m) {
          if (m < mq) {
            const float4 b = *reinterpret_cast<const float4*>(&sq[(jg + 8 * m) * WR_KP + k]);
            acc[m] += a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w;
          }
        }
      }
    }
    __syncthreads();
  }
  // the scale: 16 lanes per row, rows tid/16 and tid/16 + 16
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    for (int off = 8; off > 0; off >>= 1) ss[e] += __shfl_xor(ss[e], off, 64);
    const int64_t tok = t0 + (tid >> 4) + 16 * e;
    if ((tid & 15) == 0 && tok < n_tok) r[tok] = rsqrtf(ss[e] / (float)d + eps);
  }
  const int64_t tok = t0 + tc;
  if (tok < n_tok) {
#pragma unroll
    for (int m = 0; m < WR_MQ; ++m) {
      const int jj = jg + 8 * m;
      if (m < mq && jj < nq) dots[(int64_t)jj * dots_jstride + tok] = acc[m];
    }
  }
}

// LDS written by some lanes of a wave and read by others of the same wave: complete the writes, keep the order
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ---------------------------------------------------------------------------------------------------------------
// write step on the matrix cores (bf16 updates): the scores are a (tokens x d) . (d x queries) product. Each fp32
// query row is held as three bf16 parts q = hi + mid + lo (the split is exact to ~2^-24 relative); the update is
// exactly bf16 after its rounding, so three bf16 MFMAs with fp32 accumulation give fp32-accurate scores.
// A workgroup takes WM_TT tokens (WM_MB 16-row blocks); its 4 waves split d into 64-column chunks. In a chunk, lane
// quad g holds columns [8g, 8g + 8) and [32 + 8g, 40 + 8g) of its row (one 8-element k-group per MFMA), so each
// load instruction covers 64 contiguous bytes of every row it touches; the wave's V tile of the chunk goes through
// LDS and is stored by 8 lanes per row, whole 128-byte lines per instruction (stored as 64-byte halves, memory saw
// 1.3x the bytes of V). The wave partials of the scores meet in LDS in a fixed order. A wave requests the next
// chunk's rows before it works on the current one.
// v_mfma_f32_16x16x32_bf16 operands: lane l holds row (l % 16) of A and column (l % 16) of B over the k-group of its
// quad (l / 16); the result holds rows 4 (l / 16) + i, i < 4, of column l % 16.
// ---------------------------------------------------------------------------------------------------------------
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

#ifndef LDR_WM_MB
#define LDR_WM_MB 4           // write: 16-token blocks per workgroup (each query-part load serves all of them)
#endif
constexpr int WM_MB = LDR_WM_MB;   // 16-token blocks per workgroup
constexpr int WM_TT = 16 * WM_MB;   // tokens per workgroup
static_assert(WM_MB == 1 || WM_MB == 2 || WM_MB == 4, "write: 1, 2 or 4 16-token blocks per workgroup");
#ifndef LDR_WM_DEPTH
#define LDR_WM_DEPTH 1        // whole-row write: 256-column steps of rows in flight
#endif
constexpr int WM_DEPTH = LDR_WM_DEPTH;
#ifndef LDR_WM_QPF
#define LDR_WM_QPF 0          // whole-row write: request the next step's query parts a step ahead
#endif
#ifndef LDR_WM_DBUF
#define LDR_WM_DBUF 0         // whole-row write: two LDS tiles alternated, one barrier per step
#endif
constexpr bool WM_QPF = LDR_WM_QPF, WM_DBUF = LDR_WM_DBUF;
static_assert(WM_DEPTH >= 1 && WM_DEPTH <= 3, "write: 1..3 steps of rows in flight");
// k_write_rows maps its 4 waves x 16 rows onto the workgroup's tokens: it takes 64-token workgroups only
constexpr bool WM_ROWS = LDR_WM_ROWS && WM_MB == 4;
constexpr int WM_KC = 64;   // columns per chunk
constexpr int WM_QS = 8;    // column step between the quads of a wave
constexpr int WM_HS = 32;   // column step between a lane's two k-groups

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 u) { return __builtin_bit_cast(bf16x8_t, u); }

// The matrix cores' A operands of 8 stored update values (one 16-byte vector). A bf16 update is its own operand. An
// fp16 value e is the exact sum of two bf16 values, hi = bf16(e) and lo = e - hi (e has 11 significant bits, hi takes
// the top 8 and lo the rest; bf16 spans fp16's exponent range), so the products with hi and lo give e's share exactly
// and the scores keep the bf16 updates' accuracy.
template <typename T> struct MfmaA;
template <> struct MfmaA<bf16_t> {
  static constexpr int NP = 1;
  static __device__ __forceinline__ void split(uint4 u, uint4 (&a)[1]) { a[0] = u; }
};
template <> struct MfmaA<_Float16> {
  static constexpr int NP = 2;
  static __device__ __forceinline__ void split(uint4 u, uint4 (&a)[2]) {
    float e[8], hi[8];
    IO<_Float16>::unpack(IO<_Float16>::Raw{u}, e);
    a[0] = make_uint4(pack2(e[0], e[1]), pack2(e[2], e[3]), pack2(e[4], e[5]), pack2(e[6], e[7]));
    IO<bf16_t>::unpack(IO<bf16_t>::Raw{a[0]}, hi);
#pragma unroll
    for (int k = 0; k < 8; ++k) e[k] -= hi[k];   // exact
    a[1] = make_uint4(pack2(e[0], e[1]), pack2(e[2], e[3]), pack2(e[4], e[5]), pack2(e[6], e[7]));
  }
};

// The bf16 parts of the read queries in the matrix cores' operand order (written once per stack by
// k_split_queries): for chunk c of 64 columns, 16-query block b, part p (hi, mid, lo) and k-group half hf, the 64
// lanes' 16-byte operands are consecutive -- qt[(((c nbq + b) 3 + p) 2 + hf) 64 + l], lane l holding query
// 16 b + l mod 16 at columns 64 c + 8 (l / 16) + 32 hf .. + 8 (zeros past the last query and past d) -- so one wave
// load is 1 KiB of whole cache lines. A write scores the queries j_lo .. nq - 1: blocks b0 = j_lo / 16 .. nbq - 1,
// the rows below j_lo computed and not stored.
struct QTile {
  const uint4* qt;
  int nbq;    // 16-query blocks in the table
  int b0;     // first block scored
  int j_lo;   // first query stored (dots points at its slice)
  int nq;     // queries in the table
};

template <typename T, int NB>   // 16-bit updates; NB 16-query blocks scored (from block qt.b0); NB = 0: no scores
__global__ __launch_bounds__(WG) void k_write_mfma(const T* __restrict__ h, const T* __restrict__ x,
                                                   T* __restrict__ v, float* __restrict__ r, QTile qt,
                                                   float* __restrict__ dots, int64_t n_tok, int d,
                                                   int64_t dots_jstride, float eps) {
  using AP = MfmaA<T>;
  constexpr int NBA = NB > 0 ? NB : 1;   // array extents
  __shared__ f32x4_t s_part[4][WM_MB][NBA][64];
  __shared__ float s_ss[4][WM_MB][16];
  __shared__ uint4 s_v[4][WM_TT][WM_KC / 8 + 1];   // each wave's V tile of a chunk (a 16-byte pad per row)
  const int tid = (int)threadIdx.x, w = tid >> 6, l = tid & 63, row = l & 15, quad = l >> 4;
  const int64_t t0 = (int64_t)blockIdx.x * WM_TT;
  f32x4_t acc[WM_MB][NBA];
#pragma unroll
  for (int mb = 0; mb < WM_MB; ++mb)
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[mb][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float ss[WM_MB];
#pragma unroll
  for (int mb = 0; mb < WM_MB; ++mb) ss[mb] = 0.f;
  int64_t roff[WM_MB];
  bool tok_ok[WM_MB];
#pragma unroll
  for (int mb = 0; mb < WM_MB; ++mb) {
    const int64_t tok = t0 + 16 * mb + row;
    tok_ok[mb] = tok < n_tok;
    roff[mb] = (tok_ok[mb] ? tok : n_tok - 1) * (int64_t)d;
  }
  const int nchunks = (d + WM_KC - 1) / WM_KC;
  // a chunk's h and x rows: every 16-token block, the lane's two 8-column k-groups (clamped in bounds)
  auto load_hx = [&](int c, uint4 (&hr)[WM_MB][2], uint4 (&xr)[WM_MB][2]) {
    const int col = c * WM_KC + quad * WM_QS;
#pragma unroll
    for (int mb = 0; mb < WM_MB; ++mb)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int cc = col + WM_HS * hf < d ? col + WM_HS * hf : 0;
        hr[mb][hf] = ld_nt16(h + roff[mb] + cc);
        xr[mb][hf] = *reinterpret_cast<const uint4*>(x + roff[mb] + cc);
      }
  };
  uint4 hr[WM_MB][2], xr[WM_MB][2];
  if (w < nchunks) load_hx(w, hr, xr);
  for (int c = w; c < nchunks; c += 4) {   // wave-uniform trip count
    const int col = c * WM_KC + quad * WM_QS;
    bool col_ok[2];
    int cc[2];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      col_ok[hf] = col + WM_HS * hf < d;
      cc[hf] = col_ok[hf] ? col + WM_HS * hf : 0;
    }
    // the chunk's query parts (cache-resident), requested before the data is touched
    uint4 qv[3][NBA][2];
#pragma unroll
    for (int p = 0; p < 3 * (NB > 0); ++p)
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
          qv[p][b][hf] = qt.qt[((((int64_t)c * qt.nbq + qt.b0 + b) * 3 + p) * 2 + hf) * 64 + l];

    uint4 hc[WM_MB][2], xc[WM_MB][2];   // this chunk's rows; the next chunk's are requested now
#pragma unroll
    for (int mb = 0; mb < WM_MB; ++mb)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) { hc[mb][hf] = hr[mb][hf]; xc[mb][hf] = xr[mb][hf]; }
    if (c + 4 < nchunks) load_hx(c + 4, hr, xr);   // uniform branch
    uint4 va[WM_MB][2][AP::NP];
#pragma unroll
    for (int mb = 0; mb < WM_MB; ++mb)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        float hv[8], xv[8], vv[8];
        IO<T>::unpack(typename IO<T>::Raw{hc[mb][hf]}, hv);
        IO<T>::unpack(typename IO<T>::Raw{xc[mb][hf]}, xv);
        const bool ok = tok_ok[mb] && col_ok[hf];
#pragma unroll
        for (int k = 0; k < 8; ++k) vv[k] = ok ? hv[k] - xv[k] : 0.f;
        T rounded[8];
        IO<T>::store(rounded, vv);
        const uint4 u = *reinterpret_cast<const uint4*>(rounded);
        AP::split(u, va[mb][hf]);
        float rv[8];
        IO<T>::unpack(typename IO<T>::Raw{u}, rv);   // the stored (rounded) update
#pragma unroll
        for (int k = 0; k < 8; ++k) ss[mb] = __builtin_fmaf(rv[k], rv[k], ss[mb]);   // k_rstd_chunks' order
        s_v[w][16 * mb + row][quad + 4 * hf] = u;
      }
    wave_lds_sync();
#pragma unroll
    for (int k = 0; k < WM_TT * 8 / 64; ++k) {   // 8 lanes per token row
      const int e = l + 64 * k, t = e >> 3, u8 = e & 7;
      const int64_t tok = t0 + t;
      const int col8 = c * WM_KC + 8 * u8;
      const uint4 u = s_v[w][t][u8];
      // non-temporal: the read that follows streams V[s] with its other sources, and dirty cached lines would be
      // written back in the middle of its stream
      if (tok < n_tok && col8 < d)
        __builtin_nontemporal_store(u32x4{u.x, u.y, u.z, u.w}, reinterpret_cast<u32x4*>(v + tok * (int64_t)d + col8));
    }
    wave_lds_sync();   // the tile is read before the next chunk overwrites it
#pragma unroll
    for (int p = 0; p < 3 * (NB > 0); ++p)
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
#pragma unroll
          for (int mb = 0; mb < WM_MB; ++mb)   // (columns past d: zero operands on both sides)
#pragma unroll
            for (int a = 0; a < AP::NP; ++a)
              acc[mb][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(va[mb][hf][a]), as_bf16x8(qv[p][b][hf]),
                                                                   acc[mb][b], 0, 0, 0);
        }
  }
#pragma unroll
  for (int mb = 0; mb < WM_MB; ++mb) {
    ss[mb] += __shfl_xor(ss[mb], 16, 64);
    ss[mb] += __shfl_xor(ss[mb], 32, 64);
    if (quad == 0) s_ss[w][mb][row] = ss[mb];
#pragma unroll
    for (int b = 0; b < NB; ++b) s_part[w][mb][b][l] = acc[mb][b];
  }
  __syncthreads();
  if (tid < 16 * WM_MB) {
    const int mb = tid >> 4, rr = tid & 15;
    const float tot = ((s_ss[0][mb][rr] + s_ss[1][mb][rr]) + s_ss[2][mb][rr]) + s_ss[3][mb][rr];
    const int64_t tok = t0 + tid;
    if (tok < n_tok) r[tok] = rsqrtf(tot / (float)d + eps);
  }
  if constexpr (NB > 0) {   // the scores (NB = 0 writes none)
    for (int e = tid; e < WM_MB * NB * 64; e += WG) {
      const int mb = e / (NB * 64), rem = e - mb * NB * 64, b = rem >> 6, ll = rem & 63;
      const f32x4_t sum = ((s_part[0][mb][b][ll] + s_part[1][mb][b][ll]) + s_part[2][mb][b][ll]) + s_part[3][mb][b][ll];
      const int jj = 16 * (qt.b0 + b) + (ll & 15);   // the query; dots points at query j_lo's slice
      if (jj < qt.j_lo || jj >= qt.nq) continue;
      const int64_t tok = t0 + 16 * mb + 4 * (ll >> 4);
      float* dst = dots + (int64_t)(jj - qt.j_lo) * dots_jstride + tok;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (tok + i < n_tok) dst[i] = sum[i];
    }
  }
}

// The write with rows streamed whole (d a multiple of 256): per 256-column step, wave w moves 16 rows of h and x in
// 512-byte row segments (32 lanes per row), stores V row-major and puts it in an LDS tile; then each wave runs the
// matrix-core product of its 64-column quarter (chunk 4 step + w, as k_write_mfma's chunks) on the tile. The chunk
// order per wave, the operands and the order of every sum are k_write_mfma's: V, R and the scores are its bits.
template <typename T, int NB>
__global__ __launch_bounds__(WG) void k_write_rows(const T* __restrict__ h, const T* __restrict__ x,
                                                   T* __restrict__ v, float* __restrict__ r, QTile qt,
                                                   float* __restrict__ dots, int64_t n_tok, int d,
                                                   int64_t dots_jstride, float eps) {
  static_assert(WM_MB == 4, "k_write_rows: its 4 waves x 16 rows are the workgroup's 64 tokens");
  using AP = MfmaA<T>;
  constexpr int NBA = NB > 0 ? NB : 1;
  constexpr int KS = 4 * WM_KC;   // columns per step
  __shared__ f32x4_t s_part[4][WM_MB][NBA][64];
  __shared__ float s_ss[4][WM_MB][16];
  // the step's V tile (a 16-byte pad per row); with WM_DBUF two tiles alternate between steps, so a step needs one
  // barrier (its tile is written, then read; the next step writes the other tile)
  __shared__ uint4 s_a[WM_DBUF ? 2 : 1][WM_TT][KS / 8 + 1];
  const int tid = (int)threadIdx.x, w = tid >> 6, l = tid & 63, row = l & 15, quad = l >> 4;
  const int64_t t0 = (int64_t)blockIdx.x * WM_TT;
  f32x4_t acc[WM_MB][NBA];
#pragma unroll
  for (int mb = 0; mb < WM_MB; ++mb)
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[mb][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float ss[WM_MB];
#pragma unroll
  for (int mb = 0; mb < WM_MB; ++mb) ss[mb] = 0.f;
  // this lane's rows in the streaming layout: 16 w + 2 i + (l / 32), i < 8, vector column l % 32 of the step
  const int lr = l & 31, lh = l >> 5;
  int64_t rof[8];
  bool rok[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int64_t tok = t0 + 16 * w + 2 * i + lh;
    rok[i] = tok < n_tok;
    rof[i] = (rok[i] ? tok : n_tok - 1) * (int64_t)d;
  }
  auto load_rows = [&](int st, uint4 (&hr)[8], uint4 (&xr)[8]) {
    const int col = st * KS + lr * 8;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      hr[i] = ld_nt16(h + rof[i] + col);   // non-temporal: see ld_nt16
      xr[i] = *reinterpret_cast<const uint4*>(x + rof[i] + col);
    }
  };
  const int nsteps = d / KS;
  // one 256-column step; its rows arrive in (hb, xb), which then take the rows of step st + WM_DEPTH: WM_DEPTH steps
  // of rows are in flight while a step is worked on
  // the query parts of this wave's chunk of step st (cache-resident)
  auto load_q = [&](int st, uint4 (&qv)[3][NBA][2]) {
    const int c = 4 * st + w;
#pragma unroll
    for (int p = 0; p < 3 * (NB > 0); ++p)
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
          qv[p][b][hf] = qt.qt[((((int64_t)c * qt.nbq + qt.b0 + b) * 3 + p) * 2 + hf) * 64 + l];
  };
  uint4 qcur[3][NBA][2], qnext[3][NBA][2];   // WM_QPF: the next step's parts are requested a step ahead
  if (WM_QPF && NB > 0) load_q(0, qcur);
  auto step = [&](int st, uint4 (&hb)[8], uint4 (&xb)[8]) {
    uint4 (&qv)[3][NBA][2] = qcur;
    if (NB > 0) {
      if (!WM_QPF) load_q(st, qcur);
      else if (st + 1 < nsteps) load_q(st + 1, qnext);
    }
    auto& tile = s_a[WM_DBUF ? (st & 1) : 0];
    uint4 hc[8], xc[8];   // this step's rows; the buffer now takes the rows WM_DEPTH steps ahead
#pragma unroll
    for (int i = 0; i < 8; ++i) { hc[i] = hb[i]; xc[i] = xb[i]; }
    if (st + WM_DEPTH < nsteps) load_rows(st + WM_DEPTH, hb, xb);   // uniform branch
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float hv[8], xv[8], vv[8];
      IO<T>::unpack(typename IO<T>::Raw{hc[i]}, hv);
      IO<T>::unpack(typename IO<T>::Raw{xc[i]}, xv);
#pragma unroll
      for (int k = 0; k < 8; ++k) vv[k] = rok[i] ? hv[k] - xv[k] : 0.f;
      T rounded[8];
      IO<T>::store(rounded, vv);
      const uint4 ru = *reinterpret_cast<const uint4*>(rounded);
      const u32x4 u{ru.x, ru.y, ru.z, ru.w};
      // non-temporal: the read that follows streams V[s] with its other sources
      if (rok[i]) __builtin_nontemporal_store(u, reinterpret_cast<u32x4*>(v + rof[i] + st * KS + lr * 8));
      tile[16 * w + 2 * i + lh][lr] = make_uint4(u.x, u.y, u.z, u.w);
    }
    __syncthreads();
    uint4 va[WM_MB][2][AP::NP];
#pragma unroll
    for (int mb = 0; mb < WM_MB; ++mb)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const uint4 u = tile[16 * mb + row][w * (WM_KC / 8) + quad + 4 * hf];
        AP::split(u, va[mb][hf]);
        float rv[8];
        IO<T>::unpack(typename IO<T>::Raw{u}, rv);
#pragma unroll
        for (int k = 0; k < 8; ++k) ss[mb] = __builtin_fmaf(rv[k], rv[k], ss[mb]);   // k_rstd_chunks' order
      }
    if (!WM_DBUF) __syncthreads();   // the tile is read before the next step overwrites it
#pragma unroll
    for (int p = 0; p < 3 * (NB > 0); ++p)
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
#pragma unroll
          for (int mb = 0; mb < WM_MB; ++mb)
#pragma unroll
            for (int a = 0; a < AP::NP; ++a)
              acc[mb][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(va[mb][hf][a]), as_bf16x8(qv[p][b][hf]),
                                                                   acc[mb][b], 0, 0, 0);
        }
    if (WM_QPF && NB > 0) {
#pragma unroll
      for (int p = 0; p < 3; ++p)
#pragma unroll
        for (int b = 0; b < NBA; ++b)
#pragma unroll
          for (int hf = 0; hf < 2; ++hf) qcur[p][b][hf] = qnext[p][b][hf];
    }
  };
  uint4 hr[WM_DEPTH][8], xr[WM_DEPTH][8];
#pragma unroll
  for (int k = 0; k < WM_DEPTH; ++k)
    if (k < nsteps) load_rows(k, hr[k], xr[k]);
  for (int st = 0; st < nsteps; st += WM_DEPTH) {
#pragma unroll
    for (int k = 0; k < WM_DEPTH; ++k)
      if (st + k < nsteps) step(st + k, hr[k], xr[k]);   // uniform branch; the buffer index is static
  }
#pragma unroll
  for (int mb = 0; mb < WM_MB; ++mb) {
    ss[mb] += __shfl_xor(ss[mb], 16, 64);
    ss[mb] += __shfl_xor(ss[mb], 32, 64);
    if (quad == 0) s_ss[w][mb][row] = ss[mb];
#pragma unroll
    for (int b = 0; b < NB; ++b) s_part[w][mb][b][l] = acc[mb][b];
  }
  __syncthreads();
  if (tid < 16 * WM_MB) {
    const int mb = tid >> 4, rr = tid & 15;
    const float tot = ((s_ss[0][mb][rr] + s_ss[1][mb][rr]) + s_ss[2][mb][rr]) + s_ss[3][mb][rr];
    const int64_t tok = t0 + tid;
    if (tok < n_tok) r[tok] = rsqrtf(tot / (float)d + eps);
  }
  if constexpr (NB > 0) {   // the scores (NB = 0 writes none)
    for (int e = tid; e < WM_MB * NB * 64; e += WG) {
      const int mb = e / (NB * 64), rem = e - mb * NB * 64, b = rem >> 6, ll = rem & 63;
      const f32x4_t sum = ((s_part[0][mb][b][ll] + s_part[1][mb][b][ll]) + s_part[2][mb][b][ll]) + s_part[3][mb][b][ll];
      const int jj = 16 * (qt.b0 + b) + (ll & 15);   // the query; dots points at query j_lo's slice
      if (jj < qt.j_lo || jj >= qt.nq) continue;
      const int64_t tok = t0 + 16 * mb + 4 * (ll >> 4);
      float* dst = dots + (int64_t)(jj - qt.j_lo) * dots_jstride + tok;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (tok + i < n_tok) dst[i] = sum[i];
    }
  }
}

// The write of fp32 updates on the matrix cores. Each stored value v is split into three bf16 parts,
// v = a0 + a1 + a2 with a0 = bf16(v), a1 = bf16(v - a0), a2 = bf16(v - a0 - a1) (both differences exact in fp32), as
// the queries are in the operand table; of the nine products a_i q_j the six with i + j <= 2 are accumulated, the
// others being below 2^-24 of the score's terms. The layout is k_write_mfma's (lane quad g holds columns 8g.. and
// 32 + 8g.. of its row in each 64-column chunk; the scale sums in k_rstd_chunks' order) with 32-token workgroups
// (fp32 rows take twice the registers); a chunk's values go to LDS and into their parts before the next chunk's rows
// are requested into the same registers, and the V tile is stored by 16 lanes per row, non-temporally.
constexpr int W32_MB = 2, W32_TT = 16 * W32_MB;

__device__ __forceinline__ void split3(const float (&e)[8], uint4 (&a)[3]) {
  float rem[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) rem[k] = e[k];
#pragma unroll
  for (int p = 0; p < 3; ++p) {
    a[p] = make_uint4(pack2(rem[0], rem[1]), pack2(rem[2], rem[3]), pack2(rem[4], rem[5]), pack2(rem[6], rem[7]));
    if (p < 2) {
      float part[8];
      IO<bf16_t>::unpack(IO<bf16_t>::Raw{a[p]}, part);
#pragma unroll
      for (int k = 0; k < 8; ++k) rem[k] -= part[k];   // exact
    }
  }
}

template <int NB>   // NB 16-query blocks scored (from block qt.b0); NB = 0: no scores
__global__ __launch_bounds__(WG) void k_write_mfma32(const float* __restrict__ h, const float* __restrict__ x,
                                                     float* __restrict__ v, float* __restrict__ r, QTile qt,
                                                     float* __restrict__ dots, int64_t n_tok, int d,
                                                     int64_t dots_jstride, float eps) {
  constexpr int NBA = NB > 0 ? NB : 1;
  __shared__ f32x4_t s_part[4][W32_MB][NBA][64];
  __shared__ float s_ss[4][W32_MB][16];
  __shared__ float4 s_v[4][W32_TT][WM_KC / 4 + 1];   // each wave's V tile of a chunk (a 16-byte pad per row)
  const int tid = (int)threadIdx.x, w = tid >> 6, l = tid & 63, row = l & 15, quad = l >> 4;
  const int64_t t0 = (int64_t)blockIdx.x * W32_TT;
  f32x4_t acc[W32_MB][NBA];
#pragma unroll
  for (int mb = 0; mb < W32_MB; ++mb)
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[mb][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float ss[W32_MB];
#pragma unroll
  for (int mb = 0; mb < W32_MB; ++mb) ss[mb] = 0.f;
  int64_t roff[W32_MB];
  bool tok_ok[W32_MB];
#pragma unroll
  for (int mb = 0; mb < W32_MB; ++mb) {
    const int64_t tok = t0 + 16 * mb + row;
    tok_ok[mb] = tok < n_tok;
    roff[mb] = (tok_ok[mb] ? tok : n_tok - 1) * (int64_t)d;
  }
  const int nchunks = (d + WM_KC - 1) / WM_KC;
  using Raw = IO<float>::Raw;
  Raw hr[W32_MB][2], xr[W32_MB][2];
  auto load_hx = [&](int c) {   // a chunk's h and x rows: every 16-token block, the lane's two k-groups
    const int col = c * WM_KC + quad * WM_QS;
#pragma unroll
    for (int mb = 0; mb < W32_MB; ++mb)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int cc = col + WM_HS * hf < d ? col + WM_HS * hf : 0;
        hr[mb][hf] = IO<float>::raw_str(h + roff[mb] + cc);   // non-temporal, as the 16-bit writes' h
        xr[mb][hf] = IO<float>::raw(x + roff[mb] + cc);
      }
  };
  if (w < nchunks) load_hx(w);
  for (int c = w; c < nchunks; c += 4) {   // wave-uniform trip count
    const int col = c * WM_KC + quad * WM_QS;
    uint4 qv[3][NBA][2];   // the chunk's query parts (cache-resident)
#pragma unroll
    for (int p = 0; p < 3 * (NB > 0); ++p)
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
          qv[p][b][hf] = qt.qt[((((int64_t)c * qt.nbq + qt.b0 + b) * 3 + p) * 2 + hf) * 64 + l];
    uint4 va[W32_MB][2][3];
#pragma unroll
    for (int mb = 0; mb < W32_MB; ++mb)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        float hv[8], xv[8], vv[8];
        IO<float>::unpack(hr[mb][hf], hv);
        IO<float>::unpack(xr[mb][hf], xv);
        const bool ok = tok_ok[mb] && col + WM_HS * hf < d;
#pragma unroll
        for (int k = 0; k < 8; ++k) vv[k] = ok ? hv[k] - xv[k] : 0.f;
#pragma unroll
        for (int k = 0; k < 8; ++k) ss[mb] = __builtin_fmaf(vv[k], vv[k], ss[mb]);   // k_rstd_chunks' order
        split3(vv, va[mb][hf]);
        const int u4 = 2 * (quad + 4 * hf);
        s_v[w][16 * mb + row][u4] = make_float4(vv[0], vv[1], vv[2], vv[3]);
        s_v[w][16 * mb + row][u4 + 1] = make_float4(vv[4], vv[5], vv[6], vv[7]);
      }
    if (c + 4 < nchunks) load_hx(c + 4);   // uniform branch; the registers are free again
    wave_lds_sync();
#pragma unroll
    for (int k = 0; k < W32_TT * (WM_KC / 4) / 64; ++k) {   // 16 lanes per token row
      const int e = l + 64 * k, t = e >> 4, u = e & 15;
      const int64_t tok = t0 + t;
      const int col4 = c * WM_KC + 4 * u;
      const float4 f = s_v[w][t][u];
      // non-temporal: the read that follows streams V[s] with its other sources
      if (tok < n_tok && col4 < d)
        __builtin_nontemporal_store(u32x4{__float_as_uint(f.x), __float_as_uint(f.y), __float_as_uint(f.z),
                                          __float_as_uint(f.w)},
                                    reinterpret_cast<u32x4*>(v + tok * (int64_t)d + col4));
    }
    wave_lds_sync();   // the tile is read before the next chunk overwrites it
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
#pragma unroll
        for (int mb = 0; mb < W32_MB; ++mb)   // a_i q_j, i + j <= 2 (columns past d: zero operands on both sides)
#pragma unroll
          for (int i = 0; i < 3; ++i)
#pragma unroll
            for (int j = 0; j + i < 3; ++j)
              acc[mb][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(va[mb][hf][i]), as_bf16x8(qv[j][b][hf]),
                                                                   acc[mb][b], 0, 0, 0);
  }
#pragma unroll
  for (int mb = 0; mb < W32_MB; ++mb) {
    ss[mb] += __shfl_xor(ss[mb], 16, 64);
    ss[mb] += __shfl_xor(ss[mb], 32, 64);
    if (quad == 0) s_ss[w][mb][row] = ss[mb];
#pragma unroll
    for (int b = 0; b < NB; ++b) s_part[w][mb][b][l] = acc[mb][b];
  }
  __syncthreads();
  if (tid < 16 * W32_MB) {
    const int mb = tid >> 4, rr = tid & 15;
    const float tot = ((s_ss[0][mb][rr] + s_ss[1][mb][rr]) + s_ss[2][mb][rr]) + s_ss[3][mb][rr];
    const int64_t tok = t0 + tid;
    if (tok < n_tok) r[tok] = rsqrtf(tot / (float)d + eps);
  }
  if constexpr (NB > 0) {   // the scores (NB = 0 writes none)
    for (int e = tid; e < W32_MB * NB * 64; e += WG) {
      const int mb = e / (NB * 64), rem = e - mb * NB * 64, b = rem >> 6, ll = rem & 63;
      const f32x4_t sum = ((s_part[0][mb][b][ll] + s_part[1][mb][b][ll]) + s_part[2][mb][b][ll]) + s_part[3][mb][b][ll];
      const int jj = 16 * (qt.b0 + b) + (ll & 15);   // the query; dots points at query j_lo's slice
      if (jj < qt.j_lo || jj >= qt.nq) continue;
      const int64_t tok = t0 + 16 * mb + 4 * (ll >> 4);
      float* dst = dots + (int64_t)(jj - qt.j_lo) * dots_jstride + tok;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (tok + i < n_tok) dst[i] = sum[i];
    }
  }
}

// The fp32 write with whole rows (d a multiple of 256). Per 256-column step each wave moves 8 token rows of h and x,
// a lane two 16-byte pieces of a row 128 columns apart, so each load instruction covers 512 consecutive bytes of
// two rows (k_write_mfma32's layout strides 32 bytes between lanes); V is stored row-major from there and put in an
// LDS tile, from which each wave takes its 64-column chunk of the step in k_write_mfma32's layout. The chunks per
// wave and the order of every sum are k_write_mfma32's, so V, R and the scores are its bits.
template <int NB>   // NB 16-query blocks scored (from block qt.b0); NB = 0: no scores
__global__ __launch_bounds__(WG) void k_write_rows32(const float* __restrict__ h, const float* __restrict__ x,
                                                     float* __restrict__ v, float* __restrict__ r, QTile qt,
                                                     float* __restrict__ dots, int64_t n_tok, int d,
                                                     int64_t dots_jstride, float eps) {
  constexpr int NBA = NB > 0 ? NB : 1;
  constexpr int KS = 4 * WM_KC;   // columns per step
  __shared__ f32x4_t s_part[4][W32_MB][NBA][64];
  __shared__ float s_ss[4][W32_MB][16];
  __shared__ float4 s_a[W32_TT][KS / 4 + 1];   // the step's V tile (a 16-byte pad per row)
  const int tid = (int)threadIdx.x, w = tid >> 6, l = tid & 63, row = l & 15, quad = l >> 4;
  const int64_t t0 = (int64_t)blockIdx.x * W32_TT;
  f32x4_t acc[W32_MB][NBA];
#pragma unroll
  for (int mb = 0; mb < W32_MB; ++mb)
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[mb][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float ss[W32_MB];
#pragma unroll
  for (int mb = 0; mb < W32_MB; ++mb) ss[mb] = 0.f;
  // this lane's rows in the streaming layout: 8 w + 2 i + (l / 32), i < 4; float4 columns l % 32 and 32 + l % 32
  constexpr int RI = W32_TT / 8;
  const int lr = l & 31, lh = l >> 5;
  int64_t rof[RI];
  bool rok[RI];
#pragma unroll
  for (int i = 0; i < RI; ++i) {
    const int64_t tok = t0 + 8 * w + 2 * i + lh;
    rok[i] = tok < n_tok;
    rof[i] = (rok[i] ? tok : n_tok - 1) * (int64_t)d;
  }
  auto load_rows = [&](int st, uint4 (&hr)[RI][2], uint4 (&xr)[RI][2]) {
    const int col = st * KS + lr * 4;
#pragma unroll
    for (int i = 0; i < RI; ++i)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        hr[i][hh] = ld_nt16(h + rof[i] + col + 128 * hh);   // non-temporal: see ld_nt16
        xr[i][hh] = *reinterpret_cast<const uint4*>(x + rof[i] + col + 128 * hh);
      }
  };
  const int nsteps = d / KS;
  uint4 hb[RI][2], xb[RI][2];
  load_rows(0, hb, xb);
  for (int st = 0; st < nsteps; ++st) {
    const int c = 4 * st + w;   // this wave's chunk of the step
    uint4 qv[3][NBA][2];        // its query parts (cache-resident)
#pragma unroll
    for (int p = 0; p < 3 * (NB > 0); ++p)
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
          qv[p][b][hf] = qt.qt[((((int64_t)c * qt.nbq + qt.b0 + b) * 3 + p) * 2 + hf) * 64 + l];
    uint4 hc[RI][2], xc[RI][2];   // this step's rows; the buffer now takes the next step's
#pragma unroll
    for (int i = 0; i < RI; ++i)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) { hc[i][hh] = hb[i][hh]; xc[i][hh] = xb[i][hh]; }
    if (st + 1 < nsteps) load_rows(st + 1, hb, xb);   // uniform branch
#pragma unroll
    for (int i = 0; i < RI; ++i)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const float4 hv = *reinterpret_cast<const float4*>(&hc[i][hh]);
        const float4 xv = *reinterpret_cast<const float4*>(&xc[i][hh]);
        const float4 vv = rok[i] ? make_float4(hv.x - xv.x, hv.y - xv.y, hv.z - xv.z, hv.w - xv.w)
                                 : make_float4(0.f, 0.f, 0.f, 0.f);
        // non-temporal: the read that follows streams V[s] with its other sources
        if (rok[i])
          __builtin_nontemporal_store(u32x4{__float_as_uint(vv.x), __float_as_uint(vv.y), __float_as_uint(vv.z),
                                            __float_as_uint(vv.w)},
                                      reinterpret_cast<u32x4*>(v + rof[i] + st * KS + lr * 4 + 128 * hh));
        s_a[8 * w + 2 * i + lh][lr + 32 * hh] = vv;
      }
    __syncthreads();
    uint4 va[W32_MB][2][3];
#pragma unroll
    for (int mb = 0; mb < W32_MB; ++mb)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int u4 = 16 * w + 2 * quad + 8 * hf;   // k_write_mfma32's columns 8 quad + 32 hf of chunk c
        const float4 a = s_a[16 * mb + row][u4], b = s_a[16 * mb + row][u4 + 1];
        const float vv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int k = 0; k < 8; ++k) ss[mb] = __builtin_fmaf(vv[k], vv[k], ss[mb]);   // k_rstd_chunks' order
        split3(vv, va[mb][hf]);
      }
    __syncthreads();   // the tile is read before the next step overwrites it
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
#pragma unroll
        for (int mb = 0; mb < W32_MB; ++mb)   // a_i q_j, i + j <= 2, in k_write_mfma32's order
#pragma unroll
          for (int i = 0; i < 3; ++i)
#pragma unroll
            for (int j = 0; j + i < 3; ++j)
              acc[mb][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(va[mb][hf][i]), as_bf16x8(qv[j][b][hf]),
                                                                   acc[mb][b], 0, 0, 0);
  }
#pragma unroll
  for (int mb = 0; mb < W32_MB; ++mb) {
    ss[mb] += __shfl_xor(ss[mb], 16, 64);
    ss[mb] += __shfl_xor(ss[mb], 32, 64);
    if (quad == 0) s_ss[w][mb][row] = ss[mb];
#pragma unroll
    for (int b = 0; b < NB; ++b) s_part[w][mb][b][l] = acc[mb][b];
  }
  __syncthreads();
  if (tid < 16 * W32_MB) {
    const int mb = tid >> 4, rr = tid & 15;
    const float tot = ((s_ss[0][mb][rr] + s_ss[1][mb][rr]) + s_ss[2][mb][rr]) + s_ss[3][mb][rr];
    const int64_t tok = t0 + tid;
    if (tok < n_tok) r[tok] = rsqrtf(tot / (float)d + eps);
  }
  if constexpr (NB > 0) {   // the scores (NB = 0 writes none)
    for (int e = tid; e < W32_MB * NB * 64; e += WG) {
      const int mb = e / (NB * 64), rem = e - mb * NB * 64, b = rem >> 6, ll = rem & 63;
      const f32x4_t sum = ((s_part[0][mb][b][ll] + s_part[1][mb][b][ll]) + s_part[2][mb][b][ll]) + s_part[3][mb][b][ll];
      const int jj = 16 * (qt.b0 + b) + (ll & 15);   // the query; dots points at query j_lo's slice
      if (jj < qt.j_lo || jj >= qt.nq) continue;
      const int64_t tok = t0 + 16 * mb + 4 * (ll >> 4);
      float* dst = dots + (int64_t)(jj - qt.j_lo) * dots_jstride + tok;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (tok + i < n_tok) dst[i] = sum[i];
    }
  }
}

// the fp32 write kernel: rows streamed whole when d is whole 256-column steps (LDR_W32_ROWS), else the matrix
// cores' layout; both give the same bits
template <int NB>
auto write32_kernel(bool rows) {
  if constexpr (LDR_W32_ROWS) {
    if (rows) return &k_write_rows32<NB>;
  }
  return &k_write_mfma32<NB>;
}

// the write kernel for bf16 updates: rows streamed whole when d is whole 256-column steps (and the build keeps
// 64-token workgroups), else the matrix cores' layout; both give the same bits
template <typename T, int NB>
auto write_kernel(bool rows) {
  if constexpr (WM_ROWS) {
    if (rows) return &k_write_rows<T, NB>;
  }
  return &k_write_mfma<T, NB>;
}

// the three bf16 parts of fp32 query values, q = hi + mid + lo, into the operand table (QTile's layout)
__global__ __launch_bounds__(WG) void k_split_queries(const float* __restrict__ q, uint4* __restrict__ qt, int nq,
                                                      int d, int nbq, int64_t n_vec) {
  for (int64_t e = (int64_t)blockIdx.x * WG + threadIdx.x; e < n_vec; e += (int64_t)gridDim.x * WG) {
    const int l = (int)(e & 63);
    int64_t rest = e >> 6;
    const int hf = (int)(rest & 1);
    rest >>= 1;
    const int p = (int)(rest % 3);
    rest /= 3;
    const int b = (int)(rest % nbq);
    const int64_t c = rest / nbq;
    const int j = 16 * b + (l & 15);
    const int64_t col0 = c * 64 + 8 * (l >> 4) + 32 * hf;
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 8; k += 2) {
      uint32_t two = 0;
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const int64_t col = col0 + k + kk;
        const float a = (j < nq && col < d) ? q[(int64_t)j * d + col] : 0.f;
        const __bf16 hi = (__bf16)a;
        const float r1 = a - (float)hi;
        const __bf16 mid = (__bf16)r1;
        const __bf16 lo = (__bf16)(r1 - (float)mid);
        const __bf16 part = p == 0 ? hi : (p == 1 ? mid : lo);
        two |= (uint32_t)__builtin_bit_cast(bf16_t, part) << (16 * kk);
      }
      w[k / 2] = two;
    }
    qt[e] = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

inline int64_t query_blocks(int64_t nq) { return (nq + 15) / 16; }
inline int64_t query_chunks(int64_t d) { return (d + 63) / 64; }

// ---------------------------------------------------------------------------------------------------------------
// online scores: out[i][tok] = q . v_i[tok]  (the read without a stored score table)
// ---------------------------------------------------------------------------------------------------------------
template <typename T, int VPT, int C>
__global__ __launch_bounds__(WG) void k_dots(SrcTab src, int n, const float* __restrict__ q, float* __restrict__ out,
                                             int64_t out_stride, int64_t n_tok, int d, int tpr) {
  __shared__ float red[4 * C];
  const Rows R(d, tpr);
  float qv[VPT][8];
#pragma unroll
  for (int v = 0; v < VPT; ++v) {
    const int c8 = R.c8(v);
    if (c8 < R.d8) load_f32x8(q + c8 * 8, qv[v]);
    else {
#pragma unroll
      for (int k = 0; k < 8; ++k) qv[v][k] = 0.f;
    }
  }
  const int64_t groups = (n_tok + R.rpw - 1) / R.rpw;
  for (int64_t gi = blockIdx.x; gi < groups; gi += gridDim.x) {
    const int64_t tok = gi * R.rpw + R.rs;
    const bool valid = tok < n_tok;
    const int64_t roff = (valid ? tok : n_tok - 1) * (int64_t)d;
    int i0 = 0;
    for (; i0 + C <= n; i0 += C) {
      typename IO<T>::Raw raw[C][VPT];
#pragma unroll
      for (int c = 0; c < C; ++c)
#pragma unroll
        for (int v = 0; v < VPT; ++v) raw[c][v] = IO<T>::raw_nt(static_cast<const T*>(src.v[i0 + c]) + roff + R.off(v));
      float pd[C];
#pragma unroll
      for (int c = 0; c < C; ++c) {
        pd[c] = 0.f;
#pragma unroll
        for (int v = 0; v < VPT; ++v) {
          float e[8];
          IO<T>::unpack(raw[c][v], e);
#pragma unroll
          for (int k = 0; k < 8; ++k) pd[c] += qv[v][k] * e[k];
        }
      }
      row_sum<C>(pd, tpr, red);
      if (valid && R.lr == 0) {
#pragma unroll
        for (int c = 0; c < C; ++c) out[(int64_t)(i0 + c) * out_stride + tok] = pd[c];
      }
    }
    for (; i0 < n; ++i0) {
      float pd[1] = {0.f};
#pragma unroll
      for (int v = 0; v < VPT; ++v) {
        float e[8];
        IO<T>::load(static_cast<const T*>(src.v[i0]) + roff + R.off(v), e);
#pragma unroll
        for (int k = 0; k < 8; ++k) pd[0] += qv[v][k] * e[k];
      }
      row_sum<1>(pd, tpr, red);
      if (valid && R.lr == 0) out[(int64_t)i0 * out_stride + tok] = pd[0];
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------
// read forward: softmax weights from the raw scores, then out = base + sum_i w_i v_i in one pass over the sources.
// With STAGE (the tile's output rows fit in LDS: 16 bf16 rows of d = 2048), the rows go to LDS as they finish and
// the tile's consecutive rows are written at its end as one contiguous burst: the read/write turnarounds of the HBM
// come once per tile instead of once per row (a stream probe: 6.3 TB/s with 64 KiB bursts against 5.6 TB/s with
// each row written after its reads).
// ---------------------------------------------------------------------------------------------------------------
// big-tile launch: workgroups of RF_BIG_LANES lanes, tiles of RF_BIG_TT tokens staged in RF_BIG_STAGE bytes
constexpr int RF_BIG_LANES = 512, RF_BIG_TT = 32, RF_BIG_STAGE = 131072;

template <typename T, int VPT, bool BLEND, bool STAGE, int NTH = WG>
__global__ __launch_bounds__(NTH) void k_read_fwd(SrcTab src, int n, const float* __restrict__ dots, int64_t dots_stride,
                                                 const T* __restrict__ base, const T* __restrict__ h0, float beta,
                                                 Coef cf, float inv, T* __restrict__ out, float* __restrict__ tc,
                                                 float* __restrict__ prob, float* __restrict__ next_prior,
                                                 int64_t n_tok, int d, int tpr,
                                                 int tt) {
  // the logits [i][t] during a tile's prologue; with STAGE, then the tile's output rows, written out together at
  // its end (the launch picks STAGE when the tile's rows fit)
  constexpr int STAGE_BYTES = NTH > WG ? RF_BIG_STAGE : RF_STAGE_BYTES;
  constexpr int SL = MAXS * (TT_MAX + 1), SB = STAGE && STAGE_BYTES / 4 > SL ? STAGE_BYTES / 4 : SL;
  __shared__ __align__(16) float s_big[SB];
  float* s_l = s_big;
  __shared__ float s_w[TT_MAX * SP];           // cbar, then the weights [t][i]
  __shared__ float s_c0[MAXS], s_lc[MAXS], s_p0[MAXS], s_M;
  __shared__ gptr_f32 s_rp[MAXS];   // the sources' scale rows (see fetch)
  const Rows R(d, tpr, NTH);
  const int tid = (int)threadIdx.x;
  // A tile's scores, scales and cbar, PRO_K entries per lane at a time: fetch issues a chunk's loads (clamped
  // in-bounds addresses; none is used before all are issued), commit writes the logits and cbar to LDS -- a memory
  // round trip per chunk instead of one per entry. Their lane index is opaque, so the index math is formed in each
  // tile (hoisted out of the tile loop, its registers would stay live through the row stream). A lane's scale
  // addresses come from LDS: read from the kernel's argument table at a per-lane index, each would be a memory
  // round trip of its own before its load.
  const int nt = n * tt;
  float zv[PRO_K], rv[PRO_K], cv[PRO_K];
  auto fetch = [&](int64_t t0, int c) {
    const int lane = opaque(tid) + c;
#pragma unroll
    for (int k = 0; k < PRO_K; ++k) {
      const int idx = min(lane + k * NTH, nt - 1);
      const int i = idx / tt, t = idx - i * tt;                  // source-major: coalesced over tokens
      const int64_t tok = min(t0 + t, n_tok - 1);
      zv[k] = dots[(int64_t)i * dots_stride + tok];
      rv[k] = s_rp[i][tok];
      const int t2 = idx / n, i2 = idx - t2 * n;                 // token-major: coalesced over [tok][i]
      cv[k] = cbar_load(cf, min(t0 + t2, n_tok - 1), i2, dots);
    }
  };
  auto commit = [&](int64_t t0, int c) {
    const int lane = opaque(tid) + c;
#pragma unroll
    for (int k = 0; k < PRO_K; ++k) {
      const int idx = lane + k * NTH;
      if (idx < nt) {
        const int i = idx / tt, t = idx - i * tt;
        float l = s_lc[i];
        if (t0 + t < n_tok) l = zv[k] * rv[k] * inv + s_lc[i];
        s_l[i * (TT_MAX + 1) + t] = l;
        const int t2 = idx / n, i2 = idx - t2 * n;
        s_w[t2 * SP + i2] = t0 + t2 < n_tok ? cbar_value(cf, cv[k], i2) : 0.f;
      }
    }
  };
  const int64_t tiles = (n_tok + tt - 1) / tt;
  load_prior(cf, n, s_c0, s_lc, &s_M, src, s_rp, dots);
  const float M = s_M;
  if (next_prior && blockIdx.x == 0 && tid < n) next_prior[tid] = s_c0[tid];
  const int lpt = NTH / tt;   // lanes per token in the softmax
  const int ns = (n + lpt - 1) / lpt;
  if (tid < lpt) {   // p0 = softmax(lc), a per-read constant: once, by the lanes of one token
    float p0[8];
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const int i = tid + m * lpt;
      p0[m] = (i < n) ? s_lc[i] : -INFINITY;
    }
    softmax_lanes(p0, lpt, ns);
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const int i = tid + m * lpt;
      if (i < n) s_p0[i] = p0[m];
    }
  }
  for (int64_t tile = blockIdx.x; tile < tiles; tile += gridDim.x) {
    const int64_t t0 = tile * tt;
#pragma unroll 1
    for (int c = 0; c < nt; c += PRO_K * NTH) {
      fetch(t0, c);
      commit(t0, c);
    }
    __syncthreads();
    {
      const int t = tid / lpt, j = tid - t * lpt;
      const int64_t tok = t0 + t;
      float ps[8];
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        const int i = j + m * lpt;
        ps[m] = (i < n) ? s_l[i * (TT_MAX + 1) + t] : -INFINITY;
      }
      softmax_lanes(ps, lpt, ns);
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        const int i = j + m * lpt;
        if (i < n) {
          const float tcv = s_c0[i] + M * (ps[m] - s_p0[i]);
          s_w[t * SP + i] = tcv - s_w[t * SP + i];
          if (tok < n_tok) {
            tc[tok * n + i] = tcv;
            if (prob) prob[tok * n + i] = ps[m];   // for the backward only
          }
        }
      }
    }
    __syncthreads();
    for (int rr = R.rs; rr < tt; rr += R.rpw) {
      const int64_t tok = t0 + rr;
      if (tok >= n_tok) break;
      const float* wrow = &s_w[rr * SP];
      const int64_t roff = tok * (int64_t)d;
      constexpr int U = std::is_same<T, float>::value ? LDR_RF_U_F32 : STAGE ? LDR_RF_STAGE_U : LDR_RF_UNROLL;
      using Raw = typename IO<T>::Raw;
      float acc[VPT][8];
#pragma unroll
      for (int v = 0; v < VPT; ++v) IO<T>::load(base + roff + R.off(v), acc[v]);
      if (BLEND) {   // iteration end: base = proposal + beta (h0 - proposal), each step rounded as the caller's ops
#pragma clang fp contract(off)   // three separately rounded operations, as torch runs them (no fused multiply-add)
#pragma unroll
        for (int v = 0; v < VPT; ++v) {
          float hv[8];
          IO<T>::load(h0 + roff + R.off(v), hv);
#pragma unroll
          for (int k = 0; k < 8; ++k)
            acc[v][k] = IO<T>::round(acc[v][k] + IO<T>::round(beta * IO<T>::round(hv[k] - acc[v][k])));
        }
      }
      int i = 0;
      for (; i + U <= n; i += U) {
        Raw raw[U][VPT];
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int v = 0; v < VPT; ++v) raw[u][v] = IO<T>::raw_str(static_cast<const T*>(src.v[i + u]) + roff + R.off(v));
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const float w = wrow[i + u];
#pragma unroll
          for (int v = 0; v < VPT; ++v) {
            float e[8];
            IO<T>::unpack(raw[u][v], e);
#pragma unroll
            for (int k = 0; k < 8; ++k) acc[v][k] += w * e[k];
          }
        }
      }
      // the rest (fewer than U sources) in batches of 4, 2 and 1, each batch's loads in flight together
      auto batch = [&](auto nb_tag) {
        constexpr int NB = decltype(nb_tag)::value;
        Raw raw[NB][VPT];
#pragma unroll
        for (int u = 0; u < NB; ++u)
#pragma unroll
          for (int v = 0; v < VPT; ++v) raw[u][v] = IO<T>::raw_str(static_cast<const T*>(src.v[i + u]) + roff + R.off(v));
        // the loads stay ahead of the sums (the scheduler would otherwise interleave them with the fp16 kernels'
        // mixed-precision multiply-adds, one register set reused, each load then waited for alone)
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < NB; ++u) {
          const float w = wrow[i + u];
#pragma unroll
          for (int v = 0; v < VPT; ++v) {
            float e[8];
            IO<T>::unpack(raw[u][v], e);
#pragma unroll
            for (int k = 0; k < 8; ++k) acc[v][k] += w * e[k];
          }
        }
        i += NB;
      };
      if (U > 4 && i + 4 <= n) batch(std::integral_constant<int, 4>());
      if (U > 2 && i + 2 <= n) batch(std::integral_constant<int, 2>());
      if (i < n) batch(std::integral_constant<int, 1>());
#pragma unroll
      for (int v = 0; v < VPT; ++v)
        if (R.act(v))
          IO<T>::store(STAGE ? reinterpret_cast<T*>(s_big) + rr * d + R.c8(v) * 8 : out + roff + R.c8(v) * 8, acc[v]);
    }
    if (STAGE) {   // the tile's rows are consecutive tokens: one contiguous region, written in one burst
      __syncthreads();
      const int64_t rows = (int64_t)tt < n_tok - t0 ? (int64_t)tt : n_tok - t0;
      const int64_t nv = rows * d * (int64_t)sizeof(T) / 16;
      const uint4* src4 = reinterpret_cast<const uint4*>(s_big);
      uint4* dst4 = reinterpret_cast<uint4*>(out + t0 * (int64_t)d);
      for (int64_t e = tid; e < nv; e += NTH) dst4[e] = src4[e];
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------------------------------------------
// read forward with online scores in one pass over the sources (rows inside one wave, tpr <= 64). Per token row and
// source i: the raw score q . v_i (row sum), the logit l_i = score r_i inv + lc_i, and an online softmax against a
// reference maximum m that moves only when a logit passes it by more than RF_LAZY (the running sums are then
// rescaled): S = sum_i e_i and P = sum_i e_i v_i with e_i = exp(l_i - m), beside
// acc = base + sum_i (c0_i - cbar_i - M p0_i) v_i (p0 = softmax(lc) is a per-read constant); at the row's end
// out = acc + (M / S) P = base + sum_i (tc_i - cbar_i) v_i. A zero query is the exact case p = p0: the weights are
// then c0_i - cbar_i and P is not formed, so a zero query with cbar == c0 gives out == base bitwise. tc and p come
// from the row's logits at its end (the softmax of the stored-score read, so equal logits give tc == c0 bitwise);
// the raw scores are stored for the backward.
// ---------------------------------------------------------------------------------------------------------------
constexpr float RF_LAZY = 8.f;   // e^8 < 3000: the running sums stay far from overflow between rescales

template <typename T, int VPT, bool BLEND, int PD>
__global__ __launch_bounds__(WG) __attribute__((amdgpu_waves_per_eu(LDR_ON_WAVES)))
void k_read_online(SrcTab src, int n, const float* __restrict__ q, float* __restrict__ dots, int64_t dots_stride,
                   const T* __restrict__ base, const T* __restrict__ h0, float beta, Coef cf, float inv,
                   T* __restrict__ out, float* __restrict__ tc, float* __restrict__ prob,
                   float* __restrict__ next_prior, int64_t n_tok, int d, int tpr) {
  __shared__ float s_lg[WG / 8][MAXS];   // each row's logits (rows have at least 8 lanes)
  __shared__ float s_wt[WG / 8][MAXS];   // each row's fixed weights
  __shared__ float s_rs[WG / 8][MAXS];   // each row's source scales
  __shared__ float s_c0[MAXS], s_lc[MAXS], s_p0[MAXS], s_M;
  __shared__ __align__(16) float s_q[64 * 4 * 8];   // the query, zero past d (rows of <= 64 lanes x 4 vectors)
  __shared__ int s_qnz;
  __shared__ gptr_f32 s_rp[MAXS];   // the sources' scale rows, as in the read forward's prologue
  using Raw = typename IO<T>::Raw;
  const Rows R(d, tpr);
  const int tid = (int)threadIdx.x;
  if (tid == 0) s_qnz = 0;
  load_prior(cf, n, s_c0, s_lc, &s_M, src, s_rp, q);   // barriers inside: s_qnz is cleared before anyone sets it
  const float M = s_M;
  if (next_prior && blockIdx.x == 0 && tid < n) next_prior[tid] = s_c0[tid];
  bool nz = false;
  float qk[64 * 4 * 8 / WG];   // every load out before the first is used (at a clamped column, the value then zeroed)
#pragma unroll
  for (int j = 0; j < 64 * 4 * 8 / WG; ++j) qk[j] = q[min(tid + j * WG, d - 1)];
#pragma unroll
  for (int j = 0; j < 64 * 4 * 8 / WG; ++j) {
    const int k = tid + j * WG;
    const float x = k < d ? qk[j] : 0.f;
    s_q[k] = x;
    nz |= x != 0.f;
  }
  if (nz) s_qnz = 1;   // every writer stores the same value
  const int ns = (n + tpr - 1) / tpr;
  if (R.rs == 0) {     // p0 = softmax(lc), a per-read constant: once, by the lanes of one row
    float p0[8];
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const int i = R.lr + m * tpr;
      p0[m] = i < n ? s_lc[i] : -INFINITY;
    }
    softmax_lanes(p0, tpr, ns);
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const int i = R.lr + m * tpr;
      if (i < n) s_p0[i] = p0[m];
    }
  }
  __syncthreads();
  const bool qz = s_qnz == 0;   // workgroup-uniform
  float* lg = s_lg[R.rs];
  float* wt = s_wt[R.rs];
  float* rsc = s_rs[R.rs];
  const int64_t groups = (n_tok + R.rpw - 1) / R.rpw;
  for (int64_t gi = blockIdx.x; gi < groups; gi += gridDim.x) {
    const int64_t tok = gi * R.rpw + R.rs;
    const bool valid = tok < n_tok;
    const int64_t tk = valid ? tok : n_tok - 1;   // rows past the end recompute the last token, store nothing
    const int64_t roff = tk * (int64_t)d;
    auto load_src = [&](int i, Raw (&rw)[VPT]) {
#pragma unroll
      for (int v = 0; v < VPT; ++v) rw[v] = IO<T>::raw_str(static_cast<const T*>(src.v[i]) + roff + R.off(v));
    };
    // the row's first sources and its base are requested before its scalars, so one memory round trip brings all
    // three (the scalars first were two: theirs, then the rows')
    Raw buf[PD][VPT];   // a ring of PD sources in flight: source i lives in buf[i % PD]
#pragma unroll
    for (int j = 0; j < PD; ++j)
      if (j < n) load_src(j, buf[j]);
    Raw braw[VPT];
#pragma unroll
    for (int v = 0; v < VPT; ++v) braw[v] = IO<T>::raw(base + roff + R.off(v));
    for (int i = R.lr; i < n; i += tpr) {           // the row's per-source scalars, spread over its lanes
      const float cb = cbar_value(cf, cbar_load(cf, tk, i, q), i);   // both loads out before either is used
      const float rv = s_rp[i][tk];
      wt[i] = qz ? s_c0[i] - cb : (s_c0[i] - cb) - M * s_p0[i];
      rsc[i] = rv;
    }
    float acc[VPT][8], P[VPT][8];
#pragma unroll
    for (int v = 0; v < VPT; ++v) IO<T>::unpack(braw[v], acc[v]);
    if (BLEND) {   // iteration end: base = proposal + beta (h0 - proposal), each step rounded as the caller's ops
#pragma clang fp contract(off)   // three separately rounded operations, as torch runs them (no fused multiply-add)
#pragma unroll
      for (int v = 0; v < VPT; ++v) {
        float hv[8];
        IO<T>::load(h0 + roff + R.off(v), hv);
#pragma unroll
        for (int k = 0; k < 8; ++k)
          acc[v][k] = IO<T>::round(acc[v][k] + IO<T>::round(beta * IO<T>::round(hv[k] - acc[v][k])));
      }
    }
#pragma unroll
    for (int v = 0; v < VPT; ++v)
#pragma unroll
      for (int k = 0; k < 8; ++k) P[v][k] = 0.f;
    float S = 0.f, mref = -INFINITY;
    wave_lds_sync();
    auto dotq = [&](const Raw (&rw)[VPT]) {   // the query slice comes from LDS (no registers held for it)
      asm volatile("" ::: "memory");           // read here, not hoisted out of the source loop into registers
      float a = 0.f;
#pragma unroll
      for (int v = 0; v < VPT; ++v) {
        float e[8], qx[8];
        IO<T>::unpack(rw[v], e);
        const float4* qp = reinterpret_cast<const float4*>(s_q + R.c8(v) * 8);
        const float4 q0 = qp[0], q1 = qp[1];
        qx[0] = q0.x; qx[1] = q0.y; qx[2] = q0.z; qx[3] = q0.w;
        qx[4] = q1.x; qx[5] = q1.y; qx[6] = q1.z; qx[7] = q1.w;
#pragma unroll
        for (int k = 0; k < 8; ++k) a += qx[k] * e[k];
      }
      return a;
    };
    // one source once its raw score is known: the logit, the online sums, the fixed-weight sum
    auto take = [&](int i, float score, const Raw (&rw)[VPT]) {
      const float l = score * rsc[i] * inv + s_lc[i];
      if (R.lr == 0) {
        lg[i] = l;
        if (valid) dots[(int64_t)i * dots_stride + tok] = score;
      }
      float ex = 0.f;
      if (!qz) {
        if (l > mref + RF_LAZY) {   // first source (mref = -inf: a = 0 on zero sums), or a far larger logit
          const float a = expf(mref - l);
          S *= a;
#pragma unroll
          for (int v = 0; v < VPT; ++v)
#pragma unroll
            for (int k = 0; k < 8; ++k) P[v][k] *= a;
          mref = l;
        }
        ex = expf(l - mref);
        S += ex;
      }
      const float w = wt[i];
#pragma unroll
      for (int v = 0; v < VPT; ++v) {
        float e[8];
        IO<T>::unpack(rw[v], e);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          if (!qz) P[v][k] += ex * e[k];
          acc[v][k] += w * e[k];
        }
      }
    };
    auto one = [&](int i, Raw (&rw)[VPT]) {   // source i, then its slot refilled with source i + PD
      float pd[1] = {dotq(rw)};
      row_sum<1>(pd, tpr, nullptr);
      take(i, pd[0], rw);
      if (i + PD < n) load_src(i + PD, rw);
    };
    int i0 = 0;
    for (; i0 + PD <= n; i0 += PD) {
#pragma unroll
      for (int j = 0; j < PD; ++j) one(i0 + j, buf[j]);
    }
#pragma unroll
    for (int j = 0; j < PD; ++j)
      if (i0 + j < n) one(i0 + j, buf[j]);
    if (!qz) {
      const float f = M / S;
#pragma unroll
      for (int v = 0; v < VPT; ++v)
#pragma unroll
        for (int k = 0; k < 8; ++k) acc[v][k] += f * P[v][k];
    }
    if (valid) {
#pragma unroll
      for (int v = 0; v < VPT; ++v)
        if (R.act(v)) IO<T>::store(out + roff + R.c8(v) * 8, acc[v]);
    }
    wave_lds_sync();
    float ps[8];
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const int i = R.lr + m * tpr;
      ps[m] = i < n ? lg[i] : -INFINITY;
    }
    softmax_lanes(ps, tpr, ns);
    if (valid) {
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        const int i = R.lr + m * tpr;
        if (i < n) {
          tc[tok * n + i] = s_c0[i] + M * (ps[m] - s_p0[i]);
          if (prob) prob[tok * n + i] = ps[m];   // for the backward only
        }
      }
    }
    wave_lds_sync();   // this row's scalars are read before the next row overwrites them
  }
}

// ---------------------------------------------------------------------------------------------------------------
// backward pass 1: the only re-read of the sources
// ---------------------------------------------------------------------------------------------------------------
constexpr int B1_GRID = LDR_B1_GRID;
constexpr int B1_MAX_VPT = LDR_B1_MAX_VPT;

// two waves per SIMD (two workgroups per CU): the fp32 rows' instantiations need it said (else 254 registers and 16
// accumulation registers, one workgroup per CU; with it 256 and 60 bytes of scratch: 14.07 -> 14.01 ms per pass at
// config 4); the 16-bit ones fit it anyway
template <typename T, int VPT, int C>
__global__ __launch_bounds__(WG) __attribute__((amdgpu_waves_per_eu(2))) void k_bwd1(SrcTab src, int n, const T* __restrict__ g, const float* __restrict__ gt,
                                             const float* __restrict__ prob, const float* __restrict__ dots,
                                             int64_t dots_stride, const float* __restrict__ tcp, Coef cf, float inv,
                                             float* __restrict__ dcbar, int dcbar_cols, PtrTab dr, int dr_accum,
                                             float* __restrict__ wz, int64_t wz_stride, float* __restrict__ dq_part,
                                             int64_t dq_stride,
                                             T* __restrict__ g_prop, T* __restrict__ g_h0, float beta, int64_t n_tok,
                                             int d, int tpr, int tt) {
  // LDS: six [TT_MAX][SP] scalar planes (probability, scale, upstream tc gradient, g.v, raw score then dr, and
  // tc - cbar) during the tiles; the first d floats are reused for the workgroup's dq sum at the end.
  // fp32 updates: g . v_i summed in fp64 (each product rounded to fp32, the d-term sum and the lane reduction in
  // fp64; the products exact would take the registers of a second wave) and gp, Sacc formed from it in fp64. The
  // query gradient of a chain's last reads sums p (gp_i - Sacc) r v over every token, and the fp32 sum of g . v was
  // the largest error left in it at the headline shape in fp32 (1.05e-5 of its RMS; 6.2e-6 with this, 3.6e-6 with
  // the row-local sums below).
  constexpr bool GD64 = LDR_B1_GD64 && std::is_same<T, float>::value;
  typedef typename std::conditional<GD64, double, float>::type Acc;
  __shared__ float lds[6 * TT_MAX * SP];
  __shared__ float s_sacc[TT_MAX], s_c0[MAXS], s_lc[MAXS], s_M;
  __shared__ gptr_f32 s_rp[MAXS];   // the sources' scale rows, as in the read forward's prologue
  __shared__ gptr_f32w s_drp[MAXS]; // the sources' dr rows (the same: no argument-table read per entry)
  __shared__ Acc red[4 * C];
  float* s_p = lds;
  float* s_r = lds + 1 * TT_MAX * SP;
  float* s_gt = lds + 2 * TT_MAX * SP;
  float* s_gd = lds + 3 * TT_MAX * SP;
  float* s_dz = lds + 4 * TT_MAX * SP;
  float* s_w = lds + 5 * TT_MAX * SP;
  const Rows R(d, tpr);
  const int tid = (int)threadIdx.x;
  // A tile's per-token scalars, PRO_K entries per lane at a time: fetch issues a chunk's loads (clamped in-bounds
  // addresses; none is used before all are issued), commit writes them to LDS -- a memory round trip per chunk
  // instead of one per entry (the lane index opaque, as in the read forward).
  const int nt = n * tt;
  float pv[PRO_K], gv[PRO_K], wv[PRO_K], cv[PRO_K], rv[PRO_K], zv[PRO_K];
  const float* gtp = gt ? gt : prob;   // without gt: prob's entries loaded and not used (a load under no condition)
  auto fetch = [&](int64_t t0, int c) {
    const int lane = opaque(tid) + c;
#pragma unroll
    for (int k = 0; k < PRO_K; ++k) {
      const int idx = min(lane + k * WG, nt - 1);
      const int t = idx / n, i = idx - t * n;                    // token-major: [tok][i]
      const int64_t tok = min(t0 + t, n_tok - 1);
      pv[k] = prob[tok * n + i];
      gv[k] = gtp[tok * n + i];
      wv[k] = tcp[tok * n + i];
      cv[k] = cbar_load(cf, tok, i, tcp);
      const int i2 = idx / tt, t2 = idx - i2 * tt;               // source-major: scales and raw scores
      const int64_t tok2 = min(t0 + t2, n_tok - 1);
      rv[k] = s_rp[i2][tok2];
      zv[k] = dots[i2 * dots_stride + tok2];
    }
  };
  auto commit = [&](int64_t t0, int c) {
    const int lane = opaque(tid) + c;
#pragma unroll
    for (int k = 0; k < PRO_K; ++k) {
      const int idx = lane + k * WG;
      if (idx < nt) {
        const int t = idx / n, i = idx - t * n;
        const bool ok = t0 + t < n_tok;
        s_p[t * SP + i] = ok ? pv[k] : 0.f;
        s_gt[t * SP + i] = ok && gt ? gv[k] : 0.f;
        s_w[t * SP + i] = ok ? wv[k] - cbar_value(cf, cv[k], i) : 0.f;
        const int i2 = idx / tt, t2 = idx - i2 * tt;
        const bool ok2 = t0 + t2 < n_tok;
        s_r[t2 * SP + i2] = ok2 ? rv[k] : 1.f;
        s_dz[t2 * SP + i2] = ok2 ? zv[k] : 0.f;                  // q . v_i until the epilogue
      }
    }
  };
  const int64_t tiles = (n_tok + tt - 1) / tt;
  load_prior(cf, n, s_c0, s_lc, &s_M, src, s_rp, tcp, &dr, s_drp);
  const float M = s_M;
  float dqa[VPT][8];
#pragma unroll
  for (int v = 0; v < VPT; ++v)
#pragma unroll
    for (int k = 0; k < 8; ++k) dqa[v][k] = 0.f;
  const int nfull = (n - LDR_B1_KEEP_LAST) - (n - LDR_B1_KEEP_LAST) % C;   // sources in whole chunks
  const int rows_per_slot = (tt + R.rpw - 1) / R.rpw;
  typename IO<T>::Raw gq[VPT];     // the row's g, kept packed (fewer registers), unpacked where used
  typename IO<T>::Raw cur[C][VPT];  // the row's chunk of sources being reduced
  auto load_chunk = [&](int64_t roff, int i0, typename IO<T>::Raw (&rw)[C][VPT]) {
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
      for (int v = 0; v < VPT; ++v) rw[c][v] = IO<T>::raw_nt(static_cast<const T*>(src.v[i0 + c]) + roff + R.off(v));
  };
  // a row's first loads: its g and its first chunk of sources
  auto start_row = [&](int64_t t0, int rk) {
    const int64_t tok = t0 + R.rs + rk * R.rpw;
    const int64_t roff = (tok < n_tok ? tok : n_tok - 1) * (int64_t)d;
#pragma unroll
    for (int v = 0; v < VPT; ++v) {
      gq[v] = IO<T>::raw(g + roff + R.off(v));   // just written by the caller: cached, not streamed
      if (!R.act(v)) gq[v] = IO<T>::zero();
    }
    if (nfull > 0) load_chunk(roff, 0, cur);
  };
  for (int64_t tile = blockIdx.x; tile < tiles; tile += gridDim.x) {
    const int64_t t0 = tile * tt;
    // the tile's first row is requested after the prologue's first loads and before they are waited for (waiting
    // for older loads does not wait for younger ones), so the prologue's round trip overlaps the row stream's start
    fetch(t0, 0);
    start_row(t0, 0);
    commit(t0, 0);
#pragma unroll 1
    for (int c = PRO_K * WG; c < nt; c += PRO_K * WG) {
      fetch(t0, c);
      commit(t0, c);
    }
    __syncthreads();
    for (int rk = 0; rk < rows_per_slot; ++rk) {   // uniform trip count: row_sum may hold barriers
      const int rr = R.rs + rk * R.rpw;            // < tt: tt is a multiple of rpw
      const int64_t tok = t0 + rr;
      const bool valid = tok < n_tok;
      const int64_t roff = (valid ? tok : n_tok - 1) * (int64_t)d;
      if (rk > 0) start_row(t0, rk);
      if ((g_prop || g_h0) && valid) {   // the blend's gradients: beta g to h0, g - beta g to the proposal
#pragma clang fp contract(off)   // a product and a difference, each rounded as autograd rounds them (no fma)
#pragma unroll
        for (int v = 0; v < VPT; ++v) {
          if (!R.act(v)) continue;
          float gb[8], gpv[8];
          float gvv[8];
          IO<T>::unpack(gq[v], gvv);
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            gb[k] = IO<T>::round(beta * gvv[k]);
            gpv[k] = gvv[k] - gb[k];
          }
          if (g_h0) IO<T>::store(g_h0 + roff + R.c8(v) * 8, gb);
          if (g_prop) IO<T>::store(g_prop + roff + R.c8(v) * 8, gpv);
        }
      }
      // dq of the row is sum_i p_i r_i (gp_i - Sacc) v_i, with Sacc known only after the last source: the row's
      // a = sum_i p_i r_i gp_i v_i and b = sum_i p_i r_i v_i, then a - Sacc b joins the running dq. The two terms
      // largely cancel, so they meet in the row's own registers before the (much longer) running sum takes the
      // difference: adding a to the running dq directly and subtracting Sacc b there was measured to leave twice
      // the fp32 error in the headline chain's query gradient.
      float a[VPT][8], b[VPT][8];
#pragma unroll
      for (int v = 0; v < VPT; ++v)
#pragma unroll
        for (int k = 0; k < 8; ++k) a[v][k] = b[v][k] = 0.f;
      Acc sacc = 0;
      // one source's share once its g.v is known: the scalars, the two accumulators, g.v to LDS
      auto take = [&](int i, Acc gd, const typename IO<T>::Raw (&rw)[VPT]) {
        const float p = s_p[rr * SP + i];
        const float pr = p * s_r[rr * SP + i];
        const Acc gp = (Acc)M * (gd + (Acc)s_gt[rr * SP + i]);
        sacc += (Acc)p * gp;
        const float alpha = (float)((Acc)pr * gp);
#pragma unroll
        for (int v = 0; v < VPT; ++v) {
          float e[8];
          IO<T>::unpack(rw[v], e);
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            a[v][k] += alpha * e[k];
            b[v][k] += pr * e[k];
          }
        }
        if (R.lr == 0) s_gd[rr * SP + i] = (float)gd;
      };
      auto dotc = [&](const typename IO<T>::Raw (&rw)[VPT]) {
        Acc acc = 0;
#pragma unroll
        for (int v = 0; v < VPT; ++v) {
          float e[8];
          IO<T>::unpack(rw[v], e);
          float gvv[8];
          IO<T>::unpack(gq[v], gvv);
#pragma unroll
          for (int k = 0; k < 8; ++k) acc += (Acc)(gvv[k] * e[k]);
        }
        return acc;
      };
      auto rsum = [&](auto& pd) {
        if constexpr (GD64)
          row_sum_d(pd, tpr, red);
        else
          row_sum(pd, tpr, red);
      };
      int i0 = 0;
      for (; i0 < nfull; i0 += C) {   // the next chunk's loads in flight while this one is reduced
        typename IO<T>::Raw nxt[C][VPT];
        if (i0 + C < nfull) load_chunk(roff, i0 + C, nxt);
        Acc pd[C];
#pragma unroll
        for (int c = 0; c < C; ++c) pd[c] = dotc(cur[c]);
        rsum(pd);
        if (valid) {
#pragma unroll
          for (int c = 0; c < C; ++c) take(i0 + c, pd[c], cur[c]);
        }
#pragma unroll
        for (int c = 0; c < C; ++c)
#pragma unroll
          for (int v = 0; v < VPT; ++v) cur[c][v] = nxt[c][v];
      }
      for (; i0 < n; ++i0) {
        typename IO<T>::Raw raw[1][VPT];
        // the newest source, through the caches: the update gradient of that source runs next and reads it again,
        // and the 256 MB last-level cache keeps it there while the non-temporal stream of the others passes
        // (c4: the update gradients 6.70 -> 6.43 ms per pass, backward pass 1 +0.05 ms)
        if (LDR_B1_KEEP_LAST && i0 == n - 1) {
#pragma unroll
          for (int v = 0; v < VPT; ++v) raw[0][v] = IO<T>::raw(static_cast<const T*>(src.v[i0]) + roff + R.off(v));
        } else {
#pragma unroll
          for (int v = 0; v < VPT; ++v) raw[0][v] = IO<T>::raw_nt(static_cast<const T*>(src.v[i0]) + roff + R.off(v));
        }
        Acc pd[1] = {dotc(raw[0])};
        rsum(pd);
        if (valid) take(i0, pd[0], raw[0]);
      }
      if (valid) {
        const float sf = (float)sacc;
#pragma unroll
        for (int v = 0; v < VPT; ++v)
#pragma unroll
          for (int k = 0; k < 8; ++k) dqa[v][k] += a[v][k] - sf * b[v][k];
        if (R.lr == 0) s_sacc[rr] = sf;
      }
    }
    __syncthreads();
    for (int idx = tid; idx < n * tt; idx += WG) {   // token-major: dcbar, dz
      const int t = idx / n, i = idx - t * n;
      const int64_t tok = t0 + t;
      if (tok < n_tok) {
        const float gd = s_gd[t * SP + i];
        const float gp = M * (gd + s_gt[t * SP + i]);
        const float dz = s_p[t * SP + i] * (gp - s_sacc[t]);
        if (i < dcbar_cols) dcbar[tok * dcbar_cols + i] = -(cf.lam * gd);
        s_dz[t * SP + i] = dz * s_dz[t * SP + i] * inv;   // dr = dz z / r = dz (q . v) / sqrt(d)
        s_gd[t * SP + i] = dz;
      }
    }
    __syncthreads();
    for (int idx = tid; idx < n * tt; idx += WG) {   // source-major: dr, wz
      const int i = idx / tt, t = idx - i * tt;
      const int64_t tok = t0 + t;
      if (tok < n_tok) {
        const gptr_f32w dri = s_drp[i];
        const float drv = s_dz[t * SP + i];
        dri[tok] = dr_accum ? dri[tok] + drv : drv;
        const float dz = s_gd[t * SP + i];
        *reinterpret_cast<float2*>(wz + 2 * ((int64_t)i * wz_stride + tok)) =
            make_float2(s_w[t * SP + i], dz * s_r[t * SP + i] * inv);
      }
    }
    __syncthreads();
  }
  // the workgroup's dq: row slots add their columns in a fixed order
  float* s_dq = lds;
  for (int k = 0; k < R.rpw; ++k) {
    if (R.rs == k) {
#pragma unroll
      for (int v = 0; v < VPT; ++v) {
        const int c8 = R.c8(v);
        if (c8 < R.d8) {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float val = dqa[v][e] * inv;
            s_dq[c8 * 8 + e] = (k == 0) ? val : s_dq[c8 * 8 + e] + val;
          }
        }
      }
    }
    __syncthreads();
  }
  for (int c = tid; c < d; c += WG) dq_part[(int64_t)blockIdx.x * dq_stride + c] = s_dq[c];
}

// out[c] = sum_p part[p][c]: 16 columns per workgroup, 16 row groups (rows p = group mod 16) added in a fixed order
// out = round(sum_j round(beta * g_j)): the iteration-end blends' shares of h0's gradient, summed once in fp32;
// per_read: each share added in T (rounded after every addition), in table order, as autograd adds them
template <typename T, int VPT>
__global__ __launch_bounds__(WG) void k_blend_sum(PtrTab g, int m, float beta, int per_read, T* __restrict__ out,
                                                  int64_t n_tok, int d, int tpr) {
#pragma clang fp contract(off)
  const Rows R(d, tpr);
  const int64_t groups = (n_tok + R.rpw - 1) / R.rpw;
  for (int64_t gi = blockIdx.x; gi < groups; gi += gridDim.x) {
    const int64_t tok = gi * R.rpw + R.rs;
    const int64_t roff = (tok < n_tok ? tok : n_tok - 1) * (int64_t)d;
    float acc[VPT][8];
#pragma unroll
    for (int v = 0; v < VPT; ++v)
#pragma unroll
      for (int x = 0; x < 8; ++x) acc[v][x] = 0.f;
    for (int j = 0; j < m; ++j) {
      float e[VPT][8];
#pragma unroll
      for (int v = 0; v < VPT; ++v) IO<T>::unpack(IO<T>::raw_nt(static_cast<const T*>(g.p[j]) + roff + R.off(v)), e[v]);
#pragma unroll
      for (int v = 0; v < VPT; ++v)
#pragma unroll
        for (int x = 0; x < 8; ++x) {
          const float t = IO<T>::round(beta * e[v][x]);
          acc[v][x] = !per_read ? acc[v][x] + t : (j == 0 ? t : IO<T>::round(acc[v][x] + t));
        }
    }
    if (tok < n_tok) {
#pragma unroll
      for (int v = 0; v < VPT; ++v)
        if (R.act(v)) IO<T>::store(out + roff + R.c8(v) * 8, acc[v]);
    }
  }
}

__global__ __launch_bounds__(WG) void k_reduce_rows(const float* __restrict__ part, int64_t rows, int d,
                                                    float* __restrict__ out) {
  __shared__ float s[WG];
  const int tid = (int)threadIdx.x, cl = tid & 15, grp = tid >> 4;
  const int c = blockIdx.x * 16 + cl;
  float acc = 0.f;
  if (c < d) {
    int64_t p = grp;
    for (; p + 7 * 16 < rows; p += 8 * 16) {
      float a[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) a[u] = part[(p + 16 * u) * d + c];
#pragma unroll
      for (int u = 0; u < 8; ++u) acc += a[u];
    }
    for (; p < rows; p += 16) acc += part[p * d + c];
  }
  s[tid] = acc;
  __syncthreads();
  if (grp == 0 && c < d) {
    float t = s[cl];
    for (int k = 1; k < 16; ++k) t += s[k * 16 + cl];
    out[c] = t;
  }
}

// One read's share of a source's gradient, w g + dzr q, with one explicit fused multiply-add (the product dzr q
// rounded first): the list layout's per-read term, and the stacked layout's when it rounds per read.
__device__ __forceinline__ float bwd2_term(float w, float g, float dzr, float q) { return __builtin_fmaf(w, g, dzr * q); }

// ---------------------------------------------------------------------------------------------------------------
// backward pass 2, list layout: dv_i (=|+=) w_i g + dzr_i q
// ---------------------------------------------------------------------------------------------------------------
template <typename T, int VPT>
__global__ __launch_bounds__(WG) void k_bwd2_list(PtrTab dv, int n, int accum, const T* __restrict__ g,
                                                  const float* __restrict__ q, const float* __restrict__ wz,
                                                  int64_t wz_stride, int64_t n_tok, int d, int tpr) {
  const Rows R(d, tpr);
  float qv[VPT][8];
#pragma unroll
  for (int v = 0; v < VPT; ++v) load_f32x8(q + R.off(v), qv[v]);
  const int64_t groups = (n_tok + R.rpw - 1) / R.rpw;
  for (int64_t gi = blockIdx.x; gi < groups; gi += gridDim.x) {
    const int64_t tok = gi * R.rpw + R.rs;
    if (tok >= n_tok) continue;
    const int64_t roff = tok * (int64_t)d;
    float gv[VPT][8];
#pragma unroll
    for (int v = 0; v < VPT; ++v) IO<T>::load(g + roff + R.off(v), gv[v]);
    for (int i = 0; i < n; ++i) {
      const float2 s = *reinterpret_cast<const float2*>(wz + 2 * ((int64_t)i * wz_stride + tok));
      T* dvi = static_cast<T*>(dv.p[i]) + roff;
      float prev[VPT][8];
      if (accum) {
#pragma unroll
        for (int v = 0; v < VPT; ++v) IO<T>::load(dvi + R.off(v), prev[v]);
      }
#pragma unroll
      for (int v = 0; v < VPT; ++v) {
        float o[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) o[k] = bwd2_term(s.x, gv[v][k], s.y, qv[v][k]);
        if (accum) {
#pragma unroll
          for (int k = 0; k < 8; ++k) o[k] = prev[v][k] + IO<T>::round(o[k]);
        }
        if (R.act(v)) IO<T>::store(dvi + R.c8(v) * 8, o);
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------
// stacked layout: the finished gradient of one update from every read that held it, plus its scale's term
// ---------------------------------------------------------------------------------------------------------------
// token rows per lane, sharing each query load (fewer when the lane holds 3+ vectors of a row: registers)
constexpr int as_rb(int vpt, bool f32 = false) { return vpt >= 3 ? (f32 ? LDR_AS_RB_F32 : 2) : LDR_AS_RB; }
// reads per batch of loads: fp32 rows two (c4 fp32: the update gradients 16.0 -> 14.8 ms per pass, with one wave per
// row; either setting takes bf16's from 6.4 to 7.0-7.8 ms)
template <typename T> constexpr int as_jb() { return std::is_same<T, float>::value ? LDR_AS_JB_F32 : LDR_AS_JB; }

// ADD_LAST: add is the output gradient of the last read in tab. PER_READ: each read's share rounded to T and added
// to the running gradient in T, in table order, then the scale's term rounded and added -- the roundings of the list
// layout, whose per-read gradients autograd adds in backward order (the host orders the table so) -- instead of one
// fp32 sum rounded once.
template <typename T, int VPT, bool ADD_LAST, bool PER_READ>
__global__ __launch_bounds__(WG) void k_dv_assemble(AsmTab tab, int m, const T* __restrict__ vsrc,
                                                    const float* __restrict__ r, const float* __restrict__ gr,
                                                    const T* __restrict__ add, float add_beta,
                                                    T* __restrict__ dv, T* __restrict__ dv_neg, int64_t n_tok, int d,
                                                    int tpr) {
  constexpr int AS_RB = as_rb(VPT, std::is_same<T, float>::value);
  const Rows R(d, tpr);
  const int64_t rows_per_tile = (int64_t)R.rpw * AS_RB;
  const int64_t tiles = (n_tok + rows_per_tile - 1) / rows_per_tile;
  for (int64_t tile = blockIdx.x; tile < tiles; tile += gridDim.x) {
    int64_t tok[AS_RB], tokc[AS_RB], roff[AS_RB];
#pragma unroll
    for (int k = 0; k < AS_RB; ++k) {
      tok[k] = tile * rows_per_tile + R.rs + (int64_t)k * R.rpw;
      tokc[k] = tok[k] < n_tok ? tok[k] : n_tok - 1;
      roff[k] = tokc[k] * (int64_t)d;
    }
    float acc[AS_RB][VPT][8];
#pragma unroll
    for (int k = 0; k < AS_RB; ++k)
#pragma unroll
      for (int v = 0; v < VPT; ++v)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[k][v][e] = 0.f;
    // one read's share: w g + dzr q for the tile's rows, as two explicit fused multiply-adds (so every kernel
    // variant and every read accumulate with the same roundings, whatever the compiler would contract)
    int taken = 0;   // reads added so far (PER_READ: the first share is the running gradient itself)
    auto take_row = [&](const typename IO<T>::Raw (&raw)[AS_RB][VPT], const float2 (&sc)[AS_RB],
                        const float (&qv)[VPT][8]) {
#pragma unroll
      for (int k = 0; k < AS_RB; ++k)
#pragma unroll
        for (int v = 0; v < VPT; ++v) {
          float e[8];
          IO<T>::unpack(raw[k][v], e);
#pragma unroll
          for (int x = 0; x < 8; ++x) {
            if (PER_READ) {
              const float t = IO<T>::round(bwd2_term(sc[k].x, e[x], sc[k].y, qv[v][x]));
              acc[k][v][x] = taken == 0 ? t : IO<T>::round(acc[k][v][x] + t);
            } else {
              acc[k][v][x] = __builtin_fmaf(sc[k].y, qv[v][x], __builtin_fmaf(sc[k].x, e[x], acc[k][v][x]));
            }
          }
        }
      ++taken;
    };
    // JB reads per batch: their g rows (and query columns) are all in flight before the first multiply-add
    auto batch = [&](int j0, auto jb_tag) {
      constexpr int JB = decltype(jb_tag)::value;
      typename IO<T>::Raw raw[JB][AS_RB][VPT];
      float2 sc[JB][AS_RB];
      float qv[JB][VPT][8];
#pragma unroll
      for (int b = 0; b < JB; ++b) {
        const T* gj = static_cast<const T*>(tab.g[j0 + b]);
#pragma unroll
        for (int k = 0; k < AS_RB; ++k)
#pragma unroll
          for (int v = 0; v < VPT; ++v) raw[b][k][v] = IO<T>::raw_nt(gj + roff[k] + R.off(v));
#pragma unroll
        for (int k = 0; k < AS_RB; ++k) sc[b][k] = *reinterpret_cast<const float2*>(tab.wz[j0 + b] + 2 * tokc[k]);
#pragma unroll
        for (int v = 0; v < VPT; ++v) load_f32x8(tab.q[j0 + b] + R.off(v), qv[b][v]);
      }
#pragma unroll
      for (int b = 0; b < JB; ++b) take_row(raw[b], sc[b], qv[b]);
    };
    const int mm = ADD_LAST ? m - 1 : m;
    int j = 0;
    constexpr int JB = as_jb<T>();
    for (; j + JB <= mm; j += JB) batch(j, std::integral_constant<int, JB>());
    for (; j < mm; ++j) batch(j, std::integral_constant<int, 1>());
    typename IO<T>::Raw last[AS_RB][VPT];   // ADD_LAST: the last read's rows, kept for the added gradient
    if (ADD_LAST) {
      const T* gj = static_cast<const T*>(tab.g[m - 1]);
      float2 sc[AS_RB];
      float qv[VPT][8];
#pragma unroll
      for (int k = 0; k < AS_RB; ++k)
#pragma unroll
        for (int v = 0; v < VPT; ++v) last[k][v] = IO<T>::raw(gj + roff[k] + R.off(v));   // backward pass 1 just read it
#pragma unroll
      for (int k = 0; k < AS_RB; ++k) sc[k] = *reinterpret_cast<const float2*>(tab.wz[m - 1] + 2 * tokc[k]);
#pragma unroll
      for (int v = 0; v < VPT; ++v) load_f32x8(tab.q[m - 1] + R.off(v), qv[v]);
      take_row(last, sc, qv);
    }
    // the tile's last loads, all requested before the first is used (the scales and their gradients and, for 16-bit
    // rows, the updates' rows and the added gradient's rows): per token row in turn they were two memory round trips
    // each (c4: the update gradients 6.44 -> 6.29 ms per pass). fp32 rows, and rows of 3 or more vectors per lane,
    // load per token row still: their registers would cost some instantiations a wave per SIMD (the fp32 update
    // gradients 14.41 -> 14.66 ms with only the scales' loads taken first).
    constexpr bool EPI_ROWS = !std::is_same<T, float>::value && VPT <= 2;
    constexpr int ER = EPI_ROWS ? AS_RB : 1;
    float rs[ER], grs[ER];
    typename IO<T>::Raw er[ER][VPT], ar[ER][VPT];
    if constexpr (EPI_ROWS) {
      const float* grp = gr ? gr : r;   // without gr: r's entries loaded again and not used
#pragma unroll
      for (int k = 0; k < ER; ++k) {
        rs[k] = r[tokc[k]];
        grs[k] = grp[tokc[k]];
#pragma unroll
        for (int v = 0; v < VPT; ++v) er[k][v] = IO<T>::raw(vsrc + roff[k] + R.off(v));
      }
      if (!ADD_LAST && add) {
#pragma unroll
        for (int k = 0; k < ER; ++k)
#pragma unroll
          for (int v = 0; v < VPT; ++v) ar[k][v] = IO<T>::raw(add + roff[k] + R.off(v));
      }
    }
#pragma unroll
    for (int k = 0; k < AS_RB; ++k) {
      const int ke = EPI_ROWS ? k : 0;
      const float rv = EPI_ROWS ? rs[ke] : r[tokc[k]];
      const float c = gr ? (EPI_ROWS ? grs[ke] : gr[tokc[k]]) * (-rv * rv * rv) / (float)d : 0.f;
      float e[VPT][8], a[VPT][8];
#pragma unroll
      for (int v = 0; v < VPT; ++v) {
        if constexpr (EPI_ROWS) IO<T>::unpack(er[ke][v], e[v]);
        else IO<T>::load(vsrc + roff[k] + R.off(v), e[v]);
      }
      if (add) {   // a gradient of the write's h from elsewhere, added as autograd would add it
        if (ADD_LAST) {   // the rows already in registers
#pragma unroll
          for (int v = 0; v < VPT; ++v) IO<T>::unpack(last[k][v], a[v]);
        } else {
#pragma unroll
          for (int v = 0; v < VPT; ++v) {
            if constexpr (EPI_ROWS) IO<T>::unpack(ar[ke][v], a[v]);
            else IO<T>::load(add + roff[k] + R.off(v), a[v]);
          }
        }
        if (add_beta != 0.f) {   // add is the output gradient g of an iteration-end blend: its proposal's share
#pragma clang fp contract(off)
#pragma unroll
          for (int v = 0; v < VPT; ++v)
#pragma unroll
            for (int x = 0; x < 8; ++x) a[v][x] = IO<T>::round(a[v][x] - IO<T>::round(add_beta * a[v][x]));
        }
      }
#pragma unroll
      for (int v = 0; v < VPT; ++v) {
#pragma unroll
        for (int x = 0; x < 8; ++x) {
          if (PER_READ) {   // the scale's term as the scale node's backward rounds it, added last
#pragma clang fp contract(off)   // the product rounded on its own (in fp32 too), as that node stores it
            if (gr) {
              const float gx = IO<T>::round(c * e[v][x]);
              acc[k][v][x] = m == 0 ? gx : IO<T>::round(acc[k][v][x] + gx);
            }
          } else {
            acc[k][v][x] = __builtin_fmaf(c, e[v][x], acc[k][v][x]);
          }
        }
        if (tok[k] < n_tok && R.act(v)) {
          if (dv_neg) {
            if (LDR_AS_STORES & 2) IO<T>::store_neg(dv_neg + roff[k] + R.c8(v) * 8, acc[k][v]);
            else IO<T>::store_neg_nt(dv_neg + roff[k] + R.c8(v) * 8, acc[k][v]);
          }
          if (add) {
#pragma unroll
            for (int x = 0; x < 8; ++x) acc[k][v][x] = IO<T>::round(acc[k][v][x]) + a[v][x];
          }
          if (LDR_AS_STORES & 1) IO<T>::store(dv + roff[k] + R.c8(v) * 8, acc[k][v]);
          else IO<T>::store_nt(dv + roff[k] + R.c8(v) * 8, acc[k][v]);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------
// any-shape kernels (the *_any entry points): rows of any width d >= 1 at element alignment and up to
// LDR_ANY_MAX_SOURCES sources, whose addresses come from DEVICE arrays. One wave per token row, the row's columns
// strided over its 64 lanes (each load instruction covers consecutive elements), row sums by the lane reduction
// above; per-source scalars of the row in LDS. They compute what the row-layout kernels compute (the same formulas,
// and for the elementwise ones the same order of every rounding), for the shapes those do not take: d not a
// multiple of 8 or above LDR_MAX_WIDTH, more than LDR_MAX_SOURCES sources, rows not 16-byte aligned.
// ---------------------------------------------------------------------------------------------------------------
constexpr int ANY_MAXS = LDR_ANY_MAX_SOURCES;
constexpr int ANY_WAVES = WG / 64;

// softmax of a[0..n) in place by the 64 lanes of one wave (all active): p = exp(l - max) / sum, as softmax_lanes
__device__ __forceinline__ void wave_softmax(float* a, int n) {
  const int lane = (int)threadIdx.x & 63;
  float mx = -INFINITY;
  for (int i = lane; i < n; i += 64) mx = fmaxf(mx, a[i]);
  mx = lanes_reduce(mx, 64, MaxOp());
  float s = 0.f;
  for (int i = lane; i < n; i += 64) {
    const float e = (a[i] == -INFINITY) ? 0.f : expf(a[i] - mx);
    a[i] = e;
    s += e;
  }
  s = lanes_reduce(s, 64, AddOp());
  for (int i = lane; i < n; i += 64) a[i] = a[i] / s;
  wave_lds_sync();
}

// per-read constants for up to ANY_MAXS sources: c0, lc = log(max(c0, 1e-8)), p0 = softmax(lc) (by the softmax
// every row uses, so equal logits give equal bits), and M = sum c0 in source order; the whole workgroup calls
__device__ void any_prior(const Coef& c, int n, float* s_c0, float* s_lc, float* s_p0, float* s_M) {
  const int tid = (int)threadIdx.x;
  for (int i = tid; i < n; i += (int)blockDim.x) {
    const float v = i < c.c0_cols ? c.lam * c.c0[i] : c.lam;
    s_c0[i] = v;
    s_lc[i] = logf(fmaxf(v, 1e-8f));
    s_p0[i] = s_lc[i];
  }
  __syncthreads();
  if (tid < 64) wave_softmax(s_p0, n);
  if (tid == 0) {
    float m = 0.f;
    for (int i = 0; i < n; ++i) m += s_c0[i];
    *s_M = m;
  }
  __syncthreads();
}

template <typename T> __device__ __forceinline__ const T* any_row(const uint64_t* tab, int i, int64_t off) {
  return reinterpret_cast<const T*>(tab[i]) + off;
}

// The read (k_read_fwd / k_read_online): scores (stored, or formed here when q is given and kept in dots), the
// softmax, tc, p, and out = base + sum_i (tc_i - cbar_i) v_i (base blended with h0 at an iteration end).
// Dynamic LDS: c0, lc, p0 [n], M, then one [n] row of logits / weights per wave.
template <typename T, bool BLEND>
__global__ __launch_bounds__(WG) void k_any_read(const uint64_t* __restrict__ tv, const uint64_t* __restrict__ tr,
                                                 int n, const float* __restrict__ q, float* __restrict__ dots,
                                                 int64_t dots_stride, const T* __restrict__ base,
                                                 const T* __restrict__ h0, float beta, Coef cf, float inv,
                                                 T* __restrict__ out, float* __restrict__ tc, float* __restrict__ prob,
                                                 float* __restrict__ next_prior, int64_t n_tok, int64_t d) {
  extern __shared__ float any_lds[];
  const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float* s_c0 = any_lds;
  float* s_lc = s_c0 + n;
  float* s_p0 = s_lc + n;
  float* s_M = s_p0 + n;
  float* s_l = s_M + 4 + wave * n;
  any_prior(cf, n, s_c0, s_lc, s_p0, s_M);
  const float M = *s_M;
  if (next_prior && blockIdx.x == 0)
    for (int i = tid; i < n; i += WG) next_prior[i] = s_c0[i];
  for (int64_t tok = (int64_t)blockIdx.x * ANY_WAVES + wave; tok < n_tok; tok += (int64_t)gridDim.x * ANY_WAVES) {
    const int64_t roff = tok * d;
    if (q) {   // online scores: q . v_i, kept for the backward
      for (int i = 0; i < n; ++i) {
        const T* v = any_row<T>(tv, i, roff);
        float a = 0.f;
        for (int64_t k = lane; k < d; k += 64) a += q[k] * ld1(v + k);
        a = lanes_reduce(a, 64, AddOp());
        if (lane == 0) {
          dots[(int64_t)i * dots_stride + tok] = a;
          s_l[i] = a * reinterpret_cast<const float*>(tr[i])[tok] * inv + s_lc[i];
        }
      }
    } else {
      for (int i = lane; i < n; i += 64)
        s_l[i] = dots[(int64_t)i * dots_stride + tok] * reinterpret_cast<const float*>(tr[i])[tok] * inv + s_lc[i];
    }
    wave_lds_sync();
    wave_softmax(s_l, n);
    for (int i = lane; i < n; i += 64) {
      const float p = s_l[i];
      const float tcv = s_c0[i] + M * (p - s_p0[i]);
      tc[tok * n + i] = tcv;
      if (prob) prob[tok * n + i] = p;   // for the backward only
      s_l[i] = tcv - coef_cbar(cf, tok, i);
    }
    wave_lds_sync();
    for (int64_t k = lane; k < d; k += 64) {
      float acc = ld1(base + roff + k);
      if (BLEND) {   // base = proposal + beta (h0 - proposal), each step rounded as the caller's ops
#pragma clang fp contract(off)
        const float hv = ld1(h0 + roff + k);
        acc = IO<T>::round(acc + IO<T>::round(beta * IO<T>::round(hv - acc)));
      }
      for (int i = 0; i < n; ++i) acc += s_l[i] * ld1(any_row<T>(tv, i, roff) + k);
      st1(out + roff + k, acc);
    }
    wave_lds_sync();   // the row's weights are read before the next row overwrites them
  }
}

// Backward pass 1 (k_bwd1): g . v_i, then per source dz = p (M (g.v + gt) - Sacc), dcbar = -lam g.v, dr (+)= dz
// (q . v) / sqrt(d), the (w, dz r / sqrt(d)) pair, and the row's share of dq, sum_i dz_i r_i v_i, added into the
// wave's partial row dq_part[blockIdx.x] (one wave per workgroup; scaled by 1/sqrt(d) at the end); the blend's
// gradients when asked. Dynamic LDS: g.v, p, M (g.v + gt), dz r [n].
template <typename T>
__global__ __launch_bounds__(64) void k_any_bwd1(const uint64_t* __restrict__ tv, const uint64_t* __restrict__ tr, int n,
                                                 const T* __restrict__ g, const float* __restrict__ gt,
                                                 const float* __restrict__ prob, const float* __restrict__ dots,
                                                 int64_t dots_stride, const float* __restrict__ tcp, Coef cf,
                                                 float inv, float* __restrict__ dcbar, int dcbar_cols,
                                                 const uint64_t* __restrict__ tdr, int dr_accum,
                                                 float* __restrict__ wz, int64_t wz_stride,
                                                 float* __restrict__ dq_part, int64_t dq_stride,
                                                 T* __restrict__ g_prop, T* __restrict__ g_h0, float beta,
                                                 int64_t n_tok, int64_t d) {
  extern __shared__ float any_lds[];
  const int lane = (int)threadIdx.x;
  float* s_gd = any_lds;
  float* s_p = s_gd + n;
  float* s_gp = s_p + n;
  float* s_c = s_gp + n;
  float M = 0.f;   // sum c0 in source order, as any_prior forms it (each product rounded before the sum)
  {
#pragma clang fp contract(off)
    for (int i = 0; i < n; ++i) M += i < cf.c0_cols ? cf.lam * cf.c0[i] : cf.lam;
  }
  float* dqp = dq_part + (int64_t)blockIdx.x * dq_stride;
  for (int64_t k = lane; k < d; k += 64) dqp[k] = 0.f;
  for (int64_t tok = blockIdx.x; tok < n_tok; tok += gridDim.x) {
    const int64_t roff = tok * d;
    if (g_prop || g_h0) {   // the blend's gradients: beta g to h0, g - beta g to the proposal
#pragma clang fp contract(off)
      for (int64_t k = lane; k < d; k += 64) {
        const float gv = ld1(g + roff + k);
        const float gb = IO<T>::round(beta * gv);
        if (g_h0) st1(g_h0 + roff + k, gb);
        if (g_prop) st1(g_prop + roff + k, gv - gb);
      }
    }
    for (int i = 0; i < n; ++i) {
      const T* v = any_row<T>(tv, i, roff);
      float a = 0.f;
      for (int64_t k = lane; k < d; k += 64) a += ld1(g + roff + k) * ld1(v + k);
      a = lanes_reduce(a, 64, AddOp());
      if (lane == 0) s_gd[i] = a;
    }
    wave_lds_sync();
    for (int i = lane; i < n; i += 64) {
      s_p[i] = prob[tok * n + i];
      s_gp[i] = M * (s_gd[i] + (gt ? gt[tok * n + i] : 0.f));
    }
    wave_lds_sync();
    float sacc = 0.f;   // every lane forms the same sum, in source order
    for (int i = 0; i < n; ++i) sacc += s_p[i] * s_gp[i];
    for (int i = lane; i < n; i += 64) {
      const float gd = s_gd[i];
      const float dz = s_p[i] * (s_gp[i] - sacc);
      if (i < dcbar_cols) dcbar[tok * dcbar_cols + i] = -(cf.lam * gd);
      float* dri = reinterpret_cast<float*>(tdr[i]);
      const float drv = dz * dots[(int64_t)i * dots_stride + tok] * inv;
      dri[tok] = dr_accum ? dri[tok] + drv : drv;
      const float r = reinterpret_cast<const float*>(tr[i])[tok];
      *reinterpret_cast<float2*>(wz + 2 * ((int64_t)i * wz_stride + tok)) =
          make_float2(tcp[tok * n + i] - coef_cbar(cf, tok, i), dz * r * inv);
      s_c[i] = dz * r;
    }
    wave_lds_sync();
    for (int64_t k = lane; k < d; k += 64) {
      float a = 0.f;
      for (int i = 0; i < n; ++i) a += s_c[i] * ld1(any_row<T>(tv, i, roff) + k);
      dqp[k] += a;
    }
    wave_lds_sync();   // the row's scalars are read before the next row overwrites them
  }
  for (int64_t k = lane; k < d; k += 64) dqp[k] *= inv;
}

// The update gradient (k_dv_assemble): per element, the reads' shares w g + dzr q in table order as two explicit
// fused multiply-adds each, the scale's term, then dv_neg = -dv and the added gradient -- the same roundings in the
// same order as k_dv_assemble, so the same bits for the same table.
template <typename T, bool PER_READ>
__global__ __launch_bounds__(WG) void k_any_dv_assemble(const uint64_t* __restrict__ tg, const uint64_t* __restrict__ twz,
                                                        const uint64_t* __restrict__ tq, int m,
                                                        const T* __restrict__ vsrc, const float* __restrict__ r,
                                                        const float* __restrict__ gr, const T* __restrict__ add,
                                                        float add_beta, T* __restrict__ dv, T* __restrict__ dv_neg,
                                                        int64_t n_tok, int64_t d) {
  const int lane = (int)threadIdx.x & 63, wave = (int)threadIdx.x >> 6;
  for (int64_t tok = (int64_t)blockIdx.x * ANY_WAVES + wave; tok < n_tok; tok += (int64_t)gridDim.x * ANY_WAVES) {
    const int64_t roff = tok * d;
    const float rv = r[tok];
    const float c = gr ? gr[tok] * (-rv * rv * rv) / (float)d : 0.f;
    for (int64_t k = lane; k < d; k += 64) {
      float acc = 0.f;
      for (int j = 0; j < m; ++j) {
        const float2 sc = *reinterpret_cast<const float2*>(reinterpret_cast<const float*>(twz[j]) + 2 * tok);
        const float e = ld1(any_row<T>(tg, j, roff) + k);
        const float q = reinterpret_cast<const float*>(tq[j])[k];
        if (PER_READ) {
          const float t = IO<T>::round(bwd2_term(sc.x, e, sc.y, q));
          acc = j == 0 ? t : IO<T>::round(acc + t);
        } else {
          acc = __builtin_fmaf(sc.y, q, __builtin_fmaf(sc.x, e, acc));
        }
      }
      if (PER_READ) {
#pragma clang fp contract(off)
        if (gr) {
          const float gx = IO<T>::round(c * ld1(vsrc + roff + k));
          acc = m == 0 ? gx : IO<T>::round(acc + gx);
        }
      } else {
        acc = __builtin_fmaf(c, ld1(vsrc + roff + k), acc);
      }
      if (dv_neg) st1(dv_neg + roff + k, -acc);
      if (add) {   // a gradient of the write's h from elsewhere, added as autograd would add it
        float a = ld1(add + roff + k);
        if (add_beta != 0.f) {   // the proposal's share of an iteration-end blend's output gradient
#pragma clang fp contract(off)
          a = IO<T>::round(a - IO<T>::round(add_beta * a));
        }
        acc = IO<T>::round(acc) + a;
      }
      st1(dv + roff + k, acc);
    }
  }
}

// Backward pass 2, list layout (k_bwd2_list): dv_i (=|+=) w_i g + dzr_i q, the accumulation rounded as autograd's
template <typename T>
__global__ __launch_bounds__(WG) void k_any_bwd2_list(const uint64_t* __restrict__ tdv, int n, int accum,
                                                      const T* __restrict__ g, const float* __restrict__ q,
                                                      const float* __restrict__ wz, int64_t wz_stride, int64_t n_tok,
                                                      int64_t d) {
  const int lane = (int)threadIdx.x & 63, wave = (int)threadIdx.x >> 6;
  for (int64_t tok = (int64_t)blockIdx.x * ANY_WAVES + wave; tok < n_tok; tok += (int64_t)gridDim.x * ANY_WAVES) {
    const int64_t roff = tok * d;
    for (int i = 0; i < n; ++i) {
      const float2 s = *reinterpret_cast<const float2*>(wz + 2 * ((int64_t)i * wz_stride + tok));
      T* dvi = reinterpret_cast<T*>(tdv[i]) + roff;
      for (int64_t k = lane; k < d; k += 64) {
        float o = bwd2_term(s.x, ld1(g + roff + k), s.y, q[k]);
        if (accum) o = ld1(dvi + k) + IO<T>::round(o);
        st1(dvi + k, o);
      }
    }
  }
}

// out = round(sum_j round(beta * g_j)) in table order, or with per_read each addition rounded (k_blend_sum)
template <typename T>
__global__ __launch_bounds__(WG) void k_any_blend_sum(const uint64_t* __restrict__ tg, int m, float beta, int per_read,
                                                      T* __restrict__ out, int64_t n_tok, int64_t d) {
#pragma clang fp contract(off)
  const int64_t total = n_tok * d;
  for (int64_t e = (int64_t)blockIdx.x * WG + threadIdx.x; e < total; e += (int64_t)gridDim.x * WG) {
    float acc = 0.f;
    for (int j = 0; j < m; ++j) {
      const float t = IO<T>::round(beta * ld1(reinterpret_cast<const T*>(tg[j]) + e));
      acc = !per_read ? acc + t : (j == 0 ? t : IO<T>::round(acc + t));
    }
    st1(out + e, acc);
  }
}

// ---------------------------------------------------------------------------------------------------------------
// host side: argument checks, layout choice, dispatch
// ---------------------------------------------------------------------------------------------------------------
int row_layout(int64_t d, int* vpt, int* tpr, int max_vpt = 4, bool wave_rows = true, int force_vpt = 0,
               bool big_vpt = false) {
  if (d <= 0 || (d & 7) || d > LDR_MAX_WIDTH) return LDR_E_SHAPE;
  const int64_t d8 = d >> 3;
  if (force_vpt > 0) {   // a fixed number of vectors per lane: the narrowest power-of-two row that covers d
    int t = 8;
    while ((int64_t)force_vpt * t < d8 && t < WG) t <<= 1;
    if ((int64_t)force_vpt * t < d8) return LDR_E_SHAPE;
    *vpt = force_vpt;
    *tpr = t;
    return LDR_OK;
  }
  int64_t best = INT64_MAX;
  int bv = 0, bt = 0;
  for (int v = 1; v <= max_vpt; ++v) {
    for (int t = 8; t <= WG; t <<= 1) {
      if ((int64_t)v * t < d8) continue;
      // waste first, then rows inside one wave (if asked), then fewer (or more) vectors per lane
      const int64_t key = ((int64_t)v * t - d8) * 16 + (wave_rows && t > 64 ? 8 : 0) + (big_vpt ? 5 - v : v);
      if (key < best) { best = key; bv = v; bt = t; }
    }
  }
  if (!bv) return LDR_E_SHAPE;
  *vpt = bv;
  *tpr = bt;
  return LDR_OK;
}

inline bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool dtype_ok(int dt) { return dt == LDR_F32 || dt == LDR_BF16 || dt == LDR_F16; }
inline int64_t elt_bytes(int dt) { return dt == LDR_F32 ? 4 : 2; }
// a token-sized buffer: required, except that with no tokens it may be NULL (torch's empty tensors are)
inline bool tok_ptr(const void* p, int64_t n_tok) { return p != nullptr || n_tok == 0; }
inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline unsigned grid_of(int64_t blocks, int64_t cap) { return (unsigned)(blocks < 1 ? 1 : (blocks < cap ? blocks : cap)); }
inline int launched() { return (int)hipGetLastError(); }

// tokens per tile of the tiled kernels: at least one row per row slot
inline int tile_tokens(int tpr) { const int rpw = WG / tpr; return rpw > 16 ? rpw : 16; }

#ifndef LDR_B1_TT
#define LDR_B1_TT 32          // backward pass 1: tokens per tile (at least one row per row slot)
#endif
// a power of two <= TT_MAX: the tile is then a multiple of the rows per workgroup and fits the LDS planes
static_assert(LDR_B1_TT >= 1 && LDR_B1_TT <= TT_MAX && (LDR_B1_TT & (LDR_B1_TT - 1)) == 0,
              "backward pass 1: tokens per tile must be a power of two <= 32");
inline int b1_tile(int tpr) { const int t = tile_tokens(tpr); return t > LDR_B1_TT ? t : LDR_B1_TT; }
inline int rf_tile(int tpr) { const int t = tile_tokens(tpr); return t > LDR_RF_TT ? t : LDR_RF_TT; }

int fill_src(SrcTab& s, const uint64_t* v, const uint64_t* r, int64_t n, int64_t n_tok) {
  if (!v || n < 1 || n > MAXS) return LDR_E_ARG;
  for (int64_t i = 0; i < n; ++i) {
    s.v[i] = reinterpret_cast<const void*>(v[i]);
    if (!tok_ptr(s.v[i], n_tok)) return LDR_E_ARG;
    if (!al16(s.v[i])) return LDR_E_ALIGN;
    s.r[i] = r ? reinterpret_cast<const float*>(r[i]) : nullptr;
    if (r && !tok_ptr(s.r[i], n_tok)) return LDR_E_ARG;
  }
  for (int64_t i = n; i < MAXS; ++i) { s.v[i] = nullptr; s.r[i] = nullptr; }
  return LDR_OK;
}

#define LDR_VPT_SWITCH(VPT_RT, ...)                              \
  switch (VPT_RT) {                                              \
    case 1: { constexpr int VPT = 1; __VA_ARGS__; } break;       \
    case 2: { constexpr int VPT = 2; __VA_ARGS__; } break;       \
    case 3: { constexpr int VPT = 3; __VA_ARGS__; } break;       \
    case 4: { constexpr int VPT = 4; __VA_ARGS__; } break;       \
    default: return LDR_E_SHAPE;                                 \
  }

#define LDR_DTYPE_SWITCH(DT, ...)                                \
  if ((DT) == LDR_BF16) { typedef bf16_t T; __VA_ARGS__; }       \
  else if ((DT) == LDR_F16) { typedef _Float16 T; __VA_ARGS__; } \
  else { typedef float T; __VA_ARGS__; }

template <int VPT> struct Chunk { static constexpr int C = VPT == 1 ? 8 : 4; };
// one-pass online read: sources in flight per row (enough bytes in flight to cover the HBM latency)
template <int VPT> struct OnlineDepth {
  static constexpr int PD = VPT <= 2 ? 2 * LDR_ON_PD : VPT >= 4 ? LDR_ON_PD_VPT4 : LDR_ON_PD;
};
// backward pass 1: sources per row reduction (one LDS exchange per chunk when a row spans two waves)
template <int VPT> struct B1Chunk { static constexpr int C = LDR_B1_C > 0 ? LDR_B1_C : (VPT == 1 ? 8 : VPT == 2 ? 4 : 1); };

}  // namespace

// ---------------------------------------------------------------------------------------------------------------
// the workspace of ldr_read_bwd1_noalloc: backward pass 1's query-gradient partials (one row of d fp32 per
// workgroup) in a device array the library holds on every GPU it runs on, sized for the widest row and the most
// workgroups pass 1 launches (512 x 8192 fp32 = 16 MiB with the default launch settings)
// ---------------------------------------------------------------------------------------------------------------
#define LDR_NOALLOC_PART_FLOATS ((int64_t)LDR_B1_GRID * LDR_MAX_WIDTH)
static __device__ __align__(256) float scratch[LDR_NOALLOC_PART_FLOATS];

namespace {

constexpr int SCRATCH_DEVICES = 64;
// scratch's address on each device, looked up once per device (each GPU holds its own copy of the array); a race
// between two first calls on one device stores the same address twice
std::atomic<float*> g_scratch[SCRATCH_DEVICES];

// the address of `scratch` on the device `st` runs on (the current device for the null stream)
int scratch_on(hipStream_t st, float** out) {
  int cur = 0;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) return (int)e;
  int dev = cur;
  if (st) {
    hipDevice_t sd = 0;
    if ((e = hipStreamGetDevice(st, &sd)) != hipSuccess) return (int)e;
    dev = (int)sd;
  }
  if (dev < 0 || dev >= SCRATCH_DEVICES) return LDR_E_ARG;
  float* p = g_scratch[dev].load(std::memory_order_acquire);
  if (!p) {
    if (dev != cur && (e = hipSetDevice(dev)) != hipSuccess) return (int)e;
    void* a = nullptr;
    e = hipGetSymbolAddress(&a, HIP_SYMBOL(scratch));
    if (dev != cur) {
      const hipError_t back = hipSetDevice(cur);
      if (e == hipSuccess) e = back;
    }
    if (e != hipSuccess) return (int)e;
    if (!a) return (int)hipErrorInvalidSymbol;
    p = static_cast<float*>(a);
    g_scratch[dev].store(p, std::memory_order_release);
  }
  *out = p;
  return LDR_OK;
}

// a vector of fp32 zeros, by a kernel (no memset node in a captured graph)
__global__ __launch_bounds__(WG) void k_zero(float* __restrict__ p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * WG + threadIdx.x; i < n; i += (int64_t)gridDim.x * WG) p[i] = 0.f;
}

}  // namespace

// ===============================================================================================================
// C ABI
// ===============================================================================================================
extern "C" {

int ldr_abi_version(void) { return LDR_ABI_VERSION; }

const char* ldr_strerror(int code) {
  switch (code) {
    case LDR_OK: return "ok";
    case LDR_E_ARG: return "loopback_read: invalid argument (null pointer, bad count or flag)";
    case LDR_E_SHAPE:
      return "loopback_read: unsupported shape (d a multiple of 8 up to 8192 and 1 <= n <= 64; *_any: d >= 1, "
             "1 <= n <= 1024)";
    case LDR_E_ALIGN: return "loopback_read: a vector pointer is not 16-byte aligned (*_any: not element-aligned)";
    case LDR_E_DTYPE: return "loopback_read: dtype must be LDR_F32, LDR_BF16 or LDR_F16";
    default: return code > 0 ? hipGetErrorString((hipError_t)code) : "loopback_read: unknown error";
  }
}

int ldr_row_layout(int64_t d, int* vpt, int* tpr) {
  if (!vpt || !tpr) return LDR_E_ARG;
  return row_layout(d, vpt, tpr);
}

int64_t ldr_read_bwd1_parts(int64_t n_tok, int64_t d) {
  int vpt, tpr;
  if (n_tok < 1 || row_layout(d, &vpt, &tpr, B1_MAX_VPT, LDR_B1_WAVE_ROWS, LDR_B1_VPT, true) != LDR_OK) return 0;
  return grid_of(cdiv(n_tok, b1_tile(tpr)), B1_GRID);
}

int ldr_rstd_fwd(const void* x, float* r, int64_t n_tok, int64_t d, float eps, int dtype, void* stream) {
  if (!dtype_ok(dtype)) return LDR_E_DTYPE;
  if (n_tok < 0 || d < 1 || !tok_ptr(x, n_tok) || !tok_ptr(r, n_tok)) return LDR_E_ARG;
  if (n_tok == 0) return LDR_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  int vpt, tpr;
  if (!al16(x) || row_layout(d, &vpt, &tpr) != LDR_OK) {   // any other row: scalar loads
    const unsigned grid = grid_of(cdiv(n_tok, WG / 64), 8192);
    LDR_DTYPE_SWITCH(dtype, hipLaunchKernelGGL((k_rstd_fwd_any<T>), dim3(grid), dim3(WG), 0, st,
                                                static_cast<const T*>(x), r, n_tok, d, eps))
    return launched();
  }
  // the write kernels' summation order (the same bits as the scale a stacked write stores): the matrix-core writes'
  // chunks, or the vector-unit write's in a build that forms the scores there
  const unsigned grid = grid_of(cdiv(n_tok, WG / 16), 8192);
  if (LDR_WRITE_VALU) {
    LDR_DTYPE_SWITCH(dtype, hipLaunchKernelGGL(k_rstd_valu<T>, dim3(grid), dim3(WG), 0, st,
                                                static_cast<const T*>(x), r, n_tok, (int)d, eps))
  } else {
    LDR_DTYPE_SWITCH(dtype, hipLaunchKernelGGL(k_rstd_chunks<T>, dim3(grid), dim3(WG), 0, st,
                                                static_cast<const T*>(x), r, n_tok, (int)d, eps))
  }
  return launched();
}

int ldr_rstd_bwd(const void* x, const float* r, const float* gr, void* gx, int64_t n_tok, int64_t d, int dtype,
                 void* stream) {
  if (!dtype_ok(dtype)) return LDR_E_DTYPE;
  if (n_tok < 0 || d < 1 || !tok_ptr(x, n_tok) || !tok_ptr(r, n_tok) || !tok_ptr(gr, n_tok) || !tok_ptr(gx, n_tok))
    return LDR_E_ARG;
  if (n_tok == 0) return LDR_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  int vpt, tpr;
  if (!al16(x) || !al16(gx) || row_layout(d, &vpt, &tpr) != LDR_OK) {   // any other row
    const unsigned grid = grid_of(cdiv(n_tok, WG / 64), 8192);
    LDR_DTYPE_SWITCH(dtype, hipLaunchKernelGGL((k_rstd_bwd_any<T>), dim3(grid), dim3(WG), 0, st,
                                                static_cast<const T*>(x), r, gr, static_cast<T*>(gx), n_tok, d))
    return launched();
  }
  const unsigned grid = grid_of(cdiv(n_tok, WG / tpr), 8192);
  LDR_DTYPE_SWITCH(dtype, LDR_VPT_SWITCH(vpt, hipLaunchKernelGGL((k_rstd_bwd<T, VPT>), dim3(grid), dim3(WG), 0, st,
                                                                  static_cast<const T*>(x), r, gr, static_cast<T*>(gx),
                                                                  n_tok, (int)d, tpr)))
  return launched();
}

int ldr_write_dots(const void* h, const void* x, void* v_out, float* r_out, const float* q, const void* qb,
                   int64_t nq, int64_t j_lo, float* dots, int64_t n_tok, int64_t d, int64_t dots_jstride, float eps,
                   int dtype, void* stream) {
  if (!dtype_ok(dtype)) return LDR_E_DTYPE;
  if (n_tok < 0 || !tok_ptr(h, n_tok) || !tok_ptr(x, n_tok) || !tok_ptr(v_out, n_tok) || !tok_ptr(r_out, n_tok) ||
      nq < 0 || j_lo < 0 || j_lo > nq)
    return LDR_E_ARG;
  if (nq > LDR_MAX_QUERIES) return LDR_E_SHAPE;
  const bool scores = j_lo < nq;
  const bool valu = LDR_WRITE_VALU;   // scores on the vector units, from the fp32 queries (a comparison build)
  if (scores && (!tok_ptr(dots, n_tok) || dots_jstride < n_tok)) return LDR_E_ARG;
  if (scores && ((valu && !q) || (!valu && !qb))) return LDR_E_ARG;
  if (!al16(h) || !al16(x) || !al16(v_out) || (scores && valu && !al16(q)) || (scores && !valu && !al16(qb)))
    return LDR_E_ALIGN;
  if (d <= 0 || (d & 7) || d > LDR_MAX_WIDTH) return LDR_E_SHAPE;
  if (n_tok == 0) return LDR_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (!valu && dtype == LDR_F32) {   // fp32 updates: split into three bf16 parts on the matrix cores
    const int nbq = (int)query_blocks(nq), b0 = (int)(j_lo / 16);
    const QTile qtl{static_cast<const uint4*>(qb), nbq, b0, (int)j_lo, (int)nq};
    const int nb = scores ? nbq - b0 : 0;
    const unsigned grid = (unsigned)cdiv(n_tok, W32_TT);
    const float* hf = static_cast<const float*>(h);
    const float* xf = static_cast<const float*>(x);
    float* vf = static_cast<float*>(v_out);
    const bool rows = d % (4 * WM_KC) == 0;   // rows streamed whole when d is whole steps
#define LDR_W32_LAUNCH(NBV)                                                                                   \
  hipLaunchKernelGGL((write32_kernel<NBV>(rows)), dim3(grid), dim3(WG), 0, st, hf, xf, vf, r_out, qtl, dots, n_tok, \
                     (int)d, dots_jstride, eps)
    switch (nb) {
      case 0: LDR_W32_LAUNCH(0); break;
      case 1: LDR_W32_LAUNCH(1); break;
      case 2: LDR_W32_LAUNCH(2); break;
      case 3: LDR_W32_LAUNCH(3); break;
      default: LDR_W32_LAUNCH(4); break;
    }
#undef LDR_W32_LAUNCH
  } else if (!valu) {   // matrix-core scores from the operand table of the nq queries (bf16 and fp16 updates)
    const unsigned grid = (unsigned)cdiv(n_tok, WM_TT);
    const int nbq = (int)query_blocks(nq), b0 = (int)(j_lo / 16);
    const QTile qtl{static_cast<const uint4*>(qb), nbq, b0, (int)j_lo, (int)nq};
    const int nb = scores ? nbq - b0 : 0;
    const bool rows = d % (4 * WM_KC) == 0;   // rows streamed whole when d is whole steps
#define LDR_WM_LAUNCH(NBV)                                                                                        \
  if (dtype == LDR_BF16)                                                                                          \
    hipLaunchKernelGGL((write_kernel<bf16_t, NBV>(rows)), dim3(grid), dim3(WG), 0, st,                            \
                       static_cast<const bf16_t*>(h), static_cast<const bf16_t*>(x), static_cast<bf16_t*>(v_out), \
                       r_out, qtl, dots, n_tok, (int)d, dots_jstride, eps);                                       \
  else                                                                                                            \
    hipLaunchKernelGGL((write_kernel<_Float16, NBV>(rows)), dim3(grid), dim3(WG), 0, st,                          \
                       static_cast<const _Float16*>(h), static_cast<const _Float16*>(x),                          \
                       static_cast<_Float16*>(v_out), r_out, qtl, dots, n_tok, (int)d, dots_jstride, eps)
    switch (nb) {
      case 0: LDR_WM_LAUNCH(0); break;
      case 1: LDR_WM_LAUNCH(1); break;
      case 2: LDR_WM_LAUNCH(2); break;
      case 3: LDR_WM_LAUNCH(3); break;
      default: LDR_WM_LAUNCH(4); break;
    }
#undef LDR_WM_LAUNCH
  } else {   // vector-unit scores from the fp32 queries (a build with LDR_WRITE_VALU)
    const unsigned grid = (unsigned)cdiv(n_tok, WR_TT);
    const float* qj = scores ? q + j_lo * d : nullptr;
    LDR_DTYPE_SWITCH(dtype, hipLaunchKernelGGL((k_write_dots<T>), dim3(grid), dim3(WG), 0, st,
                                               static_cast<const T*>(h), static_cast<const T*>(x),
                                               static_cast<T*>(v_out), r_out, qj, dots, n_tok, (int)d,
                                               (int)(nq - j_lo), dots_jstride, eps))
  }
  return launched();
}

int64_t ldr_query_parts_elems(int64_t nq, int64_t d) {
  if (nq < 0 || nq > LDR_MAX_QUERIES || d <= 0 || d > LDR_MAX_WIDTH) return 0;
  return query_chunks(d) * query_blocks(nq) * 3 * 2 * 64 * 8;
}

int ldr_split_queries(const float* q, int64_t nq, int64_t d, void* qb, void* stream) {
  if (nq < 0 || d <= 0 || (nq > 0 && (!q || !qb))) return LDR_E_ARG;
  if (nq > LDR_MAX_QUERIES || d > LDR_MAX_WIDTH) return LDR_E_SHAPE;
  if (!al16(qb)) return LDR_E_ALIGN;
  if (nq == 0) return LDR_OK;
  const int64_t n_vec = ldr_query_parts_elems(nq, d) / 8;
  const unsigned grid = grid_of(cdiv(n_vec, WG), 1024);
  hipLaunchKernelGGL(k_split_queries, dim3(grid), dim3(WG), 0, static_cast<hipStream_t>(stream), q,
                     static_cast<uint4*>(qb), (int)nq, (int)d, (int)query_blocks(nq), n_vec);
  return launched();
}

int ldr_dots_online(const uint64_t* src_v, int64_t n, const float* q, float* out, int64_t out_stride,
                    int64_t n_tok, int64_t d, int dtype, void* stream) {
  if (!dtype_ok(dtype)) return LDR_E_DTYPE;
  if (n_tok < 0 || !q || !tok_ptr(out, n_tok) || out_stride < n_tok) return LDR_E_ARG;
  if (!al16(q)) return LDR_E_ALIGN;
  SrcTab s;
  int e = fill_src(s, src_v, nullptr, n, n_tok);
  if (e) return e;
  int vpt, tpr;
  if ((e = row_layout(d, &vpt, &tpr))) return e;
  if (n_tok == 0) return LDR_OK;
  const unsigned grid = grid_of(cdiv(n_tok, WG / tpr), 4096);
  hipStream_t st = static_cast<hipStream_t>(stream);
  LDR_DTYPE_SWITCH(dtype, LDR_VPT_SWITCH(vpt, hipLaunchKernelGGL((k_dots<T, VPT, Chunk<VPT>::C>), dim3(grid), dim3(WG),
                                                                  0, st, s, (int)n, q, out, out_stride, n_tok, (int)d,
                                                                  tpr)))
  return launched();
}

int ldr_read_fwd(const uint64_t* src_v, const uint64_t* src_r, int64_t n, const float* dots, int64_t dots_stride,
                 const void* base, const void* h0, float beta, const float* cbar, int64_t cbar_cols, const float* c0,
                 int64_t c0_cols, float lam, float inv_sqrt_d, void* out, float* tc, float* p, float* next_prior,
                 int64_t n_tok, int64_t d, int dtype, void* stream) {
  if (!dtype_ok(dtype)) return LDR_E_DTYPE;
  if (!src_r || n_tok < 0 || !tok_ptr(dots, n_tok) || dots_stride < n_tok || !tok_ptr(base, n_tok) ||
      !tok_ptr(cbar, n_tok) || !c0 || !tok_ptr(out, n_tok) || !tok_ptr(tc, n_tok))
    return LDR_E_ARG;
  if ((cbar_cols != n && cbar_cols != n - 1) || (c0_cols != n && c0_cols != n - 1)) return LDR_E_ARG;
  if (!al16(base) || !al16(out) || (h0 && !al16(h0))) return LDR_E_ALIGN;
  SrcTab s;
  int e = fill_src(s, src_v, src_r, n, n_tok);
  if (e) return e;
  int vpt, tpr;
  if ((e = row_layout(d, &vpt, &tpr, LDR_RF_MAX_VPT, true, LDR_RF_VPT))) return e;
  if (n_tok == 0 && !next_prior) return LDR_OK;
  const Coef cf{cbar, (int)cbar_cols, c0, (int)c0_cols, lam};
  const int64_t row_bytes = d * elt_bytes(dtype);
  // 512-lane workgroups with 32-token tiles whose output (at most 128 KiB) is written as one burst, one workgroup
  // per CU, whenever the tile's rows fit and the read has enough sources to repay the launch's higher fixed cost;
  // rows of 4-8 KiB (fp32 rows of 2048) take 16-token tiles there, a token's softmax still over 32 lanes as in the
  // 256-lane launch's 8-token tiles for such rows (the same bits; fp32 headline read forward 15.15 -> 14.26 ms per
  // pass); else 256-lane workgroups, 16-token tiles, 64 KiB bursts when they fit
  int big_tt = RF_BIG_TT;
  if (LDR_RF_HALF_TT && big_tt * row_bytes > RF_BIG_STAGE) big_tt /= 2;
  const bool big = LDR_RF_BIG && (n + 2) * row_bytes >= LDR_RF_BIG_MIN_ROW_BYTES && RF_BIG_LANES / tpr <= big_tt &&
                   big_tt * row_bytes <= RF_BIG_STAGE;
  int tt = big ? big_tt : rf_tile(tpr);
  // rows too long for a tile's output to fit the staging space (fp32 rows of 2048, bf16 rows of 3072 and more): half
  // the tokens per tile, while that still gives every row slot a row, so the output still goes out in bursts
  if (LDR_RF_HALF_TT && !big && RF_STAGE_BYTES > 0 && tt * row_bytes > RF_STAGE_BYTES &&
      (tt / 2) * row_bytes <= RF_STAGE_BYTES && tt / 2 >= WG / tpr)
    tt /= 2;
  const unsigned grid = big ? grid_of(cdiv(n_tok, tt), LDR_RF_BIG_GRID)
                            : grid_of(cdiv(n_tok, tt), LDR_RF_GRID);   // no tokens: one workgroup writes next_prior
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool stage = big || (RF_STAGE_BYTES > 0 && tt * row_bytes <= RF_STAGE_BYTES);
#define LDR_RF_LAUNCH(BL, SG, NTH)                                                                                 \
  LDR_DTYPE_SWITCH(dtype, LDR_VPT_SWITCH(vpt, hipLaunchKernelGGL((k_read_fwd<T, VPT, BL, SG, NTH>), dim3(grid),       \
                                                                  dim3(NTH), 0, st, s, (int)n, dots, dots_stride,  \
                                                                  static_cast<const T*>(base),                     \
                                                                  static_cast<const T*>(h0), beta, cf, inv_sqrt_d, \
                                                                  static_cast<T*>(out), tc, p, next_prior, n_tok,  \
                                                                  (int)d, tpr, tt)))
  if (big && h0) {
    LDR_RF_LAUNCH(true, true, RF_BIG_LANES);
  } else if (big) {
    LDR_RF_LAUNCH(false, true, RF_BIG_LANES);
  } else if (h0 && stage) {
    LDR_RF_LAUNCH(true, true, WG);
  } else if (h0) {
    LDR_RF_LAUNCH(true, false, WG);
  } else if (stage) {
    LDR_RF_LAUNCH(false, true, WG);
  } else {
    LDR_RF_LAUNCH(false, false, WG);
  }
#undef LDR_RF_LAUNCH
  return launched();
}

int ldr_read_fwd_online(const uint64_t* src_v, const uint64_t* src_r, int64_t n, const float* q, float* dots,
                        int64_t dots_stride, const void* base, const void* h0, float beta, const float* cbar,
                        int64_t cbar_cols, const float* c0, int64_t c0_cols, float lam, float inv_sqrt_d, void* out,
                        float* tc, float* p, float* next_prior, int64_t n_tok, int64_t d, int dtype, void* stream) {
  if (!dtype_ok(dtype)) return LDR_E_DTYPE;
  if (!src_r || !q || n_tok < 0 || !tok_ptr(dots, n_tok) || dots_stride < n_tok || !tok_ptr(base, n_tok) ||
      !tok_ptr(cbar, n_tok) || !c0 || !tok_ptr(out, n_tok) || !tok_ptr(tc, n_tok))
    return LDR_E_ARG;
  if ((cbar_cols != n && cbar_cols != n - 1) || (c0_cols != n && c0_cols != n - 1)) return LDR_E_ARG;
  if (!al16(q) || !al16(base) || !al16(out) || (h0 && !al16(h0))) return LDR_E_ALIGN;
  SrcTab s;
  int e = fill_src(s, src_v, src_r, n, n_tok);
  if (e) return e;
  int vpt, tpr;
  if ((e = row_layout(d, &vpt, &tpr, LDR_RF_MAX_VPT, true, LDR_RF_VPT))) return e;
  if (tpr > 64) {   // rows across waves: the scores first, then the stored-score read (two passes)
    if ((e = ldr_dots_online(src_v, n, q, dots, dots_stride, n_tok, d, dtype, stream))) return e;
    return ldr_read_fwd(src_v, src_r, n, dots, dots_stride, base, h0, beta, cbar, cbar_cols, c0, c0_cols, lam,
                        inv_sqrt_d, out, tc, p, next_prior, n_tok, d, dtype, stream);
  }
  if (n_tok == 0 && !next_prior) return LDR_OK;   // no tokens: one workgroup writes next_prior
  const Coef cf{cbar, (int)cbar_cols, c0, (int)c0_cols, lam};
  const unsigned grid = grid_of(cdiv(n_tok, WG / tpr), LDR_ON_GRID);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (h0) {
    LDR_DTYPE_SWITCH(dtype, LDR_VPT_SWITCH(vpt, hipLaunchKernelGGL((k_read_online<T, VPT, true, OnlineDepth<VPT>::PD>),
                                                                    dim3(grid), dim3(WG), 0, st, s, (int)n, q, dots,
                                                                    dots_stride, static_cast<const T*>(base),
                                                                    static_cast<const T*>(h0), beta, cf, inv_sqrt_d,
                                                                    static_cast<T*>(out), tc, p, next_prior, n_tok,
                                                                    (int)d, tpr)))
  } else {
    LDR_DTYPE_SWITCH(dtype, LDR_VPT_SWITCH(vpt, hipLaunchKernelGGL((k_read_online<T, VPT, false, OnlineDepth<VPT>::PD>),
                                                                    dim3(grid), dim3(WG), 0, st, s, (int)n, q, dots,
                                                                    dots_stride, static_cast<const T*>(base), nullptr,
                                                                    beta, cf, inv_sqrt_d, static_cast<T*>(out), tc, p,
                                                                    next_prior, n_tok, (int)d, tpr)))
  }
  return launched();
}

int ldr_read_bwd1(const uint64_t* src_v, const uint64_t* src_r, int64_t n, const void* g, const float* gt,
                  const float* p, const float* dots, int64_t dots_stride, const float* tc, const float* cbar,
                  int64_t cbar_cols,
                  const float* c0, int64_t c0_cols, float lam, float inv_sqrt_d, float* dcbar, int64_t dcbar_cols,
                  const uint64_t* dr, int dr_accum, float* wz, int64_t wz_stride, float* dq_part,
                  int64_t dq_part_stride, void* g_prop,
                  void* g_h0, float beta, int64_t n_tok, int64_t d, int dtype, void* stream) {
  if (!dtype_ok(dtype)) return LDR_E_DTYPE;
  if (!src_r || n_tok < 0 || !tok_ptr(g, n_tok) || !tok_ptr(p, n_tok) || !tok_ptr(dots, n_tok) ||
      dots_stride < n_tok || !tok_ptr(tc, n_tok) || !tok_ptr(cbar, n_tok) || !c0 || !tok_ptr(dcbar, n_tok) || !dr ||
      !tok_ptr(wz, n_tok) || !dq_part || wz_stride < n_tok || dq_part_stride < d ||
      (dr_accum != 0 && dr_accum != 1))
    return LDR_E_ARG;
  if ((cbar_cols != n && cbar_cols != n - 1) || (c0_cols != n && c0_cols != n - 1) || dcbar_cols < 0 ||
      dcbar_cols > n)
    return LDR_E_ARG;
  if (!al16(g) || (g_prop && !al16(g_prop)) || (g_h0 && !al16(g_h0))) return LDR_E_ALIGN;
  SrcTab s;
  int e = fill_src(s, src_v, src_r, n, n_tok);
  if (e) return e;
  PtrTab drt;
  for (int64_t i = 0; i < MAXS; ++i) {
    drt.p[i] = i < n ? reinterpret_cast<void*>(dr[i]) : nullptr;
    if (i < n && !tok_ptr(drt.p[i], n_tok)) return LDR_E_ARG;
  }
  int vpt, tpr;
  if ((e = row_layout(d, &vpt, &tpr, B1_MAX_VPT, LDR_B1_WAVE_ROWS, LDR_B1_VPT, true))) return e;
  if (n_tok == 0) return LDR_OK;
  const Coef cf{cbar, (int)cbar_cols, c0, (int)c0_cols, lam};
  const int tt = b1_tile(tpr);
  const unsigned grid = grid_of(cdiv(n_tok, tt), B1_GRID);
  hipStream_t st = static_cast<hipStream_t>(stream);
  LDR_DTYPE_SWITCH(dtype, LDR_VPT_SWITCH(vpt, hipLaunchKernelGGL((k_bwd1<T, VPT, B1Chunk<VPT>::C>), dim3(grid),
                                                                  dim3(WG), 0, st, s, (int)n, static_cast<const T*>(g),
                                                                  gt, p, dots, dots_stride, tc, cf, inv_sqrt_d, dcbar,
                                                                  (int)dcbar_cols, drt, dr_accum, wz, wz_stride,
                                                                  dq_part, dq_part_stride, static_cast<T*>(g_prop),
                                                                  static_cast<T*>(g_h0), beta, n_tok, (int)d, tpr,
                                                                  tt)))
  return launched();
}

int ldr_read_bwd1_noalloc(const uint64_t* src_v, const uint64_t* src_r, int64_t n, const void* g, const float* gt,
                          const float* p, const float* dots, int64_t dots_stride, const float* tc, const float* cbar,
                          int64_t cbar_cols, const float* c0, int64_t c0_cols, float lam, float inv_sqrt_d,
                          float* dcbar, int64_t dcbar_cols, const uint64_t* dr, int dr_accum, float* wz,
                          int64_t wz_stride, float* dq, void* g_prop, void* g_h0, float beta, int64_t n_tok, int64_t d,
                          int dtype, void* stream) {
  if (!dq) return LDR_E_ARG;
  int vpt, tpr;
  int e = row_layout(d, &vpt, &tpr, B1_MAX_VPT, LDR_B1_WAVE_ROWS, LDR_B1_VPT, true);
  if (e) return e;
  const int64_t parts = ldr_read_bwd1_parts(n_tok, d);
  if (parts * d > LDR_NOALLOC_PART_FLOATS) return LDR_E_SHAPE;   // the partials would not fit the workspace
  hipStream_t st = static_cast<hipStream_t>(stream);
  float* ws = nullptr;
  if ((e = scratch_on(st, &ws))) return e;
  // every argument check of ldr_read_bwd1 runs before its launch; it launches nothing for an empty batch
  if ((e = ldr_read_bwd1(src_v, src_r, n, g, gt, p, dots, dots_stride, tc, cbar, cbar_cols, c0, c0_cols, lam,
                         inv_sqrt_d, dcbar, dcbar_cols, dr, dr_accum, wz, wz_stride, ws, d, g_prop, g_h0, beta, n_tok,
                         d, dtype, stream)))
    return e;
  if (n_tok == 0) {   // a sum over no tokens
    hipLaunchKernelGGL(k_zero, dim3(grid_of(cdiv(d, WG), 64)), dim3(WG), 0, st, dq, d);
    return launched();
  }
  return ldr_reduce_rows(ws, parts, d, dq, stream);
}

int ldr_reduce_rows(const float* part, int64_t rows, int64_t d, float* out, void* stream) {
  if (!part || !out || rows < 1 || d < 1) return LDR_E_ARG;
  const unsigned grid = (unsigned)cdiv(d, 16);
  hipLaunchKernelGGL(k_reduce_rows, dim3(grid), dim3(WG), 0, static_cast<hipStream_t>(stream), part, rows, (int)d,
                     out);
  return launched();
}

int ldr_blend_sum(const uint64_t* g, int64_t m, float beta, int per_read, void* out, int64_t n_tok, int64_t d,
                  int dtype, void* stream) {
  if (!dtype_ok(dtype)) return LDR_E_DTYPE;
  if (per_read != 0 && per_read != 1) return LDR_E_ARG;
  if (m < 1 || m > MAXS) return LDR_E_SHAPE;
  if (!g || !tok_ptr(out, n_tok) || n_tok < 0) return LDR_E_ARG;
  if (!al16(out)) return LDR_E_ALIGN;
  PtrTab t;
  for (int64_t j = 0; j < MAXS; ++j) {
    t.p[j] = j < m ? reinterpret_cast<void*>(g[j]) : nullptr;
    if (j < m && !tok_ptr(t.p[j], n_tok)) return LDR_E_ARG;
    if (j < m && !al16(t.p[j])) return LDR_E_ALIGN;
  }
  int vpt, tpr, e = row_layout(d, &vpt, &tpr);
  if (e) return e;
  if (n_tok == 0) return LDR_OK;
  const unsigned grid = grid_of(cdiv(n_tok, WG / tpr), 4096);
  hipStream_t st = static_cast<hipStream_t>(stream);
  LDR_DTYPE_SWITCH(dtype, LDR_VPT_SWITCH(vpt, hipLaunchKernelGGL((k_blend_sum<T, VPT>), dim3(grid), dim3(WG), 0, st,
                                                                  t, (int)m, beta, per_read, static_cast<T*>(out),
                                                                  n_tok, (int)d, tpr)))
  return launched();
}

int ldr_read_bwd2_list(const uint64_t* dv, int64_t n, int accum, const void* g, const float* q, const float* wz,
                       int64_t wz_stride, int64_t n_tok, int64_t d, int dtype, void* stream) {
  if (!dtype_ok(dtype)) return LDR_E_DTYPE;
  if (!dv || n < 1 || n > MAXS || !tok_ptr(g, n_tok) || !q || !tok_ptr(wz, n_tok) || wz_stride < n_tok || n_tok < 0 ||
      (accum != 0 && accum != 1))
    return n > MAXS ? LDR_E_SHAPE : LDR_E_ARG;
  if (!al16(g) || !al16(q)) return LDR_E_ALIGN;
  PtrTab t;
  for (int64_t i = 0; i < MAXS; ++i) {
    t.p[i] = i < n ? reinterpret_cast<void*>(dv[i]) : nullptr;
    if (i < n && !tok_ptr(t.p[i], n_tok)) return LDR_E_ARG;
    if (i < n && !al16(t.p[i])) return LDR_E_ALIGN;
  }
  int vpt, tpr, e = row_layout(d, &vpt, &tpr);
  if (e) return e;
  if (n_tok == 0) return LDR_OK;
  const unsigned grid = grid_of(cdiv(n_tok, WG / tpr), 8192);
  hipStream_t st = static_cast<hipStream_t>(stream);
  LDR_DTYPE_SWITCH(dtype, LDR_VPT_SWITCH(vpt, hipLaunchKernelGGL((k_bwd2_list<T, VPT>), dim3(grid), dim3(WG), 0, st, t,
                                                                  (int)n, accum, static_cast<const T*>(g), q, wz,
                                                                  wz_stride, n_tok, (int)d, tpr)))
  return launched();
}

int ldr_dv_assemble(const uint64_t* g, const uint64_t* wz, const uint64_t* q, int64_t m, const void* v,
                    const float* r, const float* gr, const void* add, float add_beta, int per_read, void* dv,
                    void* dv_neg, int64_t n_tok, int64_t d, int dtype, void* stream) {
  if (!dtype_ok(dtype)) return LDR_E_DTYPE;
  if (per_read != 0 && per_read != 1) return LDR_E_ARG;
  if (m < 0 || m > MAXS) return LDR_E_SHAPE;
  if ((m > 0 && (!g || !wz || !q)) || !tok_ptr(v, n_tok) || !tok_ptr(r, n_tok) || !tok_ptr(dv, n_tok) || n_tok < 0)
    return LDR_E_ARG;
  if (!al16(v) || !al16(dv) || (dv_neg && !al16(dv_neg)) || (add && !al16(add))) return LDR_E_ALIGN;
  AsmTab t;
  for (int64_t j = 0; j < MAXS; ++j) {
    t.g[j] = j < m ? reinterpret_cast<const void*>(g[j]) : nullptr;
    t.wz[j] = j < m ? reinterpret_cast<const float*>(wz[j]) : nullptr;
    t.q[j] = j < m ? reinterpret_cast<const float*>(q[j]) : nullptr;
    if (j < m && (!tok_ptr(t.g[j], n_tok) || !tok_ptr(t.wz[j], n_tok) || !t.q[j])) return LDR_E_ARG;
    if (j < m && (!al16(t.g[j]) || !al16(t.q[j]) || (reinterpret_cast<uintptr_t>(t.wz[j]) & 7u))) return LDR_E_ALIGN;
  }
  const int max_vpt = dtype == LDR_F32 ? LDR_AS_MAX_VPT_F32 : LDR_AS_MAX_VPT;
  int vpt, tpr, e = row_layout(d, &vpt, &tpr, max_vpt, false, LDR_AS_VPT, true);
  if (e == LDR_E_SHAPE && !LDR_AS_VPT) e = row_layout(d, &vpt, &tpr, 4, false, 0, true);   // rows past 3 x 256 x 8
  if (e) return e;
  if (n_tok == 0) return LDR_OK;
  const unsigned grid = grid_of(cdiv(n_tok, (WG / tpr) * as_rb(vpt, dtype == LDR_F32)), LDR_AS_GRID);
  hipStream_t st = static_cast<hipStream_t>(stream);
  // the added gradient is often the last read's output gradient itself (the proposal of that read is this write's
  // h): then its rows are read once
  const bool add_last = add && m > 0 && add == t.g[m - 1];
#define LDR_AS_LAUNCH(AL, PR)                                                                                     \
  LDR_DTYPE_SWITCH(dtype, LDR_VPT_SWITCH(vpt, hipLaunchKernelGGL((k_dv_assemble<T, VPT, AL, PR>), dim3(grid), dim3(WG),\
                                                                  0, st, t, (int)m, static_cast<const T*>(v), r, gr, \
                                                                  static_cast<const T*>(add), add_beta,            \
                                                                  static_cast<T*>(dv), static_cast<T*>(dv_neg),    \
                                                                  n_tok, (int)d, tpr)))
  if (add_last && per_read) {
    LDR_AS_LAUNCH(true, true)
  } else if (add_last) {
    LDR_AS_LAUNCH(true, false)
  } else if (per_read) {
    LDR_AS_LAUNCH(false, true)
  } else {
    LDR_AS_LAUNCH(false, false)
  }
#undef LDR_AS_LAUNCH
  return launched();
}

// ---------------------------------------------------------------------------------------------------------------
// any-shape entry points: per-source addresses in device arrays, rows of any width at element alignment
// ---------------------------------------------------------------------------------------------------------------
static inline bool al_elt(const void* p, int dtype) {
  return (reinterpret_cast<uintptr_t>(p) & (uintptr_t)(elt_bytes(dtype) - 1)) == 0;
}
static inline unsigned any_row_grid(int64_t n_tok, int64_t cap) { return grid_of(cdiv(n_tok, ANY_WAVES), cap); }

int ldr_read_fwd_any(const uint64_t* src_v, const uint64_t* src_r, int64_t n, const float* q, float* dots,
                     int64_t dots_stride, const void* base, const void* h0, float beta, const float* cbar,
                     int64_t cbar_cols, const float* c0, int64_t c0_cols, float lam, float inv_sqrt_d, void* out,
                     float* tc, float* p, float* next_prior, int64_t n_tok, int64_t d, int dtype, void* stream) {
  if (!dtype_ok(dtype)) return LDR_E_DTYPE;
  if (n < 1 || n > ANY_MAXS || d < 1) return LDR_E_SHAPE;
  if (!src_v || !src_r || n_tok < 0 || !tok_ptr(dots, n_tok) || dots_stride < n_tok || !tok_ptr(base, n_tok) ||
      !tok_ptr(cbar, n_tok) || !c0 || !tok_ptr(out, n_tok) || !tok_ptr(tc, n_tok))
    return LDR_E_ARG;
  if ((cbar_cols != n && cbar_cols != n - 1) || (c0_cols != n && c0_cols != n - 1)) return LDR_E_ARG;
  if (!al_elt(base, dtype) || !al_elt(out, dtype) || (h0 && !al_elt(h0, dtype))) return LDR_E_ALIGN;
  if (n_tok == 0 && !next_prior) return LDR_OK;
  const Coef cf{cbar, (int)cbar_cols, c0, (int)c0_cols, lam};
  const size_t lds = sizeof(float) * (size_t)((3 + ANY_WAVES) * n + 4);
  const unsigned grid = any_row_grid(n_tok, 4096);   // no tokens: one workgroup writes next_prior
  hipStream_t st = static_cast<hipStream_t>(stream);
#define LDR_ANY_READ(BL)                                                                                          \
  LDR_DTYPE_SWITCH(dtype, hipLaunchKernelGGL((k_any_read<T, BL>), dim3(grid), dim3(WG), lds, st, src_v, src_r,    \
                                             (int)n, q, dots, dots_stride, static_cast<const T*>(base),           \
                                             static_cast<const T*>(h0), beta, cf, inv_sqrt_d, static_cast<T*>(out), \
                                             tc, p, next_prior, n_tok, d))
  if (h0) {
    LDR_ANY_READ(true)
  } else {
    LDR_ANY_READ(false)
  }
#undef LDR_ANY_READ
  return launched();
}

int ldr_read_bwd1_any(const uint64_t* src_v, const uint64_t* src_r, int64_t n, const void* g, const float* gt,
                      const float* p, const float* dots, int64_t dots_stride, const float* tc, const float* cbar,
                      int64_t cbar_cols, const float* c0, int64_t c0_cols, float lam, float inv_sqrt_d, float* dcbar,
                      int64_t dcbar_cols, const uint64_t* dr, int dr_accum, float* wz, int64_t wz_stride,
                      float* dq_part, int64_t dq_parts, int64_t dq_part_stride, void* g_prop, void* g_h0, float beta,
                      int64_t n_tok, int64_t d, int dtype, void* stream) {
  if (!dtype_ok(dtype)) return LDR_E_DTYPE;
  if (n < 1 || n > ANY_MAXS || d < 1) return LDR_E_SHAPE;
  if (!src_v || !src_r || n_tok < 0 || !tok_ptr(g, n_tok) || !tok_ptr(p, n_tok) || !tok_ptr(dots, n_tok) ||
      dots_stride < n_tok || !tok_ptr(tc, n_tok) || !tok_ptr(cbar, n_tok) || !c0 || !tok_ptr(dcbar, n_tok) || !dr ||
      !tok_ptr(wz, n_tok) || !dq_part || wz_stride < n_tok || dq_part_stride < d || dq_parts < 1 ||
      dq_parts > 65535 || (dr_accum != 0 && dr_accum != 1))
    return LDR_E_ARG;
  if ((cbar_cols != n && cbar_cols != n - 1) || (c0_cols != n && c0_cols != n - 1) || dcbar_cols < 0 ||
      dcbar_cols > n)
    return LDR_E_ARG;
  if (!al_elt(g, dtype) || (g_prop && !al_elt(g_prop, dtype)) || (g_h0 && !al_elt(g_h0, dtype)) ||
      (reinterpret_cast<uintptr_t>(wz) & 7u))
    return LDR_E_ALIGN;
  const Coef cf{cbar, (int)cbar_cols, c0, (int)c0_cols, lam};
  const size_t lds = sizeof(float) * (size_t)(4 * n);
  hipStream_t st = static_cast<hipStream_t>(stream);
  // every partial row is written (zeros for a workgroup without tokens), so the caller sums dq_parts rows
  LDR_DTYPE_SWITCH(dtype, hipLaunchKernelGGL((k_any_bwd1<T>), dim3((unsigned)dq_parts), dim3(64), lds, st, src_v,
                                             src_r, (int)n, static_cast<const T*>(g), gt, p, dots, dots_stride, tc,
                                             cf, inv_sqrt_d, dcbar, (int)dcbar_cols, dr, dr_accum, wz, wz_stride,
                                             dq_part, dq_part_stride, static_cast<T*>(g_prop), static_cast<T*>(g_h0),
                                             beta, n_tok, d))
  return launched();
}

int ldr_dv_assemble_any(const uint64_t* g, const uint64_t* wz, const uint64_t* q, int64_t m, const void* v,
                        const float* r, const float* gr, const void* add, float add_beta, int per_read, void* dv,
                        void* dv_neg, int64_t n_tok, int64_t d, int dtype, void* stream) {
  if (!dtype_ok(dtype)) return LDR_E_DTYPE;
  if (per_read != 0 && per_read != 1) return LDR_E_ARG;
  if (m < 0 || m > ANY_MAXS || d < 1) return LDR_E_SHAPE;
  if ((m > 0 && (!g || !wz || !q)) || !tok_ptr(v, n_tok) || !tok_ptr(r, n_tok) || !tok_ptr(dv, n_tok) || n_tok < 0)
    return LDR_E_ARG;
  if (!al_elt(v, dtype) || !al_elt(dv, dtype) || (dv_neg && !al_elt(dv_neg, dtype)) || (add && !al_elt(add, dtype)))
    return LDR_E_ALIGN;
  if (n_tok == 0) return LDR_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
#define LDR_ANY_AS(PR)                                                                                            \
  LDR_DTYPE_SWITCH(dtype, hipLaunchKernelGGL((k_any_dv_assemble<T, PR>), dim3(any_row_grid(n_tok, 8192)), dim3(WG), 0, \
                                             st, g, wz, q, (int)m, static_cast<const T*>(v), r, gr,                 \
                                             static_cast<const T*>(add), add_beta, static_cast<T*>(dv),             \
                                             static_cast<T*>(dv_neg), n_tok, d))
  if (per_read) {
    LDR_ANY_AS(true)
  } else {
    LDR_ANY_AS(false)
  }
#undef LDR_ANY_AS
  return launched();
}

int ldr_read_bwd2_list_any(const uint64_t* dv, int64_t n, int accum, const void* g, const float* q, const float* wz,
                           int64_t wz_stride, int64_t n_tok, int64_t d, int dtype, void* stream) {
  if (!dtype_ok(dtype)) return LDR_E_DTYPE;
  if (n < 1 || n > ANY_MAXS || d < 1) return LDR_E_SHAPE;
  if (!dv || !tok_ptr(g, n_tok) || !q || !tok_ptr(wz, n_tok) || wz_stride < n_tok || n_tok < 0 ||
      (accum != 0 && accum != 1))
    return LDR_E_ARG;
  if (!al_elt(g, dtype) || (reinterpret_cast<uintptr_t>(wz) & 7u)) return LDR_E_ALIGN;
  if (n_tok == 0) return LDR_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  LDR_DTYPE_SWITCH(dtype, hipLaunchKernelGGL((k_any_bwd2_list<T>), dim3(any_row_grid(n_tok, 8192)), dim3(WG), 0, st,
                                             dv, (int)n, accum, static_cast<const T*>(g), q, wz, wz_stride, n_tok, d))
  return launched();
}

int ldr_blend_sum_any(const uint64_t* g, int64_t m, float beta, int per_read, void* out, int64_t n_tok, int64_t d,
                      int dtype, void* stream) {
  if (!dtype_ok(dtype)) return LDR_E_DTYPE;
  if (per_read != 0 && per_read != 1) return LDR_E_ARG;
  if (m < 1 || m > ANY_MAXS || d < 1) return LDR_E_SHAPE;
  if (!g || !tok_ptr(out, n_tok) || n_tok < 0) return LDR_E_ARG;
  if (!al_elt(out, dtype)) return LDR_E_ALIGN;
  if (n_tok == 0) return LDR_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  LDR_DTYPE_SWITCH(dtype, hipLaunchKernelGGL((k_any_blend_sum<T>), dim3(grid_of(cdiv(n_tok * d, WG), 8192)), dim3(WG),
                                             0, st, g, (int)m, beta, per_read, static_cast<T*>(out), n_tok, d))
  return launched();
}

}  // extern "C"
