// stream_probe.hip -- what HBM streaming the box sustains for the read kernels' access patterns.
//
// The read kernels stream n sources row by row (one 16-byte vector per lane, rows of 4 KiB) and write at most a few
// rows per row set. These probes do the same with no arithmetic: read the n sources (XOR-folded so the loads are
// not dead), optionally write one row per row set (right after its reads, or batched 16 row sets at a time); the
// write step's two-in, one-out traffic in its own layout and in whole rows; and a plain device copy. bench-side code (stream_probe.py) times
// them to give the practical ceiling each kernel's read/write mix allows, next to the 8 TB/s peak.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int MAXP = 64;
constexpr int ROWV = 256;   // 16-byte vectors per row: 4 KiB rows, one vector per lane of a 256-lane workgroup
struct Tab { const u32x4* p[MAXP]; };

// n sources of `rows` rows; with out != nullptr one row written per row set (the read forward's mix)
__global__ __launch_bounds__(256) void k_probe_read(Tab t, int n, int64_t rows, u32x4* __restrict__ out,
                                                    unsigned* __restrict__ sink) {
  const int lane = (int)threadIdx.x;
  unsigned s = 0;
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    u32x4 acc = {0u, 0u, 0u, 0u};
    int i = 0;
    for (; i + 8 <= n; i += 8) {
      u32x4 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = __builtin_nontemporal_load(t.p[i + u] + row * ROWV + lane);
#pragma unroll
      for (int u = 0; u < 8; ++u) acc ^= v[u];
    }
    for (; i < n; ++i) acc ^= __builtin_nontemporal_load(t.p[i] + row * ROWV + lane);
    if (out) out[row * ROWV + lane] = acc;
    s ^= acc.x ^ acc.y ^ acc.z ^ acc.w;
  }
  if (s == 0x9e3779b9u) sink[0] = s;   // never true for the probe's data; keeps the loads live
}

// the same mix with the written rows batched: the out rows of 16 consecutive row sets are kept in LDS and written
// together after the set's reads, one contiguous 64 KiB region (the stored-score read's staged output)
constexpr int BURST = 16;
__global__ __launch_bounds__(256) void k_probe_read_burst(Tab t, int n, int64_t rows, u32x4* __restrict__ out,
                                                          unsigned* __restrict__ sink) {
  __shared__ u32x4 s_out[BURST][ROWV];
  const int lane = (int)threadIdx.x;
  unsigned s = 0;
  for (int64_t blk = blockIdx.x; blk < rows / BURST; blk += gridDim.x) {
    for (int r = 0; r < BURST; ++r) {
      const int64_t row = blk * BURST + r;
      u32x4 acc = {0u, 0u, 0u, 0u};
      int i = 0;
      for (; i + 8 <= n; i += 8) {
        u32x4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = __builtin_nontemporal_load(t.p[i + u] + row * ROWV + lane);
#pragma unroll
        for (int u = 0; u < 8; ++u) acc ^= v[u];
      }
      for (; i < n; ++i) acc ^= __builtin_nontemporal_load(t.p[i] + row * ROWV + lane);
      s_out[r][lane] = acc;
      s ^= acc.x ^ acc.y ^ acc.z ^ acc.w;
    }
    for (int r = 0; r < BURST; ++r) out[(blk * BURST + r) * ROWV + lane] = s_out[r][lane];   // this lane's own
  }
  if (s == 0x9e3779b9u) sink[0] = s;
}

// the write step's traffic without its arithmetic: v = h ^ x over T rows of 2048 bf16 (two rows in, one out per
// token), 64 tokens per workgroup. Chunked: the write kernel's layout -- 4 waves take 64-column chunks c = w, w+4, ...;
// in a chunk, lane (row l % 16, quad l / 16) moves 16 bytes at columns 8 quad and 32 + 8 quad of four 16-row blocks,
// 128 bytes of each row. Rows: each wave moves 16 whole rows (4 vectors per lane, 1 KiB per instruction).
constexpr int WD = 2048;
__global__ __launch_bounds__(256) void k_probe_write_chunked(const u32x4* __restrict__ h, const u32x4* __restrict__ x,
                                                             u32x4* __restrict__ v) {
  const int tid = (int)threadIdx.x, w = tid >> 6, l = tid & 63, row = l & 15, quad = l >> 4;
  const int64_t t0 = (int64_t)blockIdx.x * 64;
  for (int c = w; c < WD / 64; c += 4) {
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int64_t e = ((t0 + 16 * mb + row) * WD + c * 64 + quad * 8 + 32 * hf) / 8;   // 16-byte units
        __builtin_nontemporal_store(h[e] ^ x[e], v + e);
      }
  }
}
__global__ __launch_bounds__(256) void k_probe_write_rows(const u32x4* __restrict__ h, const u32x4* __restrict__ x,
                                                          u32x4* __restrict__ v) {
  const int tid = (int)threadIdx.x, w = tid >> 6, l = tid & 63;
  const int64_t t0 = (int64_t)blockIdx.x * 64;
  for (int r = w; r < 64; r += 4) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int64_t e = (t0 + r) * (WD / 8) + k * 64 + l;
      __builtin_nontemporal_store(h[e] ^ x[e], v + e);
    }
  }
}

__global__ __launch_bounds__(256) void k_probe_copy(const u32x4* __restrict__ a, u32x4* __restrict__ b, int64_t n) {
  for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    b[i] = __builtin_nontemporal_load(a + i);
}

}  // namespace

extern "C" {

// Read n sources (host array of n device addresses, each `rows` rows of 4 KiB, 16-byte aligned), writing one row
// per row set to out when out != NULL; grid workgroups of 256 lanes. Returns 0 or a hipError_t / -1 on bad input.
int ldp_read(const uint64_t* src, int n, int64_t rows, void* out, void* sink, int grid, void* stream) {
  if (!src || n < 1 || n > MAXP || rows < 1 || !sink || grid < 1) return -1;
  Tab t;
  for (int i = 0; i < MAXP; ++i) t.p[i] = i < n ? reinterpret_cast<const u32x4*>(src[i]) : nullptr;
  for (int i = 0; i < n; ++i)
    if (!t.p[i] || (reinterpret_cast<uintptr_t>(t.p[i]) & 15u)) return -1;
  hipLaunchKernelGGL(k_probe_read, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream), t, n, rows,
                     static_cast<u32x4*>(out), static_cast<unsigned*>(sink));
  return (int)hipGetLastError();
}

// As ldp_read with out required, the written rows batched 16 row sets at a time (rows a multiple of 16).
int ldp_read_burst(const uint64_t* src, int n, int64_t rows, void* out, void* sink, int grid, void* stream) {
  if (!src || n < 1 || n > MAXP || rows < BURST || (rows % BURST) || !out || !sink || grid < 1) return -1;
  Tab t;
  for (int i = 0; i < MAXP; ++i) t.p[i] = i < n ? reinterpret_cast<const u32x4*>(src[i]) : nullptr;
  for (int i = 0; i < n; ++i)
    if (!t.p[i] || (reinterpret_cast<uintptr_t>(t.p[i]) & 15u)) return -1;
  if (reinterpret_cast<uintptr_t>(out) & 15u) return -1;
  hipLaunchKernelGGL(k_probe_read_burst, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream), t, n, rows,
                     static_cast<u32x4*>(out), static_cast<unsigned*>(sink));
  return (int)hipGetLastError();
}

// v = h ^ x over `rows` rows of 2048 bf16 (rows a multiple of 64, 16-byte aligned): which = 0 in the write kernel's
// chunked layout, 1 in whole rows per wave.
int ldp_write(const void* h, const void* x, void* v, int64_t rows, int which, void* stream) {
  if (!h || !x || !v || rows < 64 || (rows % 64) || (which != 0 && which != 1)) return -1;
  if ((reinterpret_cast<uintptr_t>(h) | reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(v)) & 15u) return -1;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (which == 0)
    hipLaunchKernelGGL(k_probe_write_chunked, dim3((unsigned)(rows / 64)), dim3(256), 0, st,
                       static_cast<const u32x4*>(h), static_cast<const u32x4*>(x), static_cast<u32x4*>(v));
  else
    hipLaunchKernelGGL(k_probe_write_rows, dim3((unsigned)(rows / 64)), dim3(256), 0, st,
                       static_cast<const u32x4*>(h), static_cast<const u32x4*>(x), static_cast<u32x4*>(v));
  return (int)hipGetLastError();
}

// b[0:bytes] = a[0:bytes] (bytes a multiple of 16).
int ldp_copy(const void* a, void* b, int64_t bytes, int grid, void* stream) {
  if (!a || !b || bytes < 16 || (bytes & 15) || grid < 1) return -1;
  hipLaunchKernelGGL(k_probe_copy, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const u32x4*>(a), static_cast<u32x4*>(b), bytes / 16);
  return (int)hipGetLastError();
}

}  // extern "C"
