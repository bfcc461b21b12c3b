// Row softmax forward and backward for gfx950.
//
// Forward  (python/intent/examples/kernels/normalization/softmax.py:12-66):
//   m = maximum_num over the row, e = exp(x - m), s = sum(e)
//   f32:        y = e * (1 / s)
//   f16, bf16:  y = cast(e / s)          (f32 math, round-to-nearest-even cast)
// Backward (python/intent/examples/kernels/backward/softmax.py:9-25):
//   proj = sum(p * dy), dx = p * (dy - proj)   (f32 accumulation; f16 storage variant casts)
//
// Design: one wavefront owns one row at a time. The row is loaded once with
// 128-bit loads (lane l of chunk c reads columns [(64c + l) * V, +V)), held in registers,
// reduced with DPP (no LDS, no barrier), and written once: one HBM read and one write per
// element, the minimum. f16 rows are held as their raw 16-bit words where that frees registers
// (x until its exponentials replace it, dy throughout), which raises the waves per SIMD.
// The 16-bit forward of rows up to 64 * 64 * 8 elements is persistent: a grid of as many waves
// as the device holds at once walks the rows with a grid stride, and each wave loads its next row
// before it computes the current one, so the reads of one row overlap the exponentials of the
// previous (16384 x 4096 f16: 46.7 against 52 us, bit-identical; one wave per row and launch
// leaves HBM idle while a whole round of waves computes).
// Rows longer than the register-resident limit, or rows whose layout rules out 128-bit
// access, use a scalar variant; rows longer than 64 * 64 scalar elements use a streaming
// variant that re-reads the row (3 passes forward, 2 backward).
#include <math.h>

#include <algorithm>
#include <mutex>
#include <type_traits>

#include "common.hpp"

namespace intent_hip {
namespace {

constexpr int kRowsPerBlock = 2;
constexpr int kBlock = kRowsPerBlock * kWave;
constexpr float kLog2e = 1.4426950408889634f;

// ---------------------------------------------------------------- vector load / store
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// 16-bit rows are read with non-temporal loads (each element is read once) and 128-bit accesses.
template <typename T, int V>
__device__ __forceinline__ void load_row_chunk(const T *p, float (&out)[V]) {
  if constexpr (V == 1) {
    out[0] = to_f32(p[0]);
  } else if constexpr (sizeof(T) == 4) {
    static_assert(V == 4, "f32 vectors hold 4 elements");
    const float4 raw = *reinterpret_cast<const float4 *>(p);
    out[0] = raw.x; out[1] = raw.y; out[2] = raw.z; out[3] = raw.w;
  } else {
    static_assert(V == 8, "16-bit vectors hold 8 elements");
    const u32x4_t raw = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = to_f32(T{static_cast<uint16_t>(raw[i] & 0xffffu)});
      out[2 * i + 1] = to_f32(T{static_cast<uint16_t>(raw[i] >> 16)});
    }
  }
}

// kStream selects non-temporal stores. The forward stores normally: in the forward -> backward
// sequence its output is the backward's input and may still be in the MALL when it is read. The
// backward's output is not read again and is streamed. Measured on the 16384 x 4096 f16 step
// (graph replays): 118.9 us with this choice, 126.0 us with both streamed, 136.1 us with
// neither.
template <typename T, int V, bool kStream>
__device__ __forceinline__ void store_row_chunk(T *p, const float (&in)[V]) {
  if constexpr (V == 1) {
    p[0] = from_f32<T>(in[0]);
  } else if constexpr (sizeof(T) == 4) {
    const f32x4_t v = {in[0], in[1], in[2], in[3]};
    if constexpr (kStream) __builtin_nontemporal_store(v, reinterpret_cast<f32x4_t *>(p));
    else *reinterpret_cast<f32x4_t *>(p) = v;
  } else {
    u32x4_t w;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = static_cast<uint32_t>(from_f32<T>(in[2 * i]).bits) |
             (static_cast<uint32_t>(from_f32<T>(in[2 * i + 1]).bits) << 16);
    if constexpr (kStream) __builtin_nontemporal_store(w, reinterpret_cast<u32x4_t *>(p));
    else *reinterpret_cast<u32x4_t *>(p) = w;
  }
}

// ---------------------------------------------------------------- element math
// exp(x - m). The f32 operator uses the library exp (ordinary IEEE f32 exp of
// x - m, ~1 ulp). The 16-bit operators round their result to 11 or 8 significant
// bits, so they use the hardware 2^x on (x - m) * log2(e): relative error below
// 4e-6 for |x - m| <= 60, far inside one f16 ulp.
template <typename T>
__device__ __forceinline__ float shifted_exp(float x, float m) {
  if constexpr (sizeof(T) == 4) {
    return expf(x - m);
  } else {
    return __builtin_amdgcn_exp2f((x - m) * kLog2e);
  }
}

// e / s for the 16-bit outputs: the quotient e * (1/s) corrected by one residual
// step, which gives the correctly rounded f32 quotient for these operand ranges
// (0 <= e <= 1 <= s), followed by the round-to-nearest-even cast.
__device__ __forceinline__ float quotient(float e, float s, float r) {
  const float q = e * r;
  return fmaf(fmaf(-q, s, e), r, q);
}

// ---------------------------------------------------------------- raw 16-bit rows
// The raw 16-bit words of one 16-byte chunk (8 elements), read once, and element i widened.
__device__ __forceinline__ u32x4_t load_words(const void *p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
}
template <typename T>
__device__ __forceinline__ float widen(const u32x4_t &w, int i) {
  const uint32_t word = w[i >> 1];
  return to_f32(T{static_cast<uint16_t>((i & 1) ? (word >> 16) : (word & 0xffffu))});
}

// ---------------------------------------------------------------- forward, persistent 16-bit rows
constexpr int kPipeBlock = 256;   // 4 waves, each its own row stream

// The raw words of one row (CHUNKS 16-byte chunks per lane; chunks past the row read column 0).
template <typename T, int CHUNKS>
__device__ __forceinline__ void load_row_words(const T *xr, int cols, int lane, u32x4_t (&w)[CHUNKS]) {
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c) {
    const int col = (c * kWave + lane) * 8;
    w[c] = load_words(xr + (col < cols ? col : 0));
  }
}

template <typename T, int CHUNKS>
__global__ __launch_bounds__(kPipeBlock) void softmax_fwd_pipe(const T *x, T *y, int64_t rows, int cols,
                                                               int64_t xs, int64_t ys) {
  constexpr int V = 8;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t stride = static_cast<int64_t>(gridDim.x) * (kPipeBlock / kWave);
  int64_t row = static_cast<int64_t>(blockIdx.x) * (kPipeBlock / kWave) + (threadIdx.x >> 6);
  if (row >= rows) return;  // wave-uniform
  u32x4_t cur[CHUNKS];
  load_row_words<T, CHUNKS>(x + row * xs, cols, lane, cur);
  for (; row < rows; row += stride) {
    const int64_t next = row + stride;   // wave-uniform
    u32x4_t nxt[CHUNKS];
    if (next < rows) load_row_words<T, CHUNKS>(x + next * xs, cols, lane, nxt);
    float m = -INFINITY;
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
      const bool live = (c * kWave + lane) * V < cols;
#pragma unroll
      for (int i = 0; i < V; ++i) m = live ? fmaxf(m, widen<T>(cur[c], i)) : m;
    }
    m = wave_max(m);
    float v[CHUNKS][V];
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
      const bool live = (c * kWave + lane) * V < cols;
#pragma unroll
      for (int i = 0; i < V; ++i) {
        v[c][i] = live ? shifted_exp<T>(widen<T>(cur[c], i), m) : 0.0f;
        s += v[c][i];
      }
    }
    s = wave_sum(s);
    const float r = 1.0f / s;
    T *yr = y + row * ys;
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
      const int col = (c * kWave + lane) * V;
      if (col < cols) {
        float o[V];
#pragma unroll
        for (int i = 0; i < V; ++i) o[i] = quotient(v[c][i], s, r);
        store_row_chunk<T, V, false>(yr + col, o);
      }
    }
    if (next < rows) {
#pragma unroll
      for (int c = 0; c < CHUNKS; ++c) cur[c] = nxt[c];
    }
  }
}

// ---------------------------------------------------------------- forward, register resident
template <typename T, int V, int CHUNKS>
__global__ __launch_bounds__(kBlock) void softmax_fwd_wave(const T *x, T *y, int64_t rows, int cols,
                                                           int64_t xs, int64_t ys) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;  // wave-uniform
  const T *xr = x + row * xs;
  if constexpr (std::is_same<T, f16_t>::value && V == 8) {
    // x stays in its raw f16 words until the exponentials replace it: 79 VGPRs instead of 90,
    // six waves per SIMD instead of five (forward of the 16384 x 4096 step, bit-identical:
    // 51.2 against 53.4 us). Loads are unconditional, as in the backward.
    u32x4_t xw[CHUNKS];
    float m = -INFINITY;
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
      const int col = (c * kWave + lane) * V;
      const bool live = col < cols;
      xw[c] = load_words(xr + (live ? col : 0));
#pragma unroll
      for (int i = 0; i < V; ++i) m = live ? fmaxf(m, widen<T>(xw[c], i)) : m;
    }
    m = wave_max(m);
    float v[CHUNKS][V];
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
      const bool live = (c * kWave + lane) * V < cols;
#pragma unroll
      for (int i = 0; i < V; ++i) {
        v[c][i] = live ? shifted_exp<T>(widen<T>(xw[c], i), m) : 0.0f;
        s += v[c][i];
      }
    }
    s = wave_sum(s);
    const float r = 1.0f / s;
    T *yr = y + row * ys;
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
      const int col = (c * kWave + lane) * V;
      if (col < cols) {
        float o[V];
#pragma unroll
        for (int i = 0; i < V; ++i) o[i] = quotient(v[c][i], s, r);
        store_row_chunk<T, V, false>(yr + col, o);
      }
    }
    return;
  }
  float v[CHUNKS][V];
  float m = -INFINITY;
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c) {
    const int col = (c * kWave + lane) * V;
    if (col < cols) {
      load_row_chunk<T, V>(xr + col, v[c]);
    } else {
#pragma unroll
      for (int i = 0; i < V; ++i) v[c][i] = -INFINITY;
    }
#pragma unroll
    for (int i = 0; i < V; ++i) m = fmaxf(m, v[c][i]);
  }
  m = wave_max(m);
  float s = 0.0f;
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c) {
    const bool live = (c * kWave + lane) * V < cols;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      v[c][i] = live ? shifted_exp<T>(v[c][i], m) : 0.0f;
      s += v[c][i];
    }
  }
  s = wave_sum(s);
  const float r = 1.0f / s;
  T *yr = y + row * ys;
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c) {
    const int col = (c * kWave + lane) * V;
    if (col < cols) {
      float o[V];
#pragma unroll
      for (int i = 0; i < V; ++i) o[i] = sizeof(T) == 4 ? v[c][i] * r : quotient(v[c][i], s, r);
      store_row_chunk<T, V, false>(yr + col, o);
    }
  }
}

// ---------------------------------------------------------------- forward, streaming
template <typename T>
__global__ __launch_bounds__(kBlock) void softmax_fwd_stream(const T *x, T *y, int64_t rows, int cols,
                                                             int64_t xs, int64_t ys) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T *xr = x + row * xs;
  float m = -INFINITY;
  for (int c = lane; c < cols; c += kWave) m = fmaxf(m, to_f32(xr[c]));
  m = wave_max(m);
  float s = 0.0f;
  for (int c = lane; c < cols; c += kWave) s += shifted_exp<T>(to_f32(xr[c]), m);
  s = wave_sum(s);
  const float r = 1.0f / s;
  T *yr = y + row * ys;
  for (int c = lane; c < cols; c += kWave) {
    const float e = shifted_exp<T>(to_f32(xr[c]), m);
    yr[c] = from_f32<T>(sizeof(T) == 4 ? e * r : quotient(e, s, r));
  }
}

// ---------------------------------------------------------------- backward, register resident
template <typename T, int V, int CHUNKS>
__global__ __launch_bounds__(kBlock) void softmax_bwd_wave(const T *p, const T *dy, T *dx, int64_t rows,
                                                           int cols, int64_t ps, int64_t dys,
                                                           int64_t dxs) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T *pr = p + row * ps;
  const T *gr = dy + row * dys;
  if constexpr (std::is_same<T, f16_t>::value && V == 8) {
    // dy stays in its raw f16 words and is widened where it is used (the FMAs take f16 operands
    // directly, v_fma_mix_f32): 81 VGPRs instead of 141, five waves per SIMD instead of three.
    // Backward of the 16384 x 4096 step, bit-identical outputs: 62.0 us, against 75.7 with both
    // rows widened at load and 68.0 with both kept raw (77 VGPRs, six waves). Every chunk is
    // loaded; one past the row end re-reads the row start and stays out of the projection
    // (conditional loads make the compiler keep widened copies live).
    float pv[CHUNKS][V];
    u32x4_t gw[CHUNKS];
    float proj = 0.0f;
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
      const int col = (c * kWave + lane) * V;
      const bool live = col < cols;
      const int at = live ? col : 0;
      load_row_chunk<T, V>(pr + at, pv[c]);
      gw[c] = load_words(gr + at);
#pragma unroll
      for (int i = 0; i < V; ++i) proj = live ? fmaf(pv[c][i], widen<T>(gw[c], i), proj) : proj;
    }
    proj = wave_sum(proj);
    T *dr = dx + row * dxs;
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
      const int col = (c * kWave + lane) * V;
      if (col < cols) {
        float o[V];
#pragma unroll
        for (int i = 0; i < V; ++i) o[i] = pv[c][i] * (widen<T>(gw[c], i) - proj);
        store_row_chunk<T, V, true>(dr + col, o);
      }
    }
    return;
  }
  float pv[CHUNKS][V], gv[CHUNKS][V];
  float proj = 0.0f;
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c) {
    const int col = (c * kWave + lane) * V;
    if (col < cols) {
      load_row_chunk<T, V>(pr + col, pv[c]);
      load_row_chunk<T, V>(gr + col, gv[c]);
    } else {
#pragma unroll
      for (int i = 0; i < V; ++i) pv[c][i] = gv[c][i] = 0.0f;
    }
#pragma unroll
    for (int i = 0; i < V; ++i) proj = fmaf(pv[c][i], gv[c][i], proj);
  }
  proj = wave_sum(proj);
  T *dr = dx + row * dxs;
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c) {
    const int col = (c * kWave + lane) * V;
    if (col < cols) {
      float o[V];
#pragma unroll
      for (int i = 0; i < V; ++i) o[i] = pv[c][i] * (gv[c][i] - proj);
      store_row_chunk<T, V, true>(dr + col, o);
    }
  }
}

template <typename T>
__global__ __launch_bounds__(kBlock) void softmax_bwd_stream(const T *p, const T *dy, T *dx, int64_t rows,
                                                             int cols, int64_t ps, int64_t dys,
                                                             int64_t dxs) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T *pr = p + row * ps;
  const T *gr = dy + row * dys;
  float proj = 0.0f;
  for (int c = lane; c < cols; c += kWave) proj = fmaf(to_f32(pr[c]), to_f32(gr[c]), proj);
  proj = wave_sum(proj);
  T *dr = dx + row * dxs;
  for (int c = lane; c < cols; c += kWave) {
    const float pc = to_f32(pr[c]);
    dr[c] = from_f32<T>(pc * (to_f32(gr[c]) - proj));
  }
}

// ---------------------------------------------------------------- variant selection
// Register-resident limits: 16 vector chunks (f32: 4096 columns, 16-bit: 8192) or
// 64 scalar chunks (4096 columns); anything longer streams.
struct Variant {
  const void *kernel;
  const char *name;
  int block = kBlock;         // threads per workgroup
  bool persistent = false;    // grid of resident waves walking the rows (rows per wave: any)
};

template <typename T>
Variant pick_fwd_pipe(int chunks) {
  switch (chunks) {
    case 1: return {reinterpret_cast<const void *>(&softmax_fwd_pipe<T, 1>), "softmax_fwd_pipe", kPipeBlock, true};
    case 2: return {reinterpret_cast<const void *>(&softmax_fwd_pipe<T, 2>), "softmax_fwd_pipe", kPipeBlock, true};
    case 4: return {reinterpret_cast<const void *>(&softmax_fwd_pipe<T, 4>), "softmax_fwd_pipe", kPipeBlock, true};
    default: return {reinterpret_cast<const void *>(&softmax_fwd_pipe<T, 8>), "softmax_fwd_pipe", kPipeBlock, true};
  }
}

template <typename T, int V>
Variant pick_fwd(int chunks) {
  switch (chunks) {
    case 1: return {reinterpret_cast<const void *>(&softmax_fwd_wave<T, V, 1>), "softmax_fwd_wave"};
    case 2: return {reinterpret_cast<const void *>(&softmax_fwd_wave<T, V, 2>), "softmax_fwd_wave"};
    case 4: return {reinterpret_cast<const void *>(&softmax_fwd_wave<T, V, 4>), "softmax_fwd_wave"};
    case 8: return {reinterpret_cast<const void *>(&softmax_fwd_wave<T, V, 8>), "softmax_fwd_wave"};
    case 16: return {reinterpret_cast<const void *>(&softmax_fwd_wave<T, V, 16>), "softmax_fwd_wave"};
    case 32:
      if constexpr (V == 1) return {reinterpret_cast<const void *>(&softmax_fwd_wave<T, 1, 32>), "softmax_fwd_wave"};
      break;
    case 64:
      if constexpr (V == 1) return {reinterpret_cast<const void *>(&softmax_fwd_wave<T, 1, 64>), "softmax_fwd_wave"};
      break;
  }
  return {reinterpret_cast<const void *>(&softmax_fwd_stream<T>), "softmax_fwd_stream"};
}

template <typename T, int V>
Variant pick_bwd(int chunks) {
  switch (chunks) {
    case 1: return {reinterpret_cast<const void *>(&softmax_bwd_wave<T, V, 1>), "softmax_bwd_wave"};
    case 2: return {reinterpret_cast<const void *>(&softmax_bwd_wave<T, V, 2>), "softmax_bwd_wave"};
    case 4: return {reinterpret_cast<const void *>(&softmax_bwd_wave<T, V, 4>), "softmax_bwd_wave"};
    case 8: return {reinterpret_cast<const void *>(&softmax_bwd_wave<T, V, 8>), "softmax_bwd_wave"};
    case 16: return {reinterpret_cast<const void *>(&softmax_bwd_wave<T, V, 16>), "softmax_bwd_wave"};
    case 32:
      if constexpr (V == 1) return {reinterpret_cast<const void *>(&softmax_bwd_wave<T, 1, 32>), "softmax_bwd_wave"};
      break;
    case 64:
      if constexpr (V == 1) return {reinterpret_cast<const void *>(&softmax_bwd_wave<T, 1, 64>), "softmax_bwd_wave"};
      break;
  }
  return {reinterpret_cast<const void *>(&softmax_bwd_stream<T>), "softmax_bwd_stream"};
}

int round_chunks(int64_t cols, int per_chunk) {
  const int64_t needed = (cols + per_chunk - 1) / per_chunk;
  int chunks = 1;
  while (chunks < needed) chunks <<= 1;
  return chunks;
}

template <typename T>
Variant select_fwd(const void *x, const void *y, int64_t cols, int64_t xs, int64_t ys) {
  constexpr int kVec = 16 / sizeof(T);
  const bool vector = cols % kVec == 0 && xs % kVec == 0 && ys % kVec == 0 && aligned(x, 16) && aligned(y, 16);
  if (vector) {
    const int chunks = round_chunks(cols, kWave * kVec);
    if constexpr (sizeof(T) == 2)
      if (chunks <= 8) return pick_fwd_pipe<T>(chunks);
    return chunks <= 16 ? pick_fwd<T, kVec>(chunks) : pick_fwd<T, kVec>(0);
  }
  const int chunks = round_chunks(cols, kWave);
  return chunks <= 64 ? pick_fwd<T, 1>(chunks) : pick_fwd<T, 1>(0);
}

template <typename T>
Variant select_bwd(const void *p, const void *dy, const void *dx, int64_t cols, int64_t ps, int64_t dys,
                   int64_t dxs) {
  constexpr int kVec = 16 / sizeof(T);
  const bool vector = cols % kVec == 0 && ps % kVec == 0 && dys % kVec == 0 && dxs % kVec == 0 &&
                      aligned(p, 16) && aligned(dy, 16) && aligned(dx, 16);
  if (vector) {
    const int chunks = round_chunks(cols, kWave * kVec);
    return chunks <= 16 ? pick_bwd<T, kVec>(chunks) : pick_bwd<T, kVec>(0);
  }
  const int chunks = round_chunks(cols, kWave);
  return chunks <= 64 ? pick_bwd<T, 1>(chunks) : pick_bwd<T, 1>(0);
}

// Input rows may overlap (any non-negative stride, e.g. a broadcast row); output
// rows may not.
int check_extents(int64_t rows, int64_t cols, int64_t in0, int64_t in1, int64_t out) {
  if (rows < 0 || cols < 0) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "negative extent");
  if (cols > INT32_MAX) return fail(INTENT_HIP_ERR_UNSUPPORTED, "softmax rows longer than 2^31-1 columns");
  if (rows > static_cast<int64_t>(UINT32_MAX) * kRowsPerBlock)
    return fail(INTENT_HIP_ERR_UNSUPPORTED, "too many softmax rows for one launch");
  if (in0 < 0 || in1 < 0) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "negative row stride");
  if (rows > 1 && out < cols)
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "output row stride smaller than the row length (overlapping rows)");
  return INTENT_HIP_OK;
}

template <typename T>
int launch_fwd(const void *x, void *y, int64_t rows, int64_t cols, int64_t xs, int64_t ys, hipStream_t stream) {
  const Variant v = select_fwd<T>(x, y, cols, xs, ys);
  const int rows_per_block = v.block / kWave;
  int64_t blocks = (rows + rows_per_block - 1) / rows_per_block;
  if (v.persistent) blocks = std::min<int64_t>(blocks, resident_blocks(v.kernel, v.block));
  const dim3 grid(static_cast<unsigned>(blocks));
  int icols = static_cast<int>(cols);
  void *args[] = {const_cast<void **>(&x), &y, &rows, &icols, &xs, &ys};
  if (hipLaunchKernel(v.kernel, grid, dim3(v.block), args, 0, stream) != hipSuccess) return launch_status(v.name);
  return INTENT_HIP_OK;
}

template <typename T>
int launch_bwd(const void *p, const void *dy, void *dx, int64_t rows, int64_t cols, int64_t ps, int64_t dys,
               int64_t dxs, hipStream_t stream) {
  const Variant v = select_bwd<T>(p, dy, dx, cols, ps, dys, dxs);
  const dim3 grid(static_cast<unsigned>((rows + kRowsPerBlock - 1) / kRowsPerBlock));
  int icols = static_cast<int>(cols);
  void *args[] = {const_cast<void **>(&p), const_cast<void **>(&dy), &dx, &rows, &icols, &ps, &dys, &dxs};
  if (hipLaunchKernel(v.kernel, grid, dim3(kBlock), args, 0, stream) != hipSuccess) return launch_status(v.name);
  return INTENT_HIP_OK;
}

}  // namespace

int softmax_fwd_resources(int dtype, int64_t rows, int64_t cols, IntentHipKernelResources *out) {
  (void)rows;
  // Resources of the 16-byte-aligned, contiguous variant for this row length.
  Variant v;
  switch (dtype) {
    case INTENT_HIP_F32: v = select_fwd<float>(nullptr, nullptr, cols, cols, cols); break;
    case INTENT_HIP_F16: v = select_fwd<f16_t>(nullptr, nullptr, cols, cols, cols); break;
    case INTENT_HIP_BF16: v = select_fwd<bf16_t>(nullptr, nullptr, cols, cols, cols); break;
    default: return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "unknown dtype code %d", dtype);
  }
  return describe_kernel(v.kernel, v.name, v.block, out);
}

int softmax_bwd_resources(int dtype, int64_t rows, int64_t cols, IntentHipKernelResources *out) {
  (void)rows;
  Variant v;
  switch (dtype) {
    case INTENT_HIP_F32: v = select_bwd<float>(nullptr, nullptr, nullptr, cols, cols, cols, cols); break;
    case INTENT_HIP_F16: v = select_bwd<f16_t>(nullptr, nullptr, nullptr, cols, cols, cols, cols); break;
    case INTENT_HIP_BF16: v = select_bwd<bf16_t>(nullptr, nullptr, nullptr, cols, cols, cols, cols); break;
    default: return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "unknown dtype code %d", dtype);
  }
  return describe_kernel(v.kernel, v.name, kBlock, out);
}

}  // namespace intent_hip

using namespace intent_hip;

extern "C" int intent_hip_softmax_fwd(int dtype, const void *x, void *y, int64_t rows, int64_t cols,
                                      int64_t x_row_stride, int64_t y_row_stride, void *stream) {
  if (int status = check_extents(rows, cols, x_row_stride, x_row_stride, y_row_stride)) return status;
  if (rows == 0 || cols == 0) return INTENT_HIP_OK;
  if (x == nullptr || y == nullptr) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "null tensor pointer");
  switch (dtype) {
    case INTENT_HIP_F32: return launch_fwd<float>(x, y, rows, cols, x_row_stride, y_row_stride, as_stream(stream));
    case INTENT_HIP_F16: return launch_fwd<f16_t>(x, y, rows, cols, x_row_stride, y_row_stride, as_stream(stream));
    case INTENT_HIP_BF16: return launch_fwd<bf16_t>(x, y, rows, cols, x_row_stride, y_row_stride, as_stream(stream));
  }
  return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "unknown dtype code %d", dtype);
}

extern "C" int intent_hip_softmax_bwd(int dtype, const void *p, const void *dy, void *dx, int64_t rows,
                                      int64_t cols, int64_t p_row_stride, int64_t dy_row_stride,
                                      int64_t dx_row_stride, void *stream) {
  if (int status = check_extents(rows, cols, p_row_stride, dy_row_stride, dx_row_stride)) return status;
  if (rows == 0 || cols == 0) return INTENT_HIP_OK;
  if (p == nullptr || dy == nullptr || dx == nullptr) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "null tensor pointer");
  switch (dtype) {
    case INTENT_HIP_F32:
      return launch_bwd<float>(p, dy, dx, rows, cols, p_row_stride, dy_row_stride, dx_row_stride, as_stream(stream));
    case INTENT_HIP_F16:
      return launch_bwd<f16_t>(p, dy, dx, rows, cols, p_row_stride, dy_row_stride, dx_row_stride, as_stream(stream));
    case INTENT_HIP_BF16:
      return launch_bwd<bf16_t>(p, dy, dx, rows, cols, p_row_stride, dy_row_stride, dx_row_stride, as_stream(stream));
  }
  return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "unknown dtype code %d", dtype);
}
