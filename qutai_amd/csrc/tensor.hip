// Element-wise and row kernels around the GEMM path (C ABI): dtype casts,
// fills, adds, batch reductions, last-two-axes transpose, row softmax and
// SwiGLU's silu(gate) * up.  Reference counterparts are cited per entry
// point in include/qutai_amd.h.
#include <algorithm>
#include <cstring>

#include "common.h"
#include "qutai_amd.h"

using namespace qa;

namespace {

constexpr int THREADS = 256;

// fp32 -> bf16 on the host with the device rule (round to nearest even, a
// NaN becomes (bits >> 16) | 0x40)
uint32_t f32_to_bf16_host(float f) {
  uint32_t bits;
  memcpy(&bits, &f, 4);
  if ((bits & 0x7fffffffu) > 0x7f800000u) return (bits >> 16) | 0x40u;
  return (bits + 0x7fffu + ((bits >> 16) & 1u)) >> 16;
}

unsigned grid_for(int64_t n, int64_t per_thread = 1) {
  int64_t blocks = (n + THREADS * per_thread - 1) / (THREADS * per_thread);
  return (unsigned)(blocks < 1 ? 1 : blocks > 1048576 ? 1048576 : blocks);
}

__device__ __forceinline__ double load_any(const void* p, int64_t i, int dtype) {
  switch (dtype) {
    case F32: return ((const float*)p)[i];
    case F64: return ((const double*)p)[i];
    case BF16: return bf16_to_f32(((const bf16_t*)p)[i]);
    default: return (double)((const int64_t*)p)[i];
  }
}

// Conversion with the reference cast semantics (tensor.cu:21-29): the value
// goes through double; bf16 is produced from its fp32 rounding.
__global__ void cast_kernel(const void* src, void* dst, int64_t n, int s, int d) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    double v = load_any(src, i, s);
    switch (d) {
      case F32: ((float*)dst)[i] = (float)v; break;
      case F64: ((double*)dst)[i] = v; break;
      case BF16: ((bf16_t*)dst)[i] = f32_to_bf16((float)v); break;
      default: ((int64_t*)dst)[i] = (int64_t)v; break;
    }
  }
}

// fp32 <-> bf16 in 16-byte pieces (8 values per lane and step); the same
// values as cast_kernel (RNE narrowing, exact widening)
__global__ void cast_f32_bf16x8(const f32x4* src, u32x4* dst, int64_t n8) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n8; i += (int64_t)gridDim.x * blockDim.x) {
    const f32x4 a = src[2 * i], b = src[2 * i + 1];
    dst[i] = u32x4{pack_bf16x2(a[0], a[1]), pack_bf16x2(a[2], a[3]), pack_bf16x2(b[0], b[1]), pack_bf16x2(b[2], b[3])};
  }
}
__global__ void cast_bf16_f32x8(const u32x4* src, f32x4* dst, int64_t n8) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n8; i += (int64_t)gridDim.x * blockDim.x) {
    const u32x4 w = src[i];
    dst[2 * i] = f32x4{__uint_as_float(w[0] << 16), __uint_as_float(w[0] & 0xffff0000u), __uint_as_float(w[1] << 16),
                       __uint_as_float(w[1] & 0xffff0000u)};
    dst[2 * i + 1] = f32x4{__uint_as_float(w[2] << 16), __uint_as_float(w[2] & 0xffff0000u),
                           __uint_as_float(w[3] << 16), __uint_as_float(w[3] & 0xffff0000u)};
  }
}
// out = a + b for fp32, 4 per lane and step
__global__ void add_f32x4(const f32x4* a, const f32x4* b, f32x4* out, int64_t n4) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (int64_t)gridDim.x * blockDim.x)
    out[i] = a[i] + b[i];
}

// 16 bytes per lane and step: the word pattern of one 16-byte piece
__global__ void fill16_kernel(u32x4* dst, int64_t n16, u32x4 word) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (int64_t)gridDim.x * blockDim.x)
    global_store(dst + i, word);
}

__global__ void fill_kernel(void* dst, int64_t n, double value, int d) {
  float f = (float)value;
  bf16_t h = f32_to_bf16(f);
  int64_t iv = (int64_t)value;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    switch (d) {
      case F32: ((float*)dst)[i] = f; break;
      case F64: ((double*)dst)[i] = value; break;
      case BF16: ((bf16_t*)dst)[i] = h; break;
      default: ((int64_t*)dst)[i] = iv; break;
    }
  }
}

__global__ void scale_kernel(const void* a, void* out, int64_t n, double factor, int d) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    if (d == F64) ((double*)out)[i] = ((const double*)a)[i] * factor;
    else if (d == F32) ((float*)out)[i] = ((const float*)a)[i] * (float)factor;
    else ((bf16_t*)out)[i] = f32_to_bf16(bf16_to_f32(((const bf16_t*)a)[i]) * (float)factor);
  }
}

// dst[z][r][c] = src[z][r][c] inside the source block, 0 outside it: a
// stack of matrices re-pitched to other row and column counts (padding or
// cropping, element size es bytes).
__global__ void repitch_kernel(const void* src, void* dst, int64_t batches, int64_t src_rows, int64_t src_cols,
                               int64_t dst_rows, int64_t dst_cols, int es) {
  const int64_t per = dst_rows * dst_cols, total = batches * per;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t z = i / per, r = (i % per) / dst_cols, c = i % dst_cols;
    const bool inside = r < src_rows && c < src_cols;
    const int64_t at = (z * src_rows + r) * src_cols + c;
    if (es == 2) ((bf16_t*)dst)[i] = inside ? ((const bf16_t*)src)[at] : (bf16_t)0;
    else ((float*)dst)[i] = inside ? ((const float*)src)[at] : 0.f;
  }
}

// Softmax backward along rows, one wave per row: dx = scale * p * (g - sum(g p))
// (the gradient rule of qutai.softmax with the input scaled by `scale`).
__device__ __forceinline__ float ld_any(const void* p, int64_t i, int d) {
  return d == F64 ? (float)((const double*)p)[i] : d == F32 ? ((const float*)p)[i] : bf16_to_f32(((const bf16_t*)p)[i]);
}
__global__ void __launch_bounds__(256) softmax_backward_kernel(const void* probs, const void* grad, void* out,
                                                              int64_t rows, int64_t width, float scale, int d) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t base = row * width;
  float dot = 0.f;
  for (int64_t j = lane; j < width; j += 64) dot += ld_any(grad, base + j, d) * ld_any(probs, base + j, d);
  for (int o = 32; o > 0; o >>= 1) dot += __shfl_xor(dot, o);
  for (int64_t j = lane; j < width; j += 64) {
    const float v = scale * ld_any(probs, base + j, d) * (ld_any(grad, base + j, d) - dot);
    if (d == F64) ((double*)out)[base + j] = v;
    else if (d == F32) ((float*)out)[base + j] = v;
    else ((bf16_t*)out)[base + j] = f32_to_bf16(v);
  }
}

// Causal mask of attention scores [rows][width]: row r is query r % length of
// its (batch, head) block and sees keys c <= offset + r % length; the others
// become -inf.
__global__ void causal_mask_kernel(const void* x, void* out, int64_t rows, int64_t width, int64_t length,
                                   int64_t offset, int d) {
  const int64_t n = rows * width;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / width, c = i - r * width;
    const bool masked = c > offset + r % length;
    if (d == F64) ((double*)out)[i] = masked ? -INFINITY : ((const double*)x)[i];
    else if (d == F32) ((float*)out)[i] = masked ? -INFINITY : ((const float*)x)[i];
    else ((bf16_t*)out)[i] = masked ? (bf16_t)0xff80 : ((const bf16_t*)x)[i];
  }
}

// out[o][j][i][e] = x[o][i][j][e] for an (outer, m, n, inner) array: two
// adjacent axes swapped, each element a run of `inner` values (es bytes each).
__global__ void swap_axes_kernel(const void* x, void* out, int64_t outer, int64_t m, int64_t n, int64_t inner,
                                 int es) {
  const int64_t total = outer * m * n * inner;
  for (int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; k < total; k += (int64_t)gridDim.x * blockDim.x) {
    const int64_t e = k % inner, rest = k / inner;
    const int64_t i = rest % m, rest2 = rest / m;  // output index order: o, j, i, e
    const int64_t j = rest2 % n, o = rest2 / n;
    const int64_t src = ((o * m + i) * n + j) * inner + e;
    if (es == 8) ((double*)out)[k] = ((const double*)x)[src];
    else if (es == 4) ((float*)out)[k] = ((const float*)x)[src];
    else ((bf16_t*)out)[k] = ((const bf16_t*)x)[src];
  }
}

__global__ void add_kernel(const void* a, const void* b, void* out, int64_t n, int d) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    if (d == F64) {
      ((double*)out)[i] = ((const double*)a)[i] + ((const double*)b)[i];
    } else if (d == F32) {
      ((float*)out)[i] = ((const float*)a)[i] + ((const float*)b)[i];
    } else {
      float v = bf16_to_f32(((const bf16_t*)a)[i]) + bf16_to_f32(((const bf16_t*)b)[i]);
      ((bf16_t*)out)[i] = f32_to_bf16(v);
    }
  }
}

// out = left + widen(right): fp32 plus bf16 (exactly widened), 4 per lane
__global__ void add_widen_kernel(const f32x4* a, const u32x2* b, f32x4* out, int64_t n4) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (int64_t)gridDim.x * blockDim.x) {
    const u32x2 w = b[i];
    out[i] = a[i] + f32x4{__uint_as_float(w[0] << 16), __uint_as_float(w[0] & 0xffff0000u),
                          __uint_as_float(w[1] << 16), __uint_as_float(w[1] & 0xffff0000u)};
  }
}

__global__ void add_widen_tail(const float* a, const bf16_t* b, float* out, int64_t begin, int64_t n) {
  for (int64_t i = begin + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    out[i] = a[i] + bf16_to_f32(b[i]);
}

__global__ void sum_middle_kernel(const void* x, void* out, int64_t outer, int64_t count, int64_t inner, int d) {
  int64_t n = outer * inner;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t o = i / inner, j = i % inner;
    if (d == F64) {
      double s = 0;
      for (int64_t c = 0; c < count; c++) s += ((const double*)x)[(o * count + c) * inner + j];
      ((double*)out)[i] = s;
    } else {
      float s = 0;
      for (int64_t c = 0; c < count; c++) s += (float)load_any(x, (o * count + c) * inner + j, d);
      if (d == F32) ((float*)out)[i] = s;
      else ((bf16_t*)out)[i] = f32_to_bf16(s);
    }
  }
}

// 32x32 tiles through LDS so both the read and the write are coalesced.
template <class T>
__global__ void transpose_kernel(const T* x, T* out, int64_t rows, int64_t cols, int64_t tiles_r, int64_t tiles_c) {
  __shared__ T tile[32][33];
  int64_t id = blockIdx.x;
  int64_t z = id / (tiles_r * tiles_c), t = id % (tiles_r * tiles_c);
  int64_t r0 = (t / tiles_c) * 32, c0 = (t % tiles_c) * 32;
  x += z * rows * cols;
  out += z * rows * cols;
  int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
  for (int j = ty; j < 32; j += 8) {
    int64_t r = r0 + j, c = c0 + tx;
    if (r < rows && c < cols) tile[j][tx] = x[r * cols + c];
  }
  __syncthreads();
  for (int j = ty; j < 32; j += 8) {
    int64_t c = c0 + j, r = r0 + tx;
    if (r < rows && c < cols) out[c * rows + r] = tile[tx][j];
  }
}

// Row softmax, one workgroup per row.  Three passes over the row (max,
// sum of exp, write) with the row kept in registers when it fits, so HBM
// sees one read and one write of the row.
template <class T, int PER>  // PER values per thread held in registers
__global__ void __launch_bounds__(THREADS) softmax_rows_kernel(const T* x, T* out, int64_t rows, int64_t width,
                                                               float scale) {
  __shared__ float red[THREADS / 64];
  int64_t row = blockIdx.x;
  if (row >= rows) return;
  const T* xr = x + row * width;
  T* yr = out + row * width;
  int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float v[PER];
  float peak = -INFINITY;
#pragma unroll
  for (int j = 0; j < PER; j++) {
    int64_t at = tid + (int64_t)j * THREADS;
    float f = -INFINITY;
    if (at < width) {
      if constexpr (sizeof(T) == 2) f = bf16_to_f32(xr[at]) * scale;
      else f = (float)xr[at] * scale;
    }
    v[j] = f;
    peak = fmaxf(peak, f);
  }
  for (int64_t at = tid + (int64_t)PER * THREADS; at < width; at += THREADS) {
    float f;
    if constexpr (sizeof(T) == 2) f = bf16_to_f32(xr[at]) * scale;
    else f = (float)xr[at] * scale;
    peak = fmaxf(peak, f);
  }
  for (int o = 32; o > 0; o >>= 1) peak = fmaxf(peak, __shfl_xor(peak, o));
  if (lane == 0) red[wave] = peak;
  __syncthreads();
  peak = red[0];
  for (int w = 1; w < THREADS / 64; w++) peak = fmaxf(peak, red[w]);
  __syncthreads();
  float total = 0.f;
#pragma unroll
  for (int j = 0; j < PER; j++) {
    v[j] = __expf(v[j] - peak);
    total += (tid + (int64_t)j * THREADS < width) ? v[j] : 0.f;
  }
  for (int64_t at = tid + (int64_t)PER * THREADS; at < width; at += THREADS) {
    float f;
    if constexpr (sizeof(T) == 2) f = bf16_to_f32(xr[at]) * scale;
    else f = (float)xr[at] * scale;
    total += __expf(f - peak);
  }
  for (int o = 32; o > 0; o >>= 1) total += __shfl_xor(total, o);
  if (lane == 0) red[wave] = total;
  __syncthreads();
  total = 0.f;
  for (int w = 0; w < THREADS / 64; w++) total += red[w];
  float inv = 1.0f / total;
#pragma unroll
  for (int j = 0; j < PER; j++) {
    int64_t at = tid + (int64_t)j * THREADS;
    if (at < width) {
      if constexpr (sizeof(T) == 2) yr[at] = f32_to_bf16(v[j] * inv);
      else yr[at] = v[j] * inv;
    }
  }
  for (int64_t at = tid + (int64_t)PER * THREADS; at < width; at += THREADS) {
    float f;
    if constexpr (sizeof(T) == 2) {
      f = bf16_to_f32(xr[at]) * scale;
      yr[at] = f32_to_bf16(__expf(f - peak) * inv);
    } else {
      f = (float)xr[at] * scale;
      yr[at] = __expf(f - peak) * inv;
    }
  }
}

// Row softmax, one wavefront per row (4 rows per 256-thread workgroup):
// 16-byte loads (8 bf16 or 4 fp32 per lane), the row kept in registers for
// up to 64 * V * CH elements, max and sum reduced inside the wavefront (no
// LDS, no barrier).  HBM sees one read and one write of every row; the
// register-held part is read with the nontemporal hint and every store
// carries it (config 3's 1 GiB of score rows: 365 -> 345 us); chunks beyond
// it are read three times and keep plain loads.
template <class T, int CH>  // CH 16-byte chunks per lane held in registers
__global__ void __launch_bounds__(256) softmax_rows_wave(const T* x, T* out, int64_t rows, int64_t width,
                                                         float scale) {
  constexpr int V = 16 / sizeof(T);
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const u32x4* xr = reinterpret_cast<const u32x4*>(x + row * width);
  u32x4* yr = reinterpret_cast<u32x4*>(out + row * width);
  const int chunks = (int)(width / V);
  auto unpack = [&](u32x4 w, float (&f)[V]) {
    if constexpr (sizeof(T) == 2) {
#pragma unroll
      for (int q = 0; q < 4; q++) {
        f[2 * q] = __uint_as_float(w[q] << 16) * scale;
        f[2 * q + 1] = __uint_as_float(w[q] & 0xffff0000u) * scale;
      }
    } else {
#pragma unroll
      for (int q = 0; q < 4; q++) f[q] = __uint_as_float(w[q]) * scale;
    }
  };
  auto pack = [&](const float (&f)[V]) {
    u32x4 w;
    if constexpr (sizeof(T) == 2) {
#pragma unroll
      for (int q = 0; q < 4; q++) w[q] = pack_bf16x2(f[2 * q], f[2 * q + 1]);
    } else {
#pragma unroll
      for (int q = 0; q < 4; q++) w[q] = __float_as_uint(f[q]);
    }
    return w;
  };
  float v[CH][V];
  float peak = -INFINITY;
#pragma unroll
  for (int c = 0; c < CH; c++) {
    int at = lane + 64 * c;
    if (at < chunks) {
      unpack(global_load_nt<u32x4>(xr + at), v[c]);
#pragma unroll
      for (int e = 0; e < V; e++) peak = fmaxf(peak, v[c][e]);
    }
  }
  for (int at = lane + 64 * CH; at < chunks; at += 64) {
    float f[V];
    unpack(xr[at], f);
#pragma unroll
    for (int e = 0; e < V; e++) peak = fmaxf(peak, f[e]);
  }
  for (int o = 32; o > 0; o >>= 1) peak = fmaxf(peak, __shfl_xor(peak, o));
  float total = 0.f;
#pragma unroll
  for (int c = 0; c < CH; c++) {
    if (lane + 64 * c < chunks) {
#pragma unroll
      for (int e = 0; e < V; e++) {
        v[c][e] = __expf(v[c][e] - peak);
        total += v[c][e];
      }
    }
  }
  for (int at = lane + 64 * CH; at < chunks; at += 64) {
    float f[V];
    unpack(xr[at], f);
#pragma unroll
    for (int e = 0; e < V; e++) total += __expf(f[e] - peak);
  }
  for (int o = 32; o > 0; o >>= 1) total += __shfl_xor(total, o);
  const float inv = 1.0f / total;
#pragma unroll
  for (int c = 0; c < CH; c++) {
    int at = lane + 64 * c;
    if (at < chunks) {
#pragma unroll
      for (int e = 0; e < V; e++) v[c][e] *= inv;
      global_store_nt(yr + at, pack(v[c]));
    }
  }
  for (int at = lane + 64 * CH; at < chunks; at += 64) {
    float f[V];
    unpack(xr[at], f);
#pragma unroll
    for (int e = 0; e < V; e++) f[e] = __expf(f[e] - peak) * inv;
    global_store_nt(yr + at, pack(f));
  }
}

__global__ void softmax_rows_f64(const double* x, double* out, int64_t rows, int64_t width, double scale) {
  __shared__ double red[THREADS];
  int64_t row = blockIdx.x;
  const double* xr = x + row * width;
  double* yr = out + row * width;
  int tid = threadIdx.x;
  double peak = -INFINITY;
  for (int64_t at = tid; at < width; at += THREADS) peak = fmax(peak, xr[at] * scale);
  red[tid] = peak;
  __syncthreads();
  for (int s = THREADS / 2; s; s >>= 1) {
    if (tid < s) red[tid] = fmax(red[tid], red[tid + s]);
    __syncthreads();
  }
  peak = red[0];
  __syncthreads();
  double total = 0;
  for (int64_t at = tid; at < width; at += THREADS) total += exp(xr[at] * scale - peak);
  red[tid] = total;
  __syncthreads();
  for (int s = THREADS / 2; s; s >>= 1) {
    if (tid < s) red[tid] += red[tid + s];
    __syncthreads();
  }
  total = red[0];
  for (int64_t at = tid; at < width; at += THREADS) yr[at] = exp(xr[at] * scale - peak) / total;
}

// Softmax along an axis that is not the last: x viewed as
// [outer][width][inner], one lane per (o, j) column, consecutive lanes on
// consecutive j so every pass over the axis is coalesced.  Three passes
// (max, sum of exp, write), as the reference's softmax_forward
// (src/qutai/backends/cuda/nn.cu:67-76), in fp32 (fp64 for fp64).
template <class T, class R>
__global__ void __launch_bounds__(THREADS) softmax_cols_kernel(const T* x, T* out, int64_t outer, int64_t width,
                                                               int64_t inner, R scale) {
  auto load = [&](int64_t i) -> R {
    if constexpr (sizeof(T) == 2) return (R)bf16_to_f32(x[i]) * scale;
    else return (R)x[i] * scale;
  };
  const int64_t total = outer * inner;
  for (int64_t i = (int64_t)blockIdx.x * THREADS + threadIdx.x; i < total; i += (int64_t)gridDim.x * THREADS) {
    const int64_t base = (i / inner) * width * inner + i % inner;
    R peak = load(base);
    for (int64_t c = 1; c < width; c++) peak = fmax(peak, load(base + c * inner));
    R sum = 0;
    for (int64_t c = 0; c < width; c++) sum += exp(load(base + c * inner) - peak);
    const R inv = R(1) / sum;
    for (int64_t c = 0; c < width; c++) {
      const R v = exp(load(base + c * inner) - peak) * inv;
      if constexpr (sizeof(T) == 2) out[base + c * inner] = f32_to_bf16((float)v);
      else out[base + c * inner] = (T)v;
    }
  }
}

// silu(gate) * up with silu_f (common.h).  With bf16 storage the silu output
// is itself a bf16 tensor before the multiply (two roundings), as in the
// unfused SwiGLU of the reference.
// bf16, 8 elements (16 bytes) per thread and step.
__global__ void silu_mul_bf16x8(const u32x4* g, const u32x4* u, u32x4* out, int64_t n8) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n8; i += (int64_t)gridDim.x * blockDim.x) {
    u32x4 a = g[i], b = u[i], r;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      float lo = bf16_to_f32(f32_to_bf16(silu_f(__uint_as_float(a[q] << 16)))) * __uint_as_float(b[q] << 16);
      float hi = bf16_to_f32(f32_to_bf16(silu_f(__uint_as_float(a[q] & 0xffff0000u)))) *
                 __uint_as_float(b[q] & 0xffff0000u);
      r[q] = pack_bf16x2(lo, hi);
    }
    out[i] = r;
  }
}

__global__ void silu_mul_kernel(const void* g, const void* u, void* out, int64_t n, int d) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    if (d == BF16) {
      float s = bf16_to_f32(f32_to_bf16(silu_f(bf16_to_f32(((const bf16_t*)g)[i]))));
      ((bf16_t*)out)[i] = f32_to_bf16(s * bf16_to_f32(((const bf16_t*)u)[i]));
    } else if (d == F32) {
      ((float*)out)[i] = silu_f(((const float*)g)[i]) * ((const float*)u)[i];
    } else {
      double v = ((const double*)g)[i];
      double s = v >= 0 ? 1.0 / (1.0 + exp(-v)) : exp(v) / (1.0 + exp(v));
      ((double*)out)[i] = (v * s) * ((const double*)u)[i];
    }
  }
}

__global__ void add_rows_kernel(const void* x, const void* bias, void* out, int64_t rows, int64_t cols, int d) {
  int64_t n = rows * cols;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t c = i % cols;
    if (d == F64) {
      ((double*)out)[i] = ((const double*)x)[i] + ((const double*)bias)[c];
    } else if (d == F32) {
      ((float*)out)[i] = ((const float*)x)[i] + ((const float*)bias)[c];
    } else {
      float v = bf16_to_f32(((const bf16_t*)x)[i]) + bf16_to_f32(((const bf16_t*)bias)[c]);
      ((bf16_t*)out)[i] = f32_to_bf16(v);
    }
  }
}

// Gradients of y = silu(g) * u: dg = dy * u * s * (1 + g (1 - s)), du = dy * silu(g)
// (the derivative of lm_silu, lm.cu:54, times the multiply's rule).  bf16:
// 8 elements (16 bytes of each operand) per thread and step, s from the
// hardware exp2 / reciprocal (sigmoid_f, common.h).
__global__ void silu_mul_backward_bf16x8(const u32x4* dy, const u32x4* g, const u32x4* u, u32x4* dg, u32x4* du,
                                         int64_t n8) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n8; i += (int64_t)gridDim.x * blockDim.x) {
    const u32x4 y8 = dy[i], g8 = g[i], u8 = u[i];
    u32x4 a8, b8;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      float a[2], b[2];
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const float y = __uint_as_float(h ? y8[q] & 0xffff0000u : y8[q] << 16);
        const float v = __uint_as_float(h ? g8[q] & 0xffff0000u : g8[q] << 16);
        const float w = __uint_as_float(h ? u8[q] & 0xffff0000u : u8[q] << 16);
        const float s = sigmoid_f(v);
        a[h] = y * w * s * (1.f + v * (1.f - s));
        b[h] = y * (v * s);
      }
      a8[q] = pack_bf16x2(a[0], a[1]);
      b8[q] = pack_bf16x2(b[0], b[1]);
    }
    dg[i] = a8;
    du[i] = b8;
  }
}

__global__ void silu_mul_backward_kernel(const void* dy, const void* g, const void* u, void* dg, void* du, int64_t n,
                                         int d) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    if (d == F64) {
      double v = ((const double*)g)[i], w = ((const double*)u)[i], y = ((const double*)dy)[i];
      double s = v >= 0 ? 1.0 / (1.0 + exp(-v)) : exp(v) / (1.0 + exp(v));
      ((double*)dg)[i] = y * w * s * (1.0 + v * (1.0 - s));
      ((double*)du)[i] = y * (v * s);
    } else {
      float v, w, y;
      if (d == F32) {
        v = ((const float*)g)[i]; w = ((const float*)u)[i]; y = ((const float*)dy)[i];
      } else {
        v = bf16_to_f32(((const bf16_t*)g)[i]); w = bf16_to_f32(((const bf16_t*)u)[i]);
        y = bf16_to_f32(((const bf16_t*)dy)[i]);
      }
      float s = sigmoid_f(v);
      float a = y * w * s * (1.f + v * (1.f - s)), b = y * (v * s);
      if (d == F32) {
        ((float*)dg)[i] = a; ((float*)du)[i] = b;
      } else {
        ((bf16_t*)dg)[i] = f32_to_bf16(a); ((bf16_t*)du)[i] = f32_to_bf16(b);
      }
    }
  }
}

bool float_dtype(int d) { return d == F32 || d == F64 || d == BF16; }

}  // namespace

extern "C" {

int qutai_amd_cast(const void* src, void* dst, int64_t n, int src_dtype, int dst_dtype, void* stream) {
  if (n < 0) return QA_EINVAL;
  for (int d : {src_dtype, dst_dtype})
    if (!float_dtype(d) && d != I64) return QA_EINVAL;
  if (n == 0) return QA_OK;
  hipStream_t s = (hipStream_t)stream;
  int64_t head = 0;
  const bool aligned = ((uintptr_t)src | (uintptr_t)dst) % 16 == 0;
  if (aligned && src_dtype == F32 && dst_dtype == BF16) {
    head = n / 8 * 8;
    if (head)
      hipLaunchKernelGGL(cast_f32_bf16x8, dim3(grid_for(head / 8)), dim3(THREADS), 0, s, (const f32x4*)src,
                         (u32x4*)dst, head / 8);
  } else if (aligned && src_dtype == BF16 && dst_dtype == F32) {
    head = n / 8 * 8;
    if (head)
      hipLaunchKernelGGL(cast_bf16_f32x8, dim3(grid_for(head / 8)), dim3(THREADS), 0, s, (const u32x4*)src,
                         (f32x4*)dst, head / 8);
  }
  if (head < n) {
    const int64_t so = head * (src_dtype == BF16 ? 2 : src_dtype == F32 ? 4 : 8);
    const int64_t d_o = head * (dst_dtype == BF16 ? 2 : dst_dtype == F32 ? 4 : 8);
    hipLaunchKernelGGL(cast_kernel, dim3(grid_for(n - head)), dim3(THREADS), 0, s, (const char*)src + so,
                       (char*)dst + d_o, n - head, src_dtype, dst_dtype);
  }
  return (int)hipGetLastError();
}

int qutai_amd_fill(void* dst, int64_t n, double value, int dtype, void* stream) {
  if (n < 0 || (!float_dtype(dtype) && dtype != I64)) return QA_EINVAL;
  if (n == 0) return QA_OK;
  if (!dst) return QA_EINVAL;
  hipStream_t s = (hipStream_t)stream;
  const int es = dtype == BF16 ? 2 : dtype == F32 ? 4 : 8;
  if ((uintptr_t)dst % 16 == 0 && n * es >= 16) {
    // whole 16-byte pieces with one repeated word pattern, the rest element-wise
    uint32_t w[4];
    if (dtype == BF16) {
      const uint32_t h = f32_to_bf16_host((float)value);
      w[0] = w[1] = w[2] = w[3] = h | (h << 16);
    } else if (dtype == F32) {
      const float f = (float)value;
      uint32_t u;
      memcpy(&u, &f, 4);
      w[0] = w[1] = w[2] = w[3] = u;
    } else {
      uint64_t u;
      if (dtype == F64) memcpy(&u, &value, 8);
      else { const int64_t iv = (int64_t)value; memcpy(&u, &iv, 8); }
      w[0] = w[2] = (uint32_t)u;
      w[1] = w[3] = (uint32_t)(u >> 32);
    }
    const int64_t n16 = n * es / 16, done = n16 * 16 / es;
    hipLaunchKernelGGL(fill16_kernel, dim3(grid_for(n16)), dim3(THREADS), 0, s, (u32x4*)dst, n16,
                       u32x4{w[0], w[1], w[2], w[3]});
    if (done < n)
      hipLaunchKernelGGL(fill_kernel, dim3(1), dim3(THREADS), 0, s, (void*)((char*)dst + done * es), n - done, value,
                         dtype);
    return (int)hipGetLastError();
  }
  hipLaunchKernelGGL(fill_kernel, dim3(grid_for(n)), dim3(THREADS), 0, s, dst, n, value, dtype);
  return (int)hipGetLastError();
}

int qutai_amd_add(const void* left, const void* right, void* out, int64_t n, int dtype, void* stream) {
  if (n < 0 || !float_dtype(dtype)) return QA_EINVAL;
  if (n == 0) return QA_OK;
  int64_t head = 0;
  if (dtype == F32 && ((uintptr_t)left | (uintptr_t)right | (uintptr_t)out) % 16 == 0) {
    head = n / 4 * 4;
    if (head)
      hipLaunchKernelGGL(add_f32x4, dim3(grid_for(head / 4)), dim3(THREADS), 0, (hipStream_t)stream,
                         (const f32x4*)left, (const f32x4*)right, (f32x4*)out, head / 4);
  }
  if (head < n) {
    const int64_t off = head * (dtype == BF16 ? 2 : dtype == F32 ? 4 : 8);
    hipLaunchKernelGGL(add_kernel, dim3(grid_for(n - head)), dim3(THREADS), 0, (hipStream_t)stream,
                       (const char*)left + off, (const char*)right + off, (char*)out + off, n - head, dtype);
  }
  return (int)hipGetLastError();
}

int qutai_amd_add_widen(const float* left, const void* right, float* out, int64_t n, void* stream) {
  if (n < 0 || (n > 0 && (!left || !right || !out))) return QA_EINVAL;
  if (n == 0) return QA_OK;
  int64_t head = 0;
  if (((uintptr_t)left | (uintptr_t)out) % 16 == 0 && (uintptr_t)right % 8 == 0) {
    head = n / 4 * 4;
    if (head)
      hipLaunchKernelGGL(add_widen_kernel, dim3(grid_for(head / 4)), dim3(THREADS), 0, (hipStream_t)stream,
                         (const f32x4*)left, (const u32x2*)right, (f32x4*)out, head / 4);
  }
  if (head < n)
    hipLaunchKernelGGL(add_widen_tail, dim3(grid_for(n - head)), dim3(THREADS), 0, (hipStream_t)stream, left,
                       (const bf16_t*)right, out, head, n);
  return (int)hipGetLastError();
}

int qutai_amd_scale(const void* x, void* out, int64_t n, double factor, int dtype, void* stream) {
  if (n < 0 || !float_dtype(dtype)) return QA_EINVAL;
  if (n == 0) return QA_OK;
  hipLaunchKernelGGL(scale_kernel, dim3(grid_for(n)), dim3(THREADS), 0, (hipStream_t)stream, x, out, n, factor, dtype);
  return (int)hipGetLastError();
}

int qutai_amd_repitch(const void* src, void* dst, int64_t batches, int64_t src_rows, int64_t src_cols,
                      int64_t dst_rows, int64_t dst_cols, int dtype, void* stream) {
  if (batches < 0 || src_rows < 0 || src_cols < 0 || dst_rows < 0 || dst_cols < 0) return QA_EINVAL;
  if (dtype != BF16 && dtype != F32) return QA_EINVAL;
  const int64_t n = batches * dst_rows * dst_cols;
  if (n == 0) return QA_OK;
  if (!src || !dst) return QA_EINVAL;
  hipLaunchKernelGGL(repitch_kernel, dim3(grid_for(n)), dim3(THREADS), 0, (hipStream_t)stream, src, dst, batches,
                     src_rows, src_cols, dst_rows, dst_cols, dtype == BF16 ? 2 : 4);
  return (int)hipGetLastError();
}

int qutai_amd_add_rows(const void* x, const void* bias, void* out, int64_t rows, int64_t cols, int dtype,
                       void* stream) {
  if (rows < 0 || cols < 0 || !float_dtype(dtype)) return QA_EINVAL;
  if (rows * cols == 0) return QA_OK;
  hipLaunchKernelGGL(add_rows_kernel, dim3(grid_for(rows * cols)), dim3(THREADS), 0, (hipStream_t)stream, x, bias,
                     out, rows, cols, dtype);
  return (int)hipGetLastError();
}

int qutai_amd_sum_middle(const void* x, void* out, int64_t outer, int64_t count, int64_t inner, int dtype,
                         void* stream) {
  if (outer < 0 || count < 0 || inner < 0 || !float_dtype(dtype)) return QA_EINVAL;
  if (outer * inner == 0) return QA_OK;
  hipLaunchKernelGGL(sum_middle_kernel, dim3(grid_for(outer * inner)), dim3(THREADS), 0, (hipStream_t)stream, x,
                     out, outer, count, inner, dtype);
  return (int)hipGetLastError();
}

int qutai_amd_swap_axes(const void* x, void* out, int64_t outer, int64_t m, int64_t n, int64_t inner, int dtype,
                        void* stream) {
  if (outer < 0 || m < 0 || n < 0 || inner < 0 || !float_dtype(dtype)) return QA_EINVAL;
  const int64_t total = outer * m * n * inner;
  if (total == 0) return QA_OK;
  if (!x || !out) return QA_EINVAL;
  hipLaunchKernelGGL(swap_axes_kernel, dim3(grid_for(total)), dim3(THREADS), 0, (hipStream_t)stream, x, out, outer, m,
                     n, inner, dtype == F64 ? 8 : dtype == F32 ? 4 : 2);
  return (int)hipGetLastError();
}

int qutai_amd_transpose_last2(const void* x, void* out, int64_t batch, int64_t rows, int64_t cols, int dtype,
                              void* stream) {
  if (batch < 0 || rows < 0 || cols < 0 || !float_dtype(dtype)) return QA_EINVAL;
  if (batch * rows * cols == 0) return QA_OK;
  int64_t tr = (rows + 31) / 32, tc = (cols + 31) / 32;
  int64_t blocks = batch * tr * tc;
  if (blocks > 0x7fffffff) return QA_EINVAL;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == F64)
    hipLaunchKernelGGL(transpose_kernel<double>, dim3((unsigned)blocks), dim3(256), 0, s, (const double*)x,
                       (double*)out, rows, cols, tr, tc);
  else if (dtype == F32)
    hipLaunchKernelGGL(transpose_kernel<float>, dim3((unsigned)blocks), dim3(256), 0, s, (const float*)x,
                       (float*)out, rows, cols, tr, tc);
  else
    hipLaunchKernelGGL(transpose_kernel<bf16_t>, dim3((unsigned)blocks), dim3(256), 0, s, (const bf16_t*)x,
                       (bf16_t*)out, rows, cols, tr, tc);
  return (int)hipGetLastError();
}

int qutai_amd_softmax_rows(const void* x, void* out, int64_t rows, int64_t width, double scale, int dtype,
                           void* stream) {
  if (rows < 0 || width < 0 || !float_dtype(dtype)) return QA_EINVAL;
  if (rows == 0 || width == 0) return QA_OK;
  if (rows > 0x7fffffff) return QA_EINVAL;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == F64)
    hipLaunchKernelGGL(softmax_rows_f64, dim3((unsigned)rows), dim3(THREADS), 0, s, (const double*)x, (double*)out,
                       rows, width, scale);
  else {
    // vector path: whole 16-byte chunks per row and 16-byte aligned rows
    int64_t v = dtype == F32 ? 4 : 8;
    bool vec = width % v == 0 && (uintptr_t)x % 16 == 0 && (uintptr_t)out % 16 == 0;
    unsigned groups = (unsigned)((rows + 3) / 4);
    if (vec && dtype == F32)
      hipLaunchKernelGGL((softmax_rows_wave<float, 8>), dim3(groups), dim3(256), 0, s, (const float*)x, (float*)out,
                         rows, width, (float)scale);
    else if (vec)
      hipLaunchKernelGGL((softmax_rows_wave<bf16_t, 4>), dim3(groups), dim3(256), 0, s, (const bf16_t*)x,
                         (bf16_t*)out, rows, width, (float)scale);
    else if (dtype == F32)
      hipLaunchKernelGGL((softmax_rows_kernel<float, 8>), dim3((unsigned)rows), dim3(THREADS), 0, s,
                         (const float*)x, (float*)out, rows, width, (float)scale);
    else
      hipLaunchKernelGGL((softmax_rows_kernel<bf16_t, 8>), dim3((unsigned)rows), dim3(THREADS), 0, s,
                         (const bf16_t*)x, (bf16_t*)out, rows, width, (float)scale);
  }
  return (int)hipGetLastError();
}

int qutai_amd_softmax(const void* x, void* out, int64_t outer, int64_t width, int64_t inner, double scale,
                      int dtype, void* stream) {
  if (outer < 0 || width < 0 || inner < 1 || !float_dtype(dtype)) return QA_EINVAL;
  if (inner == 1) return qutai_amd_softmax_rows(x, out, outer, width, scale, dtype, stream);
  if (outer == 0 || width == 0) return QA_OK;
  if (!x || !out) return QA_EINVAL;
  const int64_t columns = outer * inner;
  const unsigned blocks = (unsigned)std::min<int64_t>((columns + THREADS - 1) / THREADS, 65536);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == F64)
    hipLaunchKernelGGL((softmax_cols_kernel<double, double>), dim3(blocks), dim3(THREADS), 0, s, (const double*)x,
                       (double*)out, outer, width, inner, scale);
  else if (dtype == F32)
    hipLaunchKernelGGL((softmax_cols_kernel<float, float>), dim3(blocks), dim3(THREADS), 0, s, (const float*)x,
                       (float*)out, outer, width, inner, (float)scale);
  else
    hipLaunchKernelGGL((softmax_cols_kernel<bf16_t, float>), dim3(blocks), dim3(THREADS), 0, s, (const bf16_t*)x,
                       (bf16_t*)out, outer, width, inner, (float)scale);
  return (int)hipGetLastError();
}

int qutai_amd_softmax_backward(const void* probs, const void* grad, void* out, int64_t rows, int64_t width,
                               double scale, int dtype, void* stream) {
  if (rows < 0 || width < 0 || !float_dtype(dtype)) return QA_EINVAL;
  if (rows == 0 || width == 0) return QA_OK;
  if (!probs || !grad || !out || (rows + 3) / 4 > 0x7fffffff) return QA_EINVAL;
  hipLaunchKernelGGL(softmax_backward_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, (hipStream_t)stream,
                     probs, grad, out, rows, width, (float)scale, dtype);
  return (int)hipGetLastError();
}

int qutai_amd_causal_mask(const void* x, void* out, int64_t rows, int64_t width, int64_t length, int64_t offset,
                          int dtype, void* stream) {
  if (rows < 0 || width < 0 || length <= 0 || offset < 0 || !float_dtype(dtype)) return QA_EINVAL;
  if (rows == 0 || width == 0) return QA_OK;
  if (!x || !out) return QA_EINVAL;
  hipLaunchKernelGGL(causal_mask_kernel, dim3(grid_for(rows * width)), dim3(THREADS), 0, (hipStream_t)stream, x, out,
                     rows, width, length, offset, dtype);
  return (int)hipGetLastError();
}

int qutai_amd_silu_mul(const void* gate, const void* up, void* out, int64_t n, int dtype, void* stream) {
  if (n < 0 || !float_dtype(dtype)) return QA_EINVAL;
  if (n == 0) return QA_OK;
  if (dtype == BF16 && n % 8 == 0 && (uintptr_t)gate % 16 == 0 && (uintptr_t)up % 16 == 0 &&
      (uintptr_t)out % 16 == 0) {
    hipLaunchKernelGGL(silu_mul_bf16x8, dim3(grid_for(n / 8)), dim3(THREADS), 0, (hipStream_t)stream,
                       (const u32x4*)gate, (const u32x4*)up, (u32x4*)out, n / 8);
    return (int)hipGetLastError();
  }
  hipLaunchKernelGGL(silu_mul_kernel, dim3(grid_for(n)), dim3(THREADS), 0, (hipStream_t)stream, gate, up, out, n,
                     dtype);
  return (int)hipGetLastError();
}

int qutai_amd_silu_mul_backward(const void* dy, const void* gate, const void* up, void* dgate, void* dup, int64_t n,
                                int dtype, void* stream) {
  if (n < 0 || !float_dtype(dtype)) return QA_EINVAL;
  if (n == 0) return QA_OK;
  const bool aligned = ((uintptr_t)dy | (uintptr_t)gate | (uintptr_t)up | (uintptr_t)dgate | (uintptr_t)dup) % 16 == 0;
  if (dtype == BF16 && n % 8 == 0 && aligned) {
    hipLaunchKernelGGL(silu_mul_backward_bf16x8, dim3(grid_for(n / 8)), dim3(THREADS), 0, (hipStream_t)stream,
                       (const u32x4*)dy, (const u32x4*)gate, (const u32x4*)up, (u32x4*)dgate, (u32x4*)dup, n / 8);
    return (int)hipGetLastError();
  }
  hipLaunchKernelGGL(silu_mul_backward_kernel, dim3(grid_for(n)), dim3(THREADS), 0, (hipStream_t)stream, dy, gate, up,
                     dgate, dup, n, dtype);
  return (int)hipGetLastError();
}

}  // extern "C"
