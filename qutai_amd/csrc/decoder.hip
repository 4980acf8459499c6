// Decoder glue kernels of the lm path (C ABI `qutai_amd_embedding`, `_rms_norm`,
// `_silu`, `_rope`, `_head_*`): the element-wise and row work around the
// contractions that a `Decoder.loss` step needs (src/qutai/backends/cuda/lm.cu:
// 30-59, 417-444, driven by src/qutai/backends/cuda_lm.py:64-228, 584-660).
// Activations are bf16 or fp32; statistics, RMSNorm/embedding weights and
// every sum are fp32 (the reference's accumulation type for both).  All
// reductions run in a fixed order, so results are bit-repeatable.
#include "common.h"
#include "qutai_amd.h"

using namespace qa;

namespace {

template <class T> __device__ __forceinline__ float get(const T* p, int64_t i);
template <> __device__ __forceinline__ float get<float>(const float* p, int64_t i) { return p[i]; }
template <> __device__ __forceinline__ float get<bf16_t>(const bf16_t* p, int64_t i) { return bf16_to_f32(p[i]); }
template <class T> __device__ __forceinline__ void put(T* p, int64_t i, float x);
template <> __device__ __forceinline__ void put<float>(float* p, int64_t i, float x) { p[i] = x; }
template <> __device__ __forceinline__ void put<bf16_t>(bf16_t* p, int64_t i, float x) { p[i] = f32_to_bf16(x); }

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

constexpr int ROWS_PER_BLOCK = 4;  // one wave per row, 4 waves per workgroup

unsigned blocks_for(int64_t n, int64_t per_block = 256) {
  int64_t b = (n + per_block - 1) / per_block;
  return (unsigned)(b < 1 ? 1 : b > (1 << 20) ? (1 << 20) : b);
}
#define GRID_STRIDE(i, n) \
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < (n); i += (int64_t)gridDim.x * blockDim.x)

// out[r][j] = w[ids[r]][j], fp32 table -> activation dtype (lm.cu:30)
template <class T>
__global__ void embedding_kernel(const float* w, const int64_t* ids, T* out, int64_t n, int64_t width) {
  GRID_STRIDE(i, n) put<T>(out, i, w[ids[i / width] * width + i % width]);
}

// out[tokens[g]][f] = sum over the rows of group g (input order) of grad[row][f]
// (lm.cu:32-38), added to the old value when accumulating; rows of tokens
// that do not occur are not touched.
template <class T>
__global__ void embedding_grad_kernel(const T* g, const int64_t* tokens, const int64_t* offsets,
                                      const int64_t* rows, float* out, int64_t n, int64_t width, int accumulate) {
  GRID_STRIDE(i, n) {
    const int64_t group = i / width, f = i % width;
    float total = 0.f;
    for (int64_t p = offsets[group]; p < offsets[group + 1]; p++) total += get<T>(g, rows[p] * width + f);
    float* at = out + tokens[group] * width + f;
    *at = accumulate ? *at + total : total;
  }
}

// The same two with 4 features per thread (16-byte table rows and fp32
// gradient rows, 8-byte bf16 rows): one workgroup per token row / per
// group, the index arithmetic once per row.  Same sums in the same order.
template <class T>
__global__ void __launch_bounds__(256) embedding_rows(const float* w, const int64_t* ids, T* out, int64_t width) {
  const int64_t r = blockIdx.x;
  const float* src = w + ids[r] * width;
  T* dst = out + r * width;
  for (int64_t c = (int64_t)threadIdx.x * 4; c < width; c += 1024) {
    const float4 v = *(const float4*)(src + c);
    if constexpr (sizeof(T) == 2)
      *(uint2*)(dst + c) = make_uint2(pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w));
    else
      *(float4*)(dst + c) = v;
  }
}

template <class T>
__global__ void __launch_bounds__(256) embedding_grad_rows(const T* g, const int64_t* tokens, const int64_t* offsets,
                                                           const int64_t* rows, float* out, int64_t width,
                                                           int accumulate) {
  const int64_t group = blockIdx.x, p0 = offsets[group], p1 = offsets[group + 1];
  float* dst = out + tokens[group] * width;
  for (int64_t c = (int64_t)threadIdx.x * 4; c < width; c += 1024) {
    float t[4] = {0.f, 0.f, 0.f, 0.f};
    for (int64_t p = p0; p < p1; p++) {
      const T* src = g + rows[p] * width + c;
      float v[4];
      if constexpr (sizeof(T) == 2) {
        const uint2 raw = *(const uint2*)src;
        v[0] = __uint_as_float(raw.x << 16);
        v[1] = __uint_as_float(raw.x & 0xffff0000u);
        v[2] = __uint_as_float(raw.y << 16);
        v[3] = __uint_as_float(raw.y & 0xffff0000u);
      } else {
        const float4 x = *(const float4*)src;
        v[0] = x.x, v[1] = x.y, v[2] = x.z, v[3] = x.w;
      }
#pragma unroll
      for (int e = 0; e < 4; e++) t[e] += v[e];
    }
    float4 o = make_float4(t[0], t[1], t[2], t[3]);
    if (accumulate) {
      const float4 old = *(const float4*)(dst + c);
      o = make_float4(old.x + t[0], old.y + t[1], old.z + t[2], old.w + t[3]);
    }
    *(float4*)(dst + c) = o;
  }
}

// RMSNorm forward, one wave per row: inv = 1/sqrt(mean(x^2) + eps),
// out = x * inv * w (fp32 out and inv, lm.cu:39-45)
template <class T>
__global__ void __launch_bounds__(256) rms_kernel(const T* x, const float* w, float* out, float* inv, int64_t rows,
                                                  int64_t width, float eps, bf16_t* out16) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + row * width;
  float total = 0.f;
  for (int64_t j = lane; j < width; j += 64) {
    const float v = get<T>(xr, j);
    total += v * v;
  }
  const float scale = 1.f / sqrtf(wave_sum(total) / (float)width + eps);
  if (lane == 0) inv[row] = scale;
  for (int64_t j = lane; j < width; j += 64) {
    const float y = get<T>(xr, j) * scale * w[j];
    out[row * width + j] = y;
    if (out16) out16[row * width + j] = f32_to_bf16(y);
  }
}

// dx = inv * (g w - x inv^2 mean(g w x)), one wave per row (lm.cu:46-51)
template <class T>
__global__ void __launch_bounds__(256) rms_dx_kernel(const float* g, const T* x, const float* w, const float* inv,
                                                     T* dx, int64_t rows, int64_t width) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6);
  if (row >= rows) return;
  float total = 0.f;
  for (int64_t j = lane; j < width; j += 64) total += g[row * width + j] * w[j] * get<T>(x, row * width + j);
  const float projected = wave_sum(total) / (float)width, scale = inv[row];
  for (int64_t j = lane; j < width; j += 64) {
    const int64_t at = row * width + j;
    put<T>(dx, at, scale * (g[at] * w[j] - get<T>(x, at) * scale * scale * projected));
  }
}

// dw[j] = sum_r g x inv over rows (lm.cu:52): chunks of RC rows write
// partial sums, then one thread per column adds the chunks in order
constexpr int RC = 64;
constexpr int RCB = 16;  // rows per workgroup of the one-pass backward (enough workgroups for 4096 rows)
template <class T>
__global__ void rms_dw_partial_kernel(const float* g, const T* x, const float* inv, float* partial, int64_t rows,
                                      int64_t width) {
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t chunk = blockIdx.y;
  if (j >= width) return;
  const int64_t r0 = chunk * RC, r1 = min(rows, r0 + RC);
  float total = 0.f;
  for (int64_t r = r0; r < r1; r++) total += g[r * width + j] * get<T>(x, r * width + j) * inv[r];
  partial[chunk * width + j] = total;
}
__global__ void rms_dw_final_kernel(const float* partial, float* dw, int64_t chunks, int64_t width) {
  GRID_STRIDE(j, width) {
    float total = 0.f;
    for (int64_t c = 0; c < chunks; c++) total += partial[c * width + j];
    dw[j] = total;
  }
}

// Rows of width 256*NI (NI <= 8, e.g. d_model 2048): lane l owns columns
// 4 l + 256 i, i < NI, read and written 16 bytes at a time; the forward keeps
// the row in registers between the sum of squares and the output.
template <class T, int NI>
__device__ __forceinline__ void load_cols(const T* row, int lane, f32x4 (&v)[NI]) {
#pragma unroll
  for (int i = 0; i < NI; i++) {
    const int64_t c = 4 * lane + 256 * i;
    if constexpr (sizeof(T) == 2) {
      const u32x2 w = global_load<u32x2>(row + c);
      v[i] = f32x4{__uint_as_float(w[0] << 16), __uint_as_float(w[0] & 0xffff0000u), __uint_as_float(w[1] << 16),
                   __uint_as_float(w[1] & 0xffff0000u)};
    } else {
      v[i] = global_load<f32x4>(row + c);
    }
  }
}
template <class T, int NI>
__device__ __forceinline__ void store_cols(T* row, int lane, const f32x4 (&v)[NI]) {
#pragma unroll
  for (int i = 0; i < NI; i++) {
    const int64_t c = 4 * lane + 256 * i;
    if constexpr (sizeof(T) == 2) global_store(row + c, u32x2{pack_bf16x2(v[i][0], v[i][1]), pack_bf16x2(v[i][2], v[i][3])});
    else global_store(row + c, v[i]);
  }
}

template <class T, int NI>
__global__ void __launch_bounds__(256) rms_cols_kernel(const T* x, const float* w, float* out, float* inv,
                                                       int64_t rows, float eps, bf16_t* out16) {
  constexpr int W = 256 * NI;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6);
  if (row >= rows) return;
  f32x4 v[NI], wv[NI];
  load_cols<T, NI>(x + row * W, lane, v);
  load_cols<float, NI>(w, lane, wv);
  float total = 0.f;
#pragma unroll
  for (int i = 0; i < NI; i++) total += v[i][0] * v[i][0] + v[i][1] * v[i][1] + v[i][2] * v[i][2] + v[i][3] * v[i][3];
  const float scale = 1.f / sqrtf(wave_sum(total) / (float)W + eps);
  if (lane == 0) inv[row] = scale;
#pragma unroll
  for (int i = 0; i < NI; i++) v[i] = v[i] * scale * wv[i];
  store_cols<float, NI>(out + row * W, lane, v);
  // the bf16 copy of the bf16-path products (the cast kernel's rounding)
  if (out16) store_cols<bf16_t, NI>(out16 + row * W, lane, v);
}

// Backward in one pass over g and x: a workgroup takes RCB rows (wave k the
// rows k, k + 4, ...), writes dx per row and sums g x inv per column in
// registers; the four waves' column sums are added in wave order through LDS
// into the workgroup's row of `partial` (rms_dw_final adds the chunks).
template <class T, int NI>
__global__ void __launch_bounds__(256) rms_backward_cols_kernel(const float* g, const T* x, const float* w,
                                                                const float* inv, const float* residual, T* dx,
                                                                float* partial, int64_t rows) {
  constexpr int W = 256 * NI;
  __shared__ f32x4 sums[4][W / 4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t r0 = (int64_t)blockIdx.x * RCB, r1 = min(rows, r0 + RCB);
  f32x4 wv[NI], acc[NI];
  load_cols<float, NI>(w, lane, wv);
#pragma unroll
  for (int i = 0; i < NI; i++) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int64_t r = r0 + wave; r < r1; r += 4) {
    f32x4 gv[NI], xv[NI];
    load_cols<float, NI>(g + r * W, lane, gv);
    load_cols<T, NI>(x + r * W, lane, xv);
    float total = 0.f;
#pragma unroll
    for (int i = 0; i < NI; i++) {
      const f32x4 t = gv[i] * wv[i] * xv[i];
      total += t[0] + t[1] + t[2] + t[3];
    }
    const float projected = wave_sum(total) / (float)W, scale = inv[r];
#pragma unroll
    for (int i = 0; i < NI; i++) {
      acc[i] += gv[i] * xv[i] * scale;
      gv[i] = scale * (gv[i] * wv[i] - xv[i] * (scale * scale * projected));
    }
    if (residual) {  // fp32 only: dx = residual + dx, one rounding (may be dx itself)
      f32x4 rv[NI];
      load_cols<float, NI>(residual + r * W, lane, rv);
#pragma unroll
      for (int i = 0; i < NI; i++) gv[i] = rv[i] + gv[i];
    }
    store_cols<T, NI>(dx + r * W, lane, gv);
  }
#pragma unroll
  for (int i = 0; i < NI; i++) sums[wave][lane + 64 * i] = acc[i];
  __syncthreads();
  for (int q = threadIdx.x; q < W / 4; q += 256) {
    f32x4 t = sums[0][q];
#pragma unroll
    for (int k = 1; k < 4; k++) t += sums[k][q];
    global_store(partial + (int64_t)blockIdx.x * W + 4 * q, t);
  }
}

// dw[j] = sum over chunks c of partial[c][j]: 16 parts of consecutive
// chunks, each summed in chunk order, then the parts added in order; 16
// columns per workgroup
__global__ void __launch_bounds__(256) rms_dw_final_parts(const float* partial, float* dw, int64_t chunks,
                                                          int64_t width) {
  __shared__ float part[16][16];
  const int col = threadIdx.x & 15, k = threadIdx.x >> 4;
  const int64_t j = (int64_t)blockIdx.x * 16 + col;
  const int64_t per = (chunks + 15) / 16, c0 = k * per, c1 = min(chunks, c0 + per);
  float total = 0.f;
  if (j < width) {
    // eight loads in flight, added in chunk order
    int64_t c = c0;
    for (; c + 7 < c1; c += 8) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; u++) v[u] = partial[(c + u) * width + j];
#pragma unroll
      for (int u = 0; u < 8; u++) total += v[u];
    }
    for (; c < c1; c++) total += partial[c * width + j];
  }
  part[k][col] = total;
  __syncthreads();
  if (k == 0 && j < width) {
    float sum = part[0][col];
    for (int q = 1; q < 16; q++) sum += part[q][col];
    dw[j] = sum;
  }
}

// silu (backward = 0) or its derivative times g (lm.cu:54), s = sigmoid_f
// (common.h)
template <class T>
__global__ void silu_kernel(const T* x, const T* g, T* out, int64_t n, int backward) {
  GRID_STRIDE(i, n) {
    const float v = get<T>(x, i), s = sigmoid_f(v);
    put<T>(out, i, backward ? get<T>(g, i) * s * (1.f + v * (1.f - s)) : v * s);
  }
}

// (x0, x1) at `at` rotated by the angle with sine s and cosine c, the
// contractions spelled out so that every kernel rounds the same way
template <class T>
__device__ __forceinline__ void rotate_pair(const T* x, T* out, int64_t at, int64_t to, float s, float c) {
  const float x0 = get<T>(x, at), x1 = get<T>(x, at + 1);
  put<T>(out, to, fmaf(x0, c, -(x1 * s)));
  put<T>(out, to + 1, fmaf(x0, s, x1 * c));
}

// rotary embedding of the pairs (2i, 2i+1) of [batch][time][heads][dim]:
// angle (offset + t) * theta^(-d/dim), d = 2 (i mod dim/2); inverse rotates
// back (lm.cu:55-59).  A position's heads*dim values start x_row (out_row)
// elements after the previous position's: heads*dim for a contiguous block,
// more for a column slice of a wider matrix.
template <class T>
__global__ void rope_kernel(const T* x, T* out, int64_t pairs, int64_t time, int64_t heads, int64_t dim, float theta,
                            int64_t offset, int inverse, int64_t x_row, int64_t out_row) {
  const int64_t per = heads * (dim / 2);
  GRID_STRIDE(i, pairs) {
    const int64_t bt = i / per, within = 2 * (i % per), d = (i % (dim / 2)) * 2, t = bt % time;
    const float a = (float)(offset + t) * powf(theta, -(float)d / (float)dim) * (inverse ? -1.f : 1.f);
    float s, c;
    sincosf(a, &s, &c);
    rotate_pair<T>(x, out, bt * x_row + within, bt * out_row + within, s, c);
  }
}

// The same rotation with the angle's sine and cosine computed once per
// (position, pair) and applied to every head: one lane per (b t, pair),
// looping over the heads (the angle does not depend on the head).
template <class T>
__global__ void rope_heads_kernel(const T* x, T* out, int64_t items, int64_t time, int64_t heads, int64_t dim,
                                  float theta, int64_t offset, int inverse, int64_t x_row, int64_t out_row) {
  const int64_t half = dim / 2;
  GRID_STRIDE(i, items) {
    const int64_t bt = i / half, p = i % half, d = 2 * p, t = bt % time;
    const float a = (float)(offset + t) * powf(theta, -(float)d / (float)dim) * (inverse ? -1.f : 1.f);
    float s, c;
    sincosf(a, &s, &c);
    for (int64_t h = 0; h < heads; h++) {
      rotate_pair<T>(x, out, bt * x_row + h * dim + d, bt * out_row + h * dim + d, s, c);
    }
  }
}

// The same rotation with 16-byte accesses: a lane takes the P = 16 /
// (2 sizeof(T)) consecutive pairs of one position that share a 16-byte chunk
// (their angles computed once, with the expressions above, so the bits are
// the same) in up to HB heads, whose chunks it loads together before
// rotating and storing them.  Bases and row pitches 16-byte aligned, dim a
// multiple of 2P.
constexpr int ROPE_HB = 8;
template <class T>
__global__ void rope_heads_vec(const T* x, T* out, int64_t items, int64_t time, int64_t heads, int64_t dim,
                               float theta, int64_t offset, int inverse, int64_t x_row, int64_t out_row) {
  constexpr int P = 16 / (2 * (int)sizeof(T));
  const int64_t groups = dim / (2 * P), blocks = (heads + ROPE_HB - 1) / ROPE_HB;
  GRID_STRIDE(i, items) {
    const int64_t g = i % groups, hb = (i / groups) % blocks, bt = i / (groups * blocks), t = bt % time;
    float s[P], c[P];
#pragma unroll
    for (int q = 0; q < P; q++) {
      const int64_t d = 2 * (g * P + q);
      const float a = (float)(offset + t) * powf(theta, -(float)d / (float)dim) * (inverse ? -1.f : 1.f);
      sincosf(a, &s[q], &c[q]);
    }
    const int64_t h0 = hb * ROPE_HB;
    const int n = (int)(heads - h0 < ROPE_HB ? heads - h0 : ROPE_HB);
    const T* src = x + bt * x_row + h0 * dim + 2 * g * P;
    T* dst = out + bt * out_row + h0 * dim + 2 * g * P;
    u32x4 w[ROPE_HB];
#pragma unroll
    for (int h = 0; h < ROPE_HB; h++)
      if (h < n) w[h] = global_load<u32x4>(src + h * dim);
#pragma unroll
    for (int h = 0; h < ROPE_HB; h++) {
      if (h >= n) break;
      float v[2 * P];
      if constexpr (sizeof(T) == 2) {
#pragma unroll
        for (int k = 0; k < 8; k++) v[k] = __uint_as_float(((w[h][k >> 1] >> (16 * (k & 1))) & 0xffffu) << 16);
      } else {
#pragma unroll
        for (int k = 0; k < 4; k++) v[k] = __uint_as_float(w[h][k]);
      }
      float y[2 * P];
#pragma unroll
      for (int q = 0; q < P; q++) {
        y[2 * q] = fmaf(v[2 * q], c[q], -(v[2 * q + 1] * s[q]));
        y[2 * q + 1] = fmaf(v[2 * q], s[q], v[2 * q + 1] * c[q]);
      }
      u32x4 r;
      if constexpr (sizeof(T) == 2) {
#pragma unroll
        for (int k = 0; k < 4; k++)
          r[k] = (uint32_t)f32_to_bf16(y[2 * k]) | ((uint32_t)f32_to_bf16(y[2 * k + 1]) << 16);
      } else {
#pragma unroll
        for (int k = 0; k < 4; k++) r[k] = __float_as_uint(y[k]);
      }
      global_store(dst + h * dim, r);
    }
  }
}

// rows start.. of the (time-1)-long prediction positions of every sequence
// (lm.cu:425-427); backward adds the rows back into the [.. time ..] layout
template <class T>
__global__ void head_rows_kernel(const T* x, T* out, int64_t n, int64_t start, int64_t width, int64_t time,
                                 int backward) {
  GRID_STRIDE(i, n) {
    const int64_t row = start + i / width;
    const int64_t at = ((row / (time - 1)) * time + row % (time - 1)) * width + i % width;
    if (backward) put<T>(out, at, get<T>(out, at) + get<T>(x, i));
    else put<T>(out, i, get<T>(x, at));
  }
}

// Loss head rows: one 256-thread workgroup per row of logits.  Each thread
// keeps a running (max, sum of exp(v - max)) over its 16-byte chunks of the
// row (one exp per element; the sum is rescaled when the max grows), the
// pairs are merged across the wave and then across the 4 waves in LDS, in a
// fixed order.  The gradient kernel's second pass re-reads the row, which the
// first pass has just brought into L2.
constexpr int HEAD_THREADS = 256;

struct MaxSum {
  float m, s;
};

__device__ __forceinline__ MaxSum merge(MaxSum a, MaxSum b) {
  const float m = fmaxf(a.m, b.m);
  if (m == -INFINITY) return {m, 0.f};
  return {m, a.s * expf(a.m - m) + b.s * expf(b.m - m)};
}

// exp(x) for x <= 0 (a logit minus its row's running max) as the hardware
// exp2 of x log2(e): one multiply and one v_exp_f32 instead of the library
// expf's range reduction; relative error about |x| 2^-24 (4e-7 at x = -10),
// far inside the fp32 parity bar of the loss and its gradient.
__device__ __forceinline__ float exp_shifted(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }

// Fold up to 8 values (n of them valid) into the running pair.
__device__ __forceinline__ MaxSum fold(MaxSum a, const float* v, int n) {
  float top = v[0];
  for (int i = 1; i < n; i++) top = fmaxf(top, v[i]);
  if (top > a.m) {
    a.s = a.m == -INFINITY ? 0.f : a.s * expf(a.m - top);
    a.m = top;
  }
  for (int i = 0; i < n; i++) a.s += exp_shifted(v[i] - a.m);
  return a;
}

template <class T> constexpr int chunk_of() { return 16 / (int)sizeof(T); }

template <class T>
__device__ __forceinline__ void load_chunk(const T* p, float* v) {
  if constexpr (sizeof(T) == 2) {
    const uint4 raw = *(const uint4*)p;
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  } else {
    const float4 raw = *(const float4*)p;
    v[0] = raw.x, v[1] = raw.y, v[2] = raw.z, v[3] = raw.w;
  }
}

// (max, sum of exp(v - max)) of one row, the same value in every thread.
template <class T>
__device__ MaxSum row_max_sum(const T* l, int64_t vocab, bool vec) {
  __shared__ MaxSum partial[HEAD_THREADS / 64];
  MaxSum a = {-INFINITY, 0.f};
  constexpr int V = chunk_of<T>();
  float v[8];
  if (vec) {
    // four chunks in flight per thread, then their folds in column order
    constexpr int64_t STEP = (int64_t)HEAD_THREADS * V;
    int64_t c = (int64_t)threadIdx.x * V;
    for (; c + 3 * STEP < vocab; c += 4 * STEP) {
      float w[4][8];
#pragma unroll
      for (int u = 0; u < 4; u++) load_chunk<T>(l + c + u * STEP, w[u]);
#pragma unroll
      for (int u = 0; u < 4; u++) a = fold(a, w[u], V);
    }
    for (; c < vocab; c += STEP) {
      load_chunk<T>(l + c, v);
      a = fold(a, v, V);
    }
  } else {
    for (int64_t c = threadIdx.x; c < vocab; c += HEAD_THREADS) {
      v[0] = get<T>(l, c);
      a = fold(a, v, 1);
    }
  }
#pragma unroll
  for (int o = 32; o; o >>= 1) a = merge(a, {__shfl_xor(a.m, o), __shfl_xor(a.s, o)});
  if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = a;
  __syncthreads();
  MaxSum total = partial[0];
#pragma unroll
  for (int w = 1; w < HEAD_THREADS / 64; w++) total = merge(total, partial[w]);
  return total;
}

// out[row] = log(sum exp(l - max)) - (l[label] - max), 0 for label -100
// (lm.cu:430-433)
template <class T>
__global__ void __launch_bounds__(HEAD_THREADS) head_loss_kernel(const T* logits, const int64_t* labels, float* out,
                                                                 int64_t vocab, bool vec) {
  const int64_t row = blockIdx.x;
  const int64_t label = labels[row];
  if (label == -100) {
    if (threadIdx.x == 0) out[row] = 0.f;
    return;
  }
  const T* l = logits + row * vocab;
  const MaxSum t = row_max_sum<T>(l, vocab, vec);
  if (threadIdx.x == 0) out[row] = logf(t.s) - (get<T>(l, label) - t.m);
}

// in place: logits = g * factor * (softmax - onehot(label)); label -100 -> 0
// (lm.cu:434-440)
template <class T>
__global__ void __launch_bounds__(HEAD_THREADS) head_gradient_kernel(T* logits, const int64_t* labels,
                                                                     const float* gradient, int64_t vocab,
                                                                     float factor, bool vec) {
  const int64_t row = blockIdx.x;
  const int64_t label = labels[row];
  T* l = logits + row * vocab;
  constexpr int V = chunk_of<T>();
  if (label == -100) {
    for (int64_t c = threadIdx.x; c < vocab; c += HEAD_THREADS) put<T>(l, c, 0.f);
    return;
  }
  const MaxSum t = row_max_sum<T>(l, vocab, vec);
  const float scale = gradient[0] * factor, inv = 1.f / t.s;
  if (vec) {
    float v[8];
    for (int64_t c = (int64_t)threadIdx.x * V; c < vocab; c += HEAD_THREADS * V) {
      load_chunk<T>(l + c, v);
#pragma unroll
      for (int i = 0; i < V; i++) v[i] = scale * (exp_shifted(v[i] - t.m) * inv - (c + i == label ? 1.f : 0.f));
      if constexpr (sizeof(T) == 2) {
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; i++) w[i] = (uint32_t)f32_to_bf16(v[2 * i]) | ((uint32_t)f32_to_bf16(v[2 * i + 1]) << 16);
        *(uint4*)(l + c) = make_uint4(w[0], w[1], w[2], w[3]);
      } else {
        *(float4*)(l + c) = make_float4(v[0], v[1], v[2], v[3]);
      }
    }
  } else {
    for (int64_t c = threadIdx.x; c < vocab; c += HEAD_THREADS)
      put<T>(l, c, scale * (exp_shifted(get<T>(l, c) - t.m) * inv - (c == label ? 1.f : 0.f)));
  }
}

// Vocabulary-blocked loss head.  The logits of all prediction rows are made
// one block of vocabulary columns at a time ([rows][cols] holding columns
// col0 .. col0+cols of the [rows][vocab] logits), so the weight gradient of a
// block is one GEMM over all rows, written once, instead of a read-modify-write
// of the whole [vocab][width] gradient per block of rows.  Per row, stats
// holds the running (max, sum of exp(v - max)) over the blocks seen so far and
// picked the label's logit.
template <class T>
__global__ void __launch_bounds__(HEAD_THREADS) head_block_stats_kernel(const T* logits, const int64_t* labels,
                                                                        float* stats, float* picked, int64_t cols,
                                                                        int64_t col0, int first, bool vec) {
  const int64_t row = blockIdx.x;
  const int64_t label = labels[row];
  if (label == -100) return;
  const T* l = logits + row * cols;
  const MaxSum t = row_max_sum<T>(l, cols, vec);
  if (threadIdx.x == 0) {
    const MaxSum m = first ? t : merge({stats[2 * row], stats[2 * row + 1]}, t);
    stats[2 * row] = m.m;
    stats[2 * row + 1] = m.s;
    if (label >= col0 && label < col0 + cols) picked[row] = get<T>(l, label - col0);
  }
}

// out[r] = log(sum) + max - picked (the row's cross entropy), 0 for label -100
__global__ void head_block_loss_kernel(const float* stats, const float* picked, const int64_t* labels, float* out,
                                       int64_t rows) {
  GRID_STRIDE(r, rows) out[r] = labels[r] == -100 ? 0.f : logf(stats[2 * r + 1]) + stats[2 * r] - picked[r];
}

// in place over one block: g * factor * (exp(v - max) / sum - onehot(label))
template <class T>
__global__ void __launch_bounds__(HEAD_THREADS) head_block_gradient_kernel(T* logits, const int64_t* labels,
                                                                           const float* stats, const float* gradient,
                                                                           int64_t cols, int64_t col0, float factor,
                                                                           bool vec) {
  const int64_t row = blockIdx.x;
  const int64_t label = labels[row] == -100 ? -100 : labels[row] - col0;
  T* l = logits + row * cols;
  constexpr int V = chunk_of<T>();
  if (labels[row] == -100) {
    for (int64_t c = threadIdx.x; c < cols; c += HEAD_THREADS) put<T>(l, c, 0.f);
    return;
  }
  const float m = stats[2 * row], inv = 1.f / stats[2 * row + 1], scale = gradient[0] * factor;
  if (vec) {
    float v[8];
    for (int64_t c = (int64_t)threadIdx.x * V; c < cols; c += HEAD_THREADS * V) {
      load_chunk<T>(l + c, v);
#pragma unroll
      for (int i = 0; i < V; i++) v[i] = scale * (exp_shifted(v[i] - m) * inv - (c + i == label ? 1.f : 0.f));
      if constexpr (sizeof(T) == 2) {
        *(uint4*)(l + c) = make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                                      pack_bf16x2(v[6], v[7]));
      } else {
        *(float4*)(l + c) = make_float4(v[0], v[1], v[2], v[3]);
      }
    }
  } else {
    for (int64_t c = threadIdx.x; c < cols; c += HEAD_THREADS)
      put<T>(l, c, scale * (exp_shifted(get<T>(l, c) - m) * inv - (c == label ? 1.f : 0.f)));
  }
}

// The same with 16-byte chunks: one workgroup per selected row (the row
// index arithmetic once per row), rows of whole chunks and aligned bases.
// The backward add is the elementwise one (fp32 sum, one rounding).
template <class T>
__global__ void __launch_bounds__(256) head_rows_vec(const T* x, T* out, int64_t start, int64_t width, int64_t time,
                                                     int backward) {
  constexpr int V = 16 / (int)sizeof(T);
  const int64_t i = blockIdx.x, row = start + i;
  const int64_t at = (row / (time - 1)) * time + row % (time - 1);
  const T* src = x + (backward ? i : at) * width;
  T* dst = out + (backward ? at : i) * width;
  for (int64_t c = (int64_t)threadIdx.x * V; c < width; c += 256 * V) {
    if (!backward) {
      *(uint4*)(dst + c) = *(const uint4*)(src + c);
      continue;
    }
    float a[8], b[8];
    load_chunk<T>(src + c, a);
    load_chunk<T>(dst + c, b);
#pragma unroll
    for (int e = 0; e < V; e++) b[e] += a[e];
    if constexpr (sizeof(T) == 2)
      *(uint4*)(dst + c) = make_uint4(pack_bf16x2(b[0], b[1]), pack_bf16x2(b[2], b[3]), pack_bf16x2(b[4], b[5]),
                                      pack_bf16x2(b[6], b[7]));
    else
      *(float4*)(dst + c) = make_float4(b[0], b[1], b[2], b[3]);
  }
}

bool act_dtype(int d) { return d == F32 || d == BF16; }

// rows of whole 256-column groups, at most 2048 wide, 16-byte aligned base
bool cols_path(const void* p, int64_t width) {
  return width % 256 == 0 && width <= 2048 && (uintptr_t)p % 16 == 0;
}

// 16-byte chunks need an aligned base and rows that are whole chunks
bool vec_rows(const void* p, int64_t vocab, int per_chunk) {
  return (uintptr_t)p % 16 == 0 && vocab % per_chunk == 0;
}

}  // namespace

extern "C" {

int qutai_amd_embedding(const float* weight, const int64_t* ids, void* out, int64_t count, int64_t width,
                        int out_dtype, void* stream) {
  if (count < 0 || width < 0 || !act_dtype(out_dtype)) return QA_EINVAL;
  const int64_t n = count * width;
  if (n == 0) return QA_OK;
  hipStream_t s = (hipStream_t)stream;
  if (width % 4 == 0 && (uintptr_t)weight % 16 == 0 && (uintptr_t)out % 16 == 0 && count <= 0x7fffffff) {
    if (out_dtype == BF16)
      hipLaunchKernelGGL(embedding_rows<bf16_t>, dim3((unsigned)count), dim3(256), 0, s, weight, ids, (bf16_t*)out,
                         width);
    else
      hipLaunchKernelGGL(embedding_rows<float>, dim3((unsigned)count), dim3(256), 0, s, weight, ids, (float*)out,
                         width);
    return (int)hipGetLastError();
  }
  if (out_dtype == BF16)
    hipLaunchKernelGGL(embedding_kernel<bf16_t>, dim3(blocks_for(n)), dim3(256), 0, s, weight, ids, (bf16_t*)out, n,
                       width);
  else
    hipLaunchKernelGGL(embedding_kernel<float>, dim3(blocks_for(n)), dim3(256), 0, s, weight, ids, (float*)out, n,
                       width);
  return (int)hipGetLastError();
}

int qutai_amd_embedding_backward(const void* gradient, const int64_t* tokens, const int64_t* offsets,
                                 const int64_t* rows, float* out, int64_t groups, int64_t width, int dtype,
                                 int accumulate, void* stream) {
  if (groups < 0 || width < 0 || !act_dtype(dtype)) return QA_EINVAL;
  const int64_t n = groups * width;
  if (n == 0) return QA_OK;
  hipStream_t s = (hipStream_t)stream;
  if (width % 4 == 0 && (uintptr_t)gradient % 16 == 0 && (uintptr_t)out % 16 == 0 && groups <= 0x7fffffff) {
    if (dtype == BF16)
      hipLaunchKernelGGL(embedding_grad_rows<bf16_t>, dim3((unsigned)groups), dim3(256), 0, s,
                         (const bf16_t*)gradient, tokens, offsets, rows, out, width, accumulate ? 1 : 0);
    else
      hipLaunchKernelGGL(embedding_grad_rows<float>, dim3((unsigned)groups), dim3(256), 0, s, (const float*)gradient,
                         tokens, offsets, rows, out, width, accumulate ? 1 : 0);
    return (int)hipGetLastError();
  }
  if (dtype == BF16)
    hipLaunchKernelGGL(embedding_grad_kernel<bf16_t>, dim3(blocks_for(n)), dim3(256), 0, s, (const bf16_t*)gradient,
                       tokens, offsets, rows, out, n, width, accumulate ? 1 : 0);
  else
    hipLaunchKernelGGL(embedding_grad_kernel<float>, dim3(blocks_for(n)), dim3(256), 0, s, (const float*)gradient,
                       tokens, offsets, rows, out, n, width, accumulate ? 1 : 0);
  return (int)hipGetLastError();
}

int qutai_amd_rms_norm(const void* x, const float* weight, float* out, float* inverse, int64_t rows, int64_t width,
                       double eps, int dtype, void* stream) {
  return qutai_amd_rms_norm_bf16(x, weight, out, nullptr, inverse, rows, width, eps, dtype, stream);
}

int qutai_amd_rms_norm_bf16(const void* x, const float* weight, float* out, void* out_bf16, float* inverse,
                            int64_t rows, int64_t width, double eps, int dtype, void* stream) {
  if (rows < 0 || width <= 0 || !act_dtype(dtype)) return QA_EINVAL;
  if (rows == 0) return QA_OK;
  const unsigned blocks = (unsigned)((rows + ROWS_PER_BLOCK - 1) / ROWS_PER_BLOCK);
  hipStream_t s = (hipStream_t)stream;
  bf16_t* out16 = (bf16_t*)out_bf16;
  if (cols_path(x, width) && cols_path(weight, width) && cols_path(out, width) &&
      (!out16 || (uintptr_t)out16 % 8 == 0)) {
    const bool bf = dtype == BF16;
    switch (width / 256) {
#define QA_RMS(N)                                                                                                   \
  case N:                                                                                                           \
    if (bf) hipLaunchKernelGGL((rms_cols_kernel<bf16_t, N>), dim3(blocks), dim3(256), 0, s, (const bf16_t*)x, weight, \
                               out, inverse, rows, (float)eps, out16);                                              \
    else hipLaunchKernelGGL((rms_cols_kernel<float, N>), dim3(blocks), dim3(256), 0, s, (const float*)x, weight, out,   \
                            inverse, rows, (float)eps, out16);                                                      \
    break;
      QA_RMS(1) QA_RMS(2) QA_RMS(3) QA_RMS(4) QA_RMS(5) QA_RMS(6) QA_RMS(7) QA_RMS(8)
#undef QA_RMS
    }
    return (int)hipGetLastError();
  }
  if (dtype == BF16)
    hipLaunchKernelGGL(rms_kernel<bf16_t>, dim3(blocks), dim3(256), 0, s, (const bf16_t*)x, weight, out, inverse,
                       rows, width, (float)eps, out16);
  else
    hipLaunchKernelGGL(rms_kernel<float>, dim3(blocks), dim3(256), 0, s, (const float*)x, weight, out, inverse, rows,
                       width, (float)eps, out16);
  return (int)hipGetLastError();
}

int64_t qutai_amd_rms_norm_workspace(int64_t rows, int64_t width) {
  return rows <= 0 || width <= 0 ? 0 : ((rows + RCB - 1) / RCB) * width;
}

int qutai_amd_rms_norm_backward(const float* gradient, const void* x, const float* weight, const float* inverse,
                                const float* residual, void* dx, float* dweight, float* partial, int64_t rows,
                                int64_t width, int dtype, void* stream) {
  if (rows < 0 || width <= 0 || !act_dtype(dtype) || (residual && (dtype != F32 || residual == dx)))
    return QA_EINVAL;
  hipStream_t s = (hipStream_t)stream;
  if (rows == 0) return QA_OK;
  if (!partial) return QA_EWORKSPACE;
  const unsigned blocks = (unsigned)((rows + ROWS_PER_BLOCK - 1) / ROWS_PER_BLOCK);
  const int64_t chunks = (rows + RC - 1) / RC;
  if (chunks > 65535) return QA_EINVAL;
  const dim3 grid((unsigned)((width + 255) / 256), (unsigned)chunks);
  if (cols_path(gradient, width) && cols_path(x, width) && cols_path(weight, width) && cols_path(dx, width) &&
      cols_path(partial, width) && (!residual || cols_path(residual, width))) {
    const bool bf = dtype == BF16;
    const int64_t groups = (rows + RCB - 1) / RCB;
    switch (width / 256) {
#define QA_RMSB(N)                                                                                                 \
  case N:                                                                                                          \
    if (bf) hipLaunchKernelGGL((rms_backward_cols_kernel<bf16_t, N>), dim3((unsigned)groups), dim3(256), 0, s,      \
                               gradient, (const bf16_t*)x, weight, inverse, nullptr, (bf16_t*)dx, partial, rows);   \
    else hipLaunchKernelGGL((rms_backward_cols_kernel<float, N>), dim3((unsigned)groups), dim3(256), 0, s, gradient, \
                            (const float*)x, weight, inverse, residual, (float*)dx, partial, rows);                \
    break;
      QA_RMSB(1) QA_RMSB(2) QA_RMSB(3) QA_RMSB(4) QA_RMSB(5) QA_RMSB(6) QA_RMSB(7) QA_RMSB(8)
#undef QA_RMSB
    }
    hipLaunchKernelGGL(rms_dw_final_parts, dim3((unsigned)((width + 15) / 16)), dim3(256), 0, s, partial, dweight,
                       groups, width);
    return (int)hipGetLastError();
  }
  if (dtype == BF16) {
    hipLaunchKernelGGL(rms_dx_kernel<bf16_t>, dim3(blocks), dim3(256), 0, s, gradient, (const bf16_t*)x, weight,
                       inverse, (bf16_t*)dx, rows, width);
    hipLaunchKernelGGL(rms_dw_partial_kernel<bf16_t>, grid, dim3(256), 0, s, gradient, (const bf16_t*)x, inverse,
                       partial, rows, width);
  } else {
    hipLaunchKernelGGL(rms_dx_kernel<float>, dim3(blocks), dim3(256), 0, s, gradient, (const float*)x, weight,
                       inverse, (float*)dx, rows, width);
    if (residual) {
      const int rc = qutai_amd_add(residual, dx, dx, rows * width, QA_F32, stream);
      if (rc != QA_OK) return rc;
    }
    hipLaunchKernelGGL(rms_dw_partial_kernel<float>, grid, dim3(256), 0, s, gradient, (const float*)x, inverse,
                       partial, rows, width);
  }
  hipLaunchKernelGGL(rms_dw_final_kernel, dim3(blocks_for(width)), dim3(256), 0, s, partial, dweight, chunks, width);
  return (int)hipGetLastError();
}

int qutai_amd_silu(const void* x, const void* gradient, void* out, int64_t n, int backward, int dtype,
                   void* stream) {
  if (n < 0 || !act_dtype(dtype) || (backward && !gradient)) return QA_EINVAL;
  if (n == 0) return QA_OK;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == BF16)
    hipLaunchKernelGGL(silu_kernel<bf16_t>, dim3(blocks_for(n)), dim3(256), 0, s, (const bf16_t*)x,
                       (const bf16_t*)gradient, (bf16_t*)out, n, backward ? 1 : 0);
  else
    hipLaunchKernelGGL(silu_kernel<float>, dim3(blocks_for(n)), dim3(256), 0, s, (const float*)x,
                       (const float*)gradient, (float*)out, n, backward ? 1 : 0);
  return (int)hipGetLastError();
}

int qutai_amd_rope_rows(const void* x, void* out, int64_t batch, int64_t time, int64_t heads, int64_t dim,
                        double theta, int64_t offset, int inverse, int64_t x_row, int64_t out_row, int dtype,
                        void* stream) {
  if (batch < 0 || time < 0 || heads < 0 || dim <= 0 || dim % 2 || !act_dtype(dtype)) return QA_EINVAL;
  if (x_row < heads * dim || out_row < heads * dim) return QA_EINVAL;
  const int64_t pairs = batch * time * heads * dim / 2;
  if (pairs == 0) return QA_OK;
  hipStream_t s = (hipStream_t)stream;
  if (heads > 1) {  // one angle per (position, pair), shared by the heads
    const int64_t es = dtype == BF16 ? 2 : 4, P = 16 / (2 * es);
    if (dim % (2 * P) == 0 && (uintptr_t)x % 16 == 0 && (uintptr_t)out % 16 == 0 && (x_row * es) % 16 == 0 &&
        (out_row * es) % 16 == 0) {
      const int64_t items = batch * time * (dim / (2 * P)) * ((heads + ROPE_HB - 1) / ROPE_HB);
      if (dtype == BF16)
        hipLaunchKernelGGL(rope_heads_vec<bf16_t>, dim3(blocks_for(items)), dim3(256), 0, s, (const bf16_t*)x,
                           (bf16_t*)out, items, time, heads, dim, (float)theta, offset, inverse ? 1 : 0, x_row,
                           out_row);
      else
        hipLaunchKernelGGL(rope_heads_vec<float>, dim3(blocks_for(items)), dim3(256), 0, s, (const float*)x,
                           (float*)out, items, time, heads, dim, (float)theta, offset, inverse ? 1 : 0, x_row,
                           out_row);
      return (int)hipGetLastError();
    }
    const int64_t items = batch * time * dim / 2;
    if (dtype == BF16)
      hipLaunchKernelGGL(rope_heads_kernel<bf16_t>, dim3(blocks_for(items)), dim3(256), 0, s, (const bf16_t*)x,
                         (bf16_t*)out, items, time, heads, dim, (float)theta, offset, inverse ? 1 : 0, x_row, out_row);
    else
      hipLaunchKernelGGL(rope_heads_kernel<float>, dim3(blocks_for(items)), dim3(256), 0, s, (const float*)x,
                         (float*)out, items, time, heads, dim, (float)theta, offset, inverse ? 1 : 0, x_row, out_row);
    return (int)hipGetLastError();
  }
  if (dtype == BF16)
    hipLaunchKernelGGL(rope_kernel<bf16_t>, dim3(blocks_for(pairs)), dim3(256), 0, s, (const bf16_t*)x, (bf16_t*)out,
                       pairs, time, heads, dim, (float)theta, offset, inverse ? 1 : 0, x_row, out_row);
  else
    hipLaunchKernelGGL(rope_kernel<float>, dim3(blocks_for(pairs)), dim3(256), 0, s, (const float*)x, (float*)out,
                       pairs, time, heads, dim, (float)theta, offset, inverse ? 1 : 0, x_row, out_row);
  return (int)hipGetLastError();
}

int qutai_amd_rope(const void* x, void* out, int64_t batch, int64_t time, int64_t heads, int64_t dim, double theta,
                   int64_t offset, int inverse, int dtype, void* stream) {
  return qutai_amd_rope_rows(x, out, batch, time, heads, dim, theta, offset, inverse, heads * dim, heads * dim, dtype,
                             stream);
}

int qutai_amd_head_rows(const void* x, void* out, int64_t count, int64_t start, int64_t width, int64_t time,
                        int backward, int dtype, void* stream) {
  if (count < 0 || start < 0 || width < 0 || time < 2 || !act_dtype(dtype)) return QA_EINVAL;
  const int64_t n = count * width;
  if (n == 0) return QA_OK;
  hipStream_t s = (hipStream_t)stream;
  const int per = dtype == BF16 ? 8 : 4;
  if (width % per == 0 && (uintptr_t)x % 16 == 0 && (uintptr_t)out % 16 == 0 && count <= 0x7fffffff) {
    if (dtype == BF16)
      hipLaunchKernelGGL(head_rows_vec<bf16_t>, dim3((unsigned)count), dim3(256), 0, s, (const bf16_t*)x,
                         (bf16_t*)out, start, width, time, backward ? 1 : 0);
    else
      hipLaunchKernelGGL(head_rows_vec<float>, dim3((unsigned)count), dim3(256), 0, s, (const float*)x, (float*)out,
                         start, width, time, backward ? 1 : 0);
    return (int)hipGetLastError();
  }
  if (dtype == BF16)
    hipLaunchKernelGGL(head_rows_kernel<bf16_t>, dim3(blocks_for(n)), dim3(256), 0, s, (const bf16_t*)x,
                       (bf16_t*)out, n, start, width, time, backward ? 1 : 0);
  else
    hipLaunchKernelGGL(head_rows_kernel<float>, dim3(blocks_for(n)), dim3(256), 0, s, (const float*)x, (float*)out,
                       n, start, width, time, backward ? 1 : 0);
  return (int)hipGetLastError();
}

int qutai_amd_head_loss(const void* logits, const int64_t* labels, float* out, int64_t rows, int64_t vocab,
                        int dtype, void* stream) {
  if (rows < 0 || vocab <= 0 || !act_dtype(dtype)) return QA_EINVAL;
  if (rows == 0) return QA_OK;
  if (rows > 0x7fffffff) return QA_EINVAL;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == BF16)
    hipLaunchKernelGGL(head_loss_kernel<bf16_t>, dim3((unsigned)rows), dim3(HEAD_THREADS), 0, s,
                       (const bf16_t*)logits, labels, out, vocab, vec_rows(logits, vocab, 8));
  else
    hipLaunchKernelGGL(head_loss_kernel<float>, dim3((unsigned)rows), dim3(HEAD_THREADS), 0, s, (const float*)logits,
                       labels, out, vocab, vec_rows(logits, vocab, 4));
  return (int)hipGetLastError();
}

int qutai_amd_head_gradient(void* logits, const int64_t* labels, const float* gradient, int64_t rows, int64_t vocab,
                            double factor, int dtype, void* stream) {
  if (rows < 0 || vocab <= 0 || !act_dtype(dtype)) return QA_EINVAL;
  if (rows == 0) return QA_OK;
  if (rows > 0x7fffffff) return QA_EINVAL;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == BF16)
    hipLaunchKernelGGL(head_gradient_kernel<bf16_t>, dim3((unsigned)rows), dim3(HEAD_THREADS), 0, s,
                       (bf16_t*)logits, labels, gradient, vocab, (float)factor, vec_rows(logits, vocab, 8));
  else
    hipLaunchKernelGGL(head_gradient_kernel<float>, dim3((unsigned)rows), dim3(HEAD_THREADS), 0, s, (float*)logits,
                       labels, gradient, vocab, (float)factor, vec_rows(logits, vocab, 4));
  return (int)hipGetLastError();
}

int qutai_amd_head_block_stats(const void* logits, const int64_t* labels, float* stats, float* picked, int64_t rows,
                               int64_t cols, int64_t col0, int first, int dtype, void* stream) {
  if (rows < 0 || cols <= 0 || col0 < 0 || !act_dtype(dtype) || !labels || !stats || !picked) return QA_EINVAL;
  if (rows == 0) return QA_OK;
  if (rows > 0x7fffffff) return QA_EINVAL;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == BF16)
    hipLaunchKernelGGL(head_block_stats_kernel<bf16_t>, dim3((unsigned)rows), dim3(HEAD_THREADS), 0, s,
                       (const bf16_t*)logits, labels, stats, picked, cols, col0, first ? 1 : 0,
                       vec_rows(logits, cols, 8));
  else
    hipLaunchKernelGGL(head_block_stats_kernel<float>, dim3((unsigned)rows), dim3(HEAD_THREADS), 0, s,
                       (const float*)logits, labels, stats, picked, cols, col0, first ? 1 : 0,
                       vec_rows(logits, cols, 4));
  return (int)hipGetLastError();
}

int qutai_amd_head_block_loss(const float* stats, const float* picked, const int64_t* labels, float* out,
                              int64_t rows, void* stream) {
  if (rows < 0 || !stats || !picked || !labels || !out) return QA_EINVAL;
  if (rows == 0) return QA_OK;
  hipLaunchKernelGGL(head_block_loss_kernel, dim3(blocks_for(rows)), dim3(256), 0, (hipStream_t)stream, stats,
                     picked, labels, out, rows);
  return (int)hipGetLastError();
}

int qutai_amd_head_block_gradient(void* logits, const int64_t* labels, const float* stats, const float* gradient,
                                  int64_t rows, int64_t cols, int64_t col0, double factor, int dtype, void* stream) {
  if (rows < 0 || cols <= 0 || col0 < 0 || !act_dtype(dtype) || !labels || !stats || !gradient) return QA_EINVAL;
  if (rows == 0) return QA_OK;
  if (rows > 0x7fffffff) return QA_EINVAL;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == BF16)
    hipLaunchKernelGGL(head_block_gradient_kernel<bf16_t>, dim3((unsigned)rows), dim3(HEAD_THREADS), 0, s,
                       (bf16_t*)logits, labels, stats, gradient, cols, col0, (float)factor,
                       vec_rows(logits, cols, 8));
  else
    hipLaunchKernelGGL(head_block_gradient_kernel<float>, dim3((unsigned)rows), dim3(HEAD_THREADS), 0, s,
                       (float*)logits, labels, stats, gradient, cols, col0, (float)factor,
                       vec_rows(logits, cols, 4));
  return (int)hipGetLastError();
}

}  // extern "C"
