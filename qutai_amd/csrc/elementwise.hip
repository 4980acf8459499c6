// Tensor algebra behind the reference's generic backend functions: strided
// copies (broadcast, axis permutation, concatenation, slice reads and
// writes), element-wise binary and unary arithmetic, and sums over one axis.
// All HBM-bound; every kernel moves 16 bytes per lane where the layout
// allows it.  Reference counterparts are cited per entry point in
// include/qutai_amd.h.
#include <type_traits>

#include "common.h"
#include "qutai_amd.h"

using namespace qa;

namespace {

constexpr int THREADS = 256;
constexpr int MAX_RANK = 8;

unsigned blocks_for(int64_t items, int64_t per_block = THREADS) {
  int64_t b = (items + per_block - 1) / per_block;
  return (unsigned)(b < 1 ? 1 : b > 65536 ? 65536 : b);
}

// ---- strided copy -------------------------------------------------------------
// dst[sum_d c_d * dst_stride_d] = src[sum_d c_d * src_stride_d] for every
// coordinate c of the index space `dims` (row-major).  A source stride of 0
// broadcasts.  Work item = one run of up to V consecutive elements of the
// innermost axis.
struct Strided {
  int rank;
  int64_t dims[MAX_RANK];
  int64_t src[MAX_RANK];
  int64_t dst[MAX_RANK];
};

template <int ES>
struct Word;
template <> struct Word<2> { typedef uint16_t T; };
template <> struct Word<4> { typedef uint32_t T; };
template <> struct Word<8> { typedef uint64_t T; };

// VEC: innermost axis contiguous in dst and contiguous (or broadcast) in src,
// its length a multiple of V and every outer offset a multiple of V, both
// bases 16-byte aligned: one 16-byte load (or a splat) and one 16-byte store.
template <int ES, bool VEC>
__global__ void __launch_bounds__(THREADS) strided_copy_kernel(const char* __restrict__ src, char* __restrict__ dst,
                                                               Strided s, int64_t items) {
  typedef typename Word<ES>::T W;
  constexpr int V = 16 / ES;
  const int r = s.rank;
  const int64_t inner = s.dims[r - 1];
  const int64_t runs = (inner + V - 1) / V;
  for (int64_t item = (int64_t)blockIdx.x * THREADS + threadIdx.x; item < items;
       item += (int64_t)gridDim.x * THREADS) {
    int64_t rest = item / runs;
    const int64_t c0 = (item - rest * runs) * V;
    int64_t so = c0 * s.src[r - 1], d_o = c0 * s.dst[r - 1];
    for (int d = r - 2; d >= 0; d--) {
      const int64_t q = rest / s.dims[d];
      const int64_t c = rest - q * s.dims[d];
      so += c * s.src[d];
      d_o += c * s.dst[d];
      rest = q;
    }
    if constexpr (VEC) {
      u32x4 v;
      if (s.src[r - 1] == 0) {
        W x = global_load<W>(reinterpret_cast<const W*>(src) + so);
        W lanes[V];
#pragma unroll
        for (int t = 0; t < V; t++) lanes[t] = x;
        v = __builtin_bit_cast(u32x4, lanes);
      } else {
        v = global_load<u32x4>(reinterpret_cast<const W*>(src) + so);
      }
      global_store(reinterpret_cast<W*>(dst) + d_o, v);
    } else {
      const int64_t n = inner - c0 < V ? inner - c0 : V;
      for (int t = 0; t < n; t++)
        global_store(reinterpret_cast<W*>(dst) + d_o + t * s.dst[r - 1],
                     global_load<W>(reinterpret_cast<const W*>(src) + so + t * s.src[r - 1]));
    }
  }
}

// ---- element-wise arithmetic ---------------------------------------------------
enum BinaryOp { OP_ADD = 0, OP_SUB = 1, OP_MUL = 2, OP_DIV = 3 };

template <class R>
__device__ __forceinline__ R binary_op(R x, R y, int op) {
  switch (op) {
    case OP_ADD: return x + y;
    case OP_SUB: return x - y;
    case OP_MUL: return x * y;
    default: return x / y;
  }
}

// 16 bytes per lane: 4 fp32, 8 bf16 (computed in fp32, one rounding) or 2 fp64.
// The binary and unary kernels may run in place (out == an input): each lane
// reads its elements before it writes them.
template <class T>
struct Lanes;
template <> struct Lanes<float> { static constexpr int V = 4; };
template <> struct Lanes<double> { static constexpr int V = 2; };
template <> struct Lanes<bf16_t> { static constexpr int V = 8; };

template <class T> struct Acc { typedef float R; };
template <> struct Acc<double> { typedef double R; };

template <class T>
__device__ __forceinline__ typename Acc<T>::R widen(T v) { return (typename Acc<T>::R)v; }
template <>
__device__ __forceinline__ float widen<bf16_t>(bf16_t v) { return bf16_to_f32(v); }
template <class T>
__device__ __forceinline__ T narrow(typename Acc<T>::R v) { return (T)v; }
template <>
__device__ __forceinline__ bf16_t narrow<bf16_t>(float v) { return f32_to_bf16(v); }

template <class T>
__global__ void __launch_bounds__(THREADS) binary_kernel(const T* a, const T* b, T* out, int64_t n, int64_t chunks, int op,
                                                         int* zero_flag) {
  typedef typename Acc<T>::R R;
  constexpr int V = Lanes<T>::V;
  bool zero = false;
  for (int64_t i = (int64_t)blockIdx.x * THREADS + threadIdx.x; i < chunks; i += (int64_t)gridDim.x * THREADS) {
    T x[V], y[V], z[V];
    *reinterpret_cast<u32x4*>(x) = global_load<u32x4>(a + i * V);
    *reinterpret_cast<u32x4*>(y) = global_load<u32x4>(b + i * V);
#pragma unroll
    for (int t = 0; t < V; t++) {
      const R yt = widen(y[t]);
      zero |= yt == R(0);
      z[t] = narrow<T>(binary_op(widen(x[t]), yt, op));
    }
    global_store(out + i * V, *reinterpret_cast<u32x4*>(z));
  }
  for (int64_t i = chunks * V + (int64_t)blockIdx.x * THREADS + threadIdx.x; i < n; i += (int64_t)gridDim.x * THREADS) {
    const R yt = widen(b[i]);
    zero |= yt == R(0);
    out[i] = narrow<T>(binary_op(widen(a[i]), yt, op));
  }
  // any zero divisor raises ZeroDivisionError on the host (a plain vector
  // store of 1 from every lane that saw one; all writers store the same value)
  if (zero_flag && op == OP_DIV && zero) global_store(zero_flag, 1);
}

enum UnaryOp {
  U_NEGATE = 0, U_SQUARE, U_SCALE, U_RELU, U_RELU_BACKWARD, U_GELU, U_GELU_BACKWARD, U_EXP, U_LOG, U_TANH, U_ATAN,
  U_TANH_BACKWARD, U_ATAN_BACKWARD, U_DIVIDE
};

template <class R>
__device__ __forceinline__ R unary_op(R x, R g, R factor, int op, bool& bad) {
  const R half = R(0.5), one = R(1);
  const R inv_sqrt2 = R(0.70710678118654752440), inv_sqrt_2pi = R(0.39894228040143267794);
  switch (op) {
    case U_NEGATE: return -x;
    case U_SQUARE: return x * x;
    case U_SCALE: return x * factor;
    case U_RELU: return x > R(0) ? x : R(0);
    case U_RELU_BACKWARD: return x > R(0) ? g : R(0);
    case U_GELU: return x * (one + erf(x * inv_sqrt2)) * half;
    case U_GELU_BACKWARD: return g * ((one + erf(x * inv_sqrt2)) * half + x * exp(-x * x * half) * inv_sqrt_2pi);
    case U_EXP: return exp(x);
    case U_LOG: bad |= !(x > R(0)); return log(x);
    case U_TANH: return tanh(x);
    case U_ATAN: return atan(x);
    case U_TANH_BACKWARD: { const R y = tanh(x); return g * (one - y * y); }
    case U_ATAN_BACKWARD: return g / (one + x * x);
    default: return x / factor;
  }
}

template <class T>
__global__ void __launch_bounds__(THREADS) unary_kernel(const T* x, const T* g, T* out, int64_t n, int64_t chunks, int op,
                                                        typename Acc<T>::R factor, int* flag) {
  typedef typename Acc<T>::R R;
  constexpr int V = Lanes<T>::V;
  bool bad = false;
  for (int64_t i = (int64_t)blockIdx.x * THREADS + threadIdx.x; i < chunks; i += (int64_t)gridDim.x * THREADS) {
    T xv[V], gv[V], z[V];
    *reinterpret_cast<u32x4*>(xv) = global_load<u32x4>(x + i * V);
    if (g) *reinterpret_cast<u32x4*>(gv) = global_load<u32x4>(g + i * V);
#pragma unroll
    for (int t = 0; t < V; t++) z[t] = narrow<T>(unary_op<R>(widen(xv[t]), g ? widen(gv[t]) : R(0), factor, op, bad));
    global_store(out + i * V, *reinterpret_cast<u32x4*>(z));
  }
  for (int64_t i = chunks * V + (int64_t)blockIdx.x * THREADS + threadIdx.x; i < n; i += (int64_t)gridDim.x * THREADS)
    out[i] = narrow<T>(unary_op<R>(widen(x[i]), g ? widen(g[i]) : R(0), factor, op, bad));
  if (flag && bad) global_store(flag, 1);
}

__global__ void set_flag_kernel(int* flag) { global_store(flag, 0); }

// ---- sums over one axis ---------------------------------------------------------
// x viewed as [outer][width][inner]; out[o][j] = sum_c x[o][c][j], accumulated
// in fp32 (fp64 for fp64) and rounded once.  The order of the partial sums is
// fixed by the launch shape alone, so results repeat bit for bit.

// inner == 1: one wave per (row, part); lanes stride over the part's
// columns, then a butterfly over the wave.  parts == 1 writes the rounded
// row sum; otherwise the fp partials of each row go to `partial[row][part]`.
template <class T>
__global__ void __launch_bounds__(THREADS) row_sum_kernel(const T* __restrict__ x, T* __restrict__ out,
                                                          typename Acc<T>::R* __restrict__ partial, int64_t rows,
                                                          int64_t width, int64_t parts, int64_t span) {
  typedef typename Acc<T>::R R;
  const int lane = threadIdx.x & 63;
  // waves stride over the items, so any number of rows fits the capped grid
  for (int64_t item = (int64_t)blockIdx.x * (THREADS / 64) + (threadIdx.x >> 6); item < rows * parts;
       item += (int64_t)gridDim.x * (THREADS / 64)) {
    const int64_t row = item / parts, part = item - row * parts;
    const int64_t lo = part * span, hi = lo + span < width ? lo + span : width;
    const T* p = x + row * width;
    R s = R(0);
    // eight loads in flight, added in the same order as one at a time
    int64_t c = lo + lane;
    for (; c + 7 * 64 < hi; c += 8 * 64) {
      T v[8];
#pragma unroll
      for (int u = 0; u < 8; u++) v[u] = p[c + u * 64];
#pragma unroll
      for (int u = 0; u < 8; u++) s += widen(v[u]);
    }
    for (; c < hi; c += 64) s += widen(p[c]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
    if (lane == 0) {
      if (parts == 1) out[row] = narrow<T>(s);
      else partial[item] = s;
    }
  }
}

// the partials of each row summed in part order
template <class T>
__global__ void __launch_bounds__(THREADS) row_partials_kernel(const typename Acc<T>::R* __restrict__ partial,
                                                               T* __restrict__ out, int64_t rows, int64_t parts) {
  typedef typename Acc<T>::R R;
  const int lane = threadIdx.x & 63;
  for (int64_t row = (int64_t)blockIdx.x * (THREADS / 64) + (threadIdx.x >> 6); row < rows;
       row += (int64_t)gridDim.x * (THREADS / 64)) {
    R s = R(0);
    for (int64_t q = lane; q < parts; q += 64) s += partial[row * parts + q];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
    if (lane == 0) out[row] = narrow<T>(s);
  }
}

// inner > 1: one lane per (o, part, j) column segment, consecutive lanes on
// consecutive j (coalesced); parts == 1 writes the rounded sum.
template <class T>
__global__ void __launch_bounds__(THREADS) col_sum_kernel(const T* __restrict__ x, T* __restrict__ out,
                                                          typename Acc<T>::R* __restrict__ partial, int64_t outer,
                                                          int64_t width, int64_t inner, int64_t parts, int64_t span) {
  typedef typename Acc<T>::R R;
  const int64_t total = outer * parts * inner;
  for (int64_t i = (int64_t)blockIdx.x * THREADS + threadIdx.x; i < total; i += (int64_t)gridDim.x * THREADS) {
    const int64_t j = i % inner, op = i / inner, part = op % parts, o = op / parts;
    const int64_t lo = part * span, hi = lo + span < width ? lo + span : width;
    const T* p = x + o * width * inner + j;
    R s = R(0);
    for (int64_t c = lo; c < hi; c++) s += widen(p[c * inner]);
    if (parts == 1) out[o * inner + j] = narrow<T>(s);
    else partial[i] = s;
  }
}

template <class T>
__global__ void __launch_bounds__(THREADS) col_partials_kernel(const typename Acc<T>::R* __restrict__ partial,
                                                               T* __restrict__ out, int64_t outer, int64_t inner,
                                                               int64_t parts) {
  typedef typename Acc<T>::R R;
  const int64_t total = outer * inner;
  for (int64_t i = (int64_t)blockIdx.x * THREADS + threadIdx.x; i < total; i += (int64_t)gridDim.x * THREADS) {
    const int64_t o = i / inner, j = i % inner;
    R s = R(0);
    for (int64_t q = 0; q < parts; q++) s += partial[(o * parts + q) * inner + j];
    out[i] = narrow<T>(s);
  }
}

// ---- gather / scatter by explicit positions -----------------------------------------
// out[i] = x[pos[i]] (element size ES)
template <int ES>
__global__ void gather_kernel(const char* __restrict__ x, const int64_t* __restrict__ pos, char* __restrict__ out,
                              int64_t n) {
  typedef typename Word<ES>::T W;
  for (int64_t i = (int64_t)blockIdx.x * THREADS + threadIdx.x; i < n; i += (int64_t)gridDim.x * THREADS)
    global_store(reinterpret_cast<W*>(out) + i, global_load<W>(reinterpret_cast<const W*>(x) + pos[i]));
}

// out[t] = sum over k in [start[t], start[t+1]) of x[order[k]], in order:
// the host groups the sources of every target position (CSR), so repeated
// positions add up deterministically and no atomics are needed.
template <class T>
__global__ void scatter_kernel(const T* __restrict__ x, const int64_t* __restrict__ start,
                               const int64_t* __restrict__ order, T* __restrict__ out, int64_t size) {
  typedef typename Acc<T>::R R;
  for (int64_t t = (int64_t)blockIdx.x * THREADS + threadIdx.x; t < size; t += (int64_t)gridDim.x * THREADS) {
    R s = R(0);
    for (int64_t k = start[t]; k < start[t + 1]; k++) s += widen(x[order[k]]);
    out[t] = narrow<T>(s);
  }
}

int element_size(int dtype) {
  switch (dtype) {
    case F32: return 4;
    case BF16: return 2;
    case F64:
    case I64: return 8;
    default: return 0;
  }
}

template <class F>
int by_float_dtype(int dtype, F f) {
  switch (dtype) {
    case F32: return f((float*)nullptr);
    case F64: return f((double*)nullptr);
    case BF16: return f((bf16_t*)nullptr);
    default: return QA_EINVAL;
  }
}

// Parts a reduction of `count` independent sums of `width` terms is split
// into, so that at least ~2048 waves (or lanes for the column form) run.
int64_t reduce_parts(int64_t count, int64_t width, int64_t target, int64_t min_span) {
  if (count >= target || width < 2 * min_span) return 1;
  int64_t parts = (target + count - 1) / count;
  const int64_t most = width / min_span;
  return parts < most ? parts : most;
}
void row_plan(int64_t rows, int64_t width, int64_t& parts, int64_t& span) {
  parts = reduce_parts(rows, width, 2048, 4096);
  span = (width + parts - 1) / parts;
  span = (span + 63) / 64 * 64;
  parts = span ? (width + span - 1) / span : 1;
  if (parts < 1) parts = 1;
}
void col_plan(int64_t columns, int64_t width, int64_t& parts, int64_t& span) {
  parts = reduce_parts(columns, width, 65536, 64);
  span = (width + parts - 1) / parts;
  parts = span ? (width + span - 1) / span : 1;
  if (parts < 1) parts = 1;
}

}  // namespace

extern "C" {

int qutai_amd_strided_copy(const void* src, void* dst, int rank, const int64_t* dims, const int64_t* src_strides,
                           const int64_t* dst_strides, int element_bytes, void* stream) {
  if (rank < 0 || rank > MAX_RANK || (rank && (!dims || !src_strides || !dst_strides)))
    return QA_EINVAL;
  if (element_bytes != 2 && element_bytes != 4 && element_bytes != 8) return QA_EINVAL;
  // drop unit axes, then merge neighbours that are contiguous on both sides
  Strided s{};
  int64_t total = 1;
  for (int d = 0; d < rank; d++) {
    if (dims[d] < 0) return QA_EINVAL;
    total *= dims[d];
  }
  if (total == 0) return QA_OK;
  if (!src || !dst) return QA_EINVAL;
  int r = 0;
  for (int d = 0; d < rank; d++) {
    if (dims[d] == 1) continue;
    if (r > 0 && s.src[r - 1] == src_strides[d] * dims[d] && s.dst[r - 1] == dst_strides[d] * dims[d]) {
      s.dims[r - 1] *= dims[d];
      s.src[r - 1] = src_strides[d];
      s.dst[r - 1] = dst_strides[d];
      continue;
    }
    s.dims[r] = dims[d];
    s.src[r] = src_strides[d];
    s.dst[r] = dst_strides[d];
    r++;
  }
  if (r == 0) {  // a single element
    s.dims[0] = 1;
    s.src[0] = s.dst[0] = 1;
    r = 1;
  }
  s.rank = r;
  const int V = 16 / element_bytes;
  bool vec = s.dst[r - 1] == 1 && (s.src[r - 1] == 1 || s.src[r - 1] == 0) && s.dims[r - 1] % V == 0 &&
             ((uintptr_t)src % 16 == 0 || s.src[r - 1] == 0) && (uintptr_t)dst % 16 == 0;
  for (int d = 0; d + 1 < r && vec; d++) vec = s.dst[d] % V == 0 && (s.src[d] % V == 0 || s.src[r - 1] == 0);
  if (s.src[r - 1] == 0 && (uintptr_t)src % element_bytes) vec = false;
  const int64_t runs = (s.dims[r - 1] + V - 1) / V;
  const int64_t items = total / s.dims[r - 1] * runs;
  hipStream_t st = (hipStream_t)stream;
  const char* a = (const char*)src;
  char* b = (char*)dst;
  const unsigned g = blocks_for(items);
  switch (element_bytes * 2 + (vec ? 1 : 0)) {
    case 4: strided_copy_kernel<2, false><<<g, THREADS, 0, st>>>(a, b, s, items); break;
    case 5: strided_copy_kernel<2, true><<<g, THREADS, 0, st>>>(a, b, s, items); break;
    case 8: strided_copy_kernel<4, false><<<g, THREADS, 0, st>>>(a, b, s, items); break;
    case 9: strided_copy_kernel<4, true><<<g, THREADS, 0, st>>>(a, b, s, items); break;
    case 16: strided_copy_kernel<8, false><<<g, THREADS, 0, st>>>(a, b, s, items); break;
    default: strided_copy_kernel<8, true><<<g, THREADS, 0, st>>>(a, b, s, items); break;
  }
  return (int)hipGetLastError();
}

int qutai_amd_binary(const void* left, const void* right, void* out, int64_t n, int op, int dtype, int* zero_flag,
                     void* stream) {
  if (n < 0 || op < OP_ADD || op > OP_DIV) return QA_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  if (zero_flag) set_flag_kernel<<<1, 1, 0, st>>>(zero_flag);
  if (n == 0) return (int)hipGetLastError();
  if (!left || !right || !out) return QA_EINVAL;
  const bool aligned = ((uintptr_t)left | (uintptr_t)right | (uintptr_t)out) % 16 == 0;
  return by_float_dtype(dtype, [&](auto* tag) {
    typedef std::remove_pointer_t<decltype(tag)> T;
    const int64_t chunks = aligned ? n / Lanes<T>::V : 0;  // 16-byte lanes, then the scalar tail
    binary_kernel<T><<<blocks_for(aligned ? n : n * Lanes<T>::V, (int64_t)THREADS * Lanes<T>::V), THREADS, 0, st>>>(
        (const T*)left, (const T*)right, (T*)out, n, chunks, op, zero_flag);
    return (int)hipGetLastError();
  });
}

int qutai_amd_unary(const void* x, const void* gradient, void* out, int64_t n, int op, double factor, int dtype,
                    int* flag, void* stream) {
  if (n < 0 || op < U_NEGATE || op > U_DIVIDE) return QA_EINVAL;
  const bool needs_g = op == U_RELU_BACKWARD || op == U_GELU_BACKWARD || op == U_TANH_BACKWARD ||
                       op == U_ATAN_BACKWARD;
  if (needs_g != (gradient != nullptr)) return QA_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  if (flag) set_flag_kernel<<<1, 1, 0, st>>>(flag);
  if (n == 0) return (int)hipGetLastError();
  if (!x || !out) return QA_EINVAL;
  const bool aligned = ((uintptr_t)x | (uintptr_t)gradient | (uintptr_t)out) % 16 == 0;
  return by_float_dtype(dtype, [&](auto* tag) {
    typedef std::remove_pointer_t<decltype(tag)> T;
    typedef typename Acc<T>::R R;
    const int64_t chunks = aligned ? n / Lanes<T>::V : 0;
    unary_kernel<T><<<blocks_for(aligned ? n : n * Lanes<T>::V, (int64_t)THREADS * Lanes<T>::V), THREADS, 0, st>>>(
        (const T*)x, (const T*)gradient, (T*)out, n, chunks, op, (R)factor, flag);
    return (int)hipGetLastError();
  });
}

size_t qutai_amd_reduce_sum_workspace_size(int64_t outer, int64_t width, int64_t inner, int dtype) {
  if (outer < 0 || width < 0 || inner < 1) return 0;
  const size_t acc = dtype == F64 ? 8 : 4;
  int64_t parts, span;
  if (inner == 1) row_plan(outer, width, parts, span);
  else col_plan(outer * inner, width, parts, span);
  return parts > 1 ? (size_t)(outer * inner * parts) * acc : 0;
}

int qutai_amd_reduce_sum(const void* x, void* out, int64_t outer, int64_t width, int64_t inner, int dtype,
                         void* workspace, size_t workspace_bytes, void* stream) {
  if (outer < 0 || width < 0 || inner < 1) return QA_EINVAL;
  if (dtype != F32 && dtype != F64 && dtype != BF16) return QA_EINVAL;
  if (outer == 0) return QA_OK;
  if (!out || (width && !x)) return QA_EINVAL;
  const size_t need = qutai_amd_reduce_sum_workspace_size(outer, width, inner, dtype);
  if (need && (!workspace || workspace_bytes < need)) return QA_EWORKSPACE;
  hipStream_t st = (hipStream_t)stream;
  return by_float_dtype(dtype, [&](auto* tag) {
    typedef std::remove_pointer_t<decltype(tag)> T;
    typedef typename Acc<T>::R R;
    R* partial = (R*)workspace;
    int64_t parts, span;
    if (inner == 1) {
      row_plan(outer, width, parts, span);
      row_sum_kernel<T><<<blocks_for(outer * parts, THREADS / 64), THREADS, 0, st>>>((const T*)x, (T*)out, partial,
                                                                                     outer, width, parts, span);
      if (parts > 1)
        row_partials_kernel<T><<<blocks_for(outer, THREADS / 64), THREADS, 0, st>>>(partial, (T*)out, outer, parts);
    } else {
      col_plan(outer * inner, width, parts, span);
      col_sum_kernel<T><<<blocks_for(outer * parts * inner), THREADS, 0, st>>>((const T*)x, (T*)out, partial, outer,
                                                                               width, inner, parts, span);
      if (parts > 1)
        col_partials_kernel<T><<<blocks_for(outer * inner), THREADS, 0, st>>>(partial, (T*)out, outer, inner, parts);
    }
    return (int)hipGetLastError();
  });
}

int qutai_amd_gather(const void* x, const int64_t* positions, void* out, int64_t n, int element_bytes, void* stream) {
  if (n < 0 || (element_bytes != 2 && element_bytes != 4 && element_bytes != 8)) return QA_EINVAL;
  if (n == 0) return QA_OK;
  if (!x || !positions || !out) return QA_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  const char* a = (const char*)x;
  char* b = (char*)out;
  if (element_bytes == 2) gather_kernel<2><<<blocks_for(n), THREADS, 0, st>>>(a, positions, b, n);
  else if (element_bytes == 4) gather_kernel<4><<<blocks_for(n), THREADS, 0, st>>>(a, positions, b, n);
  else gather_kernel<8><<<blocks_for(n), THREADS, 0, st>>>(a, positions, b, n);
  return (int)hipGetLastError();
}

int qutai_amd_scatter(const void* x, const int64_t* start, const int64_t* order, void* out, int64_t size, int dtype,
                      void* stream) {
  if (size < 0) return QA_EINVAL;
  if (size == 0) return QA_OK;
  if (!start || !out) return QA_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  return by_float_dtype(dtype, [&](auto* tag) {
    typedef std::remove_pointer_t<decltype(tag)> T;
    scatter_kernel<T><<<blocks_for(size), THREADS, 0, st>>>((const T*)x, start, order, (T*)out, size);
    return (int)hipGetLastError();
  });
}

}  // extern "C"
