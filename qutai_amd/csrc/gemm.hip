// GEMM entry points of libqutai_amd (C ABI).  The argument meaning, the
// dtype rules and the validation follow the reference GEMM boundary
// `cuda.gemm` (src/qutai/backends/cuda.py:305-362) and its kernel signature
// (src/qutai/backends/cuda/gemm.cu:35, `(a, b, out, M, K, N, sa, sb, ta, tb,
// accumulate)`); kernel choice is MI355X-specific.
#include "gemm_kernel.h"
#include "qutai_amd.h"

using namespace qa;

namespace {

template <class Kern>
__global__ void __launch_bounds__(Kern::NT) gemm_entry(GemmArgs p) {
  __shared__ __attribute__((aligned(16))) char smem[Kern::LDS_BYTES];
  Kern::run(p, smem);
}

// fp64 GEMM: plain 32x32 SIMT tiles, 2x2 outputs per thread (not an MFMA
// target; kept for the float64 storage contract of the boundary).
__global__ void __launch_bounds__(256) gemm_f64(const double* a, const double* b, double* out, int64_t M,
                                                int64_t K, int64_t N, int64_t sa, int64_t sb, int ta, int tb,
                                                int accumulate, int64_t tiles_n, int64_t tiles_m) {
  __shared__ double As[32][33], Bs[32][33];
  int x = threadIdx.x & 15, y = threadIdx.x >> 4;
  int64_t id = blockIdx.x;
  int64_t z = id / (tiles_m * tiles_n), t = id % (tiles_m * tiles_n);
  int64_t tm = t / tiles_n, tn = t % tiles_n;
  a += z * sa;
  b += z * sb;
  out += z * M * N;
  double c[2][2] = {{0, 0}, {0, 0}};
  for (int64_t k0 = 0; k0 < K; k0 += 32) {
    for (int dy = 0; dy < 2; dy++)
      for (int dx = 0; dx < 2; dx++) {
        int64_t r = tm * 32 + y + dy * 16, k = k0 + x + dx * 16;
        As[y + dy * 16][x + dx * 16] = (r < M && k < K) ? a[ta ? k * M + r : r * K + k] : 0.0;
        int64_t kk = k0 + y + dy * 16, cc = tn * 32 + x + dx * 16;
        Bs[y + dy * 16][x + dx * 16] = (kk < K && cc < N) ? b[tb ? cc * K + kk : kk * N + cc] : 0.0;
      }
    __syncthreads();
    for (int k = 0; k < 32; k++) {
      double a0 = As[y][k], a1 = As[y + 16][k], b0 = Bs[k][x], b1 = Bs[k][x + 16];
      c[0][0] = __dadd_rn(c[0][0], __dmul_rn(a0, b0));
      c[0][1] = __dadd_rn(c[0][1], __dmul_rn(a0, b1));
      c[1][0] = __dadd_rn(c[1][0], __dmul_rn(a1, b0));
      c[1][1] = __dadd_rn(c[1][1], __dmul_rn(a1, b1));
    }
    __syncthreads();
  }
  for (int dy = 0; dy < 2; dy++)
    for (int dx = 0; dx < 2; dx++) {
      int64_t r = tm * 32 + y + dy * 16, cc = tn * 32 + x + dx * 16;
      if (r < M && cc < N) {
        double v = c[dy][dx];
        if (accumulate) v += out[r * N + cc];
        out[r * N + cc] = v;
      }
    }
}

// Narrow fp32 -> bf16 (round to nearest even) into a workspace.
__global__ void narrow_f32_bf16(const float* x, bf16_t* y, int64_t n) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) y[i] = f32_to_bf16(x[i]);
}

enum Tile { TILE_L, TILE_N, TILE_W, TILE_S };

template <bool F32, bool TA, bool TB, int BM, int BN, int WM, int WN>
hipError_t launch_cfg(GemmArgs p, hipStream_t stream) {
  typedef GemmKernel<F32, TA, TB, BM, BN, WM, WN> Kern;
  int64_t tiles_n = (p.N + BN - 1) / BN;
  if (p.groups == 0) p.tiles_m = (int)((p.M + BM - 1) / BM);
  int64_t blocks = (int64_t)p.tiles_m * tiles_n * (p.groups ? 1 : p.batch);
  if (blocks <= 0) return hipSuccess;
  if (blocks > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL(gemm_entry<Kern>, dim3((unsigned)blocks), dim3(Kern::NT), 0, stream, p);
  return hipGetLastError();
}

template <bool F32, bool TA, bool TB>
hipError_t launch_tile(Tile tile, GemmArgs p, hipStream_t stream) {
  switch (tile) {
    case TILE_N: return launch_cfg<F32, TA, TB, 256, 64, 4, 1>(p, stream);
    case TILE_W: return launch_cfg<F32, TA, TB, 64, 256, 1, 4>(p, stream);
    case TILE_S: return launch_cfg<F32, TA, TB, 128, 128, 2, 2>(p, stream);
    default: return launch_cfg<F32, TA, TB, 256, 256, 2, 2>(p, stream);
  }
}

template <bool F32>
hipError_t launch_mma(Tile tile, bool ta, bool tb, const GemmArgs& p, hipStream_t stream) {
  if (ta) return tb ? launch_tile<F32, true, true>(tile, p, stream) : launch_tile<F32, true, false>(tile, p, stream);
  return tb ? launch_tile<F32, false, true>(tile, p, stream) : launch_tile<F32, false, false>(tile, p, stream);
}

// Tile choice: 256x256 when it still gives about one tile per CU, else the
// 128x128 tile; thin outputs use the 256x64 / 64x256 shapes.
Tile choose_tile(int64_t M, int64_t N, int64_t batch) {
  if (N <= 64) return TILE_N;
  if (M <= 64) return TILE_W;
  int64_t big = ((M + 255) / 256) * ((N + 255) / 256) * batch;
  if (big < 192) return TILE_S;
  return TILE_L;
}

bool aligned16(const void* p, int64_t ld, int64_t esize, int64_t stride) {
  return ((uintptr_t)p % 16 == 0) && ((ld * esize) % 16 == 0) && ((stride * esize) % 16 == 0);
}

// 4-wide output stores need 4 | ldc, 4 | batch stride and an aligned base.
bool vec_out(const void* p, int64_t ldc, int64_t stride) {
  return ((uintptr_t)p % 16 == 0) && (ldc % 4 == 0) && (stride % 4 == 0);
}

int esize_of(int dtype) { return dtype == QA_BF16 ? 2 : dtype == QA_F64 ? 8 : 4; }

}  // namespace

extern "C" {

size_t qutai_amd_gemm_workspace_size(int64_t rows, int64_t inner, int64_t cols, int64_t batch,
                                     int64_t left_stride, int64_t right_stride, int a_dtype, int b_dtype,
                                     int bf16_compute) {
  if (a_dtype == QA_F64 || b_dtype == QA_F64) return 0;
  bool mixed = bf16_compute || a_dtype == QA_BF16 || b_dtype == QA_BF16;
  if (!mixed) return 0;
  size_t bytes = 0;
  if (a_dtype == QA_F32) bytes += (size_t)((batch - 1) * left_stride + rows * inner) * 2 + 256;
  if (b_dtype == QA_F32) bytes += (size_t)((batch - 1) * right_stride + inner * cols) * 2 + 256;
  return batch > 0 ? bytes : 0;
}

int qutai_amd_gemm(const void* a, const void* b, void* out, int64_t rows, int64_t inner, int64_t cols,
                   int64_t batch, int64_t left_stride, int64_t right_stride, int transpose_left,
                   int transpose_right, int a_dtype, int b_dtype, int out_dtype, int accumulate,
                   int bf16_compute, void* workspace, size_t workspace_bytes, void* stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  if (rows < 0 || inner < 0 || cols < 0 || batch < 0 || left_stride < 0 || right_stride < 0) return QA_EINVAL;
  bool f64 = a_dtype == QA_F64 || b_dtype == QA_F64;
  for (int d : {a_dtype, b_dtype})
    if (d != QA_F32 && d != QA_BF16 && d != QA_F64) return QA_EINVAL;
  if (f64 && (a_dtype != b_dtype || out_dtype != QA_F64)) return QA_EINVAL;
  if (!f64 && out_dtype != QA_F32 && out_dtype != QA_BF16) return QA_EINVAL;
  int64_t size = batch * rows * cols;
  if (size == 0) return QA_OK;
  if (!out) return QA_EINVAL;
  if (inner > 0 && (!a || !b)) return QA_EINVAL;
  if (f64) {
    int64_t tiles_m = (rows + 31) / 32, tiles_n = (cols + 31) / 32;
    int64_t blocks = tiles_m * tiles_n * batch;
    if (blocks > 0x7fffffff) return QA_EINVAL;
    hipLaunchKernelGGL(gemm_f64, dim3((unsigned)blocks), dim3(256), 0, stream, (const double*)a, (const double*)b,
                       (double*)out, rows, inner, cols, left_stride, right_stride, transpose_left, transpose_right,
                       accumulate, tiles_n, tiles_m);
    return (int)hipGetLastError();
  }
  bool mixed = bf16_compute || a_dtype == QA_BF16 || b_dtype == QA_BF16;
  const void* A = a;
  const void* B = b;
  if (mixed) {
    size_t need = qutai_amd_gemm_workspace_size(rows, inner, cols, batch, left_stride, right_stride, a_dtype,
                                                b_dtype, bf16_compute);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need)) return QA_EWORKSPACE;
    char* ws = (char*)(((uintptr_t)workspace + 255) & ~(uintptr_t)255);
    if (a_dtype == QA_F32 && inner > 0) {
      int64_t n = (batch - 1) * left_stride + rows * inner;
      hipLaunchKernelGGL(narrow_f32_bf16, dim3((unsigned)std::min<int64_t>((n + 255) / 256, 65536)), dim3(256), 0,
                         stream, (const float*)a, (bf16_t*)ws, n);
      A = ws;
      ws += ((n * 2 + 255) / 256) * 256;
    }
    if (b_dtype == QA_F32 && inner > 0) {
      int64_t n = (batch - 1) * right_stride + inner * cols;
      hipLaunchKernelGGL(narrow_f32_bf16, dim3((unsigned)std::min<int64_t>((n + 255) / 256, 65536)), dim3(256), 0,
                         stream, (const float*)b, (bf16_t*)ws, n);
      B = ws;
    }
  }
  GemmArgs p = {};
  p.a = A;
  p.b = B;
  p.out = out;
  p.M = rows;
  p.N = cols;
  p.K = inner;
  p.lda = transpose_left ? rows : inner;
  p.ldb = transpose_right ? inner : cols;
  p.ldc = cols;
  p.sa = left_stride;
  p.sb = right_stride;
  p.sc = rows * cols;
  p.batch = batch;
  p.accumulate = accumulate ? 1 : 0;
  p.out_bf16 = out_dtype == QA_BF16;
  int es = mixed ? 2 : 4;
  p.vec_a = aligned16(A, p.lda, es, left_stride);
  p.vec_b = aligned16(B, p.ldb, es, right_stride);
  p.vec_c = vec_out(out, p.ldc, p.sc);
  p.alpha = 1.0f;
  Tile tile = choose_tile(rows, cols, batch);
  hipError_t err = mixed ? launch_mma<false>(tile, transpose_left, transpose_right, p, stream)
                         : launch_mma<true>(tile, transpose_left, transpose_right, p, stream);
  return (int)err;
}

int qutai_amd_gemm_grouped(const void* a, const void* b, void* out, const int64_t* offsets, int groups,
                           int64_t max_rows, int64_t inner, int64_t cols, int64_t expert_stride,
                           int transpose_right, int dtype, int out_dtype, int accumulate, void* stream_) {
  hipStream_t stream = (hipStream_t)stream_;
  if (groups <= 0 || max_rows < 0 || inner < 0 || cols < 0 || expert_stride < 0) return QA_EINVAL;
  if (dtype != QA_BF16 && dtype != QA_F32) return QA_EINVAL;
  if (out_dtype != QA_F32 && out_dtype != QA_BF16) return QA_EINVAL;
  if (!offsets || !out) return QA_EINVAL;
  if (max_rows == 0 || cols == 0) return QA_OK;
  GemmArgs p = {};
  p.a = a;
  p.b = b;
  p.out = out;
  p.M = max_rows;
  p.N = cols;
  p.K = inner;
  p.lda = inner;
  p.ldb = transpose_right ? inner : cols;
  p.ldc = cols;
  p.sb = expert_stride;
  p.batch = 1;
  p.accumulate = accumulate ? 1 : 0;
  p.out_bf16 = out_dtype == QA_BF16;
  int es = esize_of(dtype);
  p.vec_a = aligned16(a, p.lda, es, 0);
  p.vec_b = aligned16(b, p.ldb, es, expert_stride);
  p.vec_c = vec_out(out, p.ldc, 0);
  p.offsets = offsets;
  p.groups = groups;
  p.alpha = 1.0f;
  // Upper bound of M tiles over all groups: sum ceil(n_g / BM) <= ceil(max_rows / BM) + groups.
  Tile tile = cols <= 64 ? TILE_N : TILE_L;
  int bm = tile == TILE_N ? 256 : 256;
  p.tiles_m = (int)((max_rows + bm - 1) / bm + groups);
  bool f32 = dtype == QA_F32;
  hipError_t err = f32 ? launch_mma<true>(tile, false, transpose_right, p, stream)
                       : launch_mma<false>(tile, false, transpose_right, p, stream);
  return (int)err;
}

}  // extern "C"
