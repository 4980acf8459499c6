// MFMA GEMM core for gfx950.
//
// C[b][m][n] (+)= sum_k A(b,m,k) * B(b,k,n) with the operand index maps of
// the reference kernels (src/qutai/backends/cuda/gemm.cu:44-46):
//   A(m,k) = ta ? a[k*M + m] : a[m*K + k]      B(k,n) = tb ? b[n*K + k] : b[k*N + n]
// fp32 accumulation, one rounding to the output type in the epilogue, and
// the `accumulate` epilogue that adds the old output before that rounding
// (gemm.cu:25-32).
//
// Design (CDNA4):
//  * one workgroup computes a BM x BN output tile with WM x WN wavefronts;
//    every wave owns a (BM/WM) x (BN/WN) sub-tile of 32x32 MFMA blocks whose
//    fp32 accumulators stay in registers for the whole K loop;
//  * bf16 operands feed v_mfma_f32_32x32x16_bf16, fp32 operands feed
//    v_mfma_f32_32x32x2_f32 (true fp32 products, fp32 accumulation);
//  * A and B tiles are staged HBM -> registers -> LDS with 16-byte loads,
//    double-buffered in LDS so the loads of step k+1 are in flight while the
//    MFMAs of step k run; one barrier per K step;
//  * an operand whose K index is contiguous in HBM ("K-major") sits in LDS
//    as [row][k] and is read with ds_read_b128; an operand whose M/N index is
//    contiguous ("MN-major", e.g. B of a plain row-major A@B) keeps its HBM
//    layout [k][row] in LDS and is read with the gfx950 transpose read
//    ds_read_b64_tr_b16, so no transpose pass or register shuffle is needed;
//  * LDS rows are XOR-swizzled in 16-byte chunks so the fragment reads and the
//    staging writes are free of bank conflicts;
//  * workgroup ids are remapped so that each XCD (own L2) works on one
//    compact block of output tiles.
#pragma once
#include "common.h"

namespace qa {

struct GemmArgs {
  const void* a;
  const void* b;
  void* out;
  int64_t M, N, K;
  int64_t lda, ldb, ldc;  // leading dimensions in elements
  int64_t sa, sb, sc;     // batch strides in elements (0 = broadcast)
  int64_t batch;
  int accumulate;         // out = old + A@B
  int out_bf16;           // output element type: bf16 (1) or fp32 (0)
  int vec_a, vec_b;       // operand rows are 16-byte aligned
  int vec_c;              // output rows allow 16-byte (fp32) / 8-byte (bf16) stores
  // Grouped mode (groups > 0): group g owns rows [offsets[g], offsets[g+1])
  // of A (K-major, lda) and of out (ldc); its B operand is b + g*sb.
  const int64_t* offsets;
  int groups;
  int tiles_m;            // M tiles in the grid (grouped: an upper bound)
  float alpha;            // scale applied to A@B before the epilogue
};

template <bool F32> struct MmaTraits;
template <> struct MmaTraits<false> {  // bf16 in, fp32 accumulate
  typedef bf16_t T;
  static constexpr int E = 8;    // elements per 16-byte chunk
  static constexpr int BK = 64;  // K per LDS stage (8 chunks per K-major row)
};
template <> struct MmaTraits<true> {   // fp32 in, fp32 accumulate
  typedef float T;
  static constexpr int E = 4;
  static constexpr int BK = 32;
};

// ---- LDS swizzles ---------------------------------------------------------
// K-major tile [R][BK], 8 chunks of 16 B per row.  Fragment reads take 32
// consecutive rows at one chunk; (r ^ r>>3) & 7 makes any 8 consecutive rows,
// and any 8 rows of equal parity among 16 consecutive rows, hit different
// chunks, so 8 or 16 lanes serviced together touch distinct banks.
__device__ __forceinline__ int swz_k(int r) { return (r ^ (r >> 3)) & 7; }

// MN-major tile [BK][R] of bf16 read by ds_read_b64_tr_b16: 32 lanes read 4
// consecutive k-rows x 64 bytes; shifting each of the 4 rows into its own
// 64-byte quarter of a 256-byte bank window removes the 4-way conflict.
template <int CR> __device__ __forceinline__ int swz_mn16(int k) {
  return CR >= 16 ? (k & 3) * 4 : ((k >> 1) & 1) * 4;
}
// MN-major tile of fp32 read with ds_read_b32: the two lane halves read
// k-rows 8 apart; put them in different 128-byte bank halves.
__device__ __forceinline__ int swz_mn32(int k) { return ((k >> 3) & 1) * 8; }

template <bool F32, bool KMAJOR, int R>
struct OperandTile {
  typedef MmaTraits<F32> Tr;
  typedef typename Tr::T T;
  static constexpr int E = Tr::E, BK = Tr::BK;
  static constexpr int CHUNKS = R * BK / E;          // 16-byte chunks per stage
  static constexpr int CR = R / E;                   // chunks per MN-major row
  static constexpr int ELEMS = R * BK;

  // element offset of chunk (row, c) inside one stage
  __device__ static __forceinline__ int chunk_offset(int idx) {
    if (KMAJOR) {
      int r = idx >> 3, c = idx & 7;
      return r * BK + ((c ^ swz_k(r)) * E);
    } else {
      int k = idx / CR, c = idx % CR;
      int s = F32 ? swz_mn32(k) : swz_mn16<CR>(k);
      return k * R + ((c ^ s) * E);
    }
  }
};

template <bool F32, bool TA, bool TB, int BM, int BN, int WM, int WN>
struct GemmKernel {
  typedef MmaTraits<F32> Tr;
  typedef typename Tr::T T;
  static constexpr int E = Tr::E, BK = Tr::BK;
  static constexpr int NT = 64 * WM * WN;
  static constexpr int TM = BM / WM, TN = BN / WN;  // wave tile
  static constexpr int FM = TM / 32, FN = TN / 32;  // 32x32 blocks per wave
  static constexpr bool KA = !TA;                   // A K-major?
  static constexpr bool KB = TB;                    // B K-major?
  typedef OperandTile<F32, KA, BM> TileA;
  typedef OperandTile<F32, KB, BN> TileB;
  static constexpr int LA = TileA::CHUNKS / NT;     // chunks per thread
  static constexpr int LB = TileB::CHUNKS / NT;
  static constexpr int STAGE = (BM + BN) * BK;      // elements per stage
  static constexpr int LDS_BYTES = 2 * STAGE * (int)sizeof(T);
  static_assert(TileA::CHUNKS % NT == 0 && TileB::CHUNKS % NT == 0, "staging split");
  static_assert(TM % 32 == 0 && TN % 32 == 0, "wave tile");
  static_assert(LDS_BYTES <= 160 * 1024, "LDS");

  // One 16-byte chunk of an operand from HBM: E elements along the
  // contiguous axis starting at (outer, inner); zero outside [0,rows)x[0,cols).
  __device__ static __forceinline__ u32x4 load_chunk(const T* base, int64_t ld, int64_t outer,
                                                      int64_t inner, int64_t outer_n, int64_t inner_n,
                                                      bool vec) {
    if (vec && outer < outer_n && inner + E <= inner_n) {
      return *reinterpret_cast<const u32x4*>(base + outer * ld + inner);
    }
    T v[E];
#pragma unroll
    for (int j = 0; j < E; j++) {
      bool ok = outer < outer_n && inner + j < inner_n;
      v[j] = ok ? base[outer * ld + inner + j] : (T)0;
    }
    u32x4 r;
    __builtin_memcpy(&r, v, 16);
    return r;
  }

  // Fragment reads -----------------------------------------------------------
  // bf16, K-major: lane l takes row (l & 31), k = 16 s + 8 (l >> 5) + [0, 8).
  __device__ static __forceinline__ bf16x8 frag_k16(const T* t, int row, int s, int lane) {
    int r = row + (lane & 31);
    int c = 2 * s + (lane >> 5);
    const T* p = t + r * BK + ((c ^ swz_k(r)) * E);
    return *reinterpret_cast<const bf16x8*>(p);
  }
  // bf16, MN-major [BK][R]: two transpose reads of 4 k-values each.  Within a
  // 16-lane group, source lane i reads k-row kb + i/4, columns cb + 4 (i&3);
  // the hardware returns to lane i the 4 values of column cb + i.
  template <int R>
  __device__ static __forceinline__ bf16x8 frag_mn16(const T* t, int col0, int s, int lane) {
    constexpr int CR = R / 8;
    int g = lane >> 4, i = lane & 15;
    int cb = col0 + (g & 1) * 16 + 4 * (i & 3);
    int c = cb >> 3, w = cb & 7;
    int k0 = 16 * s + (g >> 1) * 8 + (i >> 2);
    int k1 = k0 + 4;
    const T* p0 = t + k0 * R + ((c ^ swz_mn16<CR>(k0)) * 8) + w;
    const T* p1 = t + k1 * R + ((c ^ swz_mn16<CR>(k1)) * 8) + w;
    typedef i16x4 __attribute__((address_space(3))) * lds_ptr;
    i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_ptr)(p0));
    i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_ptr)(p1));
    i16x8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return __builtin_bit_cast(bf16x8, v);
  }
  // fp32, K-major: lane takes row (l & 31), k = 16 s + 8 (l >> 5) + [0, 8).
  __device__ static __forceinline__ void frag_k32(const T* t, int row, int s, int lane, float (&v)[8]) {
    int r = row + (lane & 31);
    int c0 = 4 * s + 2 * (lane >> 5);
    f32x4 x = *reinterpret_cast<const f32x4*>(t + r * BK + ((c0 ^ swz_k(r)) * E));
    f32x4 y = *reinterpret_cast<const f32x4*>(t + r * BK + (((c0 + 1) ^ swz_k(r)) * E));
    v[0] = x[0]; v[1] = x[1]; v[2] = x[2]; v[3] = x[3];
    v[4] = y[0]; v[5] = y[1]; v[6] = y[2]; v[7] = y[3];
  }
  // fp32, MN-major [BK][R]: same k assignment, one ds_read_b32 per value.
  template <int R>
  __device__ static __forceinline__ void frag_mn32(const T* t, int col0, int s, int lane, float (&v)[8]) {
    int col = col0 + (lane & 31);
    int c = col >> 2, w = col & 3;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      int k = 16 * s + 8 * (lane >> 5) + j;
      v[j] = t[k * R + ((c ^ swz_mn32(k)) * 4) + w];
    }
  }

  __device__ static __forceinline__ void run(const GemmArgs& p, char* smem) {
    T* lds = reinterpret_cast<T*>(smem);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;

    // ---- tile scheduling -------------------------------------------------
    const int tiles_n = (int)((p.N + BN - 1) / BN);
    const int tiles_per = p.tiles_m * tiles_n;
    const int total = (int)gridDim.x;
    int pid = xcd_remap((int)blockIdx.x, total);
    int64_t bz = pid / tiles_per;
    int t = pid % tiles_per;
    // grouped ordering: 4 M-tiles per group, N fastest inside a group
    constexpr int GM = 4;
    int group = t / (GM * tiles_n);
    int first_m = group * GM;
    int gsize = min(p.tiles_m - first_m, GM);
    int tile_m = first_m + (t % (GM * tiles_n)) % gsize;
    int tile_n = (t % (GM * tiles_n)) / gsize;

    const T* A = reinterpret_cast<const T*>(p.a);
    const T* B = reinterpret_cast<const T*>(p.b);
    int64_t M = p.M, row0 = 0;
    char* outp = reinterpret_cast<char*>(p.out);
    const int osize = p.out_bf16 ? 2 : 4;
    if (p.groups > 0) {
      // locate the group that owns M-tile `tile_m`
      int64_t before = 0;
      int g = -1;
      int64_t lo = 0, hi = 0;
      for (int e = 0; e < p.groups; e++) {
        int64_t s0 = p.offsets[e], s1 = p.offsets[e + 1];
        int64_t nt = (s1 - s0 + BM - 1) / BM;
        if (g < 0 && tile_m < before + nt) { g = e; lo = s0; hi = s1; row0 = (tile_m - before) * BM; }
        before += nt;
      }
      if (g < 0) return;  // tile beyond the last group: nothing to do
      A += lo * p.lda;
      B += (int64_t)g * p.sb;
      outp += lo * p.ldc * osize;
      M = hi - lo;
    } else {
      A += bz * p.sa;
      B += bz * p.sb;
      outp += bz * p.sc * osize;
      row0 = (int64_t)tile_m * BM;
    }
    const int64_t col0 = (int64_t)tile_n * BN;
    const int64_t K = p.K, N = p.N;
    const bool vec_a = p.vec_a, vec_b = p.vec_b;

    // ---- staging -----------------------------------------------------------
    u32x4 ra[LA], rb[LB];
    auto load = [&](int64_t k0) {
#pragma unroll
      for (int i = 0; i < LA; i++) {
        int idx = tid + i * NT;
        if (KA) {  // rows of A, K contiguous
          int r = idx >> 3, c = idx & 7;
          ra[i] = load_chunk(A, p.lda, row0 + r, k0 + c * E, M, K, vec_a);
        } else {   // A^T stored [K][M]
          int k = idx / TileA::CR, c = idx % TileA::CR;
          ra[i] = load_chunk(A, p.lda, k0 + k, row0 + c * E, K, M, vec_a);
        }
      }
#pragma unroll
      for (int i = 0; i < LB; i++) {
        int idx = tid + i * NT;
        if (KB) {  // B^T stored [N][K]
          int r = idx >> 3, c = idx & 7;
          rb[i] = load_chunk(B, p.ldb, col0 + r, k0 + c * E, N, K, vec_b);
        } else {   // B stored [K][N]
          int k = idx / TileB::CR, c = idx % TileB::CR;
          rb[i] = load_chunk(B, p.ldb, k0 + k, col0 + c * E, K, N, vec_b);
        }
      }
    };
    auto store = [&](int stage) {
      T* sa = lds + stage * STAGE;
      T* sb = sa + BM * BK;
#pragma unroll
      for (int i = 0; i < LA; i++)
        *reinterpret_cast<u32x4*>(sa + TileA::chunk_offset(tid + i * NT)) = ra[i];
#pragma unroll
      for (int i = 0; i < LB; i++)
        *reinterpret_cast<u32x4*>(sb + TileB::chunk_offset(tid + i * NT)) = rb[i];
    };

    f32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
      for (int j = 0; j < FN; j++)
#pragma unroll
        for (int e = 0; e < 16; e++) acc[i][j][e] = 0.f;

    const int nk = (int)((K + BK - 1) / BK);
    if (nk > 0) {
      load(0);
      store(0);
      __syncthreads();
    }
    for (int kt = 0; kt < nk; kt++) {
      const int cur = kt & 1;
      if (kt + 1 < nk) load((int64_t)(kt + 1) * BK);
      const T* sa = lds + cur * STAGE;
      const T* sb = sa + BM * BK;
#pragma unroll
      for (int s = 0; s < BK / 16; s++) {
        if constexpr (!F32) {
          bf16x8 fa[FM], fb[FN];
#pragma unroll
          for (int i = 0; i < FM; i++)
            fa[i] = KA ? frag_k16(sa, wm * TM + i * 32, s, lane)
                       : frag_mn16<BM>(sa, wm * TM + i * 32, s, lane);
#pragma unroll
          for (int j = 0; j < FN; j++)
            fb[j] = KB ? frag_k16(sb, wn * TN + j * 32, s, lane)
                       : frag_mn16<BN>(sb, wn * TN + j * 32, s, lane);
#pragma unroll
          for (int i = 0; i < FM; i++)
#pragma unroll
            for (int j = 0; j < FN; j++)
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
        } else {
          float fa[FM][8], fb[FN][8];
#pragma unroll
          for (int i = 0; i < FM; i++) {
            if (KA) frag_k32(sa, wm * TM + i * 32, s, lane, fa[i]);
            else frag_mn32<BM>(sa, wm * TM + i * 32, s, lane, fa[i]);
          }
#pragma unroll
          for (int j = 0; j < FN; j++) {
            if (KB) frag_k32(sb, wn * TN + j * 32, s, lane, fb[j]);
            else frag_mn32<BN>(sb, wn * TN + j * 32, s, lane, fb[j]);
          }
#pragma unroll
          for (int q = 0; q < 8; q++)
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
              for (int j = 0; j < FN; j++)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i][q], fb[j][q], acc[i][j], 0, 0, 0);
        }
      }
      if (kt + 1 < nk) store(cur ^ 1);
      __syncthreads();
    }

    // ---- epilogue ---------------------------------------------------------
    Out o;
    o.ptr = outp;
    o.ldc = p.ldc;
    o.M = M;
    o.N = N;
    o.row0 = row0 + wm * TM;
    o.col0 = col0 + wn * TN;
    o.bf16 = p.out_bf16;
    o.accumulate = p.accumulate;
    o.vec = p.vec_c;
    o.alpha = p.alpha;
    float* stage = reinterpret_cast<float*>(smem) + wave * 32 * EP;
    store_rows<0>(acc, stage, o, lane);
  }

  // Output staging: each wave turns one 32-row slab of its accumulators
  // (MFMA C layout: lane l holds column l & 31 and rows
  // 8 (e/4) + 4 (l >> 5) + (e & 3) of a 32x32 block) into row-major order in
  // LDS, then writes it with 16-byte (fp32) or 8-byte (bf16) stores along
  // rows.  The row pitch EP = TN + 8 floats puts the two lane halves, which
  // write rows 4 apart, into different bank halves.
  static constexpr int EP = TN + 8;
  static_assert(WM * WN * 32 * EP * 4 <= LDS_BYTES, "epilogue staging");

  struct Out {
    char* ptr;
    int64_t ldc, M, N, row0, col0;
    int bf16, accumulate, vec;
    float alpha;
  };

  __device__ static __forceinline__ void write4(const Out& o, int64_t row, int64_t col, f32x4 v) {
    v *= o.alpha;
    int64_t at = row * o.ldc + col;
    if (o.bf16) {
      bf16_t* q = reinterpret_cast<bf16_t*>(o.ptr) + at;
      if (o.vec && col + 4 <= o.N) {
        if (o.accumulate) {
          uint2 old = *reinterpret_cast<const uint2*>(q);
          v[0] += __uint_as_float(old.x << 16);
          v[1] += __uint_as_float(old.x & 0xffff0000u);
          v[2] += __uint_as_float(old.y << 16);
          v[3] += __uint_as_float(old.y & 0xffff0000u);
        }
        uint2 w;
        w.x = pack_bf16x2(v[0], v[1]);
        w.y = pack_bf16x2(v[2], v[3]);
        *reinterpret_cast<uint2*>(q) = w;
      } else {
#pragma unroll
        for (int t = 0; t < 4; t++) {
          if (col + t < o.N) {
            float x = v[t];
            if (o.accumulate) x += bf16_to_f32(q[t]);
            q[t] = f32_to_bf16(x);
          }
        }
      }
    } else {
      float* q = reinterpret_cast<float*>(o.ptr) + at;
      if (o.vec && col + 4 <= o.N) {
        if (o.accumulate) v += *reinterpret_cast<const f32x4*>(q);
        *reinterpret_cast<f32x4*>(q) = v;
      } else {
#pragma unroll
        for (int t = 0; t < 4; t++) {
          if (col + t < o.N) {
            float x = v[t];
            if (o.accumulate) x += q[t];
            q[t] = x;
          }
        }
      }
    }
  }

  template <int I>
  __device__ static __forceinline__ void store_rows(const f32x16 (&acc)[FM][FN], float* stage, const Out& o,
                                                    int lane) {
    if constexpr (I < FM) {
      __syncthreads();  // staging area free (the K loop or the previous slab is done)
#pragma unroll
      for (int j = 0; j < FN; j++)
#pragma unroll
        for (int e = 0; e < 16; e++) {
          int r = 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
          stage[r * EP + j * 32 + (lane & 31)] = acc[I][j][e];
        }
      __syncthreads();
      constexpr int Q = TN / 4;  // float4 per staged row
      constexpr int ITERS = 32 * Q / 64;
#pragma unroll
      for (int it = 0; it < ITERS; it++) {
        int idx = it * 64 + lane;
        int r = idx / Q, q = idx % Q;
        f32x4 v = *reinterpret_cast<const f32x4*>(stage + r * EP + 4 * q);
        int64_t row = o.row0 + I * 32 + r;
        int64_t col = o.col0 + 4 * q;
        if (row < o.M && col < o.N) write4(o, row, col, v);
      }
      store_rows<I + 1>(acc, stage, o, lane);
    }
  }
};

}  // namespace qa
