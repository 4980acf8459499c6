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
//  * A and B tiles move HBM -> LDS in 16-byte chunks with buffer loads,
//    either straight into LDS (`buffer_load_dwordx4 ... lds`, DMA = true,
//    STAGES-deep ring so several K steps are in flight while the MFMAs run;
//    issued from inline assembly, see lds_load16) 
//    or through registers (DMA = false, two LDS stages); a chunk outside the
//    matrix gets an out-of-range buffer offset and reads as zeros, so the
//    loop has no branches;
//  * an operand whose K index is contiguous in HBM ("K-major") sits in LDS
//    as [row][k] and is read with ds_read_b128; an operand whose M/N index is
//    contiguous ("MN-major", e.g. B of a plain row-major A@B) keeps its HBM
//    layout [k][row] in LDS and is read with the gfx950 transpose read
//    ds_read_b64_tr_b16, so no transpose pass or register shuffle is needed;
//  * LDS rows are XOR-swizzled in 16-byte chunks so the fragment reads and the
//    stage writes are free of bank conflicts;
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
  int vec_c;              // 1: output rows allow 16-byte fp32 / 8-byte bf16 stores;
                          // 2: also 16-byte bf16 stores
  // Grouped mode (groups > 0): group g owns rows [offsets[g], offsets[g+1])
  // of A (K-major, lda) and of out (ldc); its B operand is b + g*sb.
  const int64_t* offsets;
  int groups;
  // Gathered rows (grouped mode, K-major A): when a_rows is set, row i of the
  // grouped block is row a_rows[i] of A (a_bytes = A's size in bytes, every
  // index below it), so a routed row set needs no copy of its own.
  const int64_t* a_rows;
  int64_t a_bytes;
  // Two K segments (k_head > 0; grouped mode without gathered rows): the
  // reduction runs over k < k_head from a and b, then over k_head <= k < K
  // from a_tail and b_tail at k - k_head (same leading dimensions and group
  // stride), in one accumulator: out = a op(b) + a_tail op(b_tail).  k_head
  // is a multiple of 64, so no K step straddles the join.
  const void* a_tail;
  const void* b_tail;
  int64_t k_head;
  int tiles_m;            // M tiles in the grid (grouped: an upper bound)
  float alpha;            // scale applied to A@B before the epilogue
  // Grouped-K mode (group_k = 1, batch = groups): group g reduces over the K
  // rows [offsets[g], offsets[g+1]) of A and B and writes out + g*sc.
  int group_k;
  // Split-K (k_split > 1; batch = product batch * k_split): grid batch index
  // z = b * k_split + s reduces K range [s * k_chunk, min(K, (s+1) * k_chunk))
  // of product b and writes its fp32 partial tile to out + z*sc.  k_chunk is
  // a multiple of 64, so no 16-byte chunk of a K-major row crosses a range end.
  int k_split;
  int64_t k_chunk;
  // SwiGLU mode (kernels built with SWIGLU): b is the gate weight and b2 the
  // up weight, both [N][K] (K-major, ldb, group stride sb); out receives
  // silu(gate) * up, and gate_out / up_out (when not null) the two products.
  const void* b2;
  void* gate_out;
  void* up_out;
  // Gathered K rows (grouped-K mode, MN-major B, kernels built with GATHER_B):
  // K row k of B is row b_rows[k] of b (b_bytes = b's size in bytes), so the
  // routed token rows of a weight gradient need no copy of their own; an
  // index outside b's rows reads zeros.
  const int64_t* b_rows;
  int64_t b_bytes;
};


template <bool F32> struct MmaTraits;
template <> struct MmaTraits<false> {  // bf16 in, fp32 accumulate
  typedef bf16_t T;
  static constexpr int E = 8;  // elements per 16-byte chunk
};
template <> struct MmaTraits<true> {   // fp32 in, fp32 accumulate
  typedef float T;
  static constexpr int E = 4;
};

// ---- LDS swizzles -------------------------------------------------------------
// K-major tile [R][BK] with CK 16-byte chunks per row.  Fragment reads take
// 32 consecutive rows at one logical chunk; the XOR below sends any 8
// consecutive rows (128-byte bank window) and any 16 consecutive rows
// (256-byte window) to distinct banks.
template <int CK>
__device__ __forceinline__ int swz_k(int r) {
  if constexpr (CK == 8) return (r ^ (r >> 3)) & 7;
  else return ((r >> 1) ^ (r >> 3)) & 3;  // 64-byte rows: pair parity with row/2
}

// MN-major tile [BK][R] of bf16 read by ds_read_b64_tr_b16: 32 lanes read 4
// consecutive k-rows x 64 bytes; shifting each of the 4 rows into its own
// 64-byte quarter of a 256-byte bank window removes the 4-way conflict.
// Rows of a multiple of 256 bytes (CR = 16, 32) all start in the same bank
// and take four shifts; rows of 128 or 384 bytes (CR = 8, 24) already
// alternate between the two halves of the window and take one shift per
// row pair, which also keeps the XOR inside the 8-chunk groups of a row.
template <int CR>
__device__ __forceinline__ int swz_mn16(int k) {
  return CR % 16 == 0 ? (k & 3) * 4 : ((k >> 1) & 1) * 4;
}
// MN-major tile of fp32 read with ds_read_b32: the two lane halves read
// k-rows 8 apart; put them in different 128-byte bank halves.
__device__ __forceinline__ int swz_mn32(int k) { return ((k >> 3) & 1) * 8; }

// Physical LDS chunk q of one operand stage <-> logical chunk of the tile.
// K-major: q = r * CK + p holds row r, logical chunk c = p ^ swz(r).
// MN-major: q = k * CR + p holds k-row k, logical chunk c = p ^ swz(k).
template <bool F32, bool KMAJOR, int R, int BK>
struct OperandTile {
  typedef MmaTraits<F32> Tr;
  static constexpr int E = Tr::E;
  static constexpr int CK = BK / E;        // chunks per K-major row
  static constexpr int CR = R / E;         // chunks per MN-major row
  static constexpr int CHUNKS = R * BK / E;
  static_assert(!KMAJOR || CK == 4 || CK == 8, "K-major rows of 4 or 8 chunks");

  __device__ static __forceinline__ int swz(int outer) {
    if constexpr (KMAJOR) return swz_k<CK>(outer);
    else return F32 ? swz_mn32(outer) : swz_mn16<CR>(outer);
  }
  // (outer, logical chunk) of physical chunk q
  __device__ static __forceinline__ void coords(int q, int& outer, int& c) {
    if constexpr (KMAJOR) {
      outer = q / CK;
      c = (q % CK) ^ swz(outer);
    } else {
      outer = q / CR;
      c = (q % CR) ^ swz(outer);
    }
  }
  // element offset inside the stage of logical chunk (outer, c)
  __device__ static __forceinline__ int offset(int outer, int c) {
    return KMAJOR ? outer * BK + ((c ^ swz(outer)) * E) : outer * R + ((c ^ swz(outer)) * E);
  }
};

// SWIGLU: the B tile's 32-row blocks alternate between the gate weight (even
// blocks) and the up weight (odd blocks) at the same N index, so each wave's
// two 32-column accumulator blocks hold gate and up of the same outputs and
// the epilogue writes silu(gate) * up: an output tile is BN / 2 wide.
// GATHER_B: grouped-K mode with B's K rows read through GemmArgs::b_rows.
// STREAM_A: A's copies carry the nontemporal hint (lds_load16_nt), for tiles
// that read every A element once (one column tile: the 256x64 tile of
// outputs at most 64 wide) in whole 128-byte row segments per K step (the
// host checks that A's rows start on 128-byte lines and that A is larger
// than the 256 MiB memory-side cache).
template <bool F32, bool TA, bool TB, int BM, int BN, int WM, int WN, int BK, int STAGES, bool DMA,
          bool SWIGLU = false, bool GATHER_B = false, bool STREAM_A = false>
struct GemmKernel {
  typedef MmaTraits<F32> Tr;
  typedef typename Tr::T T;
  static constexpr int E = Tr::E;
  static constexpr int NW = WM * WN;
  static constexpr int NT = 64 * NW;
  static constexpr int TM = BM / WM, TN = BN / WN;  // wave tile
  static constexpr int FM = TM / 32, FN = TN / 32;  // 32x32 blocks per wave
  static constexpr int BNO = SWIGLU ? BN / 2 : BN;  // output columns per tile
  static_assert(!SWIGLU || (!F32 && !TA && TB && DMA && FN == 2), "SwiGLU: bf16 NT, two blocks per wave");
  static_assert(!GATHER_B || (!TB && DMA && STAGES == 2), "gathered K rows: MN-major B, two-stage DMA ring");
  static_assert(!STREAM_A || (DMA && (TA ? BM : BK) * (int)sizeof(typename MmaTraits<F32>::T) % 128 == 0),
                "streamed A: direct-to-LDS copies of whole 128-byte row segments");
  static constexpr bool KA = !TA;                   // A K-major?
  static constexpr bool KB = TB;                    // B K-major?
  typedef OperandTile<F32, KA, BM, BK> TileA;
  typedef OperandTile<F32, KB, BN, BK> TileB;
  static constexpr int LA = TileA::CHUNKS / NT;     // chunks per thread and stage
  static constexpr int LB = TileB::CHUNKS / NT;
  static constexpr int STAGE = (BM + BN) * BK;      // elements per stage
  // Output staging row pitch (floats): TN + 8 puts the two lane halves, which
  // write rows 4 apart, into different bank halves.
  static constexpr int EP = TN + 8;
  static constexpr int RING_BYTES = STAGES * STAGE * (int)sizeof(T);
  static constexpr int LDS_BYTES = RING_BYTES > NW * 32 * EP * 4 ? RING_BYTES : NW * 32 * EP * 4;
  static_assert(TileA::CHUNKS % NT == 0 && TileB::CHUNKS % NT == 0, "staging split");
  static_assert(TM % 32 == 0 && TN % 32 == 0 && BK % 16 == 0, "tile shape");
  static_assert(DMA || STAGES == 2, "register staging is double-buffered");
  static_assert(STAGES >= 2 && LDS_BYTES <= 160 * 1024, "LDS");

  // Operand chunks are fetched with buffer loads: the descriptor's base is
  // the first element this workgroup reads in the current K step, every
  // lane's byte offset is fixed for the whole K loop, and a chunk outside the
  // matrix gets an offset beyond the descriptor's range, for which the
  // hardware returns zeros.  Operands whose rows are not 16-byte aligned are
  // re-laid out (zero-padded pitch) by the host entry point before the launch.
  static constexpr uint32_t OOB = 0x80000000u;
  __device__ static __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const T* base, int64_t bytes) {
    uint32_t n = bytes > 0x7ffffff0 ? 0x7ffffff0u : (uint32_t)bytes;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(base), 0, n, 0x00020000);
  }
  __device__ static __forceinline__ u32x4 fetch(__amdgpu_buffer_rsrc_t r, uint32_t offset) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, offset, 0, 0));
  }

  template <int N>
  __device__ static __forceinline__ void wait_vm() {
    wait_vmcnt<N>();
  }
  __device__ static __forceinline__ void barrier() { asm volatile("s_barrier" ::: "memory"); }

  // Fragment reads -----------------------------------------------------------
  // bf16, K-major: lane l takes row (l & 31), k = 16 s + 8 (l >> 5) + [0, 8).
  __device__ static __forceinline__ bf16x8 frag_k16(const T* t, int row, int s, int lane) {
    int r = row + (lane & 31);
    int c = 2 * s + (lane >> 5);
    return *reinterpret_cast<const bf16x8*>(t + r * BK + ((c ^ swz_k<BK / E>(r)) * E));
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
    constexpr int CK = BK / E;
    int r = row + (lane & 31);
    int c0 = 4 * s + 2 * (lane >> 5);
    f32x4 x = *reinterpret_cast<const f32x4*>(t + r * BK + ((c0 ^ swz_k<CK>(r)) * E));
    f32x4 y = *reinterpret_cast<const f32x4*>(t + r * BK + (((c0 + 1) ^ swz_k<CK>(r)) * E));
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

  // MFMAs of one LDS stage.  bf16: the fragments of k-step s+1 are read
  // while the MFMAs of step s run (two fragment register sets), and the
  // scheduler is asked to interleave one LDS read between MFMAs.
  static constexpr int READS = (KA ? 1 : 2) * FM + (KB ? 1 : 2) * FN;  // ds_read per k-step
  __device__ static __forceinline__ void frags16(const T* sa, const T* sb, bf16x8 (&fa)[FM], bf16x8 (&fb)[FN],
                                                 int wm, int wn, int s, int lane) {
#pragma unroll
    for (int i = 0; i < FM; i++)
      fa[i] = KA ? frag_k16(sa, wm * TM + i * 32, s, lane) : frag_mn16<BM>(sa, wm * TM + i * 32, s, lane);
#pragma unroll
    for (int j = 0; j < FN; j++)
      fb[j] = KB ? frag_k16(sb, wn * TN + j * 32, s, lane) : frag_mn16<BN>(sb, wn * TN + j * 32, s, lane);
  }
  __device__ static __forceinline__ void mfma16(const bf16x8 (&fa)[FM], const bf16x8 (&fb)[FN],
                                                f32x16 (&acc)[FM][FN]) {
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
      for (int j = 0; j < FN; j++)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
  }
  __device__ static __forceinline__ void compute(const T* sa, const T* sb, f32x16 (&acc)[FM][FN], int wm, int wn,
                                                 int lane) {
    if constexpr (!F32) {
      constexpr int S = BK / 16;
      bf16x8 fa[2][FM], fb[2][FN];
      frags16(sa, sb, fa[0], fb[0], wm, wn, 0, lane);
#pragma unroll
      for (int s = 0; s < S; s++) {
        if (s + 1 < S) frags16(sa, sb, fa[(s + 1) & 1], fb[(s + 1) & 1], wm, wn, s + 1, lane);
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
          for (int j = 0; j < FN; j++)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[s & 1][i], fb[s & 1][j], acc[i][j], 0, 0, 0);
      }
#ifdef QA_SCHED_INTERLEAVE
      // one group per MFMA, one LDS read after each of the first ones
#pragma unroll
      for (int s = 0; s < S; s++) {
#pragma unroll
        for (int m = 0; m < FM * FN; m++) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          if (s + 1 < S && m < READS) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
      }
#endif
    } else {
#pragma unroll
      for (int s = 0; s < BK / 16; s++) {
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
  }

  __device__ static __forceinline__ void run(const GemmArgs& p, char* smem) {
    T* lds = reinterpret_cast<T*>(smem);
    const int tid = threadIdx.x, lane = tid & 63, wave = uniform32(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;

    // ---- tile scheduling -------------------------------------------------
    const int tiles_n = (int)((p.N + BNO - 1) / BNO);
    int tiles_m = p.tiles_m;
    int total = (int)gridDim.x;
    if (p.groups > 0 && !p.group_k) {
      // grouped rows: the grid covers an upper bound of the M tiles; count
      // the real ones so that they, not the grid, are spread evenly over the
      // XCDs (surplus ids exit here instead of piling onto the last XCDs)
      int real = 0;
      for (int e = 0; e < p.groups; e++) real += (int)((p.offsets[e + 1] - p.offsets[e] + BM - 1) / BM);
      tiles_m = uniform32(real);
      total = tiles_m * tiles_n;
      if ((int)blockIdx.x >= total) return;
    }
    const int tiles_per = tiles_m * tiles_n;
    int pid = uniform32(xcd_remap((int)blockIdx.x, total));
    int64_t bz = pid / tiles_per;
    int t = pid % tiles_per;
    // grouped ordering: 4 M-tiles per group, N fastest inside a group
    constexpr int GM = 4;
    int group = t / (GM * tiles_n);
    int first_m = group * GM;
    int gsize = min(tiles_m - first_m, GM);
    int tile_m = first_m + (t % (GM * tiles_n)) % gsize;
    int tile_n = (t % (GM * tiles_n)) / gsize;

    const T* A = reinterpret_cast<const T*>(p.a);
    const T* B = reinterpret_cast<const T*>(p.b);
    const T* B2 = reinterpret_cast<const T*>(p.b2);
    const T* A_tail = reinterpret_cast<const T*>(p.a_tail);  // second K segment (k_head > 0)
    const T* B_tail = reinterpret_cast<const T*>(p.b_tail);
    int64_t M = p.M, row0 = 0, K = p.K;
    const int64_t* gather = nullptr;  // grouped mode with a_rows: this group's row indices
    const int64_t* gather_b = nullptr;  // GATHER_B: this group's K-row indices into b
    char* outp = reinterpret_cast<char*>(p.out);
    const int osize = p.out_bf16 ? 2 : 4;
    if (p.group_k) {
      // per-group K range; an empty group writes zeros (or keeps `out`)
      const int64_t k_lo = p.offsets[bz], k_hi = p.offsets[bz + 1];
      A += k_lo * (KA ? 1 : p.lda);
      if constexpr (GATHER_B) gather_b = p.b_rows + k_lo;
      else B += k_lo * (KB ? 1 : p.ldb);
      outp += bz * p.sc * osize;
      row0 = (int64_t)tile_m * BM;
      K = k_hi - k_lo;
    } else if (p.groups > 0) {
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
      if (KA && p.a_rows) gather = p.a_rows + lo;
      else A += lo * p.lda;
      B += (int64_t)g * p.sb;
      if (p.k_head > 0) {
        A_tail += lo * p.lda;
        B_tail += (int64_t)g * p.sb;
      }
      if constexpr (SWIGLU) B2 += (int64_t)g * p.sb;
      outp += lo * p.ldc * osize;
      M = hi - lo;
    } else if (p.k_split > 1) {
      const int64_t prod = bz / p.k_split, k_lo = (bz % p.k_split) * p.k_chunk;
      A += prod * p.sa + k_lo * (KA ? 1 : p.lda);
      B += prod * p.sb + k_lo * (KB ? 1 : p.ldb);
      outp += bz * p.sc * osize;
      row0 = (int64_t)tile_m * BM;
      K = (K < k_lo + p.k_chunk ? K : k_lo + p.k_chunk) - k_lo;
    } else {
      A += bz * p.sa;
      B += bz * p.sb;
      outp += bz * p.sc * osize;
      row0 = (int64_t)tile_m * BM;
    }
    A = uniform_ptr(A);
    B = uniform_ptr(B);
    A_tail = uniform_ptr(A_tail);
    B_tail = uniform_ptr(B_tail);
    const int64_t k_head = uniform64(p.k_head);
    if constexpr (SWIGLU) B2 = uniform_ptr(B2);
    outp = uniform_ptr(outp);
    M = uniform64(M);
    row0 = uniform64(row0);
    const int64_t col0 = uniform64((int64_t)tile_n * BNO);
    K = uniform64(K);
    const int64_t N = p.N;
    const int64_t lda = p.lda, ldb = p.ldb;

    f32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
      for (int j = 0; j < FN; j++)
#pragma unroll
        for (int e = 0; e < 16; e++) acc[i][j][e] = 0.f;

    const int nk = (int)((K + BK - 1) / BK);
    // descriptor of one operand for the K step starting at k0
    auto desc_a = [&](int64_t k0) {
      const bool tail = k_head > 0 && k0 >= k_head;
      const T* a = tail ? A_tail : A;
      if (tail) k0 -= k_head;
      return rsrc(KA ? a + row0 * lda + k0 : a + k0 * lda + row0,
                  (int64_t)(KA ? BM * lda : BK * lda) * (int64_t)sizeof(T));
    };
    auto desc_b = [&](int64_t k0) {
      const bool tail = k_head > 0 && k0 >= k_head;
      const T* b = tail ? B_tail : B;
      if (tail) k0 -= k_head;
      return rsrc(KB ? b + col0 * ldb + k0 : b + k0 * ldb + col0,
                  (int64_t)(KB ? BN * ldb : BK * ldb) * (int64_t)sizeof(T));
    };

    if constexpr (DMA) {
      // ---- direct-to-LDS ring: wave w, instruction j fills physical chunks
      // q = (j * NW + w) * 64 + lane, i.e. 1 KB of LDS per instruction.
      constexpr int JA = TileA::CHUNKS / (64 * NW), JB = TileB::CHUNKS / (64 * NW);
      constexpr int L = JA + JB;  // DMA instructions per wave and stage
      static_assert(TileA::CHUNKS % (64 * NW) == 0 && TileB::CHUNKS % (64 * NW) == 0, "DMA split");
      static_assert(L * (STAGES - 2) <= 63, "vmcnt range");
      uint32_t oa[JA], ob[JB];
      int ka[JA], kb[JB];  // k coordinate of the chunk (validity per K step)
      bool va[JA], vb[JB];
      // gathered rows: rows of A in the table's range [0, a_bytes / row bytes)
      const int64_t a_count = gather ? p.a_bytes / (lda * (int64_t)sizeof(T)) : 0;
#pragma unroll
      for (int j = 0; j < JA; j++) {
        int q = (j * NW + wave) * 64 + lane, outer, c;
        TileA::coords(q, outer, c);
        ka[j] = KA ? c * E : outer;
        va[j] = KA ? (row0 + outer < M) : (row0 + c * E < M);
        // gathered rows: the row index comes from the table (read only for
        // rows inside the group), the descriptor spans all of A; an index
        // outside A's rows reads zeros (its chunks get the out-of-range
        // offset; a 32-bit byte offset could otherwise wrap onto a real row)
        const int64_t src_row = KA && gather && va[j] ? gather[row0 + outer] : outer;
        if (KA && gather && va[j] && (src_row < 0 || src_row >= a_count)) va[j] = false;
        oa[j] = (uint32_t)((src_row * lda + c * E) * (int64_t)sizeof(T));
      }
      // A's descriptor base at k0 is a_tile + k0 (K-major) or + k0 * lda
      const T* a_tile = gather ? A : KA ? A + row0 * lda : A + row0;
      const T* a_tail_tile = KA ? A_tail + row0 * lda : A_tail + row0;
      const int64_t a_span = gather ? p.a_bytes : (int64_t)(KA ? BM * lda : BK * lda) * (int64_t)sizeof(T);
      bool up[JB];  // SWIGLU: instruction j copies up-weight rows
#pragma unroll
      for (int j = 0; j < JB; j++) {
        int q = (j * NW + wave) * 64 + lane, outer, c;
        TileB::coords(q, outer, c);
        // SWIGLU: tile row `outer` is row (outer / 64) * 32 + outer % 32 of the
        // gate (outer / 32 even) or up (odd) weight; one instruction covers 8
        // rows, all in one 32-row block
        if constexpr (SWIGLU) outer = ((outer >> 6) << 5) + (outer & 31);
        up[j] = SWIGLU && (((j * NW + wave) >> 2) & 1);
        ob[j] = (uint32_t)(((int64_t)outer * ldb + c * E) * (int64_t)sizeof(T));
        kb[j] = KB ? c * E : outer;
        vb[j] = KB ? (col0 + outer < N) : (col0 + c * E < N);
        if constexpr (GATHER_B) ob[j] = (uint32_t)(c * E * (int)sizeof(T));  // byte offset inside a source row
      }
      // GATHER_B: the source rows of this lane's chunks for the stage issued
      // next (rows[]) and the one after (rows_next[], loaded one K step ahead
      // so that the copies never wait for their index); -1 = no row (past the
      // group's K range or N), read as zeros like an index outside b.
      const int64_t b_count = GATHER_B ? p.b_bytes / (ldb * (int64_t)sizeof(T)) : 0;
      int64_t rows[GATHER_B ? JB : 1], rows_next[GATHER_B ? JB : 1];
      auto fetch_rows = [&](int64_t (&dst)[GATHER_B ? JB : 1], int64_t k0) {
        if constexpr (GATHER_B) {
#pragma unroll
          for (int j = 0; j < JB; j++) dst[j] = (vb[j] && k0 + kb[j] < K) ? gather_b[k0 + kb[j]] : -1;
        }
      };
      char* base = reinterpret_cast<char*>(lds);
      // copies of one stage, optionally only instructions [first, last)
      auto issue_range = [&](int stage, int64_t k0, int first, int last) {
        // the second K segment reads a_tail / b_tail at k0 - k_head
        const bool tail = k_head > 0 && k0 >= k_head;
        const int64_t kk = tail ? k0 - k_head : k0;
        const T* at = tail ? a_tail_tile : a_tile;
        const T* bt = tail ? B_tail : B;
        const u32x4 da = lds_rsrc(KA ? at + kk : at + kk * lda, a_span);
        const u32x4 db = GATHER_B ? lds_rsrc(B + col0, p.b_bytes - col0 * (int64_t)sizeof(T))
                                  : lds_rsrc(KB ? bt + col0 * ldb + kk : bt + kk * ldb + col0,
                                             (int64_t)(KB ? BN * ldb : BK * ldb) * (int64_t)sizeof(T));
        const u32x4 db2 = SWIGLU ? lds_rsrc(B2 + col0 * ldb + k0, (int64_t)BN * ldb * (int64_t)sizeof(T)) : db;
        const int64_t krem = K - k0;
        char* sa = base + stage * STAGE * (int)sizeof(T);
        char* sb = sa + BM * BK * (int)sizeof(T);
#pragma unroll
        for (int j = 0; j < JA; j++)
          if (j >= first && j < last)
          {
            const uint32_t off = (va[j] && ka[j] < krem) ? oa[j] : OOB;
            if constexpr (STREAM_A) lds_load16_nt(da, sa + (j * NW + wave) * 1024, off);
            else lds_load16(da, sa + (j * NW + wave) * 1024, off);
          }
#pragma unroll
        for (int j = 0; j < JB; j++)
          if (JA + j >= first && JA + j < last) {
            uint32_t off = (vb[j] && kb[j] < krem) ? ob[j] : OOB;
            if constexpr (GATHER_B) {
              // the row's 32-bit byte offset from b + col0 (b is below 2 GiB)
              const int64_t r = rows[j];
              off = (r >= 0 && r < b_count) ? (uint32_t)(r * ldb * (int64_t)sizeof(T)) + ob[j] : OOB;
            }
            lds_load16(up[j] ? db2 : db, sb + (j * NW + wave) * 1024, off);
          }
      };
      auto issue = [&](int stage, int64_t k0) { issue_range(stage, k0, 0, L); };
      if constexpr (GATHER_B) {
        // two stages: stage 0's rows now, stage 1's ahead of the loop
        fetch_rows(rows, 0);
        if (nk > 0) issue(0, 0);
        fetch_rows(rows_next, BK);
      } else {
#pragma unroll
        for (int st = 0; st < STAGES - 1; st++)
          if (st < nk) issue(st, (int64_t)st * BK);
      }
      for (int kt = 0; kt < nk; kt++) {
        // this wave's copies of stage kt are done when at most the copies of
        // the (up to STAGES-2) younger stages are still outstanding
        const int younger = min(STAGES - 2, nk - 1 - kt);
        if (younger >= 3) wait_vm<(STAGES >= 5 ? 3 : 0) * L>();
        else if (younger == 2) wait_vm<(STAGES >= 4 ? 2 : 0) * L>();
        else if (younger == 1) wait_vm<L>();
        else wait_vm<0>();
        barrier();  // every wave's copies of stage kt are in LDS; stage kt-1 is free
        if constexpr (GATHER_B) {
          // rows_next (loaded during the previous step, complete after the
          // vmcnt wait above) belong to stage kt + 1, issued in this step
#pragma unroll
          for (int j = 0; j < JB; j++) rows[j] = rows_next[j];
          fetch_rows(rows_next, (int64_t)(kt + 2) * BK);
        }
        const T* sa = lds + (kt % STAGES) * STAGE;
        const bool more = kt + STAGES - 1 < nk;
        const int next = (kt + STAGES - 1) % STAGES;
        const int64_t k_next = (int64_t)(kt + STAGES - 1) * BK;
        if constexpr (!F32) {
          // the next stage's copies in two slices, issued in the first two
          // k-steps between the fragment reads and the MFMAs (all copies at
          // once stall the issuing wave; spreading them over every k-step
          // leaves the last slice too little time)
          constexpr int S = BK / 16, PER = S >= 2 ? (L + 1) / 2 : L;
          const T* sb = sa + BM * BK;
          bf16x8 fa[2][FM], fb[2][FN];
          frags16(sa, sb, fa[0], fb[0], wm, wn, 0, lane);
#pragma unroll
          for (int s = 0; s < S; s++) {
            if (more && s * PER < L) issue_range(next, k_next, s * PER, (s + 1) * PER < L ? (s + 1) * PER : L);
            if (s + 1 < S) frags16(sa, sb, fa[(s + 1) & 1], fb[(s + 1) & 1], wm, wn, s + 1, lane);
            mfma16(fa[s & 1], fb[s & 1], acc);
          }
        } else {
          if (more) issue(next, k_next);
          compute(sa, sa + BM * BK, acc, wm, wn, lane);
        }
      }
      static_assert(STAGES <= 5, "wait table covers up to 3 younger stages");
    } else {
      // ---- register staging, two LDS stages --------------------------------
      uint32_t oa[LA], ob[LB];
      int ka[LA], kb[LB];
      bool va[LA], vb[LB];
#pragma unroll
      for (int i = 0; i < LA; i++) {
        int idx = tid + i * NT;
        int outer = KA ? idx / TileA::CK : idx / TileA::CR;
        int c = KA ? idx % TileA::CK : idx % TileA::CR;
        oa[i] = (uint32_t)(((int64_t)outer * lda + c * E) * (int64_t)sizeof(T));
        ka[i] = KA ? c * E : outer;
        va[i] = KA ? (row0 + outer < M) : (row0 + c * E < M);
      }
#pragma unroll
      for (int i = 0; i < LB; i++) {
        int idx = tid + i * NT;
        int outer = KB ? idx / TileB::CK : idx / TileB::CR;
        int c = KB ? idx % TileB::CK : idx % TileB::CR;
        ob[i] = (uint32_t)(((int64_t)outer * ldb + c * E) * (int64_t)sizeof(T));
        kb[i] = KB ? c * E : outer;
        vb[i] = KB ? (col0 + outer < N) : (col0 + c * E < N);
      }
      u32x4 ra[LA], rb[LB];
      auto load = [&](int64_t k0) {
        auto da = desc_a(k0);
        auto db = desc_b(k0);
        const int64_t krem = K - k0;
#pragma unroll
        for (int i = 0; i < LA; i++) ra[i] = fetch(da, (va[i] && ka[i] < krem) ? oa[i] : OOB);
#pragma unroll
        for (int i = 0; i < LB; i++) rb[i] = fetch(db, (vb[i] && kb[i] < krem) ? ob[i] : OOB);
      };
      auto store = [&](int stage) {
        T* sa = lds + stage * STAGE;
        T* sb = sa + BM * BK;
#pragma unroll
        for (int i = 0; i < LA; i++) {
          int idx = tid + i * NT;
          int outer = KA ? idx / TileA::CK : idx / TileA::CR;
          int c = KA ? idx % TileA::CK : idx % TileA::CR;
          *reinterpret_cast<u32x4*>(sa + TileA::offset(outer, c)) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < LB; i++) {
          int idx = tid + i * NT;
          int outer = KB ? idx / TileB::CK : idx / TileB::CR;
          int c = KB ? idx % TileB::CK : idx % TileB::CR;
          *reinterpret_cast<u32x4*>(sb + TileB::offset(outer, c)) = rb[i];
        }
      };
      if (nk > 0) {
        load(0);
        store(0);
        __syncthreads();
      }
      for (int kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        if (kt + 1 < nk) load((int64_t)(kt + 1) * BK);
        const T* sa = lds + cur * STAGE;
        compute(sa, sa + BM * BK, acc, wm, wn, lane);
        if (kt + 1 < nk) store(cur ^ 1);
        __syncthreads();
      }
    }

    // ---- epilogue ---------------------------------------------------------
    Out o;
    o.ptr = outp;
    o.ldc = p.ldc;
    o.M = M;
    o.N = N;
    o.row0 = row0 + wm * TM;
    o.col0 = col0 + wn * (BNO / WN);
    o.bf16 = p.out_bf16;
    o.accumulate = p.accumulate;
    o.vec = p.vec_c;
    o.alpha = p.alpha;
    float* stage = reinterpret_cast<float*>(smem) + wave * 32 * EP;
    __syncthreads();  // every wave has read the ring's last stage
    // full in-bounds wave tile: straight-line 16-byte loads (accumulate) and stores
    const bool fast = o.vec >= (o.bf16 ? 2 : 1) && o.row0 + TM <= o.M && o.col0 + BNO / WN <= o.N;
    if constexpr (SWIGLU) {
      // gate / up outputs share out's layout: same byte offset from their base
      const int64_t shift = outp - reinterpret_cast<char*>(p.out);
      Out og = o, ou = o;
      og.ptr = p.gate_out ? reinterpret_cast<char*>(p.gate_out) + shift : nullptr;
      ou.ptr = p.up_out ? reinterpret_cast<char*>(p.up_out) + shift : nullptr;
#pragma unroll
      for (int i = 0; i < FM; i++) {
        // the unfused SwiGLU's roundings: gate and up are bf16 products,
        // silu(gate) is a bf16 tensor before the multiply, one rounding after
        f32x16 g, u, y;
#pragma unroll
        for (int e = 0; e < 16; e++) {
          g[e] = bf16_to_f32(f32_to_bf16(acc[i][0][e]));
          u[e] = bf16_to_f32(f32_to_bf16(acc[i][1][e]));
          y[e] = bf16_to_f32(f32_to_bf16(silu_f(g[e]))) * u[e];
        }
        const f32x16 ys[1] = {y};
        store_slab<1>(ys, stage, o, o.row0 + i * 32, lane, fast);
        if (og.ptr) {
          const f32x16 gs[1] = {g};
          store_slab<1>(gs, stage, og, o.row0 + i * 32, lane, fast);
        }
        if (ou.ptr) {
          const f32x16 us[1] = {u};
          store_slab<1>(us, stage, ou, o.row0 + i * 32, lane, fast);
        }
      }
    } else if constexpr ((FN & (FN - 1)) == 0) {
#pragma unroll
      for (int i = 0; i < FM; i++) store_slab<FN>(acc[i], stage, o, o.row0 + i * 32, lane, fast);
    } else {  // 96-wide wave tiles: one 32-column block at a time (whole rows per store)
#pragma unroll
      for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) {
          Out oj = o;
          oj.col0 = o.col0 + 32 * j;
          const f32x16 blk[1] = {acc[i][j]};
          store_slab<1>(blk, stage, oj, o.row0 + i * 32, lane, fast);
        }
    }
  }

  // Output staging: each wave turns one 32-row slab of its accumulators
  // (MFMA C layout: lane l holds column l & 31 and rows
  // 8 (e/4) + 4 (l >> 5) + (e & 3) of a 32x32 block) into row-major order in
  // its own LDS area (row pitch EP), then writes it along rows.  The area is
  // private to the wave and a wave's LDS operations complete in order, so
  // slabs need no workgroup barrier.

  struct Out {
    char* ptr;
    int64_t ldc, M, N, row0, col0;
    int bf16, accumulate, vec;
    float alpha;
  };

  __device__ static __forceinline__ void write4(const Out& o, int64_t row, int64_t col, f32x4 v) {
    typedef __attribute__((address_space(1))) bf16_t gbf16;
    typedef __attribute__((address_space(1))) float gf32;
    v *= o.alpha;
    int64_t at = row * o.ldc + col;
    if (o.bf16) {
      gbf16* q = (gbf16*)(o.ptr) + at;
      if (col + 4 <= o.N) {
        // four whole columns: one 8-byte access; rows with an odd pitch give
        // 2-byte alignment only, which unaligned global accesses accept
        typedef unsigned u32x2a2 __attribute__((ext_vector_type(2), aligned(2)));
        typedef __attribute__((address_space(1))) u32x2a2 gu2;
        if (o.accumulate) {
          u32x2 old = *(const gu2*)q;
          v[0] += __uint_as_float(old[0] << 16);
          v[1] += __uint_as_float(old[0] & 0xffff0000u);
          v[2] += __uint_as_float(old[1] << 16);
          v[3] += __uint_as_float(old[1] & 0xffff0000u);
        }
        *(gu2*)q = u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
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
      gf32* q = (gf32*)(o.ptr) + at;
      if (col + 4 <= o.N) {
        // four whole columns: one 16-byte store; rows whose pitch is not a
        // multiple of 4 elements only give 4-byte alignment, which the
        // vector store accepts (global accesses need dword alignment only)
        typedef __attribute__((address_space(1))) f32x4 gf4;
        typedef float f32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
        typedef __attribute__((address_space(1))) f32x4a4 gf4a4;
        if (o.vec) {
          if (o.accumulate) v += *(const gf4*)q;
          *(gf4*)q = v;
        } else {
          if (o.accumulate) v += *(const gf4a4*)q;
          *(gf4a4*)q = v;
        }
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

  // One 32-row slab of NB 32x32 accumulator blocks (NB * 32 columns from
  // o.col0) to rows row_base .. row_base + 31 of the output.
  template <int NB>
  __device__ static __forceinline__ void store_slab(const f32x16 (&blk)[NB], float* stage, const Out& o,
                                                    int64_t row_base, int lane, bool fast) {
    constexpr int W = NB * 32;
#pragma unroll
    for (int j = 0; j < NB; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) {
        int r = 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
        stage[r * EP + j * 32 + (lane & 31)] = blk[j][e];
      }
    __builtin_amdgcn_wave_barrier();
    if (fast && o.bf16) {
      // lane -> 8 consecutive columns of one row: one 16-byte store each
      // (accumulate: the old values are loaded first, added in fp32)
      constexpr int Q = W / 8, ITERS = 32 * Q / 64;
      static_assert(64 % Q == 0, "whole rows per store instruction");
      bf16_t* dst = reinterpret_cast<bf16_t*>(o.ptr) + (row_base + lane / Q) * o.ldc + o.col0 + 8 * (lane % Q);
      u32x4 w[ITERS];
      if (o.accumulate) {
#pragma unroll
        for (int it = 0; it < ITERS; it++) w[it] = global_load<u32x4>(dst + it * (64 / Q) * o.ldc);
      }
#pragma unroll
      for (int it = 0; it < ITERS; it++) {
        int idx = it * 64 + lane, r = idx / Q, q = idx % Q;
        f32x4 a = *reinterpret_cast<const f32x4*>(stage + r * EP + 8 * q) * o.alpha;
        f32x4 b = *reinterpret_cast<const f32x4*>(stage + r * EP + 8 * q + 4) * o.alpha;
        if (o.accumulate) {
#pragma unroll
          for (int h = 0; h < 2; h++) {
            a[2 * h] += __uint_as_float(w[it][h] << 16);
            a[2 * h + 1] += __uint_as_float(w[it][h] & 0xffff0000u);
            b[2 * h] += __uint_as_float(w[it][2 + h] << 16);
            b[2 * h + 1] += __uint_as_float(w[it][2 + h] & 0xffff0000u);
          }
        }
        w[it] = u32x4{pack_bf16x2(a[0], a[1]), pack_bf16x2(a[2], a[3]), pack_bf16x2(b[0], b[1]),
                      pack_bf16x2(b[2], b[3])};
      }
#pragma unroll
      for (int it = 0; it < ITERS; it++) global_store_nt(dst + it * (64 / Q) * o.ldc, w[it]);
    } else if (fast) {
      constexpr int Q = W / 4, ITERS = 32 * Q / 64;
      static_assert(64 % Q == 0, "whole rows per store instruction");
      float* dst = reinterpret_cast<float*>(o.ptr) + (row_base + lane / Q) * o.ldc + o.col0 + 4 * (lane % Q);
      f32x4 v[ITERS];
      if (o.accumulate) {
#pragma unroll
        for (int it = 0; it < ITERS; it++) v[it] = global_load<f32x4>(dst + it * (64 / Q) * o.ldc);
      }
#pragma unroll
      for (int it = 0; it < ITERS; it++) {
        int idx = it * 64 + lane, r = idx / Q, q = idx % Q;
        const f32x4 x = *reinterpret_cast<const f32x4*>(stage + r * EP + 4 * q) * o.alpha;
        v[it] = o.accumulate ? v[it] + x : x;
      }
#pragma unroll
      for (int it = 0; it < ITERS; it++) global_store_nt(dst + it * (64 / Q) * o.ldc, v[it]);
    } else {
      constexpr int Q = W / 4;  // float4 per staged row
      constexpr int ITERS = 32 * Q / 64;
#pragma unroll
      for (int it = 0; it < ITERS; it++) {
        int idx = it * 64 + lane;
        int r = idx / Q, q = idx % Q;
        f32x4 v = *reinterpret_cast<const f32x4*>(stage + r * EP + 4 * q);
        int64_t row = row_base + r;
        int64_t col = o.col0 + 4 * q;
        if (row < o.M && col < o.N) write4(o, row, col, v);
      }
    }
    __builtin_amdgcn_wave_barrier();
  }
};

}  // namespace qa
