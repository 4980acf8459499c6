// Fused attention forward for D = 64, bf16 storage, fp32 accumulation
// (C ABI `qutai_amd_attention_fwd`).  O = softmax(scale * Q K^T) V without
// materialising the T x T scores: the reference's score and value products
// (src/qutai/nn/layers.py:334-354 through two batched GEMMs and a softmax, and
// the lm kernel lm_attention_bf16_d64, src/qutai/backends/cuda/lm.cu:91-157)
// in one pass over K and V.
//
// Layout of the work (gfx950, 64-wide wavefronts):
//  * a workgroup owns 256 consecutive queries of one (batch, head): 8 waves
//    of 32 queries (the default), or 4 waves of two 32-query blocks; each
//    wave keeps its Q fragments in registers for the whole kernel; two
//    workgroups run per CU (8-wave shape: four waves per SIMD);
//  * K and V advance in blocks of 64 keys, copied HBM -> LDS with
//    buffer_load ... lds into a two-stage ring (8 KiB + 8 KiB per stage); the
//    copy of block j+1 overlaps the MFMAs of block j; the softmax and the
//    value product run per 32-key half of a block;
//  * scores are computed transposed, S^T = K Q^T, with
//    v_mfma_f32_32x32x16_bf16: in the MFMA result layout lane l then holds
//    query l % 32 of its block and 16 keys of each 32-key block, so the
//    running max / sum of a query live in one lane (plus its partner lane
//    l ^ 32, exchanged once per 32-key half);
//  * the probabilities, rounded to bf16, are already in the B-operand layout
//    of the value product O^T += V^T P^T (the MFMA's k index runs over the keys
//    in the order the score layout holds them; V is read with the gfx950
//    transpose read ds_read_b64_tr_b16 in the same key order), so P never
//    leaves registers;
//  * O^T's result layout gives every lane one query, so the rescaling by
//    exp(m_old - m_new) and the final 1/l are per-lane scalars.
#include "common.h"
#include "qutai_amd.h"

#include <algorithm>
#include <cstdlib>
#include <initializer_list>

using namespace qa;

namespace {

constexpr int D = 64;          // head dimension
constexpr int KB = 64;         // keys per block
constexpr int TILE = KB * D;     // elements of one K (or V) stage

struct AttnArgs {
  const bf16_t* q;
  const bf16_t* k;
  const bf16_t* v;
  bf16_t* o;
  float* lse;  // optional natural-log sum-exp per (batch, head, token)
  int64_t batch, heads, kv_heads, time;
  // element strides of (batch, head, token) for q/o, for k/v and for lse
  int64_t qb, qh, qt, kb, kh, kt, lb, lh, lt;
  float scale_log2;  // scale * log2(e)
  float scale;
  int causal;
};

// K rows: 128 bytes = 8 chunks, swizzled like the GEMM's K-major tiles.
__device__ __forceinline__ int swz_row8(int r) { return (r ^ (r >> 3)) & 7; }
// V rows read by the transpose read in groups of 4 rows x 64 bytes.
__device__ __forceinline__ int swz_v(int r) { return ((r >> 1) & 1) * 4; }

typedef __attribute__((address_space(3))) void* lds_void;
typedef i16x4 __attribute__((address_space(3))) * lds_i16x4;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, int64_t bytes) {
  uint32_t n = bytes > 0x7ffffff0 ? 0x7ffffff0u : (uint32_t)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, n, 0x00020000);
}

// Both halves of the wavefront (lanes l and l ^ 32) hold the same query:
// the gfx950 half swap exchanges them without LDS.
__device__ __forceinline__ float pair_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// The 32 keys 32 mb + [0, 32) of a 64-key block for the wave's NQB query
// blocks (a block is processed as two such halves: fewer live registers, so
// that four waves fit per SIMD).  MASK: some key of the block is past T or
// (causal) after a query; lim[qb] is then the number of leading keys of the
// block the lane's query may see, minus 4 * half.
template <int NQB, bool MASK>
__device__ __forceinline__ void attend_half(const bf16_t* sk, const bf16_t* sv, const bf16x8 (&qf)[NQB][4],
                                            f32x16 (&o)[NQB][2], float (&m)[NQB], float (&l)[NQB],
                                            const int (&lim)[NQB], float c, int lane, int mb) {
  const int half = lane >> 5, col = lane & 31;
  // K fragments (A operand): key row 32 mb + col, d = 16 s + 8 half + [0, 8)
  bf16x8 kf[4];
#pragma unroll
  for (int s = 0; s < 4; s++) {
    int r = 32 * mb + col, ch = 2 * s + half;
    kf[s] = *reinterpret_cast<const bf16x8*>(sk + r * D + ((ch ^ swz_row8(r)) * 8));
  }
  // S^T blocks for every query block first, so the value products of one
  // query block overlap the exponentials of the next.
  f32x16 sc[NQB];
#pragma unroll
  for (int qb = 0; qb < NQB; qb++) {
    f32x16 acc = {};
#pragma unroll
    for (int st = 0; st < 4; st++) acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[st], qf[qb][st], acc, 0, 0, 0);
    sc[qb] = acc;
  }

  // ---- running max (scaled log2 domain; scale > 0, so max(s) c = max(s c)).
  // The reference point m only moves when the keys' max exceeds it by more
  // than 8 (a factor 256), so the rescaling of l and O is skipped for most
  // halves; the probabilities exp2(s c - m) then stay below 256 and the
  // result is the same softmax (the normaliser uses the same m).
  bool grow_any = false;
  float m_new[NQB];
#pragma unroll
  for (int qb = 0; qb < NQB; qb++) {
    // key of element e: 32 mb + 8 (e / 4) + 4 half + e % 4
    if (MASK) {
#pragma unroll
      for (int e = 0; e < 16; e++)
        if (32 * mb + 8 * (e >> 2) + (e & 3) >= lim[qb]) sc[qb][e] = -INFINITY;
    }
    float peak = -INFINITY;
#pragma unroll
    for (int e = 0; e < 16; e++) peak = fmaxf(peak, sc[qb][e]);
    const float cand = pair_max(peak) * c;
    const bool grow = cand > m[qb] + 8.f;  // -inf + 8 = -inf: the first visible key always moves m
    m_new[qb] = grow ? cand : m[qb];
    grow_any |= grow;
  }
  if (__builtin_amdgcn_ballot_w64(grow_any)) {
#pragma unroll
    for (int qb = 0; qb < NQB; qb++) {
      // only the lanes whose m moves rescale (an exec-masked update keeps O
      // in its registers; a wave-uniform select would make the compiler copy
      // all of O every block).  A query that has seen no valid key keeps
      // m = -inf and l = 0, O = 0.
      if (m_new[qb] != m[qb]) {
        const float alpha = __builtin_amdgcn_exp2f(m[qb] - m_new[qb]);
        m[qb] = m_new[qb];
        l[qb] *= alpha;
#pragma unroll
        for (int db = 0; db < 2; db++)
#pragma unroll
          for (int e = 0; e < 16; e++) o[qb][db][e] *= alpha;
      }
    }
  }
  const int g = lane >> 4, i = lane & 15;
#pragma unroll
  for (int qb = 0; qb < NQB; qb++) {
    // exp2(-inf - 0) = 0 for a query with no visible key yet
    const float ref = m[qb] == -INFINITY ? 0.f : m[qb];
    float sum = 0.f;
    bf16x8 pf[2];
#pragma unroll
    for (int st = 0; st < 2; st++) {
      // the normaliser sums the fp32 probabilities; the value product takes
      // them rounded to bf16 (lm.cu:131-134)
      float pv[8];
#pragma unroll
      for (int e = 0; e < 8; e++) {
        pv[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[qb][8 * st + e], c, -ref));
        sum += pv[e];
      }
      u32x4 w = {pack_bf16x2(pv[0], pv[1]), pack_bf16x2(pv[2], pv[3]), pack_bf16x2(pv[4], pv[5]),
                 pack_bf16x2(pv[6], pv[7])};
      pf[st] = __builtin_bit_cast(bf16x8, w);
    }
    l[qb] += sum;
    // V^T fragments (A operand of O^T), read just before their products so
    // they are not live across the softmax: lane = d column 32 db + col;
    // keys in the score layout order: for k-step st the 8 keys
    // 32 mb + 16 st + 4 half + {0..3} and + 8 + {0..3}.
    bf16x8 vf[2][2];  // [db][st]
#pragma unroll
    for (int db = 0; db < 2; db++)
#pragma unroll
      for (int st = 0; st < 2; st++) {
        int cb = 32 * db + (g & 1) * 16 + 4 * (i & 3);
        int kb0 = 32 * mb + 16 * st + 4 * (g >> 1) + (i >> 2);
        int kb1 = kb0 + 8;
        const bf16_t* p0 = sv + kb0 * D + (((cb >> 3) ^ swz_v(kb0)) * 8) + (cb & 7);
        const bf16_t* p1 = sv + kb1 * D + (((cb >> 3) ^ swz_v(kb1)) * 8) + (cb & 7);
        i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4)p0);
        i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4)p1);
        i16x8 w = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        vf[db][st] = __builtin_bit_cast(bf16x8, w);
      }
#pragma unroll
    for (int db = 0; db < 2; db++)
#pragma unroll
      for (int st = 0; st < 2; st++)
        o[qb][db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[db][st], pf[st], o[qb][db], 0, 0, 0);
  }
}

// One 64-key block: its two 32-key halves in key order.
template <int NQB, bool MASK>
__device__ __forceinline__ void attend_block(const bf16_t* sk, const bf16_t* sv, const bf16x8 (&qf)[NQB][4],
                                             f32x16 (&o)[NQB][2], float (&m)[NQB], float (&l)[NQB],
                                             const int (&lim)[NQB], float c, int lane) {
  attend_half<NQB, MASK>(sk, sv, qf, o, m, l, lim, c, lane, 0);
  attend_half<NQB, MASK>(sk, sv, qf, o, m, l, lim, c, lane, 1);
}

// Launch bounds of two workgroups per CU: with 8 waves (the default shape)
// that is four waves per SIMD, 128 registers, and the waves of the two
// workgroups, which pass their barriers independently, overlap one's
// exponentials with the other's MFMAs.
template <int NW, int NQB>
__global__ void __launch_bounds__(NW * 64, 2) attention_fwd_d64(AttnArgs p) {
  constexpr int QW = 32 * NQB, QPB = NW * QW, CP = 8 / NW;  // copies per wave and tile
  static_assert(CP * NW == 8 && QPB == 256, "a tile is 8 copies of 1 KiB; 256 queries per workgroup");
  __shared__ __attribute__((aligned(16))) bf16_t lds[2][2][TILE];  // [stage][K,V][64 x 64]
  const int tid = threadIdx.x, lane = tid & 63, wave = uniform32(tid >> 6);
  const int T = (int)p.time;
  const int blocks_q = (T + QPB - 1) / QPB;
  // every query block of one (batch, head) on one XCD (they share K and V in
  // its L2); within a head the longest (causal) query blocks start first
  // non-causal: every query block of one (batch, head) on one XCD (they
  // share K and V in its L2).  causal: block i takes work rank i / heads, so
  // the longest query blocks of every head are dispatched first (longest
  // first scheduling over the CUs) while block i still lands on XCD i % 8,
  // i.e. one head's blocks share an XCD when 8 divides batch * heads.
  int bh, qblk;
  if (p.causal) {
    const int nbh = (int)(p.batch * p.heads);
    bh = uniform32((int)blockIdx.x % nbh);
    qblk = uniform32(blocks_q - 1 - (int)blockIdx.x / nbh);
  } else {
    const int pid = uniform32(xcd_remap(blockIdx.x, gridDim.x));
    bh = uniform32(pid / blocks_q);
    qblk = uniform32(pid % blocks_q);
  }
  const int wg_q0 = qblk * QPB;
  const int q0 = uniform32(wg_q0 + wave * QW);
  const int b = bh / (int)p.heads, h = bh % (int)p.heads;
  const int kvh = h / (int)(p.heads / p.kv_heads);
  const bf16_t* Q = uniform_ptr(p.q + b * p.qb + h * p.qh);
  const bf16_t* K = uniform_ptr(p.k + b * p.kb + kvh * p.kh);
  const bf16_t* V = uniform_ptr(p.v + b * p.kb + kvh * p.kh);
  const int half = lane >> 5, col = lane & 31;

  // ---- Q fragments (B operand of S^T = K Q^T): lane holds query col of its
  // block, d = 16 s + 8 half + [0, 8).
  bf16x8 qf[NQB][4];
  {
    auto rq = rsrc(Q, ((int64_t)T - 1) * p.qt * 2 + D * 2);
#pragma unroll
    for (int qb = 0; qb < NQB; qb++) {
      const int t = q0 + qb * 32 + col;
#pragma unroll
      for (int s = 0; s < 4; s++) {
        uint32_t off = (uint32_t)((t * p.qt + 16 * s + 8 * half) * 2) + ((uint32_t)(t >= T) << 31);
        qf[qb][s] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rq, off, 0, 0));
      }
    }
  }

  // ---- K/V stage copies: 512 chunks of 16 bytes each; wave w, instruction
  // j fills physical chunks (j * 4 + w) * 64 + lane of K, then of V.  Rows
  // past T read as zeros (offset >= 2^31 is out of the descriptor's range).
  uint32_t ko[CP], vo[CP];
  int kr[CP];
#pragma unroll
  for (int j = 0; j < CP; j++) {
    int qidx = (j * NW + wave) * 64 + lane;
    int r = qidx >> 3, pc = qidx & 7;
    kr[j] = r;
    ko[j] = (uint32_t)((r * p.kt + ((pc ^ swz_row8(r)) * 8)) * 2);
    vo[j] = (uint32_t)((r * p.kt + ((pc ^ swz_v(r)) * 8)) * 2);
  }
  const int nkb = p.causal ? min((wg_q0 + QPB + KB - 1) / KB, (T + KB - 1) / KB) : (T + KB - 1) / KB;
  auto issue = [&](int stage, int kv0) {
    const u32x4 rk = lds_rsrc(K + (int64_t)kv0 * p.kt, (int64_t)KB * p.kt * 2);
    const u32x4 rv = lds_rsrc(V + (int64_t)kv0 * p.kt, (int64_t)KB * p.kt * 2);
#pragma unroll
    for (int j = 0; j < CP; j++) {
      uint32_t oob = (uint32_t)(kv0 + kr[j] >= T) << 31;
      char* dk = reinterpret_cast<char*>(&lds[stage][0][0]) + (j * NW + wave) * 1024;
      char* dv = reinterpret_cast<char*>(&lds[stage][1][0]) + (j * NW + wave) * 1024;
      lds_load16(rk, dk, ko[j] + oob);
      lds_load16(rv, dv, vo[j] + oob);
    }
  };

  f32x16 o[NQB][2];  // O^T blocks: d block db (rows d = 32 db + ...), columns = queries
  float m[NQB], l[NQB];
#pragma unroll
  for (int qb = 0; qb < NQB; qb++) {
    m[qb] = -INFINITY;
    l[qb] = 0.f;
#pragma unroll
    for (int db = 0; db < 2; db++) o[qb][db] = f32x16{};
  }

  // The key blocks of this wave in three uniform phases, each a loop with a
  // straight-line body (a per-block choice between masked, unmasked and
  // skipped blocks makes the compiler copy all of O at every block): blocks
  // with every key visible (all keys < T and, causal, <= the wave's first
  // query), blocks that need the mask, and (causal) blocks after every query
  // of the wave.  Every wave still passes the same nkb barriers.
  const int last_key_full = p.causal ? min(T, q0 + 1) : T;
  const int nkb_w = p.causal ? min(nkb, (q0 + QW + KB - 1) / KB) : nkb;
  const int n_full = min(nkb_w, last_key_full / KB);
  // wait for block kbk's stage, then start block kbk+1's copies
  auto advance = [&](int kbk) {
    wait_vmcnt<0>();
    asm volatile("s_barrier" ::: "memory");  // stage kbk&1 landed; the other stage is free
    if (kbk + 1 < nkb) issue((kbk & 1) ^ 1, (kbk + 1) * KB);
  };
  if (nkb > 0) issue(0, 0);
  int kbk = 0;
  for (; kbk < n_full; kbk++) {
    advance(kbk);
    const int lim[NQB] = {};
    attend_block<NQB, false>(&lds[kbk & 1][0][0], &lds[kbk & 1][1][0], qf, o, m, l, lim, p.scale_log2, lane);
  }
  for (; kbk < nkb_w; kbk++) {
    advance(kbk);
    const int kv0 = kbk * KB;
    int lim[NQB];
#pragma unroll
    for (int qb = 0; qb < NQB; qb++) {
      const int tq = q0 + qb * 32 + col;
      lim[qb] = min(T - kv0, p.causal ? tq - kv0 + 1 : KB) - 4 * half;
    }
    attend_block<NQB, true>(&lds[kbk & 1][0][0], &lds[kbk & 1][1][0], qf, o, m, l, lim, p.scale_log2, lane);
  }
  for (; kbk < nkb; kbk++) advance(kbk);

  // ---- normalise and store: lane holds query col, d = 32 db + 8 (e/4) + 4 half + e%4
#pragma unroll
  for (int qb = 0; qb < NQB; qb++) {
    const int t = q0 + qb * 32 + col;
    const float total = pair_sum(l[qb]);
    const float inv = total > 0.f ? 1.f / total : 0.f;
    if (t < T) {
      bf16_t* out = p.o + b * p.qb + h * p.qh + t * p.qt;
#pragma unroll
      for (int db = 0; db < 2; db++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
          uint2 w;
          w.x = pack_bf16x2(o[qb][db][4 * g] * inv, o[qb][db][4 * g + 1] * inv);
          w.y = pack_bf16x2(o[qb][db][4 * g + 2] * inv, o[qb][db][4 * g + 3] * inv);
          *reinterpret_cast<uint2*>(out + 32 * db + 8 * g + 4 * half) = w;
        }
      if (p.lse && half == 0) p.lse[b * p.lb + h * p.lh + t * p.lt] = (m[qb] + __log2f(total)) * 0.6931471805599453f;
    }
  }
}


// ============================================================================
// Backward (cuda_lm.attention_backward, src/qutai/backends/cuda_lm.py:278-365;
// kernels lm_attention_bf16_dq / _dkv, src/qutai/backends/cuda/lm.cu:159-285;
// oracle cpu_lm.attention_backward, cpu_lm.py:176-201):
//   P = exp(scale Q K^T - lse),  delta = rowsum(dO * O),
//   dS = P (dO V^T - delta) scale,  dQ = dS K,  dK = dS^T Q,  dV = P^T dO.
// Two kernels, each owning its outputs (no atomics, bit-repeatable):
//   * dq: a workgroup owns 256 queries of one (batch, head), streams K and V
//     like the forward and also writes delta (it has dO and O of its queries
//     in registers);
//   * dkv: a workgroup owns 256 keys of one (batch, kv head), streams Q, dO,
//     lse and delta of every query block and every head of the group, and
//     sums the group's contributions in registers.
// P and dS enter the MFMAs rounded to bf16 (the reference's d64 kernels do
// the same); all sums are fp32.
// ============================================================================

struct AttnBwdArgs {
  const bf16_t* g;  // dO
  const bf16_t* q;
  const bf16_t* k;
  const bf16_t* v;
  const bf16_t* o;
  const float* lse;
  float* delta;
  bf16_t* dq;
  bf16_t* dk;
  bf16_t* dv;
  int64_t batch, heads, kv_heads, time;
  int64_t qb, qh, qt, kb, kh, kt, lb, lh, lt;
  float c;  // scale * log2(e)
  float scale;
  int causal;
  // split > 0: each dK/dV workgroup takes one query head of its kv head's
  // group and writes unscaled fp32 partials to part_k / part_v + g *
  // part_stride (dk's element offsets); dkv_reduce sums them over g
  int split;
  float* part_k;
  float* part_v;
  int64_t part_stride;
};

constexpr float LOG2E = 1.4426950408889634f;

// Row-fragment of a [64][64] LDS tile whose 16-byte chunks are swizzled by
// swz_row8: row r, d = 16 s + 8 half + [0, 8) (A operand with k = d, or B
// operand with n = r).
__device__ __forceinline__ bf16x8 row_frag(const bf16_t* x, int r, int s, int half) {
  const int ch = 2 * s + half;
  return *reinterpret_cast<const bf16x8*>(x + r * D + ((ch ^ swz_row8(r)) * 8));
}

// Transposed fragment of the same tile: A operand whose rows are the tile's
// columns 32 db + [0, 32) and whose k index runs over the tile rows
// rb + {4 half + [0, 4), 8 + 4 half + [0, 4)} (the row order of an MFMA
// result's element index), read with ds_read_b64_tr_b16.
__device__ __forceinline__ bf16x8 tr_frag(const bf16_t* x, int db, int rb, int lane) {
  const int g = lane >> 4, i = lane & 15;
  const int cb = 32 * db + (g & 1) * 16 + 4 * (i & 3);
  const int r0 = rb + 4 * (g >> 1) + (i >> 2), r1 = r0 + 8;
  const bf16_t* p0 = x + r0 * D + (((cb >> 3) ^ swz_row8(r0)) * 8) + (cb & 7);
  const bf16_t* p1 = x + r1 * D + (((cb >> 3) ^ swz_row8(r1)) * 8) + (cb & 7);
  i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4)p0);
  i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4)p1);
  i16x8 w = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(bf16x8, w);
}

// Stage copy of a [64][64] bf16 tile (rows `stride` elements apart, rows >= rows_left read as zeros)
// by NW waves: 8 / NW 16-byte chunks per lane, physical chunk (j * NW + wave) * 64 + lane.
template <int NW>
__device__ __forceinline__ void copy_tile(bf16_t* dst, const bf16_t* src, int64_t stride, int rows_left, int wave,
                                          int lane) {
  static_assert(8 % NW == 0, "a tile is 8 copies of 1 KiB");
  const u32x4 r = lds_rsrc(src, (int64_t)KB * stride * 2);
#pragma unroll
  for (int j = 0; j < 8 / NW; j++) {
    const int qidx = (j * NW + wave) * 64 + lane;
    const int row = qidx >> 3, pc = qidx & 7;
    const uint32_t off = (uint32_t)((row * stride + ((pc ^ swz_row8(row)) * 8)) * 2) + ((uint32_t)(row >= rows_left) << 31);
    char* d = reinterpret_cast<char*>(dst) + (j * NW + wave) * 1024;
    lds_load16(r, d, off);
  }
}

// One 64-key block for the wave's NQB query blocks, as two 32-key halves
// in a loop that is not unrolled (so the second half's fragment reads are
// not hoisted over the first half's products): 127 registers, four waves
// per SIMD with two 8-wave workgroups per CU.  Every dQ accumulator still
// takes its products in the order (half 0: k-steps 0, 1), (half 1: 0, 1).
template <int NQB, bool MASK>
__device__ __forceinline__ void dq_block(const bf16_t* sk, const bf16_t* sv, const bf16x8 (&qf)[NQB][4],
                                         const bf16x8 (&gf)[NQB][4], const float (&lse2)[NQB], const float (&dl)[NQB],
                                         f32x16 (&dqt)[NQB][2], const int (&lim)[NQB], float c, float scale, int lane) {
  const int half = lane >> 5, col = lane & 31;
#pragma unroll 1
  for (int mb = 0; mb < 2; mb++) {
#pragma unroll
    for (int qb = 0; qb < NQB; qb++) {
      f32x16 st_ = {}, dp = {};
#pragma unroll
      for (int s = 0; s < 4; s++) {
        const bf16x8 kf = row_frag(sk, 32 * mb + col, s, half), vf = row_frag(sv, 32 * mb + col, s, half);
        st_ = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[qb][s], st_, 0, 0, 0);
        dp = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, gf[qb][s], dp, 0, 0, 0);
      }
      bf16x8 dsf[2];
      {
        float ds[16];
#pragma unroll
        for (int e = 0; e < 16; e++) {
          float x = st_[e];
          if (MASK && 32 * mb + 8 * (e >> 2) + (e & 3) >= lim[qb]) x = -INFINITY;
          const float pr = __builtin_amdgcn_exp2f(__builtin_fmaf(x, c, -lse2[qb]));
          ds[e] = pr * (dp[e] - dl[qb]);  // the softmax scale multiplies dQ once, at the end
        }
#pragma unroll
        for (int st = 0; st < 2; st++) {
          u32x4 w = {pack_bf16x2(ds[8 * st], ds[8 * st + 1]), pack_bf16x2(ds[8 * st + 2], ds[8 * st + 3]),
                     pack_bf16x2(ds[8 * st + 4], ds[8 * st + 5]), pack_bf16x2(ds[8 * st + 6], ds[8 * st + 7])};
          dsf[st] = __builtin_bit_cast(bf16x8, w);
        }
      }
      // dQ^T += K^T dS^T with the K^T fragments (transpose reads) of this half
#pragma unroll
      for (int db = 0; db < 2; db++)
#pragma unroll
        for (int st = 0; st < 2; st++)
          dqt[qb][db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(tr_frag(sk, db, 32 * mb + 16 * st, lane), dsf[st],
                                                                dqt[qb][db], 0, 0, 0);
    }
  }
}

template <int NW, int NQB>
__global__ void __launch_bounds__(NW * 64, 2) attention_bwd_dq_d64(AttnBwdArgs p) {
  constexpr int QW = 32 * NQB, QPB = NW * QW, CP = 8 / NW;
  static_assert(CP * NW == 8 && QPB == 256, "a tile is 8 copies of 1 KiB; 256 queries per workgroup");
  __shared__ __attribute__((aligned(16))) bf16_t lds[2][2][TILE];  // [stage][K,V][64 x 64]
  const int tid = threadIdx.x, lane = tid & 63, wave = uniform32(tid >> 6);
  const int T = (int)p.time;
  const int blocks_q = (T + QPB - 1) / QPB;
  // non-causal: every query block of one (batch, head) on one XCD (they
  // share K and V in its L2).  causal: block i takes work rank i / heads, so
  // the longest query blocks of every head are dispatched first (longest
  // first scheduling over the CUs) while block i still lands on XCD i % 8,
  // i.e. one head's blocks share an XCD when 8 divides batch * heads.
  int bh, qblk;
  if (p.causal) {
    const int nbh = (int)(p.batch * p.heads);
    bh = uniform32((int)blockIdx.x % nbh);
    qblk = uniform32(blocks_q - 1 - (int)blockIdx.x / nbh);
  } else {
    const int pid = uniform32(xcd_remap(blockIdx.x, gridDim.x));
    bh = uniform32(pid / blocks_q);
    qblk = uniform32(pid % blocks_q);
  }
  const int wg_q0 = qblk * QPB;
  const int q0 = uniform32(wg_q0 + wave * QW);
  const int b = bh / (int)p.heads, h = bh % (int)p.heads;
  const int kvh = h / (int)(p.heads / p.kv_heads);
  const int64_t qbase = b * p.qb + h * p.qh;
  const bf16_t* K = uniform_ptr(p.k + b * p.kb + kvh * p.kh);
  const bf16_t* V = uniform_ptr(p.v + b * p.kb + kvh * p.kh);
  const int half = lane >> 5, col = lane & 31;

  // Q and dO fragments (B operands: lane = query, d = 16 s + 8 half + [0, 8)),
  // delta = dO . O of the lane's query (halves summed across lanes l, l ^ 32)
  bf16x8 qf[NQB][4], gf[NQB][4];
  float lse2[NQB], dl[NQB];
  {
    const int64_t bytes = ((int64_t)T - 1) * p.qt * 2 + D * 2;
    auto rq = rsrc(p.q + qbase, bytes), rg = rsrc(p.g + qbase, bytes), ro = rsrc(p.o + qbase, bytes);
#pragma unroll
    for (int qb = 0; qb < NQB; qb++) {
      const int t = q0 + qb * 32 + col;
      float dot = 0.f;
#pragma unroll
      for (int s = 0; s < 4; s++) {
        uint32_t off = (uint32_t)((t * p.qt + 16 * s + 8 * half) * 2) + ((uint32_t)(t >= T) << 31);
        qf[qb][s] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rq, off, 0, 0));
        gf[qb][s] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rg, off, 0, 0));
        u32x4 ow = __builtin_amdgcn_raw_buffer_load_b128(ro, off, 0, 0);
        u32x4 gw = __builtin_bit_cast(u32x4, gf[qb][s]);
#pragma unroll
        for (int e = 0; e < 4; e++) {
          dot += __uint_as_float(gw[e] << 16) * __uint_as_float(ow[e] << 16);
          dot += __uint_as_float(gw[e] & 0xffff0000u) * __uint_as_float(ow[e] & 0xffff0000u);
        }
      }
      dl[qb] = pair_sum(dot);
      const int64_t li = b * p.lb + h * p.lh + (int64_t)t * p.lt;
      lse2[qb] = t < T ? p.lse[li] * LOG2E : 0.f;
      if (t < T && half == 0) p.delta[li] = dl[qb];
    }
  }

  uint32_t ko[CP];
  int kr[CP];
#pragma unroll
  for (int j = 0; j < CP; j++) {
    int qidx = (j * NW + wave) * 64 + lane;
    int r = qidx >> 3, pc = qidx & 7;
    kr[j] = r;
    ko[j] = (uint32_t)((r * p.kt + ((pc ^ swz_row8(r)) * 8)) * 2);
  }
  const int nkb = p.causal ? min((wg_q0 + QPB + KB - 1) / KB, (T + KB - 1) / KB) : (T + KB - 1) / KB;
  auto issue = [&](int stage, int kv0) {
    const u32x4 rk = lds_rsrc(K + (int64_t)kv0 * p.kt, (int64_t)KB * p.kt * 2);
    const u32x4 rv = lds_rsrc(V + (int64_t)kv0 * p.kt, (int64_t)KB * p.kt * 2);
#pragma unroll
    for (int j = 0; j < CP; j++) {
      uint32_t oob = (uint32_t)(kv0 + kr[j] >= T) << 31;
      char* dk = reinterpret_cast<char*>(&lds[stage][0][0]) + (j * NW + wave) * 1024;
      char* dv = reinterpret_cast<char*>(&lds[stage][1][0]) + (j * NW + wave) * 1024;
      lds_load16(rk, dk, ko[j] + oob);
      lds_load16(rv, dv, ko[j] + oob);
    }
  };

  f32x16 dqt[NQB][2];
#pragma unroll
  for (int qb = 0; qb < NQB; qb++)
#pragma unroll
    for (int db = 0; db < 2; db++) dqt[qb][db] = f32x16{};

  // key blocks in three uniform phases (every key visible / masked /
  // causal: after every query of the wave), each a loop with a
  // straight-line body, as in the forward; every wave passes nkb barriers
  const int last_key_full = p.causal ? min(T, q0 + 1) : T;
  const int nkb_w = p.causal ? min(nkb, (q0 + QW + KB - 1) / KB) : nkb;
  const int n_full = min(nkb_w, last_key_full / KB);
  auto advance = [&](int kbk) {
    wait_vmcnt<0>();
    asm volatile("s_barrier" ::: "memory");
    if (kbk + 1 < nkb) issue((kbk & 1) ^ 1, (kbk + 1) * KB);
  };
  if (nkb > 0) issue(0, 0);
  int kbk = 0;
  for (; kbk < n_full; kbk++) {
    advance(kbk);
    const int lim[NQB] = {};
    dq_block<NQB, false>(&lds[kbk & 1][0][0], &lds[kbk & 1][1][0], qf, gf, lse2, dl, dqt, lim, p.c, p.scale, lane);
  }
  for (; kbk < nkb_w; kbk++) {
    advance(kbk);
    const int kv0 = kbk * KB;
    int lim[NQB];
#pragma unroll
    for (int qb = 0; qb < NQB; qb++) {
      const int tq = q0 + qb * 32 + col;
      lim[qb] = min(T - kv0, p.causal ? tq - kv0 + 1 : KB) - 4 * half;
    }
    dq_block<NQB, true>(&lds[kbk & 1][0][0], &lds[kbk & 1][1][0], qf, gf, lse2, dl, dqt, lim, p.c, p.scale, lane);
  }
  for (; kbk < nkb; kbk++) advance(kbk);

#pragma unroll
  for (int qb = 0; qb < NQB; qb++) {
    const int t = q0 + qb * 32 + col;
    if (t < T) {
      bf16_t* out = p.dq + b * p.qb + h * p.qh + (int64_t)t * p.qt;
#pragma unroll
      for (int db = 0; db < 2; db++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
          uint2 w;
          const float sc = p.scale;
          w.x = pack_bf16x2(dqt[qb][db][4 * g] * sc, dqt[qb][db][4 * g + 1] * sc);
          w.y = pack_bf16x2(dqt[qb][db][4 * g + 2] * sc, dqt[qb][db][4 * g + 3] * sc);
          *reinterpret_cast<uint2*>(out + 32 * db + 8 * g + 4 * half) = w;
        }
    }
  }
}


// One 64-query block against the wave's 64 keys.  MASK: some query of the
// block is >= T or (causal) before one of the keys.
template <int NKB, bool MASK>
__device__ __forceinline__ void dkv_block(const bf16_t* sq, const bf16_t* sg, const float* slse, const float* sdl,
                                          const bf16x8 (&kf)[NKB][4], const bf16x8 (&vf)[NKB][4], f32x16 (&dvt)[2][NKB],
                                          f32x16 (&dkt)[2][NKB], int qrel_end, int key_rel, int causal, float c,
                                          float scale, int lane) {
  // qrel_end: T - (first query of the block); key_rel: (first key of the
  // wave) - (first query of the block).  Element e of a result holds query
  // 32 mq + 8 (e / 4) + 4 half + e % 4 and key 32 nb + col.
  const int half = lane >> 5, col = lane & 31;
#pragma unroll
  for (int mq = 0; mq < 2; mq++) {
    bf16x8 qa[4], ga[4];
#pragma unroll
    for (int s = 0; s < 4; s++) {
      qa[s] = row_frag(sq, 32 * mq + col, s, half);
      ga[s] = row_frag(sg, 32 * mq + col, s, half);
    }
    f32x4 l4[4], d4[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      l4[j] = *reinterpret_cast<const f32x4*>(slse + 32 * mq + 8 * j + 4 * half);
      d4[j] = *reinterpret_cast<const f32x4*>(sdl + 32 * mq + 8 * j + 4 * half);
    }
    bf16x8 pf[NKB][2], dsf[NKB][2];
#pragma unroll
    for (int nb = 0; nb < NKB; nb++) {
      f32x16 sc = {}, dp = {};
#pragma unroll
      for (int s = 0; s < 4; s++) {
        sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qa[s], kf[nb][s], sc, 0, 0, 0);
        dp = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ga[s], vf[nb][s], dp, 0, 0, 0);
      }
      float pr[16], ds[16];
#pragma unroll
      for (int e = 0; e < 16; e++) {
        float x = sc[e];
        if (MASK) {
          const int qrel = 32 * mq + 8 * (e >> 2) + 4 * half + (e & 3);
          if (qrel >= qrel_end || (causal && qrel < key_rel + 32 * nb + col)) x = -INFINITY;
        }
        // slse holds -lse * log2(e); the softmax scale multiplies dK once, at the end
        pr[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(x, c, l4[e >> 2][e & 3]));
        ds[e] = pr[e] * (dp[e] - d4[e >> 2][e & 3]);
      }
#pragma unroll
      for (int st = 0; st < 2; st++) {
        u32x4 w = {pack_bf16x2(pr[8 * st], pr[8 * st + 1]), pack_bf16x2(pr[8 * st + 2], pr[8 * st + 3]),
                   pack_bf16x2(pr[8 * st + 4], pr[8 * st + 5]), pack_bf16x2(pr[8 * st + 6], pr[8 * st + 7])};
        pf[nb][st] = __builtin_bit_cast(bf16x8, w);
        u32x4 z = {pack_bf16x2(ds[8 * st], ds[8 * st + 1]), pack_bf16x2(ds[8 * st + 2], ds[8 * st + 3]),
                   pack_bf16x2(ds[8 * st + 4], ds[8 * st + 5]), pack_bf16x2(ds[8 * st + 6], ds[8 * st + 7])};
        dsf[nb][st] = __builtin_bit_cast(bf16x8, z);
      }
    }
#pragma unroll
    for (int db = 0; db < 2; db++)
#pragma unroll
      for (int st = 0; st < 2; st++) {
        const bf16x8 got = tr_frag(sg, db, 32 * mq + 16 * st, lane);
        const bf16x8 qt = tr_frag(sq, db, 32 * mq + 16 * st, lane);
#pragma unroll
        for (int nb = 0; nb < NKB; nb++) {
          dvt[db][nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(got, pf[nb][st], dvt[db][nb], 0, 0, 0);
          dkt[db][nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qt, dsf[nb][st], dkt[db][nb], 0, 0, 0);
        }
      }
  }
}

template <int NW, int NKB>
__global__ void __launch_bounds__(NW * 64) attention_bwd_dkv_d64(AttnBwdArgs p) {
  constexpr int KW = 32 * NKB, KPB = NW * KW;  // keys per wave / per workgroup
  static_assert(8 % NW == 0 && KPB == 256, "copy split; 256 keys per workgroup");
  __shared__ __attribute__((aligned(16))) bf16_t tiles[2][2][TILE];  // [stage][Q, dO][64 x 64]
  __shared__ __attribute__((aligned(16))) float stats[2][2][KB];      // [stage][lse, delta][64]
  const int tid = threadIdx.x, lane = tid & 63, wave = uniform32(tid >> 6);
  const int T = (int)p.time;
  const int blocks_k = (T + KPB - 1) / KPB;
  // key blocks of one (batch, kv head) on one XCD; the first key blocks see
  // the most queries (causal) and start first
  // as in the forward: causal key blocks in work order (the first keys see
  // the most queries), non-causal ones grouped per XCD
  const int group = (int)(p.heads / p.kv_heads);
  const int nsplit = p.split ? group : 1;  // workgroups per (batch, kv head, key block)
  int bkh, kblk, gsel;
  if (p.causal) {
    const int nbh = (int)(p.batch * p.kv_heads) * nsplit;
    const int id = (int)blockIdx.x % nbh;
    bkh = uniform32(id / nsplit);
    gsel = uniform32(id % nsplit);
    kblk = uniform32((int)blockIdx.x / nbh);
  } else {
    const int pid = uniform32(xcd_remap(blockIdx.x, gridDim.x));
    const int rest = pid % (blocks_k * nsplit);
    bkh = uniform32(pid / (blocks_k * nsplit));
    kblk = uniform32(rest / nsplit);
    gsel = uniform32(rest % nsplit);
  }
  // query heads of the group this workgroup sums over
  const int g_lo = p.split ? gsel : 0, g_hi = p.split ? gsel + 1 : group;
  const int k0 = uniform32(kblk * KPB);
  const int kw = uniform32(k0 + wave * KW);
  const int b = bkh / (int)p.kv_heads, kvh = bkh % (int)p.kv_heads;
  const int half = lane >> 5, col = lane & 31;
  const int64_t kbase = b * p.kb + kvh * p.kh;

  // K and V of the wave's keys (B operands: lane = key 32 nb + col, d = 16 s + 8 half + [0, 8))
  bf16x8 kf[NKB][4], vf[NKB][4];
  {
    const int64_t bytes = ((int64_t)T - 1) * p.kt * 2 + D * 2;
    auto rk = rsrc(p.k + kbase, bytes), rv = rsrc(p.v + kbase, bytes);
#pragma unroll
    for (int nb = 0; nb < NKB; nb++) {
      const int key = kw + 32 * nb + col;
#pragma unroll
      for (int s = 0; s < 4; s++) {
        uint32_t off = (uint32_t)((key * p.kt + 16 * s + 8 * half) * 2) + ((uint32_t)(key >= T) << 31);
        kf[nb][s] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 0));
        vf[nb][s] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 0));
      }
    }
  }

  float lse_next = 0.f;                               // wave 0: lse of the block in flight
  const int qs0 = p.causal ? k0 : 0;                  // first query any key of the workgroup sees
  const int nq = qs0 < T ? (T - qs0 + KB - 1) / KB : 0;
  const int iterations = nq * (g_hi - g_lo);
  auto issue = [&](int stage, int it) {
    const int g = g_lo + it / nq, qs = qs0 + (it % nq) * KB;
    const int h = kvh * group + g;
    const int64_t base = b * p.qb + h * p.qh + (int64_t)qs * p.qt;
    copy_tile<NW>(&tiles[stage][0][0], p.q + base, p.qt, T - qs, wave, lane);
    copy_tile<NW>(&tiles[stage][1][0], p.g + base, p.qt, T - qs, wave, lane);
    const uint32_t off = (uint32_t)((int64_t)(qs + lane) * p.lt * 4) + ((uint32_t)(qs + lane >= T) << 31);
    if (wave == 0) {  // lse of the 64 queries into a register; stored scaled by stage_lse
      const auto r = rsrc(p.lse + b * p.lb + h * p.lh, ((int64_t)T - 1) * p.lt * 4 + 4);
      lse_next = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
    } else if (wave == 1) {  // delta straight into LDS
      const u32x4 r = lds_rsrc(p.delta + b * p.lb + h * p.lh, ((int64_t)T - 1) * p.lt * 4 + 4);
      lds_load4(r, &stats[stage][1][0], off);
    }
  };
  // wave 0 stores -lse * log2(e) of the block it loaded (after the wait for
  // its load, before the barrier that publishes the stage)
  auto stage_lse = [&](int stage) {
    if (wave == 0) {
      stats[stage][0][lane] = -lse_next * LOG2E;
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the store is in LDS before the barrier
    }
  };

  f32x16 dvt[2][NKB], dkt[2][NKB];
#pragma unroll
  for (int db = 0; db < 2; db++)
#pragma unroll
    for (int nb = 0; nb < NKB; nb++) dvt[db][nb] = dkt[db][nb] = f32x16{};

  // Per head, the query blocks come in four uniform phases, each a loop with
  // a straight-line body (a per-block choice makes the compiler copy dK and
  // dV at every block): blocks whose every query is before every key of the
  // wave (causal; skipped), masked blocks, blocks with every pair visible,
  // and masked blocks at the end of the sequence.  Every wave passes
  // `iterations` barriers.
  auto advance = [&](int it) {
    wait_vmcnt<0>();
    stage_lse(it & 1);
    asm volatile("s_barrier" ::: "memory");
    if (it + 1 < iterations) issue((it & 1) ^ 1, it + 1);
  };
  auto clampq = [&](int x, int lo) { return x < lo ? lo : x > nq ? nq : x; };
  // qs = qs0 + qi KB.  skipped: qs + KB - 1 < kw;  full: qs >= kw + KW - 1
  // (causal) and qs + KB <= T
  const int a = p.causal ? clampq((kw - qs0) / KB, 0) : 0;
  const int bq = p.causal ? clampq((kw + KW - 1 - qs0 + KB - 1) / KB, a) : a;
  const int cq = clampq((T - qs0) / KB, bq);
  auto masked = [&](int it, int qi) {
    const int qs = qs0 + qi * KB;
    dkv_block<NKB, true>(&tiles[it & 1][0][0], &tiles[it & 1][1][0], &stats[it & 1][0][0], &stats[it & 1][1][0], kf,
                         vf, dvt, dkt, T - qs, kw - qs, p.causal, p.c, p.scale, lane);
  };
  if (iterations > 0) issue(0, 0);
  int it = 0;
  for (int g = g_lo; g < g_hi; g++) {
    int qi = 0;
    for (; qi < a; qi++, it++) advance(it);
    for (; qi < bq; qi++, it++) {
      advance(it);
      masked(it, qi);
    }
    for (; qi < cq; qi++, it++) {
      advance(it);
      const int qs = qs0 + qi * KB;
      dkv_block<NKB, false>(&tiles[it & 1][0][0], &tiles[it & 1][1][0], &stats[it & 1][0][0], &stats[it & 1][1][0], kf,
                            vf, dvt, dkt, T - qs, kw - qs, p.causal, p.c, p.scale, lane);
    }
    for (; qi < nq; qi++, it++) {
      advance(it);
      masked(it, qi);
    }
  }

  // dK^T / dV^T: lane = key 32 nb + col, rows d = 32 db + 8 (e / 4) + 4 half + e % 4
  if (p.split) {
#pragma unroll
    for (int nb = 0; nb < NKB; nb++) {
      const int key = kw + 32 * nb + col;
      if (key < T) {
        const int64_t at = gsel * p.part_stride + kbase + (int64_t)key * p.kt;
#pragma unroll
        for (int db = 0; db < 2; db++)
#pragma unroll
          for (int g = 0; g < 4; g++) {
            const int d = 32 * db + 8 * g + 4 * half;
            global_store(p.part_k + at + d, f32x4{dkt[db][nb][4 * g], dkt[db][nb][4 * g + 1], dkt[db][nb][4 * g + 2],
                                                  dkt[db][nb][4 * g + 3]});
            global_store(p.part_v + at + d, f32x4{dvt[db][nb][4 * g], dvt[db][nb][4 * g + 1], dvt[db][nb][4 * g + 2],
                                                  dvt[db][nb][4 * g + 3]});
          }
      }
    }
    return;
  }
#pragma unroll
  for (int nb = 0; nb < NKB; nb++) {
    const int key = kw + 32 * nb + col;
    if (key < T) {
      bf16_t* ok = p.dk + kbase + (int64_t)key * p.kt;
      bf16_t* ov = p.dv + kbase + (int64_t)key * p.kt;
#pragma unroll
      for (int db = 0; db < 2; db++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
          uint2 wk, wv;
          const float sc = p.scale;
          wk.x = pack_bf16x2(dkt[db][nb][4 * g] * sc, dkt[db][nb][4 * g + 1] * sc);
          wk.y = pack_bf16x2(dkt[db][nb][4 * g + 2] * sc, dkt[db][nb][4 * g + 3] * sc);
          wv.x = pack_bf16x2(dvt[db][nb][4 * g], dvt[db][nb][4 * g + 1]);
          wv.y = pack_bf16x2(dvt[db][nb][4 * g + 2], dvt[db][nb][4 * g + 3]);
          *reinterpret_cast<uint2*>(ok + 32 * db + 8 * g + 4 * half) = wk;
          *reinterpret_cast<uint2*>(ov + 32 * db + 8 * g + 4 * half) = wv;
        }
    }
  }
}


// dK = scale * sum_g part_k[g], dV = sum_g part_v[g] (g in order), one
// rounding to bf16; 4 elements per lane and step.
__global__ void dkv_reduce(const float* pk, const float* pv, bf16_t* dk, bf16_t* dv, int64_t n4, int64_t stride,
                           int group, float scale) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (int64_t)gridDim.x * blockDim.x) {
    f32x4 sk = global_load<f32x4>(pk + 4 * i), sv = global_load<f32x4>(pv + 4 * i);
    for (int g = 1; g < group; g++) {
      sk += global_load<f32x4>(pk + g * stride + 4 * i);
      sv += global_load<f32x4>(pv + g * stride + 4 * i);
    }
    sk *= scale;
    global_store(dk + 4 * i, u32x2{pack_bf16x2(sk[0], sk[1]), pack_bf16x2(sk[2], sk[3])});
    global_store(dv + 4 * i, u32x2{pack_bf16x2(sv[0], sv[1]), pack_bf16x2(sv[2], sv[3])});
  }
}

// ============================================================================
// Generic path: any head dimension up to 256, fp32 or bf16 storage, fp32
// math (the reference's warp kernels lm_attention / lm_attention_delta /
// lm_attention_backward_q / _kv, src/qutai/backends/cuda/lm.cu:65-87 and
// :289-343, used by cuda_lm for everything but bf16 with D = 64).  One wave
// per query row (forward, dq) or key row (dk, dv); lane l owns dimensions
// l, l + 64, l + 128, l + 192; dot products are wave-wide sums.
// ============================================================================

struct AttnGenArgs {
  const void* g;
  const void* q;
  const void* k;
  const void* v;
  const void* o;
  float* lse;
  float* delta;
  void* dq;  // forward: the output
  void* dk;
  void* dv;
  int64_t batch, heads, kv_heads, time, dim;
  int64_t qb, qh, qt, kb, kh, kt, lb, lh, lt;
  float scale;
  int causal;
};

template <class T> __device__ __forceinline__ float ld(const void* p, int64_t i);
template <> __device__ __forceinline__ float ld<float>(const void* p, int64_t i) { return ((const float*)p)[i]; }
template <> __device__ __forceinline__ float ld<bf16_t>(const void* p, int64_t i) {
  return bf16_to_f32(((const bf16_t*)p)[i]);
}
template <class T> __device__ __forceinline__ void st(void* p, int64_t i, float x);
template <> __device__ __forceinline__ void st<float>(void* p, int64_t i, float x) { ((float*)p)[i] = x; }
template <> __device__ __forceinline__ void st<bf16_t>(void* p, int64_t i, float x) {
  ((bf16_t*)p)[i] = f32_to_bf16(x);
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int off = 32; off; off >>= 1) x += __shfl_xor(x, off);
  return x;
}

constexpr int GEN_WAVES = 4;  // rows per workgroup

// row -> (b, h, t) and its element offset in a q-shaped array
__device__ __forceinline__ void gen_row(const AttnGenArgs& p, int64_t row, int64_t heads, int64_t& b, int64_t& h,
                                        int64_t& t) {
  t = row % p.time;
  h = (row / p.time) % heads;
  b = row / (p.time * heads);
}

template <class T>
__global__ void __launch_bounds__(GEN_WAVES * 64) attention_fwd_rows(AttnGenArgs p) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * GEN_WAVES + (threadIdx.x >> 6);
  if (row >= p.batch * p.heads * p.time) return;  // whole wave
  int64_t b, h, t;
  gen_row(p, row, p.heads, b, h, t);
  const int64_t kvh = h / (p.heads / p.kv_heads);
  const int64_t qi = b * p.qb + h * p.qh + t * p.qt, kbase = b * p.kb + kvh * p.kh;
  const int D = (int)p.dim;
  float qv[4], acc[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int d = lane + 64 * j;
    qv[j] = d < D ? ld<T>(p.q, qi + d) : 0.f;
    acc[j] = 0.f;
  }
  float m = -INFINITY, l = 0.f;
  const int64_t end = p.causal ? t + 1 : p.time;
  for (int64_t s = 0; s < end; s++) {
    const int64_t ki = kbase + s * p.kt;
    float dot = 0.f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int d = lane + 64 * j;
      if (d < D) dot += qv[j] * ld<T>(p.k, ki + d);
    }
    const float x = wave_sum(dot) * p.scale;
    const float m_new = fmaxf(m, x);
    const float alpha = __expf(m - m_new), pr = __expf(x - m_new);
    l = l * alpha + pr;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int d = lane + 64 * j;
      acc[j] = acc[j] * alpha + (d < D ? pr * ld<T>(p.v, ki + d) : 0.f);
    }
    m = m_new;
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int d = lane + 64 * j;
    if (d < D) st<T>(p.dq, qi + d, acc[j] * inv);
  }
  if (p.lse && lane == 0) p.lse[b * p.lb + h * p.lh + t * p.lt] = m + __logf(l);
}

template <class T>
__global__ void __launch_bounds__(GEN_WAVES * 64) attention_bwd_q_rows(AttnGenArgs p) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * GEN_WAVES + (threadIdx.x >> 6);
  if (row >= p.batch * p.heads * p.time) return;
  int64_t b, h, t;
  gen_row(p, row, p.heads, b, h, t);
  const int64_t kvh = h / (p.heads / p.kv_heads);
  const int64_t qi = b * p.qb + h * p.qh + t * p.qt, kbase = b * p.kb + kvh * p.kh;
  const int64_t li = b * p.lb + h * p.lh + t * p.lt;
  const int D = (int)p.dim;
  float qv[4], gv[4], acc[4], dl = 0.f;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int d = lane + 64 * j;
    qv[j] = d < D ? ld<T>(p.q, qi + d) : 0.f;
    gv[j] = d < D ? ld<T>(p.g, qi + d) : 0.f;
    dl += d < D ? gv[j] * ld<T>(p.o, qi + d) : 0.f;
    acc[j] = 0.f;
  }
  dl = wave_sum(dl);
  if (lane == 0) p.delta[li] = dl;
  const float lse = p.lse[li];
  const int64_t end = p.causal ? t + 1 : p.time;
  for (int64_t s = 0; s < end; s++) {
    const int64_t ki = kbase + s * p.kt;
    float dot = 0.f, dp = 0.f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int d = lane + 64 * j;
      if (d < D) {
        dot += qv[j] * ld<T>(p.k, ki + d);
        dp += gv[j] * ld<T>(p.v, ki + d);
      }
    }
    const float pr = __expf(wave_sum(dot) * p.scale - lse);
    const float ds = pr * (wave_sum(dp) - dl) * p.scale;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int d = lane + 64 * j;
      if (d < D) acc[j] += ds * ld<T>(p.k, ki + d);
    }
  }
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int d = lane + 64 * j;
    if (d < D) st<T>(p.dq, qi + d, acc[j]);
  }
}

template <class T>
__global__ void __launch_bounds__(GEN_WAVES * 64) attention_bwd_kv_rows(AttnGenArgs p) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * GEN_WAVES + (threadIdx.x >> 6);
  if (row >= p.batch * p.kv_heads * p.time) return;
  int64_t b, kvh, s;
  gen_row(p, row, p.kv_heads, b, kvh, s);
  const int64_t ki = b * p.kb + kvh * p.kh + s * p.kt;
  const int64_t group = p.heads / p.kv_heads;
  const int D = (int)p.dim;
  float kv_[4], vv[4], ak[4], av[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int d = lane + 64 * j;
    kv_[j] = d < D ? ld<T>(p.k, ki + d) : 0.f;
    vv[j] = d < D ? ld<T>(p.v, ki + d) : 0.f;
    ak[j] = av[j] = 0.f;
  }
  for (int64_t h = kvh * group; h < (kvh + 1) * group; h++) {
    for (int64_t t = p.causal ? s : 0; t < p.time; t++) {
      const int64_t qi = b * p.qb + h * p.qh + t * p.qt;
      const int64_t li = b * p.lb + h * p.lh + t * p.lt;
      float dot = 0.f, dp = 0.f;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int d = lane + 64 * j;
        if (d < D) {
          dot += ld<T>(p.q, qi + d) * kv_[j];
          dp += ld<T>(p.g, qi + d) * vv[j];
        }
      }
      const float pr = __expf(wave_sum(dot) * p.scale - p.lse[li]);
      const float ds = pr * (wave_sum(dp) - p.delta[li]) * p.scale;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int d = lane + 64 * j;
        if (d < D) {
          ak[j] += ds * ld<T>(p.q, qi + d);
          av[j] += pr * ld<T>(p.g, qi + d);
        }
      }
    }
  }
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int d = lane + 64 * j;
    if (d < D) {
      st<T>(p.dk, ki + d, ak[j]);
      st<T>(p.dv, ki + d, av[j]);
    }
  }
}

}  // namespace

extern "C" {

}  // extern "C"

namespace {

// element strides of (batch, head, token) for q-shaped, kv-shaped and lse arrays
template <class Args>
int set_layout(Args& a, int64_t batch, int64_t heads, int64_t kv_heads, int64_t time, int64_t dim, int layout) {
  if (batch < 0 || heads <= 0 || kv_heads <= 0 || heads % kv_heads || time < 0 || dim <= 0) return QA_EINVAL;
  if (layout != 0 && layout != 1) return QA_EINVAL;
  if (time > (1 << 30) / (heads > kv_heads ? heads : kv_heads) / dim) return QA_EINVAL;  // 32-bit element offsets
  a.batch = batch;
  a.heads = heads;
  a.kv_heads = kv_heads;
  a.time = time;
  if (layout == 0) {  // [batch][heads][time][dim]
    a.qb = heads * time * dim, a.qh = time * dim, a.qt = dim;
    a.kb = kv_heads * time * dim, a.kh = time * dim, a.kt = dim;
    a.lb = heads * time, a.lh = time, a.lt = 1;
  } else {            // [batch][time][heads][dim] (the lm layout)
    a.qb = time * heads * dim, a.qh = dim, a.qt = heads * dim;
    a.kb = time * kv_heads * dim, a.kh = dim, a.kt = kv_heads * dim;
    a.lb = time * heads, a.lh = 1, a.lt = heads;
  }
  return QA_OK;
}

// Workgroup shape of every attention kernel: 8 waves (two per SIMD, so one
// wave's softmax overlaps the other's MFMAs) of 32 queries or keys, or 4
// waves of 64; QUTAI_AMD_ATTN_WAVES=4|8 overrides the default 8 (tuning).
int attention_waves() {
  static const int waves = [] {
    const char* v = getenv("QUTAI_AMD_ATTN_WAVES");
    return v && atoi(v) == 4 ? 4 : 8;
  }();
  return waves;
}

int64_t cu_count() {
  static int cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// Workspace of the dK/dV query-head split: with grouped-query attention
// (heads > kv_heads) the kernel has one workgroup per (batch, kv head, 256
// keys), too few to fill the GPU when that count is below twice the CUs;
// then each workgroup takes one query head of the group and the group's fp32
// partials are summed by dkv_reduce.  0 when no split applies.
size_t dkv_split_bytes(int64_t batch, int64_t heads, int64_t kv_heads, int64_t time) {
  if (kv_heads <= 0 || heads <= kv_heads || heads % kv_heads) return 0;
  const int64_t blocks_k = batch * kv_heads * ((time + 255) / 256);
  if (blocks_k >= 2 * cu_count()) return 0;
  return (size_t)2 * (heads / kv_heads) * batch * time * kv_heads * D * sizeof(float);
}

bool aligned16(std::initializer_list<const void*> ptrs) {
  for (const void* ptr : ptrs)
    if (!ptr || (uintptr_t)ptr % 16) return false;
  return true;
}

}  // namespace

extern "C" {

int qutai_amd_attention_fwd(const void* q, const void* k, const void* v, void* out, float* lse, int64_t batch,
                            int64_t heads, int64_t kv_heads, int64_t time, int64_t dim, int dtype, int layout,
                            double scale, int causal, void* stream) {
  if (!(scale > 0.0) || scale > 1e30) return QA_EINVAL;  // the running max assumes a positive scale
  if (!q || !k || !v || !out) return QA_EINVAL;
  if (dtype == BF16 && dim == D) {
    AttnArgs a = {};
    if (set_layout(a, batch, heads, kv_heads, time, dim, layout) != QA_OK) return QA_EINVAL;
    if (!aligned16({q, k, v, out})) return QA_EINVAL;
    if (batch * time == 0) return QA_OK;
    a.q = (const bf16_t*)q;
    a.k = (const bf16_t*)k;
    a.v = (const bf16_t*)v;
    a.o = (bf16_t*)out;
    a.lse = lse;
    a.scale = (float)scale;
    a.scale_log2 = (float)(scale * 1.4426950408889634);
    a.causal = causal ? 1 : 0;
    const int64_t qpb = 256;  // queries per workgroup in both shapes
    int64_t blocks = batch * heads * ((time + qpb - 1) / qpb);
    if (blocks > 0x7fffffff) return QA_EINVAL;
    if (attention_waves() == 8)
      hipLaunchKernelGGL((attention_fwd_d64<8, 1>), dim3((unsigned)blocks), dim3(512), 0, (hipStream_t)stream, a);
    else
      hipLaunchKernelGGL((attention_fwd_d64<4, 2>), dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, a);
    return (int)hipGetLastError();
  }
  if ((dtype != BF16 && dtype != F32) || dim > 256) return QA_EINVAL;
  AttnGenArgs a = {};
  if (set_layout(a, batch, heads, kv_heads, time, dim, layout) != QA_OK) return QA_EINVAL;
  if (batch * time == 0) return QA_OK;
  a.q = q;
  a.k = k;
  a.v = v;
  a.dq = out;
  a.lse = lse;
  a.dim = dim;
  a.scale = (float)scale;
  a.causal = causal ? 1 : 0;
  const int64_t blocks = (batch * heads * time + GEN_WAVES - 1) / GEN_WAVES;
  if (blocks > 0x7fffffff) return QA_EINVAL;
  if (dtype == BF16)
    hipLaunchKernelGGL(attention_fwd_rows<bf16_t>, dim3((unsigned)blocks), dim3(GEN_WAVES * 64), 0,
                       (hipStream_t)stream, a);
  else
    hipLaunchKernelGGL(attention_fwd_rows<float>, dim3((unsigned)blocks), dim3(GEN_WAVES * 64), 0,
                       (hipStream_t)stream, a);
  return (int)hipGetLastError();
}

size_t qutai_amd_attention_bwd_workspace_size(int64_t batch, int64_t heads, int64_t kv_heads, int64_t time,
                                              int64_t dim, int dtype) {
  if (dtype != BF16 || dim != D || batch < 0 || time < 0) return 0;
  return dkv_split_bytes(batch, heads, kv_heads, time);
}

int qutai_amd_attention_bwd(const void* grad, const void* q, const void* k, const void* v, const void* out,
                            const float* lse, void* dq, void* dk, void* dv, float* delta, void* workspace,
                            size_t workspace_bytes, int64_t batch, int64_t heads, int64_t kv_heads, int64_t time,
                            int64_t dim, int dtype, int layout, double scale, int causal, void* stream) {
  if (!(scale > 0.0) || scale > 1e30) return QA_EINVAL;
  if (!grad || !q || !k || !v || !out || !dq || !dk || !dv || !lse || !delta) return QA_EINVAL;
  if (dtype == BF16 && dim == D) {
    AttnBwdArgs a = {};
    if (set_layout(a, batch, heads, kv_heads, time, dim, layout) != QA_OK) return QA_EINVAL;
    if (!aligned16({grad, q, k, v, out, dq, dk, dv})) return QA_EINVAL;
    if (batch * time == 0) return QA_OK;
    a.g = (const bf16_t*)grad;
    a.q = (const bf16_t*)q;
    a.k = (const bf16_t*)k;
    a.v = (const bf16_t*)v;
    a.o = (const bf16_t*)out;
    a.lse = lse;
    a.delta = delta;
    a.dq = (bf16_t*)dq;
    a.dk = (bf16_t*)dk;
    a.dv = (bf16_t*)dv;
    a.scale = (float)scale;
    a.c = (float)(scale * 1.4426950408889634);
    a.causal = causal ? 1 : 0;
    // 256 queries (dq) / 256 keys (dk, dv) per workgroup in both shapes
    const int64_t blocks_q = batch * heads * ((time + 255) / 256);
    int64_t blocks_k = batch * kv_heads * ((time + 255) / 256);
    const size_t split_bytes = dkv_split_bytes(batch, heads, kv_heads, time);
    if (split_bytes && workspace && workspace_bytes >= split_bytes && (uintptr_t)workspace % 16 == 0) {
      a.split = 1;
      a.part_stride = batch * time * kv_heads * D;
      a.part_k = (float*)workspace;
      a.part_v = a.part_k + (heads / kv_heads) * a.part_stride;
      blocks_k *= heads / kv_heads;
    }
    if (blocks_q > 0x7fffffff || blocks_k > 0x7fffffff) return QA_EINVAL;
    // dq first: it writes delta, which the dkv kernel reads
    if (attention_waves() == 8)
      hipLaunchKernelGGL((attention_bwd_dq_d64<8, 1>), dim3((unsigned)blocks_q), dim3(512), 0, (hipStream_t)stream, a);
    else
      hipLaunchKernelGGL((attention_bwd_dq_d64<4, 2>), dim3((unsigned)blocks_q), dim3(256), 0, (hipStream_t)stream, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    if (attention_waves() == 8)
      hipLaunchKernelGGL((attention_bwd_dkv_d64<8, 1>), dim3((unsigned)blocks_k), dim3(512), 0, (hipStream_t)stream,
                         a);
    else
      hipLaunchKernelGGL((attention_bwd_dkv_d64<4, 2>), dim3((unsigned)blocks_k), dim3(256), 0, (hipStream_t)stream,
                         a);
    if (!a.split) return (int)hipGetLastError();
    e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    const int64_t n4 = a.part_stride / 4;
    const unsigned blocks = (unsigned)std::min<int64_t>((n4 + 255) / 256, 1 << 20);
    hipLaunchKernelGGL(dkv_reduce, dim3(blocks), dim3(256), 0, (hipStream_t)stream, (const float*)a.part_k,
                       (const float*)a.part_v, a.dk, a.dv, n4, a.part_stride, (int)(heads / kv_heads), a.scale);
    return (int)hipGetLastError();
  }
  if ((dtype != BF16 && dtype != F32) || dim > 256) return QA_EINVAL;
  AttnGenArgs a = {};
  if (set_layout(a, batch, heads, kv_heads, time, dim, layout) != QA_OK) return QA_EINVAL;
  if (batch * time == 0) return QA_OK;
  a.g = grad;
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = out;
  a.lse = const_cast<float*>(lse);
  a.delta = delta;
  a.dq = dq;
  a.dk = dk;
  a.dv = dv;
  a.dim = dim;
  a.scale = (float)scale;
  a.causal = causal ? 1 : 0;
  const int64_t blocks_q = (batch * heads * time + GEN_WAVES - 1) / GEN_WAVES;
  const int64_t blocks_k = (batch * kv_heads * time + GEN_WAVES - 1) / GEN_WAVES;
  if (blocks_q > 0x7fffffff || blocks_k > 0x7fffffff) return QA_EINVAL;
  // the q pass writes delta, which the kv pass reads
  if (dtype == BF16)
    hipLaunchKernelGGL(attention_bwd_q_rows<bf16_t>, dim3((unsigned)blocks_q), dim3(GEN_WAVES * 64), 0,
                       (hipStream_t)stream, a);
  else
    hipLaunchKernelGGL(attention_bwd_q_rows<float>, dim3((unsigned)blocks_q), dim3(GEN_WAVES * 64), 0,
                       (hipStream_t)stream, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  if (dtype == BF16)
    hipLaunchKernelGGL(attention_bwd_kv_rows<bf16_t>, dim3((unsigned)blocks_k), dim3(GEN_WAVES * 64), 0,
                       (hipStream_t)stream, a);
  else
    hipLaunchKernelGGL(attention_bwd_kv_rows<float>, dim3((unsigned)blocks_k), dim3(GEN_WAVES * 64), 0,
                       (hipStream_t)stream, a);
  return (int)hipGetLastError();
}

}  // extern "C"
