// MoE routing, token gather and weighted combine for the grouped expert
// GEMMs (C ABI).  Reference counterparts are cited per entry point in
// include/qutai_amd.h.
#include "common.h"
#include "qutai_amd.h"

using namespace qa;

namespace {

// One thread per token: fp32 softmax of the router logits, then top-k.
// Selection compares the logits themselves: softmax is monotone, so the
// order of the logits is the order of the probabilities, and comparing the
// exact inputs keeps the chosen experts identical to a float64 softmax (the
// CPU oracle, cpu_lm.py:204-216).  A strict '>' keeps the lowest expert
// index among equal values, like the stable descending sort of the oracle.
__global__ void route_select(const float* scores, float* probs, float* weights, int64_t* indices, int64_t rows,
                             int64_t experts, int64_t top_k) {
  int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const float* s = scores + r * experts;
  float peak = -INFINITY;
  for (int64_t e = 0; e < experts; e++) peak = fmaxf(peak, s[e]);
  float total = 0.f;
  for (int64_t e = 0; e < experts; e++) total += expf(s[e] - peak);
  for (int64_t e = 0; e < experts; e++) probs[r * experts + e] = expf(s[e] - peak) / total;
  float chosen = 0.f;
  for (int64_t slot = 0; slot < top_k; slot++) {
    int64_t best = -1;
    for (int64_t e = 0; e < experts; e++) {
      bool used = false;
      for (int64_t q = 0; q < slot; q++) used |= indices[r * top_k + q] == e;
      if (!used && (best < 0 || s[e] > s[best])) best = e;
    }
    indices[r * top_k + slot] = best;
    float p = probs[r * experts + best];
    weights[r * top_k + slot] = p;
    chosen += p;
  }
  for (int64_t slot = 0; slot < top_k; slot++) weights[r * top_k + slot] /= chosen;
}

// Routing for up to 32 experts and top-8 in three launches over chunks of
// 256 tokens (one thread per token), all deterministic and without atomics:
//   route_select_small  the selection of route_select with the row in
//                       registers (same expressions, so the same bits), plus
//                       the chunk's per-expert assignment counts and
//                       probability column sums (fixed shuffle tree, waves
//                       added in order);
//   route_scan          one workgroup: per expert the exclusive prefix of the
//                       chunk counts (each chunk's first position in the
//                       expert's list), counts, offsets, utilization and the
//                       aux loss from the column sums (chunk order);
//   route_scatter       per chunk: a token's rank among the chunk's tokens
//                       routed to the same expert (one ballot per expert; a
//                       token's slots have distinct experts), so positions are
//                       stable in (token, slot) order like route_pack's.
constexpr int RCHUNK = 256;

template <int E>
__global__ void __launch_bounds__(RCHUNK) route_select_small(const float* scores, float* probs, float* weights,
                                                             int64_t* indices, int64_t rows, int experts, int top_k,
                                                             int* chunk_counts, float* chunk_cols) {
  __shared__ int hist[RCHUNK / 64][E];
  __shared__ float cols[RCHUNK / 64][E];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t r = (int64_t)blockIdx.x * RCHUNK + threadIdx.x;
  const bool valid = r < rows;
  float x[E], p[E];
#pragma unroll
  for (int e = 0; e < E; e++) {
    x[e] = valid && e < experts ? scores[r * experts + e] : -INFINITY;
    p[e] = 0.f;
  }
  uint32_t used = 0;
  if (valid) {
    float peak = -INFINITY;
#pragma unroll
    for (int e = 0; e < E; e++)
      if (e < experts) peak = fmaxf(peak, x[e]);
    float total = 0.f;
#pragma unroll
    for (int e = 0; e < E; e++)
      if (e < experts) total += expf(x[e] - peak);
#pragma unroll
    for (int e = 0; e < E; e++)
      if (e < experts) {
        p[e] = expf(x[e] - peak) / total;
        probs[r * experts + e] = p[e];
      }
    float w[8], chosen = 0.f;
    for (int slot = 0; slot < top_k; slot++) {
      int best = -1;
      float bx = 0.f, bp = 0.f;
#pragma unroll
      for (int e = 0; e < E; e++)
        if (e < experts && !((used >> e) & 1u) && (best < 0 || x[e] > bx)) {
          best = e;
          bx = x[e];
          bp = p[e];
        }
      used |= 1u << best;
      indices[r * top_k + slot] = best;
      w[slot] = bp;
      chosen += bp;
    }
    for (int slot = 0; slot < top_k; slot++) weights[r * top_k + slot] = w[slot] / chosen;
  }
  if (!chunk_counts) return;
#pragma unroll
  for (int e = 0; e < E; e++) {
    if (e >= experts) break;
    const uint64_t m = __ballot((used >> e) & 1u);
    float c = p[e];
    for (int o = 32; o > 0; o >>= 1) c += __shfl_xor(c, o);
    if (lane == 0) {
      hist[wave][e] = __popcll(m);
      cols[wave][e] = c;
    }
  }
  __syncthreads();
  if ((int)threadIdx.x < experts) {
    const int e = threadIdx.x;
    int count = 0;
    float col = 0.f;
    for (int w = 0; w < RCHUNK / 64; w++) {
      count += hist[w][e];
      col += cols[w][e];
    }
    chunk_counts[(int64_t)blockIdx.x * experts + e] = count;
    chunk_cols[(int64_t)blockIdx.x * experts + e] = col;
  }
}

__global__ void __launch_bounds__(1024) route_scan(const int* chunk_counts, const float* chunk_cols, int* chunk_base,
                                                   int64_t chunks, int experts, int64_t* counts, int64_t* offsets,
                                                   float* utilization, float* aux, int64_t rows, int64_t n) {
  __shared__ int64_t total[32];
  __shared__ float colsum[32];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int e = wave; e < experts; e += 16) {
    int64_t running = 0;
    float col = 0.f;
    for (int64_t c0 = 0; c0 < chunks; c0 += 64) {
      const int64_t c = c0 + lane;
      const int v = c < chunks ? chunk_counts[c * experts + e] : 0;
      int incl = v;
      for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(incl, o);
        if (lane >= o) incl += t;
      }
      if (c < chunks) chunk_base[c * experts + e] = (int)(running + incl - v);
      running += __shfl(incl, 63);
      float f = c < chunks ? chunk_cols[c * experts + e] : 0.f;
      for (int o = 32; o > 0; o >>= 1) f += __shfl_xor(f, o);
      col += f;
    }
    if (lane == 0) {
      total[e] = running;
      colsum[e] = col;
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int64_t start = 0;
    float sum = 0.f;
    for (int e = 0; e < experts; e++) {
      counts[e] = total[e];
      offsets[e] = start;
      start += total[e];
      const float u = (float)total[e] / (float)n;
      utilization[e] = u;
      sum += u * colsum[e];
    }
    offsets[experts] = n;
    aux[0] = (float)experts * sum / (float)rows;
  }
}

template <int E>
__global__ void __launch_bounds__(RCHUNK) route_scatter(const int64_t* indices, const int* chunk_base,
                                                        const int64_t* offsets, int64_t* ids, int64_t* slots,
                                                        int64_t* locations, int64_t* order, int64_t rows, int experts,
                                                        int top_k, int64_t n) {
  __shared__ int wcount[RCHUNK / 64][E];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t r = (int64_t)blockIdx.x * RCHUNK + threadIdx.x;
  const bool valid = r < rows;
  int idx[8];
  uint32_t used = 0;
  for (int s = 0; s < top_k; s++) {
    idx[s] = valid ? (int)indices[r * top_k + s] : 0;
    if (valid) used |= 1u << idx[s];
  }
  int rank[8];
  const uint64_t below = (1ull << lane) - 1ull;
#pragma unroll
  for (int e = 0; e < E; e++) {
    if (e >= experts) break;
    const uint64_t m = __ballot((used >> e) & 1u);
    if (lane == 0) wcount[wave][e] = __popcll(m);
    for (int s = 0; s < top_k; s++)
      if (valid && idx[s] == e) rank[s] = __popcll(m & below);
  }
  __syncthreads();
  if (!valid) return;
  for (int s = 0; s < top_k; s++) {
    const int e = idx[s];
    int pos = chunk_base[(int64_t)blockIdx.x * experts + e] + rank[s];
    for (int w = 0; w < wave; w++) pos += wcount[w][e];
    const int64_t at = r * top_k + s;
    ids[e * n + pos] = r;
    slots[e * n + pos] = s;
    locations[at] = pos;
    order[offsets[e] + pos] = r;
  }
}

// One workgroup per expert: stable compaction of the (token, slot)
// assignments routed to it, in increasing assignment order.  The 16 waves
// own contiguous segments of the assignments: one pass counts each
// segment's matches (and the assignments to lower experts, whose total is
// the expert's start in `order`), a prefix over the segment counts gives
// every wave its first position, and a second pass writes positions with a
// ballot per 64 assignments -- no barrier inside the loops.
constexpr int PACKW = 16;
__global__ void __launch_bounds__(PACKW * 64) route_pack(const int64_t* indices, int64_t* counts, int64_t* ids,
                                                         int64_t* slots, int64_t* locations, int64_t* offsets,
                                                         int64_t* order, int64_t n, int64_t top_k, int64_t experts,
                                                         const float* probs, float* column) {
  __shared__ int64_t seg_count[PACKW], seg_lower[PACKW];
  __shared__ float col_part[PACKW * 64];
  const int64_t e = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t seg = (n + PACKW - 1) / PACKW;
  const int64_t lo = min(n, wave * seg), hi = min(n, lo + seg);
  // U rounds of 64 assignments per iteration: the loads are issued together
  // (the loop is latency-bound otherwise)
  constexpr int U = 8;
  int64_t count = 0, lower = 0;
  for (int64_t start = lo; start < hi; start += 64 * U) {
    int64_t x[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int64_t at = start + u * 64 + lane;
      x[u] = at < hi ? indices[at] : experts;  // `experts`: neither e nor below it
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
      count += x[u] == e;
      lower += x[u] < e;
    }
  }
  for (int o = 32; o > 0; o >>= 1) {
    count += __shfl_xor(count, o);
    lower += __shfl_xor(lower, o);
  }
  if (lane == 0) {
    seg_count[wave] = count;
    seg_lower[wave] = lower;
  }
  __syncthreads();
  int64_t base = 0, written = 0, total = 0;
  for (int w = 0; w < PACKW; w++) {
    base += seg_lower[w];
    total += seg_count[w];
    if (w < wave) written += seg_count[w];
  }
  const uint64_t below = (1ull << lane) - 1ull;
  for (int64_t start = lo; start < hi; start += 64 * U) {
    int64_t x[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int64_t at = start + u * 64 + lane;
      x[u] = at < hi ? indices[at] : experts;
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int64_t at = start + u * 64 + lane;
      const bool sel = x[u] == e;
      const uint64_t mask = __ballot(sel);
      if (sel) {
        const int64_t pos = written + __popcll(mask & below);
        // n < 2^31 (checked by the host): 32-bit division
        const uint32_t token = (uint32_t)at / (uint32_t)top_k, slot = (uint32_t)at - token * (uint32_t)top_k;
        ids[e * n + pos] = token;
        slots[e * n + pos] = slot;
        locations[at] = pos;
        order[base + pos] = token;
      }
      written += __popcll(mask);
    }
  }
  if (tid == 0) {
    counts[e] = total;
    offsets[e] = base;
    if (e == experts - 1) offsets[experts] = n;
  }
  // the expert's probability column sum (thread t: rows t, t + 1024, ...;
  // fixed-order tree), left in column[e] for route_stats
  const int64_t rows = n / top_k;
  float part = 0.f;
  for (int64_t r0 = tid; r0 < rows; r0 += U * PACKW * 64) {
    float q[U];  // U loads in flight, summed in row order
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int64_t r = r0 + (int64_t)u * PACKW * 64;
      q[u] = r < rows ? probs[r * experts + e] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < U; u++)
      if (r0 + (int64_t)u * PACKW * 64 < rows) part += q[u];
  }
  col_part[tid] = part;
  __syncthreads();
  for (int w = PACKW * 32; w > 0; w >>= 1) {
    if (tid < w) col_part[tid] += col_part[tid + w];
    __syncthreads();
  }
  if (tid == 0) column[e] = col_part[0];
}

// utilization = count / (rows * top_k); aux = experts * sum_e util_e *
// colsum_e / rows, with colsum_e (the expert's probability column sum) left
// in `utilization` by route_pack.  One wave, lanes over the experts in a
// fixed order (deterministic result).
__global__ void __launch_bounds__(64) route_stats(const int64_t* counts, float* utilization, float* aux, int64_t rows,
                                                  int64_t experts, int64_t n) {
  const int lane = threadIdx.x;
  float total = 0.f;
  for (int64_t e = lane; e < experts; e += 64) {
    const float u = (float)counts[e] / (float)n;
    total += u * utilization[e];
    utilization[e] = u;
  }
  for (int o = 32; o > 0; o >>= 1) total += __shfl_xor(total, o);
  if (lane == 0) aux[0] = (float)experts * total / (float)rows;
}

// Row gather / scatter in 16-byte pieces.
// One wavefront per gathered row (no per-element index division), 4 pieces
// per lane in flight.
__global__ void __launch_bounds__(256) gather_rows16(const u32x4* x, const int64_t* order, u32x4* out, int64_t count,
                                                     int64_t pieces, int backward) {
  constexpr int R = 4;
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= count) return;
  const int64_t src = order[r];
  const u32x4* from = backward ? x + r * pieces : x + src * pieces;
  u32x4* to = backward ? out + src * pieces : out + r * pieces;
  for (int64_t c0 = 0; c0 < pieces; c0 += 64 * R) {
    u32x4 q[R];
#pragma unroll
    for (int i = 0; i < R; i++) {
      const int64_t c = c0 + i * 64 + lane;
      if (c < pieces) q[i] = global_load<u32x4>(from + c);
    }
#pragma unroll
    for (int i = 0; i < R; i++) {
      const int64_t c = c0 + i * 64 + lane;
      if (c < pieces) global_store(to + c, q[i]);
    }
  }
}
template <class T>
__global__ void gather_rows(const T* x, const int64_t* order, T* out, int64_t count, int64_t width, int backward) {
  int64_t total = count * width;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t r = i / width, j = i % width;
    int64_t src = order[r] * width + j;
    if (backward) out[src] = x[i];
    else out[i] = x[src];
  }
}

// y[row] = sum over slots of w * expert row, fp32 sum in slot order, one
// rounding to the output type U.
template <class T, int V, class U = T>  // V values per thread
__global__ void combine_kernel(const T* eo, const float* w, const int64_t* idx, const int64_t* loc,
                               const int64_t* off, U* y, int64_t rows, int64_t width, int64_t top_k) {
  int64_t per_row = width / V;
  int64_t total = rows * per_row;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t row = i / per_row, j = (i % per_row) * V;
    float acc[V];
#pragma unroll
    for (int v = 0; v < V; v++) acc[v] = 0.f;
    for (int64_t s = 0; s < top_k; s++) {
      int64_t at = row * top_k + s;
      float f = w ? w[at] : 1.f;
      const T* src = eo + (off[idx[at]] + loc[at]) * width + j;
      float x[V];
      if constexpr (V * sizeof(T) == 16) {  // one 16-byte load (rows and base 16-byte aligned)
        const u32x4 q = global_load<u32x4>(src);
        if constexpr (sizeof(T) == 2) {
#pragma unroll
          for (int h = 0; h < 4; h++) {
            x[2 * h] = __uint_as_float(q[h] << 16);
            x[2 * h + 1] = __uint_as_float(q[h] & 0xffff0000u);
          }
        } else {
#pragma unroll
          for (int h = 0; h < 4; h++) x[h] = __uint_as_float(q[h]);
        }
      } else {
#pragma unroll
        for (int v = 0; v < V; v++) {
          if constexpr (sizeof(T) == 2) x[v] = bf16_to_f32(src[v]);
          else x[v] = (float)src[v];
        }
      }
#pragma unroll
      for (int v = 0; v < V; v++) acc[v] += f * x[v];
    }
    U* dst = y + row * width + j;
    if constexpr (sizeof(U) == 2 && V == 8) {
      global_store(dst, u32x4{pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3]), pack_bf16x2(acc[4], acc[5]),
                              pack_bf16x2(acc[6], acc[7])});
    } else if constexpr (sizeof(U) == 2 && V == 4) {
      global_store(dst, u32x2{pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3])});
    } else {
#pragma unroll
      for (int v = 0; v < V; v++) {
        if constexpr (sizeof(U) == 2) dst[v] = f32_to_bf16(acc[v]);
        else dst[v] = acc[v];
      }
    }
  }
}

// The same combine with one wavefront per token row (16-byte chunks of
// the expert rows, 4 chunks per lane and slot in flight at once): the
// routing metadata is read once per row instead of once per chunk, and the
// row's loads overlap instead of forming one dependent chain per chunk.
// Every expert row is read once, in whole lines: streamed loads.
// Same sums in the same order as combine_kernel.
template <class T, class U>
__global__ void __launch_bounds__(256) combine_rows_wave(const T* eo, const float* w, const int64_t* idx,
                                                         const int64_t* loc, const int64_t* off, U* y, int64_t rows,
                                                         int64_t width, int64_t top_k) {
  // fp32 rows hold half the values per 16-byte chunk: twice the chunks in flight
  constexpr int V = 16 / sizeof(T), R = sizeof(T) == 4 ? 8 : 4;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t chunks = width / V;
  for (int64_t c0 = 0; c0 < chunks; c0 += 64 * R) {
    float acc[R][V];
#pragma unroll
    for (int i = 0; i < R; i++)
#pragma unroll
      for (int v = 0; v < V; v++) acc[i][v] = 0.f;
    for (int64_t s = 0; s < top_k; s++) {
      const int64_t at = row * top_k + s;
      const float f = w ? w[at] : 1.f;
      const T* src = eo + (off[idx[at]] + loc[at]) * width;
      u32x4 q[R];
#pragma unroll
      for (int i = 0; i < R; i++) {
        const int64_t c = c0 + i * 64 + lane;
        q[i] = c < chunks ? global_load_nt<u32x4>(src + c * V) : u32x4{0, 0, 0, 0};
      }
#pragma unroll
      for (int i = 0; i < R; i++) {
        float x[V];
        if constexpr (sizeof(T) == 2) {
#pragma unroll
          for (int h = 0; h < 4; h++) {
            x[2 * h] = __uint_as_float(q[i][h] << 16);
            x[2 * h + 1] = __uint_as_float(q[i][h] & 0xffff0000u);
          }
        } else {
#pragma unroll
          for (int h = 0; h < 4; h++) x[h] = __uint_as_float(q[i][h]);
        }
#pragma unroll
        for (int v = 0; v < V; v++) acc[i][v] += f * x[v];
      }
    }
#pragma unroll
    for (int i = 0; i < R; i++) {
      const int64_t c = c0 + i * 64 + lane;
      if (c >= chunks) continue;
      U* dst = y + row * width + c * V;
      if constexpr (sizeof(U) == 2 && V == 8) {
        global_store(dst, u32x4{pack_bf16x2(acc[i][0], acc[i][1]), pack_bf16x2(acc[i][2], acc[i][3]),
                                pack_bf16x2(acc[i][4], acc[i][5]), pack_bf16x2(acc[i][6], acc[i][7])});
      } else if constexpr (sizeof(U) == 2) {
        global_store(dst, u32x2{pack_bf16x2(acc[i][0], acc[i][1]), pack_bf16x2(acc[i][2], acc[i][3])});
      } else {
        global_store(dst, f32x4{acc[i][0], acc[i][1], acc[i][2], acc[i][3]});
      }
    }
  }
}

// Backward of the weighted combine for every routed (token, slot) pair at
// (rows*top_k pairs, one wave each; cpu_lm.combine_backward,
// src/qutai/backends/cpu_lm.py:306-320): the pair's expert-major row
// pos = offsets[e] + loc gets d_eo[pos] = dy[row] * w[at], and
// dw[at] = dy[row] . eo[pos] (fp32 sum over the width).
template <class T>
__global__ void __launch_bounds__(256) combine_backward_kernel(const T* dy, const T* eo, const float* w,
                                                               const int64_t* idx, const int64_t* loc,
                                                               const int64_t* off, T* deo, float* dw,
                                                               int64_t pairs, int64_t width, int64_t top_k) {
  const int lane = threadIdx.x & 63;
  const int64_t at = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (at >= pairs) return;  // whole wave
  const int64_t row = at / top_k, pos = off[idx[at]] + loc[at];
  const float f = w[at];
  const T* g = dy + row * width;
  const T* x = eo + pos * width;
  T* d = deo + pos * width;
  float dot = 0.f;
  for (int64_t j = lane; j < width; j += 64) {
    float gv, xv;
    if constexpr (sizeof(T) == 2) {
      gv = bf16_to_f32(g[j]);
      xv = bf16_to_f32(x[j]);
      d[j] = f32_to_bf16(gv * f);
    } else {
      gv = (float)g[j];
      xv = (float)x[j];
      d[j] = gv * f;
    }
    dot += gv * xv;
  }
  for (int o = 32; o > 0; o >>= 1) dot += __shfl_xor(dot, o);
  if (lane == 0) dw[at] = dot;
}

// The same backward with 16-byte chunks (width a multiple of 16 / size(T),
// 16-byte aligned rows): a lane takes 4 chunks per round, their loads in
// flight together; the dot product sums each lane's chunks in order, then
// the fixed shuffle tree.
template <class T>
__global__ void __launch_bounds__(256) combine_backward_vec(const T* dy, const T* eo, const float* w,
                                                            const int64_t* idx, const int64_t* loc,
                                                            const int64_t* off, T* deo, float* dw, int64_t pairs,
                                                            int64_t width, int64_t top_k) {
  constexpr int V = 16 / sizeof(T), R = 4;
  const int lane = threadIdx.x & 63;
  const int64_t at = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (at >= pairs) return;  // whole wave
  const int64_t row = at / top_k, pos = off[idx[at]] + loc[at];
  const float f = w[at];
  const u32x4* g = reinterpret_cast<const u32x4*>(dy + row * width);
  const u32x4* x = reinterpret_cast<const u32x4*>(eo + pos * width);
  u32x4* d = reinterpret_cast<u32x4*>(deo + pos * width);
  const int64_t chunks = width / V;
  float dot = 0.f;
  auto unpack = [](const u32x4& q, float (&v)[V]) {
    if constexpr (sizeof(T) == 2) {
#pragma unroll
      for (int h = 0; h < 4; h++) {
        v[2 * h] = __uint_as_float(q[h] << 16);
        v[2 * h + 1] = __uint_as_float(q[h] & 0xffff0000u);
      }
    } else {
#pragma unroll
      for (int h = 0; h < 4; h++) v[h] = __uint_as_float(q[h]);
    }
  };
  for (int64_t c0 = 0; c0 < chunks; c0 += 64 * R) {
    u32x4 qg[R], qx[R];
#pragma unroll
    for (int i = 0; i < R; i++) {
      const int64_t c = c0 + i * 64 + lane;
      if (c < chunks) {
        qg[i] = global_load<u32x4>(g + c);
        qx[i] = global_load<u32x4>(x + c);
      }
    }
#pragma unroll
    for (int i = 0; i < R; i++) {
      const int64_t c = c0 + i * 64 + lane;
      if (c >= chunks) continue;
      float gv[V], xv[V];
      unpack(qg[i], gv);
      unpack(qx[i], xv);
      u32x4 out;
      if constexpr (sizeof(T) == 2) {
#pragma unroll
        for (int h = 0; h < 4; h++) out[h] = pack_bf16x2(gv[2 * h] * f, gv[2 * h + 1] * f);
      } else {
#pragma unroll
        for (int h = 0; h < 4; h++) out[h] = __float_as_uint(gv[h] * f);
      }
      global_store(d + c, out);
#pragma unroll
      for (int v = 0; v < V; v++) dot += gv[v] * xv[v];
    }
  }
  for (int o = 32; o > 0; o >>= 1) dot += __shfl_xor(dot, o);
  if (lane == 0) dw[at] = dot;
}

// Gradient of the router logits (cpu_lm.routing_backward,
// src/qutai/backends/cpu_lm.py:245-276), one thread per token row:
//   weights: out[e_s] = w_s (g_s - sum_t g_t w_t) for the selected experts;
//   aux:     out[e]   = g * E / rows * p_e (u_e - sum_f p_f u_f).
__global__ void route_backward_kernel(const float* g, const float* probs, const float* weights,
                                      const int64_t* indices, const float* util, float* out, int64_t rows,
                                      int64_t experts, int64_t top_k, int auxiliary) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  float* o = out + r * experts;
  const float* pr = probs + r * experts;
  if (auxiliary) {
    float center = 0.f;
    for (int64_t e = 0; e < experts; e++) center += pr[e] * util[e];
    const float scale = g[0] * (float)experts / (float)rows;
    for (int64_t e = 0; e < experts; e++) o[e] = scale * pr[e] * (util[e] - center);
  } else {
    for (int64_t e = 0; e < experts; e++) o[e] = 0.f;
    float center = 0.f;
    for (int64_t s = 0; s < top_k; s++) center += g[r * top_k + s] * weights[r * top_k + s];
    for (int64_t s = 0; s < top_k; s++)
      o[indices[r * top_k + s]] = weights[r * top_k + s] * (g[r * top_k + s] - center);
  }
}

unsigned blocks_for(int64_t n) {
  int64_t b = (n + 255) / 256;
  return (unsigned)(b < 1 ? 1 : b > 1048576 ? 1048576 : b);
}

}  // namespace

extern "C" {

size_t qutai_amd_route_workspace_size(int64_t rows, int64_t experts, int64_t top_k) {
  if (rows <= 0 || experts <= 0 || experts > 32 || top_k <= 0 || top_k > 8) return 0;
  const int64_t chunks = (rows + RCHUNK - 1) / RCHUNK;
  return (size_t)(chunks * experts * 3 * 4 + 256);
}

int qutai_amd_route(const float* scores, float* probs, float* weights, int64_t* indices, int64_t* counts,
                    int64_t* ids, int64_t* slots, int64_t* locations, int64_t* offsets, int64_t* order,
                    float* utilization, float* aux, int64_t rows, int64_t experts, int64_t top_k, void* workspace,
                    size_t workspace_bytes, void* stream) {
  if (rows < 0 || experts <= 0 || top_k <= 0 || top_k > experts) return QA_EINVAL;
  hipStream_t s = (hipStream_t)stream;
  int64_t n = rows * top_k;
  if (experts > 0x7fffffff || n >= (1ll << 31)) return QA_EINVAL;
  const size_t need = qutai_amd_route_workspace_size(rows, experts, top_k);
  if (need && workspace && workspace_bytes >= need) {
    // chunked path: select + chunk counts, scan, scatter
    const int64_t chunks = (rows + RCHUNK - 1) / RCHUNK;
    if (chunks > 0x7fffffff) return QA_EINVAL;
    int* chunk_counts = (int*)(((uintptr_t)workspace + 255) & ~(uintptr_t)255);
    float* chunk_cols = (float*)(chunk_counts + chunks * experts);
    int* chunk_base = (int*)(chunk_cols + chunks * experts);
    const int e32 = (int)experts, k32 = (int)top_k;
    if (experts <= 8) {
      hipLaunchKernelGGL(route_select_small<8>, dim3((unsigned)chunks), dim3(RCHUNK), 0, s, scores, probs, weights,
                         indices, rows, e32, k32, chunk_counts, chunk_cols);
    } else {
      hipLaunchKernelGGL(route_select_small<32>, dim3((unsigned)chunks), dim3(RCHUNK), 0, s, scores, probs, weights,
                         indices, rows, e32, k32, chunk_counts, chunk_cols);
    }
    hipLaunchKernelGGL(route_scan, dim3(1), dim3(1024), 0, s, chunk_counts, chunk_cols, chunk_base, chunks, e32,
                       counts, offsets, utilization, aux, rows, n);
    if (experts <= 8)
      hipLaunchKernelGGL(route_scatter<8>, dim3((unsigned)chunks), dim3(RCHUNK), 0, s, indices, chunk_base, offsets,
                         ids, slots, locations, order, rows, e32, k32, n);
    else
      hipLaunchKernelGGL(route_scatter<32>, dim3((unsigned)chunks), dim3(RCHUNK), 0, s, indices, chunk_base, offsets,
                         ids, slots, locations, order, rows, e32, k32, n);
    return (int)hipGetLastError();
  }
  if (rows > 0 && experts <= 8 && top_k <= 8)
    hipLaunchKernelGGL(route_select_small<8>, dim3((unsigned)((rows + RCHUNK - 1) / RCHUNK)), dim3(RCHUNK), 0, s,
                       scores, probs, weights, indices, rows, (int)experts, (int)top_k, nullptr, nullptr);
  else if (rows > 0 && experts <= 32 && top_k <= 8)
    hipLaunchKernelGGL(route_select_small<32>, dim3((unsigned)((rows + RCHUNK - 1) / RCHUNK)), dim3(RCHUNK), 0, s,
                       scores, probs, weights, indices, rows, (int)experts, (int)top_k, nullptr, nullptr);
  else if (rows > 0)
    hipLaunchKernelGGL(route_select, dim3(blocks_for(rows)), dim3(256), 0, s, scores, probs, weights, indices, rows,
                       experts, top_k);
  hipLaunchKernelGGL(route_pack, dim3((unsigned)experts), dim3(PACKW * 64), 0, s, indices, counts, ids, slots,
                     locations, offsets, order, n, top_k, experts, (const float*)probs, utilization);
  if (rows > 0)
    hipLaunchKernelGGL(route_stats, dim3(1), dim3(64), 0, s, counts, utilization, aux, rows, experts, n);
  return (int)hipGetLastError();
}

int qutai_amd_route_gather(const void* x, const int64_t* order, void* out, int64_t count, int64_t width,
                           int backward, int dtype, void* stream) {
  if (count < 0 || width < 0) return QA_EINVAL;
  if (dtype != F32 && dtype != BF16 && dtype != F64) return QA_EINVAL;
  if (count * width == 0) return QA_OK;
  hipStream_t s = (hipStream_t)stream;
  int64_t es = dtype == BF16 ? 2 : dtype == F64 ? 8 : 4;
  bool vec = (width * es) % 16 == 0 && (uintptr_t)x % 16 == 0 && (uintptr_t)out % 16 == 0;
  if (vec) {
    int64_t pieces = width * es / 16;
    if ((count + 3) / 4 > 0x7fffffff) return QA_EINVAL;
    hipLaunchKernelGGL(gather_rows16, dim3((unsigned)((count + 3) / 4)), dim3(256), 0, s, (const u32x4*)x, order,
                       (u32x4*)out, count, pieces, backward);
  } else if (dtype == BF16) {
    hipLaunchKernelGGL(gather_rows<bf16_t>, dim3(blocks_for(count * width)), dim3(256), 0, s, (const bf16_t*)x,
                       order, (bf16_t*)out, count, width, backward);
  } else if (dtype == F32) {
    hipLaunchKernelGGL(gather_rows<float>, dim3(blocks_for(count * width)), dim3(256), 0, s, (const float*)x, order,
                       (float*)out, count, width, backward);
  } else {
    hipLaunchKernelGGL(gather_rows<double>, dim3(blocks_for(count * width)), dim3(256), 0, s, (const double*)x,
                       order, (double*)out, count, width, backward);
  }
  return (int)hipGetLastError();
}

int qutai_amd_combine(const void* expert_out, const float* weights, const int64_t* indices,
                      const int64_t* locations, const int64_t* offsets, void* y, int64_t rows, int64_t width,
                      int64_t top_k, int dtype, int out_dtype, void* stream) {
  if (rows < 0 || width < 0 || top_k <= 0) return QA_EINVAL;
  if (dtype != F32 && dtype != BF16) return QA_EINVAL;
  if (out_dtype != dtype && !(dtype == F32 && out_dtype == BF16)) return QA_EINVAL;
  if (rows * width == 0) return QA_OK;
  hipStream_t s = (hipStream_t)stream;
  // vector paths: 16-byte loads of expert rows, 16- / 8-byte stores
  const bool aligned = (uintptr_t)expert_out % 16 == 0 && (uintptr_t)y % 16 == 0;
  const unsigned wave_blocks = (unsigned)((rows + 3) / 4);
  if ((rows + 3) / 4 <= 0x7fffffff && aligned) {
    if (dtype == BF16 && width % 8 == 0) {
      hipLaunchKernelGGL((combine_rows_wave<bf16_t, bf16_t>), dim3(wave_blocks), dim3(256), 0, s,
                         (const bf16_t*)expert_out, weights, indices, locations, offsets, (bf16_t*)y, rows, width,
                         top_k);
      return (int)hipGetLastError();
    }
    if (dtype == F32 && width % 4 == 0) {
      if (out_dtype == BF16)
        hipLaunchKernelGGL((combine_rows_wave<float, bf16_t>), dim3(wave_blocks), dim3(256), 0, s,
                           (const float*)expert_out, weights, indices, locations, offsets, (bf16_t*)y, rows, width,
                           top_k);
      else
        hipLaunchKernelGGL((combine_rows_wave<float, float>), dim3(wave_blocks), dim3(256), 0, s,
                           (const float*)expert_out, weights, indices, locations, offsets, (float*)y, rows, width,
                           top_k);
      return (int)hipGetLastError();
    }
  }
  if (dtype == F32 && out_dtype == BF16) {  // fp32 rows summed straight into bf16 token rows
    if (width % 4 == 0 && aligned)
      hipLaunchKernelGGL((combine_kernel<float, 4, bf16_t>), dim3(blocks_for(rows * width / 4)), dim3(256), 0, s,
                         (const float*)expert_out, weights, indices, locations, offsets, (bf16_t*)y, rows, width,
                         top_k);
    else
      hipLaunchKernelGGL((combine_kernel<float, 1, bf16_t>), dim3(blocks_for(rows * width)), dim3(256), 0, s,
                         (const float*)expert_out, weights, indices, locations, offsets, (bf16_t*)y, rows, width,
                         top_k);
    return (int)hipGetLastError();
  }
  if (dtype == BF16) {
    if (width % 8 == 0 && aligned)
      hipLaunchKernelGGL((combine_kernel<bf16_t, 8>), dim3(blocks_for(rows * width / 8)), dim3(256), 0, s,
                         (const bf16_t*)expert_out, weights, indices, locations, offsets, (bf16_t*)y, rows, width,
                         top_k);
    else
      hipLaunchKernelGGL((combine_kernel<bf16_t, 1>), dim3(blocks_for(rows * width)), dim3(256), 0, s,
                         (const bf16_t*)expert_out, weights, indices, locations, offsets, (bf16_t*)y, rows, width,
                         top_k);
  } else {
    if (width % 4 == 0 && aligned)
      hipLaunchKernelGGL((combine_kernel<float, 4>), dim3(blocks_for(rows * width / 4)), dim3(256), 0, s,
                         (const float*)expert_out, weights, indices, locations, offsets, (float*)y, rows, width,
                         top_k);
    else
      hipLaunchKernelGGL((combine_kernel<float, 1>), dim3(blocks_for(rows * width)), dim3(256), 0, s,
                         (const float*)expert_out, weights, indices, locations, offsets, (float*)y, rows, width,
                         top_k);
  }
  return (int)hipGetLastError();
}

int qutai_amd_combine_backward(const void* dy, const void* expert_out, const float* weights, const int64_t* indices,
                               const int64_t* locations, const int64_t* offsets, void* d_expert_out,
                               float* d_weights, int64_t rows, int64_t width, int64_t top_k, int dtype,
                               void* stream) {
  if (rows < 0 || width < 0 || top_k <= 0) return QA_EINVAL;
  if (dtype != F32 && dtype != BF16) return QA_EINVAL;
  const int64_t pairs = rows * top_k;
  if (pairs == 0) return QA_OK;
  const unsigned blocks = (unsigned)((pairs + 3) / 4);
  hipStream_t s = (hipStream_t)stream;
  {
    const int64_t es = dtype == BF16 ? 2 : 4;
    const bool vec = (width * es) % 16 == 0 && (uintptr_t)dy % 16 == 0 && (uintptr_t)expert_out % 16 == 0 &&
                     (uintptr_t)d_expert_out % 16 == 0;
    if (vec && dtype == BF16) {
      hipLaunchKernelGGL(combine_backward_vec<bf16_t>, dim3(blocks), dim3(256), 0, s, (const bf16_t*)dy,
                         (const bf16_t*)expert_out, weights, indices, locations, offsets, (bf16_t*)d_expert_out,
                         d_weights, pairs, width, top_k);
      return (int)hipGetLastError();
    }
    if (vec) {
      hipLaunchKernelGGL(combine_backward_vec<float>, dim3(blocks), dim3(256), 0, s, (const float*)dy,
                         (const float*)expert_out, weights, indices, locations, offsets, (float*)d_expert_out,
                         d_weights, pairs, width, top_k);
      return (int)hipGetLastError();
    }
  }
  if (dtype == BF16)
    hipLaunchKernelGGL(combine_backward_kernel<bf16_t>, dim3(blocks), dim3(256), 0, s, (const bf16_t*)dy,
                       (const bf16_t*)expert_out, weights, indices, locations, offsets, (bf16_t*)d_expert_out,
                       d_weights, pairs, width, top_k);
  else
    hipLaunchKernelGGL(combine_backward_kernel<float>, dim3(blocks), dim3(256), 0, s, (const float*)dy,
                       (const float*)expert_out, weights, indices, locations, offsets, (float*)d_expert_out,
                       d_weights, pairs, width, top_k);
  return (int)hipGetLastError();
}

int qutai_amd_route_backward(const float* gradient, const float* probs, const float* weights,
                             const int64_t* indices, const float* utilization, float* out, int64_t rows,
                             int64_t experts, int64_t top_k, int auxiliary, void* stream) {
  if (rows < 0 || experts <= 0 || top_k <= 0 || top_k > experts) return QA_EINVAL;
  if (rows == 0) return QA_OK;
  hipLaunchKernelGGL(route_backward_kernel, dim3(blocks_for(rows)), dim3(256), 0, (hipStream_t)stream, gradient,
                     probs, weights, indices, utilization, out, rows, experts, top_k, auxiliary ? 1 : 0);
  return (int)hipGetLastError();
}

}  // extern "C"
