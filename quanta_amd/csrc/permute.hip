// Stable permute of the (token, slot) list by expert id: histogram, exclusive scan and
// scatter, all in LDS, with the stable rank taken from a per-expert token bitmap so the result
// is deterministic (equal to a stable argsort) without ordered atomics.
//
// Reference: order = argsort(exp) (stable), inv = argsort(order), exp/tok gathered by order
// (src/quanta/modeling/moe.py:81-85; src/quanta/dsv4/moe.py:68,107-112). The build adds
// counts/offsets per expert and the m-tile prefix the grouped-qmm grid walks.
//
// Stable rank of slot m = t*k + s routed to expert e: the number of earlier slots with the same
// expert. Top-k routing selects distinct experts per token, so that equals the number of tokens
// t' < t that chose e: popcount of e's token bitmap below bit t. Each workgroup owns a range of
// experts (so its bitmaps fit in LDS), recomputes the full histogram for the offsets, and
// scatters only its own experts' slots; no inter-workgroup communication is needed.
#include "qmoe_internal.h"
#include "../../include/quanta_moe.h"

namespace qmoe {

constexpr int kPermThreads = 1024;
constexpr int kPermLdsWords = 12 * 1024;   // 48 KiB of bitmap + prefix words per workgroup

__device__ __forceinline__ int block_exclusive_scan(int v, int* warp_sums, int* total) {
  // 1024 threads = 16 wavefronts of 64.
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  int incl = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    int o = __shfl_up(incl, off);
    if (lane >= off) incl += o;
  }
  if (lane == 63) warp_sums[wid] = incl;
  __syncthreads();
  if (wid == 0) {
    int s = (lane < 16) ? warp_sums[lane] : 0;
    int si = s;
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) {
      int o = __shfl_up(si, off);
      if (lane >= off) si += o;
    }
    if (lane < 16) warp_sums[16 + lane] = si - s;   // exclusive prefix of wave totals
    if (lane == 15) *total = si;
  }
  __syncthreads();
  return warp_sums[16 + wid] + incl - v;
}

// Optional split tile maps (hybrid regime): experts with more than `split_rows` rows get
// m-tiles of `m_tile_big` rows in tile_map_big; the others keep m_tile-row tiles in tile_map.
__global__ void __launch_bounds__(kPermThreads) permute_kernel(
    const int32_t* __restrict__ idx, int N, int k, int E, int m_tile, int experts_per_wg,
    int words_per_expert, int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
    int32_t* __restrict__ tile_off, int32_t* __restrict__ sorted_slot, int32_t* __restrict__ inv,
    int4* __restrict__ tile_map, int max_tiles, int split_rows, int m_tile_big,
    int4* __restrict__ tile_map_big, int max_tiles_big) {
  __shared__ int hist[1024];
  __shared__ int offs[1025];
  __shared__ int scan_tmp[40];
  __shared__ uint32_t bits[kPermLdsWords / 2];
  __shared__ uint32_t pref[kPermLdsWords / 2];

  const int tid = threadIdx.x;
  const int mc = N * k;
  const int e0 = blockIdx.x * experts_per_wg;
  const int e1 = min(E, e0 + experts_per_wg);
  const int nbits = (e1 - e0) * words_per_expert;

  for (int i = tid; i < 1024; i += kPermThreads) hist[i] = 0;
  for (int i = tid; i < nbits; i += kPermThreads) bits[i] = 0u;
  __syncthreads();

  for (int m = tid; m < mc; m += kPermThreads) {
    const int e = idx[m];
    if (e < 0 || e >= E) continue;
    atomicAdd(&hist[e], 1);
    if (e >= e0 && e < e1) {
      const int t = m / k;
      atomicOr(&bits[(e - e0) * words_per_expert + (t >> 5)], 1u << (t & 31));
    }
  }
  __syncthreads();

  // Offsets (exclusive scan of counts) and the m-tile prefix.
  const int c = (tid < E) ? hist[tid] : 0;
  int total = 0;
  const int ex = block_exclusive_scan(c, scan_tmp, &scan_tmp[39]);
  total = scan_tmp[39];
  if (tid < E) offs[tid] = ex;
  if (tid == 0) offs[E] = total;
  __syncthreads();
  const int tiles = (c + m_tile - 1) / m_tile;
  const int tex = block_exclusive_scan(tiles, scan_tmp, &scan_tmp[38]);
  // hybrid split: small-tile map over the experts at or below split_rows, big-tile map over
  // the rest (block-uniform condition: tile_map_big is a kernel argument)
  int s_tiles = tiles, s_ex = tex, s_total = 0, b_tiles = 0, b_ex = 0, b_total = 0;
  if (tile_map_big) {
    const bool big = c > split_rows;
    s_tiles = big ? 0 : tiles;
    b_tiles = big ? (c + m_tile_big - 1) / m_tile_big : 0;
    s_ex = block_exclusive_scan(s_tiles, scan_tmp, &scan_tmp[37]);
    s_total = scan_tmp[37];
    b_ex = block_exclusive_scan(b_tiles, scan_tmp, &scan_tmp[36]);
    b_total = scan_tmp[36];
  }
  if (blockIdx.x == 0) {
    if (tid < E) {
      counts[tid] = c;
      offsets[tid] = ex;
      tile_off[tid] = tex;
    }
    if (tid == 0) {
      offsets[E] = total;
      tile_off[E] = scan_tmp[38];
    }
    // Per-tile descriptors {expert, first sorted position, rows, 0} for the grouped-qmm grid,
    // and a -1 sentinel in every unused entry up to max_tiles, so a workgroup resolves its tile
    // with one 16-byte load.
    if (tile_map && !tile_map_big) {
      if (tid < E)
        for (int i = 0; i < tiles; ++i)
          tile_map[tex + i] = make_int4(tid, ex + i * m_tile, min(m_tile, c - i * m_tile), 0);
      for (int t = scan_tmp[38] + tid; t < max_tiles; t += kPermThreads)
        tile_map[t] = make_int4(-1, 0, 0, 0);
    }
    if (tile_map_big) {
      if (tid < E) {
        for (int i = 0; i < s_tiles; ++i)
          tile_map[s_ex + i] = make_int4(tid, ex + i * m_tile, min(m_tile, c - i * m_tile), 0);
        for (int i = 0; i < b_tiles; ++i)
          tile_map_big[b_ex + i] =
              make_int4(tid, ex + i * m_tile_big, min(m_tile_big, c - i * m_tile_big), 0);
      }
      for (int t = s_total + tid; t < max_tiles; t += kPermThreads) tile_map[t] = make_int4(-1, 0, 0, 0);
      for (int t = b_total + tid; t < max_tiles_big; t += kPermThreads)
        tile_map_big[t] = make_int4(-1, 0, 0, 0);
    }
  }

  // Per-expert exclusive popcount prefix over the token bitmap words.
  for (int i = tid; i < nbits; i += kPermThreads) pref[i] = __popc(bits[i]);
  __syncthreads();
  for (int el = tid; el < e1 - e0; el += kPermThreads) {
    uint32_t run = 0;
    uint32_t* p = pref + el * words_per_expert;
    for (int w = 0; w < words_per_expert; ++w) {
      const uint32_t v = p[w];
      p[w] = run;
      run += v;
    }
  }
  // Own output segment starts as -1 so a malformed idx (duplicate experts within a token)
  // leaves detectable holes instead of stale data.
  if (e1 > e0)
    for (int p = offs[e0] + tid; p < offs[e1]; p += kPermThreads) sorted_slot[p] = -1;
  __syncthreads();

  for (int m = tid; m < mc; m += kPermThreads) {
    const int e = idx[m];
    if (e < 0 || e >= E) {
      if (blockIdx.x == 0) inv[m] = -1;
      continue;
    }
    if (e < e0 || e >= e1) continue;
    const int t = m / k;
    const int wi = (e - e0) * words_per_expert + (t >> 5);
    const uint32_t below = bits[wi] & ((1u << (t & 31)) - 1u);
    const int pos = offs[e] + static_cast<int>(pref[wi]) + __popc(below);
    sorted_slot[pos] = m;
    inv[m] = pos;
  }
}

int launch_permute(const int32_t* idx, int N, int k, int E, int m_tile, int32_t* counts,
                   int32_t* offsets, int32_t* tile_off, int32_t* sorted_slot, int32_t* inv,
                   int32_t* tile_map, int64_t max_tiles, hipStream_t stream, int split_rows,
                   int m_tile_big, int32_t* tile_map_big, int64_t max_tiles_big) {
  const int words = (N + 31) / 32;
  int per_wg = (kPermLdsWords / 2) / words;
  if (per_wg < 1) return fail("permute: N too large for the LDS token bitmap");
  if (per_wg > E) per_wg = E;
  const int n_wg = (E + per_wg - 1) / per_wg;
  if (tile_map && max_tiles < mtile_upper_bound(static_cast<int64_t>(N) * k, E, m_tile))
    return fail("permute: tile_map smaller than the m-tile upper bound");
  if (tile_map_big && (!tile_map || m_tile_big <= 0 ||
                       max_tiles_big < mtile_upper_bound(static_cast<int64_t>(N) * k, E, m_tile_big)))
    return fail("permute: split tile maps need both maps sized to their m-tile bounds");
  permute_kernel<<<n_wg, kPermThreads, 0, stream>>>(
      idx, N, k, E, m_tile, per_wg, words, counts, offsets, tile_off, sorted_slot, inv,
      reinterpret_cast<int4*>(tile_map), static_cast<int>(max_tiles), split_rows, m_tile_big,
      reinterpret_cast<int4*>(tile_map_big), static_cast<int>(max_tiles_big));
  return check_launch("permute");
}

}  // namespace qmoe

using namespace qmoe;

extern "C" int qmoe_permute(const int32_t* idx, int64_t N, int k, int E, int m_tile,
                            int32_t* counts, int32_t* offsets, int32_t* tile_off,
                            int32_t* sorted_slot, int32_t* inv, int32_t* tile_map,
                            int64_t max_tiles, void* stream) {
  if (N <= 0 || k <= 0 || E <= 0 || E > 1024) return fail("qmoe_permute: need N,k > 0, 1 <= E <= 1024");
  if (N * k > (int64_t(1) << 30)) return fail("qmoe_permute: N*k too large");
  if (N > 196608) return fail("qmoe_permute: N above 196608 (6144 bitmap words per expert)");
  if (m_tile <= 0) return fail("qmoe_permute: m_tile must be positive");
  if (!idx || !counts || !offsets || !tile_off || !sorted_slot || !inv)
    return fail("qmoe_permute: null pointer");
  if (max_tiles > (int64_t(1) << 30)) return fail("qmoe_permute: max_tiles too large");
  return launch_permute(idx, static_cast<int>(N), k, E, m_tile, counts, offsets, tile_off,
                        sorted_slot, inv, tile_map, max_tiles, static_cast<hipStream_t>(stream));
}
