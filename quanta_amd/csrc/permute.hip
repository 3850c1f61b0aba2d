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
#include "route_common.h"
#include "../../include/quanta_moe.h"

namespace qmoe {

constexpr int kPermThreads = 1024;
constexpr int kPermLdsWords = 12 * 1024;   // 48 KiB of bitmap + prefix words per workgroup

template <int RES>
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
  __shared__ int toffs[1025], btoffs[1025];
  const int e0 = blockIdx.x * experts_per_wg;
  const int e1 = min(E, e0 + experts_per_wg);
  const PermuteLds S{hist, offs, scan_tmp, bits, pref, toffs, btoffs};
  permute_body<RES>(idx, N, k, E, m_tile, e0, e1, words_per_expert, blockIdx.x == 0, S, counts,
                    offsets, tile_off, sorted_slot, inv, tile_map, max_tiles, split_rows,
                    m_tile_big, tile_map_big, max_tiles_big);
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
  // (the slot list resident in registers up to 48 ids per thread; longer lists in batches)
  const int64_t mc = static_cast<int64_t>(N) * k;
#define QMOE_PERM(RES)                                                                            \
  permute_kernel<RES><<<n_wg, kPermThreads, 0, stream>>>(                                         \
      idx, N, k, E, m_tile, per_wg, words, counts, offsets, tile_off, sorted_slot, inv,           \
      reinterpret_cast<int4*>(tile_map), static_cast<int>(max_tiles), split_rows, m_tile_big,    \
      reinterpret_cast<int4*>(tile_map_big), static_cast<int>(max_tiles_big))
  if (mc <= 8 * kPermThreads) QMOE_PERM(8);
  else if (mc <= 48 * kPermThreads) QMOE_PERM(48);
  else QMOE_PERM(0);
#undef QMOE_PERM
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
