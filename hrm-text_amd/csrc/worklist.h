// Device-built, cost-ordered work lists.
//
// The reference launches one FlashAttention grid per pass, sized by the longest
// prefix / suffix over all segments (models/flash_attention_prefixlm_v2.py:115-128),
// so short segments leave most of each grid idle. Here a single block scans the
// segment metadata (which lives on the device; reading it on the host would need a
// sync) and writes one item per (segment, tile) that has work, ordered by
// decreasing cost so the longest tiles are dispatched first (LPT). The main kernels
// launch items*H blocks and each block picks its item from this list.
#pragma once
#include "common.h"

namespace prefixlm {

constexpr int kPrepThreads = 1024;
constexpr int kCostBuckets = 2048;
static_assert(kCostBuckets == 2 * kPrepThreads, "the scan below gives each thread two buckets");

struct MetaParams {
  const int32_t* prefix;
  const int32_t* causal;
  const int32_t* cu;
  int numseqs;
  int total_seqlen;
  int T;
  int is_causal;
  int max_all;       // max_seqlen_all: a longer segment is inconsistent metadata
};

// ---- stored-dS block layout ---------------------------------------------------------
// The backward's stored dS (fp16 blocks of 32 queries x 64 keys, one set per head) holds
// only the blocks of attended (query tile, key group) pairs. In a segment of length L
// with prefix p (prefix_lens[s], whatever is_causal: the layout then only has blocks
// nothing writes), key group kg (keys [64 kg, 64 kg + 64)) is attended by the query
// tiles [qlo, n32), n32 = ceil(L / 32), qlo = 0 when 64 kg < p (a prefix key: every row
// sees it), else 2 kg (a suffix key: rows >= 64 kg). Blocks are key-group major within
// the segment, segments in order: block (kg, qt) of segment s is
// ds_base[s] + ds_blk_off(kg, n32, kp) + qt, kp = ceil(p / 64) the prefix key groups.
__host__ __device__ inline int ds_kp(int p, int L) {
  const int kp = (p + 63) / 64, n64 = (L + 63) / 64;
  return kp < n64 ? kp : n64;
}
// offset of block (kg, qt = 0) of a segment: sum of the earlier key groups' block
// counts (n32 each below kp, n32 - 2 j for key group j >= kp) minus qlo(kg)
__host__ __device__ inline int ds_blk_off(int kg, int n32, int kp) {
  return kg < kp ? n32 * kg : n32 * kg - kg * kg - kg + kp * (kp - 1);
}
// blocks of one segment
__host__ __device__ inline int64_t ds_seg_blocks(int p, int L) {
  if (L <= 0) return 0;
  const int n32 = (L + 31) / 32, n64 = (L + 63) / 64, kp = ds_kp(p, L);
  return (int64_t)n32 * n64 - (int64_t)n64 * (n64 - 1) + (int64_t)kp * (kp - 1);
}

// Tile cost in units of the inner loop trip count.
//   mode 0 (forward):  tile = q rows [t*tile, ...), inner loop over key tiles of `inner`
//   mode 1 (backward): tile = keys [t*tile, ...), inner loop over query tiles of `inner`
__host__ __device__ inline int tile_cost(int mode, int t, int tile, int inner, int p, int L) {
  if (mode == 0) {
    const int q1 = (t + 1) * tile < L ? (t + 1) * tile : L;
    const int kend = p > q1 ? (p < L ? p : L) : q1;
    return (kend + inner - 1) / inner;
  }
  const int k0 = t * tile;
  const int qstart = (k0 < p) ? 0 : (k0 / inner) * inner;
  return (L - qstart + inner - 1) / inner;
}

// Returns false when segment s is inconsistent: negative lengths, rows past
// total_seqlen, cu_seqlens[s+1] != cu_seqlens[s] + prefix + causal, or a length above
// max_seqlen_all (the host sizes buffers from it).
__device__ __forceinline__ bool read_segment(const MetaParams& m, int s, int* cs, int* p, int* L) {
  const int c0 = m.cu[s], c1 = m.cu[s + 1];
  const int pp = m.prefix[s], cc = m.causal[s];
  const bool ok = pp >= 0 && cc >= 0 && c0 >= 0 && (int64_t)c0 + pp + cc <= m.total_seqlen &&
                  m.total_seqlen <= m.T && c1 == c0 + pp + cc && (int64_t)pp + cc <= m.max_all;
  if (!ok) return false;
  *cs = c0;
  *p = m.is_causal ? 0 : pp;
  *L = pp + cc;
  return true;
}

// One work list: items (segment, tile) of `tile` rows, costed by tile_cost(mode, ...).
struct ListSpec {
  int mode, tile, inner, max_items;
  int2* items;
  WsHeader* hdr;
  // optional (null: none): the stored-dS block base of every segment, ds_base[s] for
  // s <= numseqs (ds_base[numseqs] = the blocks of one head), checked against ds_cap
  int32_t* ds_base;
  int ds_cap;
};
struct ListSpecs {
  ListSpec l[2];
};

constexpr int kStagedSegs = 2048;   // segments whose metadata is staged in LDS
static_assert(kStagedSegs == kCostBuckets, "tile_end is scanned with the bucket scan");

// In-place inclusive scan of v[0, kCostBuckets) (Hillis-Steele, two elements per
// thread); every thread of the workgroup must call it.
__device__ __forceinline__ void block_inclusive_scan(int* v) {
  const int tid = threadIdx.x;
  for (int off = 1; off < kCostBuckets; off <<= 1) {
    int v0 = 0, v1 = 0;
    const int i0 = tid, i1 = tid + kPrepThreads;
    if (i0 >= off) v0 = v[i0 - off];
    if (i1 >= off) v1 = v[i1 - off];
    __syncthreads();
    v[i0] += v0;
    v[i1] += v1;
    __syncthreads();
  }
}

// Workgroup b builds list specs.l[b]; workgroup 0 also zeroes zero_buf[0, n_zero).
// With up to kStagedSegs segments the metadata is read once, coalesced, and the
// (segment, tile) pairs are spread over all threads; beyond that every thread
// walks the tiles of its own segments.
__global__ __launch_bounds__(kPrepThreads) void build_worklist_kernel(MetaParams m, ListSpecs specs,
                                                                      float* zero_buf, int n_zero) {
  __shared__ int hist[kCostBuckets];
  __shared__ int scan[kCostBuckets];
  __shared__ int seg_p[kStagedSegs], seg_L[kStagedSegs];   // seg_L = -1: invalid segment
  __shared__ int tile_end[kStagedSegs];                    // inclusive scan of tiles per segment
  __shared__ int err;
  const int tid = threadIdx.x;
  const ListSpec sp = specs.l[blockIdx.x];
  const int mode = sp.mode, tile = sp.tile, inner = sp.inner, max_items = sp.max_items;
  int2* items = sp.items;
  WsHeader* hdr = sp.hdr;
  const bool staged = m.numseqs <= kStagedSegs;
  // small side buffer the next kernels accumulate into (may be null)
  if (blockIdx.x == 0)
    for (int i = tid; i < n_zero; i += kPrepThreads) zero_buf[i] = 0.f;
  for (int i = tid; i < kCostBuckets; i += kPrepThreads) {
    hist[i] = 0;
    tile_end[i] = 0;
  }
  if (tid == 0) err = (m.numseqs > 0 && m.cu[0] != 0) ? kErrCuStart : 0;
  __syncthreads();
  // validate every segment once (errors are recorded here, for either path)
  for (int s = tid; s < m.numseqs; s += kPrepThreads) {
    int cs, p, L;
    const bool ok = read_segment(m, s, &cs, &p, &L);
    if (!ok) atomicOr(&err, kErrBadSegment);
    if (staged) {
      seg_p[s] = p;
      seg_L[s] = ok ? L : -1;
      tile_end[s] = ok ? (L + tile - 1) / tile : 0;
    }
  }
  __syncthreads();
  int n_pairs = 0;
  if (staged) {
    block_inclusive_scan(tile_end);
    n_pairs = tile_end[kStagedSegs - 1];
  }
  // (segment, tile) of flat pair index i: the first segment whose tile_end exceeds i
  auto pair_at = [&](int i, int* s_out, int* t_out) {
    int lo = 0, hi = m.numseqs - 1;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (tile_end[mid] > i) hi = mid; else lo = mid + 1;
    }
    *s_out = lo;
    *t_out = i - (lo > 0 ? tile_end[lo - 1] : 0);
  };

  // pass 1: histogram of tile costs
  if (staged) {
    for (int i = tid; i < n_pairs; i += kPrepThreads) {
      int s, t;
      pair_at(i, &s, &t);
      atomicAdd(&hist[min(tile_cost(mode, t, tile, inner, seg_p[s], seg_L[s]), kCostBuckets - 1)], 1);
    }
  } else {
    for (int s = tid; s < m.numseqs; s += kPrepThreads) {
      int cs, p, L;
      if (!read_segment(m, s, &cs, &p, &L)) continue;
      const int nt = (L + tile - 1) / tile;
      for (int t = 0; t < nt; ++t) atomicAdd(&hist[min(tile_cost(mode, t, tile, inner, p, L), kCostBuckets - 1)], 1);
    }
  }
  __syncthreads();

  // exclusive start of each bucket in decreasing-cost order: start[c] = sum_{c' > c} hist[c']
  for (int i = tid; i < kCostBuckets; i += kPrepThreads) scan[i] = hist[kCostBuckets - 1 - i];
  __syncthreads();
  block_inclusive_scan(scan);
  // scan[i] is now the inclusive sum of reversed buckets 0..i
  const int total_items = scan[kCostBuckets - 1];
  for (int c = tid; c < kCostBuckets; c += kPrepThreads) {
    const int ri = kCostBuckets - 1 - c;            // reversed index of bucket c
    hist[c] = scan[ri] - hist[c];                   // exclusive start of bucket c
  }
  __syncthreads();

  // pass 2: scatter items
  if (staged) {
    for (int i = tid; i < n_pairs; i += kPrepThreads) {
      int s, t;
      pair_at(i, &s, &t);
      const int c = min(tile_cost(mode, t, tile, inner, seg_p[s], seg_L[s]), kCostBuckets - 1);
      const int pos = atomicAdd(&hist[c], 1);
      if (pos < max_items) items[pos] = make_int2(s, t);
    }
  } else {
    for (int s = tid; s < m.numseqs; s += kPrepThreads) {
      int cs, p, L;
      if (!read_segment(m, s, &cs, &p, &L)) continue;
      const int nt = (L + tile - 1) / tile;
      for (int t = 0; t < nt; ++t) {
        const int c = min(tile_cost(mode, t, tile, inner, p, L), kCostBuckets - 1);
        const int pos = atomicAdd(&hist[c], 1);
        if (pos < max_items) items[pos] = make_int2(s, t);
      }
    }
  }
  if (sp.ds_base != nullptr) {
    // exclusive scan of the segments' dS block counts: each thread sums a contiguous
    // chunk of segments (clamped: a sum above any capacity is flagged either way)
    __syncthreads();
    const int chunk = (m.numseqs + kPrepThreads - 1) / kPrepThreads;
    const int s0 = min(m.numseqs, tid * chunk), s1 = min(m.numseqs, s0 + chunk);
    auto seg_blocks = [&](int s) -> int64_t {
      const int pp = m.prefix[s], cc = m.causal[s];
      return (pp >= 0 && cc >= 0) ? ds_seg_blocks(pp, pp + cc) : 0;
    };
    int64_t local = 0;
    for (int s = s0; s < s1; ++s) local += seg_blocks(s);
    for (int i = tid; i < kCostBuckets; i += kPrepThreads) scan[i] = 0;
    __syncthreads();
    scan[tid] = (int)min(local, (int64_t)1 << 20);
    __syncthreads();
    block_inclusive_scan(scan);
    int64_t base = tid > 0 ? scan[tid - 1] : 0;
    for (int s = s0; s < s1; ++s) {
      sp.ds_base[s] = (int32_t)min(base, (int64_t)0x7fffffff);
      base += seg_blocks(s);
    }
    if (tid == 0) {
      const int total = scan[kCostBuckets - 1];
      sp.ds_base[m.numseqs] = total;
      if (total > sp.ds_cap) atomicOr(&err, kErrDsCapacity);
    }
    __syncthreads();
  }
  if (tid == 0) {
    hdr->n_items = min(total_items, max_items);
    hdr->error = err;
  }
}

}  // namespace prefixlm
