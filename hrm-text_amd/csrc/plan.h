// Host-built work lists ("plan").
//
// The same three lists the device work-list kernel builds for every call (forward
// query tiles, backward key tiles, backward query tiles), computed once on the host
// from host copies of the batch metadata -- in the data loader, next to the
// reference's compute_aux_seq_tensors_scalars (dataset_new.py:129-134,
// models/flash_attention_prefixlm_v2.py:10-24) -- and uploaded with the batch. Every
// attention call of a training step reuses it, and the calls skip the work-list
// kernel. Items are ordered by decreasing cost, ties by (segment, tile), so a plan
// is a deterministic function of the metadata.
//
// Layout: three lists, each a 64-byte WsHeader followed by int2 items (segment,
// tile), every part starting on a 256-byte boundary; list i holds
// max_items(total_seqlen, numseqs, tile_i) item slots. The header's pad words hold
// kPlanMagic, numseqs, total_seqlen, the list's tile size and (pad[4]) the stored-dS
// blocks per head of the batch. Then int32 ds_base[numseqs + 1]: the stored-dS block
// base of every segment (ds_seg_blocks, in segment order) and, last, the blocks per
// head, so that a backward with this plan can size its dS buffer to exactly the blocks
// it writes.
#pragma once
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <vector>

#include "common.h"
#include "worklist.h"

namespace prefixlm {
namespace plan {

constexpr int32_t kPlanMagic = 0x50524c32;   // "PRL2" (with the stored-dS block bases)
constexpr int kLists = 3;
constexpr size_t kAlign = 256;

inline size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

inline int64_t max_items(int32_t total, int32_t numseqs, int tile) {
  return (int64_t)(total + tile - 1) / tile + numseqs;
}

struct ListDesc {
  int mode, tile, inner;
};

struct Layout {
  size_t hdr_off[kLists], items_off[kLists];
  int64_t nmax[kLists];
  size_t ds_off;   // int32 ds_base[numseqs + 1]
  size_t bytes;
};

inline Layout layout(const ListDesc (&d)[kLists], int32_t total, int32_t numseqs) {
  Layout l{};
  size_t off = 0;
  for (int i = 0; i < kLists; ++i) {
    l.nmax[i] = max_items(total, numseqs, d[i].tile);
    l.hdr_off[i] = off;
    off += align_up(sizeof(WsHeader));
    l.items_off[i] = off;
    off += align_up(sizeof(int32_t) * 2 * (size_t)l.nmax[i]);
  }
  l.ds_off = off;
  off += align_up(sizeof(int32_t) * ((size_t)(numseqs > 0 ? numseqs : 0) + 1));
  l.bytes = off;
  return l;
}

// Validates the metadata as the device work-list kernel does (read_segment) and
// fills `out` (l.bytes bytes). Returns 0, or the WsHeader error flags.
inline int32_t build(const ListDesc (&d)[kLists], const Layout& l, const int32_t* prefix,
                     const int32_t* causal, const int32_t* cu, int32_t numseqs, int32_t total,
                     int32_t T, int is_causal, unsigned char* out) {
  int32_t err = (numseqs > 0 && cu[0] != 0) ? kErrCuStart : 0;
  for (int s = 0; s < numseqs; ++s) {
    const int64_t c0 = cu[s], c1 = cu[s + 1], pp = prefix[s], cc = causal[s];
    if (!(pp >= 0 && cc >= 0 && c0 >= 0 && c0 + pp + cc <= total && total <= T && c1 == c0 + pp + cc))
      err |= kErrBadSegment;
  }
  if (err) return err;
  memset(out, 0, l.bytes);
  // stored-dS block bases (the layout uses prefix_lens whatever is_causal)
  int32_t* ds_base = reinterpret_cast<int32_t*>(out + l.ds_off);
  int64_t ds_total = 0;
  for (int s = 0; s < numseqs; ++s) {
    ds_base[s] = (int32_t)std::min<int64_t>(ds_total, 0x7fffffff);
    ds_total += ds_seg_blocks(prefix[s], prefix[s] + causal[s]);
  }
  const int32_t ds_blocks = (int32_t)std::min<int64_t>(ds_total, 0x7fffffff);
  ds_base[numseqs > 0 ? numseqs : 0] = ds_blocks;
  struct Item {
    int cost, s, t;
  };
  std::vector<Item> v;
  for (int i = 0; i < kLists; ++i) {
    v.clear();
    for (int s = 0; s < numseqs; ++s) {
      const int L = prefix[s] + causal[s];
      const int p = is_causal ? 0 : prefix[s];
      const int nt = (L + d[i].tile - 1) / d[i].tile;
      for (int t = 0; t < nt; ++t) v.push_back({tile_cost(d[i].mode, t, d[i].tile, d[i].inner, p, L), s, t});
    }
    std::stable_sort(v.begin(), v.end(), [](const Item& a, const Item& b) { return a.cost > b.cost; });
    WsHeader h{};
    h.n_items = (int32_t)std::min<int64_t>((int64_t)v.size(), l.nmax[i]);
    h.error = 0;
    h.pad[0] = kPlanMagic;
    h.pad[1] = numseqs;
    h.pad[2] = total;
    h.pad[3] = d[i].tile;
    h.pad[4] = ds_blocks;
    memcpy(out + l.hdr_off[i], &h, sizeof(h));
    int32_t* items = reinterpret_cast<int32_t*>(out + l.items_off[i]);
    for (int32_t k = 0; k < h.n_items; ++k) {
      items[2 * k] = v[k].s;
      items[2 * k + 1] = v[k].t;
    }
  }
  return 0;
}

}  // namespace plan
}  // namespace prefixlm
