// Host-side block-sparse tile plan for the VDN-H3 local-window attention.
//
// The reference builds its key sets per window run (vdn_h3/window.py:248-270) and
// gathers the selected K/V rows into copies (vdn_h3/window.py:233-245, :411-430), or
// evaluates a per-element mask (vdn_h3/window.py:327-344). Here the same allowed-key
// rule is turned into a static list of (query block, key tile) work: query rows are
// grouped into runs of rows that share one key set, each run's key set is a handful of
// half-open intervals, and each interval is covered by block_n-aligned key tiles with
// a valid [lo, hi) sub-range. The attention kernel reads K/V in place; only the first
// and last tile of an interval carry a column mask.
#include <algorithm>
#include <cstdint>
#include <vector>

#include "common.h"

namespace {

struct Interval {
  int64_t a, b;
  bool operator==(const Interval &o) const { return a == o.a && b == o.b; }
};
using KeySet = std::vector<Interval>;

struct Geometry {
  int seq, vs, ve, frames, tpf, anchor;
  const int32_t *bounds;
};

int validate(const Geometry &g, int block_m, int block_n) {
  using vdnh3::set_error;
  if (g.anchor < VDNH3_ANCHOR_NONE || g.anchor > VDNH3_ANCHOR_BOTH)
    return set_error(VDNH3_ERR_INVALID, "anchor_frames mode %d; expected 0..3 (none, columns, rows, both)", g.anchor);
  if (g.frames <= 0 || g.tpf <= 0)
    return set_error(VDNH3_ERR_INVALID, "num_frames and tokens_per_frame must be positive");
  if (!(0 <= g.vs && g.vs <= g.ve && g.ve <= g.seq))
    return set_error(VDNH3_ERR_INVALID, "video range is outside the packed sequence");
  if (int64_t(g.ve) - g.vs != int64_t(g.frames) * g.tpf)
    return set_error(VDNH3_ERR_INVALID, "video range does not equal num_frames * tokens_per_frame");
  if (g.bounds == nullptr) return set_error(VDNH3_ERR_INVALID, "bounds must contain exactly one entry per frame");
  for (int f = 0; f < g.frames; ++f) {
    int lo = g.bounds[2 * f], hi = g.bounds[2 * f + 1];
    if (lo > f || hi < f || lo > hi)
      return set_error(VDNH3_ERR_INVALID, "bounds[%d]=(%d, %d) does not contain its query frame", f, lo, hi);
  }
  if (block_m <= 0 || block_n <= 0 || block_n > 32768)
    return set_error(VDNH3_ERR_INVALID, "invalid tile sizes block_m=%d block_n=%d", block_m, block_n);
  return VDNH3_OK;
}

KeySet merge(std::vector<Interval> pieces) {
  std::sort(pieces.begin(), pieces.end(), [](const Interval &x, const Interval &y) { return x.a < y.a; });
  KeySet out;
  for (const Interval &p : pieces) {
    if (p.a >= p.b) continue;
    if (!out.empty() && out.back().b >= p.a)
      out.back().b = std::max(out.back().b, p.b);
    else
      out.push_back(p);
  }
  return out;
}

// Key set of one video frame (the rule of vdn_h3/window.py:331-342).
KeySet frame_keys(const Geometry &g, int f) {
  const bool anchor_rows = g.anchor == VDNH3_ANCHOR_ROWS || g.anchor == VDNH3_ANCHOR_BOTH;
  const bool anchor_cols = g.anchor == VDNH3_ANCHOR_COLUMNS || g.anchor == VDNH3_ANCHOR_BOTH;
  const int last = g.frames - 1;
  if (anchor_rows && (f == 0 || f == last)) return KeySet{{0, g.seq}};
  int lo = std::max(g.bounds[2 * f], 0), hi = std::min(g.bounds[2 * f + 1], last);
  std::vector<Interval> pieces;
  pieces.push_back({0, g.vs});
  pieces.push_back({g.ve, g.seq});
  pieces.push_back({g.vs + int64_t(lo) * g.tpf, g.vs + int64_t(hi + 1) * g.tpf});
  if (anchor_cols) {
    pieces.push_back({g.vs, g.vs + int64_t(g.tpf)});
    pieces.push_back({g.vs + int64_t(last) * g.tpf, g.ve});
  }
  return merge(pieces);
}

struct Run {
  int64_t q0, q1;
  KeySet keys;
};

std::vector<Run> runs_of(const Geometry &g) {
  std::vector<Run> segs;
  const KeySet dense{{0, g.seq}};
  if (g.vs > 0) segs.push_back({0, g.vs, dense});
  for (int f = 0; f < g.frames; ++f)
    segs.push_back({g.vs + int64_t(f) * g.tpf, g.vs + int64_t(f + 1) * g.tpf, frame_keys(g, f)});
  if (g.ve < g.seq) segs.push_back({g.ve, g.seq, dense});
  std::vector<Run> runs;
  for (Run &s : segs) {
    if (!runs.empty() && runs.back().q1 == s.q0 && runs.back().keys == s.keys)
      runs.back().q1 = s.q1;
    else
      runs.push_back(std::move(s));
  }
  return runs;
}

void tiles_of(const KeySet &keys, int block_n, std::vector<int32_t> *tiles) {
  for (const Interval &iv : keys) {
    for (int64_t ks = (iv.a / block_n) * block_n; ks < iv.b; ks += block_n) {
      int64_t lo = std::max(iv.a, ks) - ks, hi = std::min(iv.b, ks + block_n) - ks;
      tiles->push_back(int32_t(ks));
      tiles->push_back(int32_t(lo | (hi << 16)));
    }
  }
}

struct Plan {
  std::vector<int32_t> items, tiles;
  int64_t pairs = 0;
};

Plan make_plan(const Geometry &g, int block_m, int block_n) {
  Plan p;
  struct Item {
    int32_t q0, q1, off, cnt;
  };
  std::vector<Item> items;
  for (const Run &r : runs_of(g)) {
    int64_t keys = 0;
    for (const Interval &iv : r.keys) keys += iv.b - iv.a;
    p.pairs += keys * (r.q1 - r.q0);
    int32_t off = int32_t(p.tiles.size() / 2);
    tiles_of(r.keys, block_n, &p.tiles);
    int32_t cnt = int32_t(p.tiles.size() / 2) - off;
    for (int64_t q = r.q0; q < r.q1; q += block_m)
      items.push_back({int32_t(q), int32_t(std::min(r.q1, q + block_m)), off, cnt});
  }
  std::stable_sort(items.begin(), items.end(), [](const Item &x, const Item &y) { return x.cnt > y.cnt; });
  for (const Item &it : items) {
    p.items.push_back(it.q0);
    p.items.push_back(it.q1);
    p.items.push_back(it.off);
    p.items.push_back(it.cnt);
  }
  return p;
}

}  // namespace

extern "C" int vdnh3_window_plan_size(int seq, int video_start, int video_end, int num_frames,
                                      int tokens_per_frame, const int32_t *bounds, int anchor_mode,
                                      int block_m, int block_n, int32_t *n_items, int32_t *n_tiles,
                                      int64_t *pairs_per_head) {
  Geometry g{seq, video_start, video_end, num_frames, tokens_per_frame, anchor_mode, bounds};
  int rc = validate(g, block_m, block_n);
  if (rc) return rc;
  Plan p = make_plan(g, block_m, block_n);
  if (n_items) *n_items = int32_t(p.items.size() / 4);
  if (n_tiles) *n_tiles = int32_t(p.tiles.size() / 2);
  if (pairs_per_head) *pairs_per_head = p.pairs;
  return VDNH3_OK;
}

extern "C" int vdnh3_window_plan_build(int seq, int video_start, int video_end, int num_frames,
                                       int tokens_per_frame, const int32_t *bounds, int anchor_mode,
                                       int block_m, int block_n, int32_t *items, int32_t n_items,
                                       int32_t *tiles, int32_t n_tiles) {
  Geometry g{seq, video_start, video_end, num_frames, tokens_per_frame, anchor_mode, bounds};
  int rc = validate(g, block_m, block_n);
  if (rc) return rc;
  Plan p = make_plan(g, block_m, block_n);
  if (int64_t(n_items) * 4 != int64_t(p.items.size()) || int64_t(n_tiles) * 2 != int64_t(p.tiles.size()))
    return vdnh3::set_error(VDNH3_ERR_INVALID, "plan buffers have %d items / %d tiles; the plan needs %zu / %zu",
                            n_items, n_tiles, p.items.size() / 4, p.tiles.size() / 2);
  std::copy(p.items.begin(), p.items.end(), items);
  std::copy(p.tiles.begin(), p.tiles.end(), tiles);
  return VDNH3_OK;
}
