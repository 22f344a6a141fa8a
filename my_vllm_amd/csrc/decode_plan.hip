// Host-side planners of the paged decode launch: the per-step scheduling the
// reference hands to FlashInfer's BatchDecodeWithPagedKVCacheWrapper.plan
// (nanovllm/layers/attention_backend.py:769-894), done here for this
// library's decode kernel.  Both cut every (sequence, KV head) segment of a
// decode batch into pieces of 8 int32:
//   {seq, page_begin, page_end, chunk, n_chunks, part_base, q_row, kv_head}
// where a segment cut into n_chunks > 1 pieces is split-K: chunk k of it
// writes partial slot (part_base + k) * Hkv + kv_head.  The merge list is the
// chunk-0 piece of every split segment, in piece order.
//
// No device code and no HIP calls: these run on the host once per step and
// only fill caller-provided arrays.
#include "mva_capi.h"

#include <algorithm>
#include <cstdint>
#include <limits>
#include <vector>

namespace mva {
namespace {

constexpr int kItemInts = 8;
constexpr int kMaxPiecePages = 128;  // the decode kernel's longest piece

struct Piece {
  int64_t begin, end;  // absolute page offsets in the batch
  int32_t seq, group;
};

// Validates the block counts and returns their prefix sums (size n + 1), or
// an empty vector after recording an error.
std::vector<int64_t> page_offsets(const int64_t* counts, int64_t n) {
  std::vector<int64_t> offsets((size_t)n + 1, 0);
  for (int64_t s = 0; s < n; ++s) {
    if (counts[s] <= 0 || counts[s] > std::numeric_limits<int32_t>::max()) {
      set_error("decode plan: every decode sequence needs 1 .. 2^31-1 pages");
      return {};
    }
    offsets[(size_t)s + 1] = offsets[(size_t)s] + counts[s];
  }
  return offsets;
}

bool rows_fit_int32(int64_t first_seq, int64_t first_q_row, int64_t n) {
  const int64_t top = std::numeric_limits<int32_t>::max();
  return first_seq >= 0 && first_q_row >= 0 && first_seq + n - 1 <= top && first_q_row + n - 1 <= top;
}

void write_piece(int32_t* row, int64_t seq_index, int64_t first_seq, int64_t first_q_row, int64_t begin,
                 int64_t end, int64_t chunk, int64_t n_chunks, int64_t part_base, int kv_head) {
  row[0] = (int32_t)(first_seq + seq_index);
  row[1] = (int32_t)begin;
  row[2] = (int32_t)end;
  row[3] = (int32_t)chunk;
  row[4] = (int32_t)n_chunks;
  row[5] = (int32_t)part_base;
  row[6] = (int32_t)(first_q_row + seq_index);
  row[7] = kv_head;
}

// Copies the chunk-0 rows of split segments into `merges`; returns their
// count, or -1 when `merge_rows` is too small.
int64_t collect_merges(const int32_t* items, int64_t num_items, int32_t* merges, int64_t merge_rows) {
  int64_t m = 0;
  for (int64_t i = 0; i < num_items; ++i) {
    const int32_t* row = items + i * kItemInts;
    if (row[3] != 0 || row[4] <= 1) continue;
    if (m >= merge_rows) return -1;
    std::copy(row, row + kItemInts, merges + m * kItemInts);
    ++m;
  }
  return m;
}

}  // namespace
}  // namespace mva

extern "C" int64_t mva_decode_plan_listed_rows(int64_t num_seqs, int64_t total_pages, int num_kv_heads,
                                               int num_groups, int max_piece_pages) {
  if (num_seqs < 0 || total_pages < 0 || num_kv_heads <= 0 || num_groups <= 0 || max_piece_pages < 1 ||
      max_piece_pages > mva::kMaxPiecePages)
    return -1;
  if (num_seqs == 0) return 0;
  const int64_t groups = std::max<int64_t>(1, std::min<int64_t>(num_groups, total_pages));
  // The range and sequence boundaries cut the pages into at most
  // groups + num_seqs - 1 intervals; an interval of L pages gives
  // ceil(L / max_piece_pages) <= L / max_piece_pages + 1 pieces.
  return (groups + num_seqs + total_pages / max_piece_pages) * num_kv_heads;
}

extern "C" int mva_decode_plan_listed(const int64_t* block_counts, int64_t num_seqs, int64_t first_seq,
                                      int64_t first_q_row, int num_kv_heads, int num_groups, int max_piece_pages,
                                      int32_t* items, int64_t item_rows, int32_t* wave_extra,
                                      int64_t wave_extra_len, int32_t* merges, int64_t merge_rows,
                                      int64_t* out_counts) {
  using namespace mva;
  if (num_seqs < 0 || num_kv_heads <= 0 || num_groups <= 0 || out_counts == nullptr || wave_extra == nullptr ||
      wave_extra_len < 1)
    return set_error("decode plan: invalid arguments");
  if (max_piece_pages < 1 || max_piece_pages > kMaxPiecePages)
    return set_error("decode plan: piece length must be in [1, 128] pages");
  for (int i = 0; i < 4; ++i) out_counts[i] = 0;
  if (num_seqs == 0) {
    wave_extra[0] = 0;
    return 0;
  }
  if (block_counts == nullptr || items == nullptr) return set_error("decode plan: invalid arguments");
  if (!rows_fit_int32(first_seq, first_q_row, num_seqs))
    return set_error("decode plan: sequence or query row index out of int32 range");
  const std::vector<int64_t> offsets = page_offsets(block_counts, num_seqs);
  if (offsets.empty()) return -1;
  const int64_t total = offsets.back();
  const int64_t groups = std::max<int64_t>(1, std::min<int64_t>(num_groups, total));
  const int64_t hkv = num_kv_heads;
  const int64_t waves = groups * hkv;
  if (waves > std::numeric_limits<int32_t>::max() || wave_extra_len < waves + 1)
    return set_error("decode plan: wave_extra needs groups * num_kv_heads + 1 entries");
  // Range g holds pages [g * total / groups, (g + 1) * total / groups),
  // evaluated as g * q + g * r / groups (total = q * groups + r) so that no
  // product overflows: g * r < groups^2 < 2^62.
  const int64_t quot = total / groups, rem = total % groups;
  auto bound = [&](int64_t g) { return g * quot + g * rem / groups; };

  // Pieces in page order: walk the union of range and sequence boundaries;
  // each interval between consecutive boundaries lies in one range and one
  // sequence and is cut into ceil(L / max_piece_pages) near-equal pieces.
  std::vector<Piece> pieces;
  pieces.reserve((size_t)(groups + num_seqs + total / max_piece_pages));
  std::vector<int64_t> group_first((size_t)groups + 1, 0);
  int64_t pos = 0, g = 0, s = 0;
  while (pos < total) {
    const int64_t end = std::min(bound(g + 1), offsets[(size_t)s + 1]);
    const int64_t len = end - pos;
    if (len <= max_piece_pages) {
      pieces.push_back({pos, end, (int32_t)s, (int32_t)g});
    } else {
      const int64_t ncut = (len + max_piece_pages - 1) / max_piece_pages;
      for (int64_t k = 0; k < ncut; ++k)
        pieces.push_back({pos + k * len / ncut, pos + (k + 1) * len / ncut, (int32_t)s, (int32_t)g});
    }
    pos = end;
    if (end == bound(g + 1)) group_first[(size_t)++g] = (int64_t)pieces.size();
    if (end == offsets[(size_t)s + 1]) ++s;
  }
  const int64_t np = (int64_t)pieces.size();
  if (np * hkv > item_rows) return set_error("decode plan: item capacity too small");
  if (np * hkv > std::numeric_limits<int32_t>::max())  // wave_extra holds int32 row indices
    return set_error("decode plan: more than 2^31-1 pieces");

  // Chunk numbers in page order, and the partial slots of split sequences.
  std::vector<int64_t> per_seq((size_t)num_seqs, 0), part_base((size_t)num_seqs, 0), chunk((size_t)np);
  for (int64_t i = 0; i < np; ++i) chunk[(size_t)i] = per_seq[(size_t)pieces[(size_t)i].seq]++;
  int64_t slots = 0;
  for (int64_t q = 0; q < num_seqs; ++q) {
    part_base[(size_t)q] = slots;
    if (per_seq[(size_t)q] > 1) slots += per_seq[(size_t)q];
  }
  if (slots > std::numeric_limits<int32_t>::max()) return set_error("decode plan: more than 2^31-1 partial slots");

  // Wavefront w = g * Hkv + h streams head h of range g's pieces: its first
  // piece at row w, the rest (page order) at rows wave_extra[w] ..
  // wave_extra[w + 1] - 1 after all first pieces.
  auto emit = [&](int64_t row, int64_t i, int h) {
    const Piece& p = pieces[(size_t)i];
    const int64_t base = offsets[(size_t)p.seq];
    write_piece(items + row * kItemInts, p.seq, first_seq, first_q_row, p.begin - base, p.end - base,
                chunk[(size_t)i], per_seq[(size_t)p.seq], part_base[(size_t)p.seq], h);
  };
  int64_t cursor = waves;
  for (int64_t gg = 0; gg < groups; ++gg)
    for (int h = 0; h < num_kv_heads; ++h) {
      const int64_t w = gg * hkv + h;
      emit(w, group_first[(size_t)gg], h);
      wave_extra[w] = (int32_t)cursor;
      for (int64_t i = group_first[(size_t)gg] + 1; i < group_first[(size_t)gg + 1]; ++i) emit(cursor++, i, h);
    }
  wave_extra[waves] = (int32_t)cursor;
  const int64_t num_merges = merges != nullptr ? collect_merges(items, cursor, merges, merge_rows) : 0;
  if (num_merges < 0) return set_error("decode plan: merge capacity too small");
  out_counts[0] = cursor;
  out_counts[1] = waves;
  out_counts[2] = slots;
  out_counts[3] = num_merges;
  return 0;
}

extern "C" int64_t mva_decode_plan_claims_rows(int64_t num_seqs, int64_t total_pages, int num_kv_heads,
                                               int min_piece_pages) {
  if (num_seqs < 0 || total_pages < 0 || num_kv_heads <= 0 || min_piece_pages < 1) return -1;
  // A segment of L pages gives ceil(L / piece) <= L / min_piece_pages + 1 pieces.
  return (total_pages / min_piece_pages + num_seqs) * num_kv_heads;
}

extern "C" int mva_decode_plan_claims(const int64_t* block_counts, int64_t num_seqs, int64_t first_seq,
                                      int64_t first_q_row, int num_kv_heads, int64_t num_waves,
                                      double pieces_per_wave, int min_piece_pages, int max_piece_pages,
                                      int32_t* items, int64_t item_rows, int32_t* merges, int64_t merge_rows,
                                      int64_t* out_counts) {
  using namespace mva;
  if (num_seqs < 0 || num_kv_heads <= 0 || out_counts == nullptr)
    return set_error("decode plan: invalid arguments");
  if (!(1 <= min_piece_pages && min_piece_pages <= max_piece_pages && max_piece_pages <= kMaxPiecePages))
    return set_error("decode plan: piece length bounds must satisfy 1 <= min <= max <= 128");
  for (int i = 0; i < 4; ++i) out_counts[i] = 0;
  if (num_seqs == 0) return 0;
  if (block_counts == nullptr || items == nullptr) return set_error("decode plan: invalid arguments");
  if (!rows_fit_int32(first_seq, first_q_row, num_seqs))
    return set_error("decode plan: sequence or query row index out of int32 range");
  const std::vector<int64_t> offsets = page_offsets(block_counts, num_seqs);
  if (offsets.empty()) return -1;
  const int64_t hkv = num_kv_heads;
  const int64_t total = offsets.back() * hkv;  // pages over all (sequence, KV head) segments
  // About pieces_per_wave pieces per wavefront, within the length bounds.
  const int64_t target =
      std::max<int64_t>(1, (int64_t)((double)num_waves * std::max(1.0, pieces_per_wave)));
  const int64_t piece =
      std::min<int64_t>(std::max<int64_t>((total + target - 1) / target, min_piece_pages), max_piece_pages);

  // Segments sequence-major, KV head fastest; each cut into ceil(L / piece)
  // near-equal pieces.  A stable bucket sort by length (longest first)
  // keeps that order among equal lengths.
  int64_t rows = 0, slots = 0;
  std::vector<int64_t> by_len((size_t)kMaxPiecePages + 2, 0);
  std::vector<int64_t> part_base((size_t)num_seqs);
  for (int64_t s = 0; s < num_seqs; ++s) {
    const int64_t len = block_counts[s];
    const int64_t n = (len + piece - 1) / piece;
    part_base[(size_t)s] = slots;
    if (n > 1) slots += n;
    for (int64_t k = 0; k < n; ++k) by_len[(size_t)((k + 1) * len / n - k * len / n)] += hkv;
    rows += n * hkv;
  }
  // Pieces are claimed by int32 index on the device.
  if (rows > std::numeric_limits<int32_t>::max()) return set_error("decode plan: more than 2^31-1 pieces");
  if (rows > item_rows) return set_error("decode plan: item capacity too small");
  if (slots > std::numeric_limits<int32_t>::max()) return set_error("decode plan: more than 2^31-1 partial slots");
  // Row where each length's pieces start, longest first.
  std::vector<int64_t> next((size_t)kMaxPiecePages + 2, 0);
  int64_t at = 0;
  for (int64_t len = kMaxPiecePages + 1; len >= 1; --len) {
    next[(size_t)len] = at;
    at += by_len[(size_t)len];
  }
  std::vector<int64_t> cut;
  for (int64_t s = 0; s < num_seqs; ++s) {
    const int64_t len = block_counts[s];
    const int64_t n = (len + piece - 1) / piece;
    cut.resize((size_t)n + 1);
    for (int64_t k = 0; k <= n; ++k) cut[(size_t)k] = k * len / n;  // the same cut for every KV head
    for (int h = 0; h < num_kv_heads; ++h)
      for (int64_t k = 0; k < n; ++k) {
        const int64_t b = cut[(size_t)k], e = cut[(size_t)k + 1];
        write_piece(items + (next[(size_t)(e - b)]++) * kItemInts, s, first_seq, first_q_row, b, e, k, n,
                    part_base[(size_t)s], h);
      }
  }
  const int64_t num_merges = merges != nullptr ? collect_merges(items, rows, merges, merge_rows) : 0;
  if (num_merges < 0) return set_error("decode plan: merge capacity too small");
  out_counts[0] = rows;
  out_counts[1] = std::max<int64_t>(1, std::min<int64_t>(num_waves, rows));
  out_counts[2] = slots;
  out_counts[3] = num_merges;
  return 0;
}
