// CPU replay of the stored-tile attention backward's addressing (test infrastructure).
//
// The dQ kernel (taylor_attention_bwd_q_kernel with STORE) writes the P and dS
// series of every visited 16 x 16 (query, key) tile into the workspace; the
// dK/dV kernel (taylor_attention_bwd_kv_mat_kernel) reads them back. This
// program runs, on the host, the kernels' own index functions
// (attn_bwd_q_item, attn_key_range, attn_tile_offset, attn_bwd_kv_item,
// attn_query_range, attn_tile_consumer_offset, attention_bwd_layout and the
// Mfma16 accumulator layouts, all __host__ __device__) for every workgroup,
// wave, lane, register and block of the two grids, and checks:
//   * every producer store and consumer load lies inside the workspace and
//     inside its own (P or dS, order) slot;
//   * no tile element is written twice;
//   * consumer loads of four values are aligned to four elements;
//   * every admissible (query, key) pair is read by exactly one consumer lane
//     per head-dim slice, from the element the producer wrote for that pair.
// Modes:
//   "current"        the layout of the built kernels, float (the one in use);
//   "current-double" the same layout with float64's accumulator rows
//                    (acc_row = 4 r + h): expected to misassign values, which
//                    is why the stored-tile kernels refuse float64 at compile time;
//   "old-double"     the float64 layout of the first stored-tile build (tile
//                    element (row_group(q) * 16 + k) * 4 + row_reg(q), consumer
//                    lane l reading elements 4 l .. 4 l + 3), the build in which
//                    a float64 run took a GPU memory fault.
// Prints one line per mode: "<mode> cases=N stores=N loads=N bounds=N dup=N
// align=N mismatch=N uncovered=N"; exit status 0.
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

#include "taylor_attention_bwd.inl"

using namespace pt;

namespace {

enum Mode { kCurrent = 0, kCurrentDouble = 1, kOldDouble = 2 };

struct Counts {
  long cases = 0, stores = 0, loads = 0, bounds = 0, dup = 0, align = 0, mismatch = 0, uncovered = 0;
};

struct Shape {
  int bh, L, S, mask;   // mask: 0 none, 1 causal, 2 window, 3 random with an empty query row
};

std::vector<uint8_t> make_mask(int L, int S, int kind, unsigned seed) {
  std::vector<uint8_t> m(static_cast<size_t>(L) * S, 0);
  std::mt19937 rng(seed);
  for (int i = 0; i < L; ++i)
    for (int j = 0; j < S; ++j) {
      if (kind == 2) m[static_cast<size_t>(i) * S + j] = (j <= i && i - j <= 37) ? 1 : 0;
      if (kind == 3) m[static_cast<size_t>(i) * S + j] = (rng() % 4 == 0 && i != L / 2) ? 1 : 0;
    }
  return m;
}

// Block ranges of a boolean mask from their definition: for each 64-row query block
// the first and one-past-last admissible key, then for each 64-key block the first
// and one-past-last admitting query ((0, 0) when none).
std::vector<int32_t> ranges_of(const std::vector<uint8_t>& m, int L, int S) {
  const int nqb = (L + 63) / 64, nkb = (S + 63) / 64;
  std::vector<int32_t> r(2 * (nqb + nkb), 0);
  for (int b = 0; b < nqb; ++b) {
    int lo = S, hi = -1;
    for (int i = b * 64; i < L && i < b * 64 + 64; ++i)
      for (int j = 0; j < S; ++j)
        if (m[static_cast<size_t>(i) * S + j]) { lo = j < lo ? j : lo; hi = j > hi ? j : hi; }
    r[2 * b] = hi >= 0 ? lo : 0;
    r[2 * b + 1] = hi >= 0 ? hi + 1 : 0;
  }
  for (int b = 0; b < nkb; ++b) {
    int lo = L, hi = -1;
    for (int i = 0; i < L; ++i)
      for (int j = b * 64; j < S && j < b * 64 + 64; ++j)
        if (m[static_cast<size_t>(i) * S + j]) { lo = i < lo ? i : lo; hi = i > hi ? i : hi; }
    r[2 * (nqb + b)] = hi >= 0 ? lo : 0;
    r[2 * (nqb + b) + 1] = hi >= 0 ? hi + 1 : 0;
  }
  return r;
}

template <typename MF>
int64_t producer_offset(Mode mode, int64_t head, int qt, int kt, int nqt, int nkt, int qi, int ki) {
  if (mode == kOldDouble)
    return attn_tile_base(head, qt, kt, nqt, nkt) + (MF::row_group(qi) * 16 + ki) * 4 + MF::row_reg(qi);
  return attn_tile_offset(head, qt, kt, nqt, nkt, qi, ki);
}

int64_t consumer_offset(Mode mode, int64_t head, int qt, int kt, int nqt, int nkt, int c, int h) {
  if (mode == kOldDouble) return attn_tile_base(head, qt, kt, nqt, nkt) + (16 * h + c) * 4;
  return attn_tile_consumer_offset(head, qt, kt, nqt, nkt, c, h);
}

template <typename T, int K, int D>
void check_case(Mode mode, const Shape& sh, Counts& n) {
  using MF = Mfma16<T>;
  using A = typename AccOf<T>::type;
  using Plan = AttnBwdPlan<T, K, D>;
  if constexpr (!Plan::fits) {
    return;
  } else {
    const int bh = sh.bh, L = sh.L, S = sh.S;
    const int causal = sh.mask == 1;
    std::vector<uint8_t> mask;
    std::vector<int32_t> ranges;
    if (sh.mask >= 2) {
      mask = make_mask(L, S, sh.mask, 1234u + L * 7u + S);
      ranges = ranges_of(mask, L, S);
    }
    const int32_t* rg = ranges.empty() ? nullptr : ranges.data();
    auto admissible = [&](int q, int k) {
      if (q < 0 || q >= L || k < 0 || k >= S) return false;
      if (causal && k > q) return false;
      if (!mask.empty() && !mask[static_cast<size_t>(q) * S + k]) return false;
      return true;
    };
    const int nqt = (L + 15) / 16, nkt = (S + 15) / 16;
    const int64_t elems = static_cast<int64_t>(bh) * nqt * nkt * 256;   // per (P or dS, order) buffer
    const AttnBwdLayout lay = attention_bwd_layout(sizeof(A), sizeof(T), K, bh, L, S, true);
    // the C ABI sizes the caller's workspace with (element, element) sizes: must agree
    const AttnBwdLayout api = attention_bwd_layout(sizeof(T), sizeof(T), K, bh, L, S, true);
    if (api.total != lay.total || lay.tiles_offset < lay.delta_bytes ||
        lay.tile_bytes < static_cast<size_t>(elems) * sizeof(T) ||
        lay.total != lay.tiles_offset + 2 * static_cast<size_t>(K + 1) * lay.tile_bytes)
      ++n.bounds;
    ++n.cases;

    // byte offset of element `at` of slot `slot` (P orders 0..K, then dS orders 0..K)
    auto slot_ok = [&](int64_t at, int slot) {
      if (at < 0 || at >= elems) return false;
      const size_t byte = lay.tiles_offset + static_cast<size_t>(slot) * lay.tile_bytes + at * sizeof(T);
      return byte + sizeof(T) <= lay.tiles_offset + static_cast<size_t>(slot + 1) * lay.tile_bytes &&
             byte + sizeof(T) <= lay.total;
    };

    // ---- producer: taylor_attention_bwd_q_kernel<T, K, D, NS_Q, STORE> ----
    std::vector<int64_t> owner(elems, -1);   // encoded (head, query, key) of the element's writer
    auto code = [&](int64_t head, int q, int k) { return (head * (L + 64) + q) * (S + 64) + k; };
    const int nqb = (L + kAttnBM - 1) / kAttnBM;
    const int slices_q = Plan::DB / Plan::NS_Q;
    for (int64_t t = 0; t < static_cast<int64_t>(nqb) * bh * slices_q; ++t) {
      int64_t head;
      int slice, q_block;
      attn_bwd_q_item(t, bh, nqb, slices_q, head, slice, q_block);
      int lo, hi;
      attn_key_range(S, q_block, causal, rg, lo, hi);
      for (int wave = 0; wave < kAttnWaves; ++wave) {
        if (!(slice == 0 && q_block + wave * kAttnQPerWave < L)) continue;   // the kernel's STORE guard
        for (int lane = 0; lane < kWave; ++lane) {
          const int c = lane % 16, h = lane / 16;
          const int my_q = q_block + wave * kAttnQPerWave + c;
          for (int kb0 = lo; kb0 < hi; kb0 += kAttnBN)
            for (int r = 0; r < 4; ++r) {
              const int key = kb0 + MF::acc_row(h, r);
              const int64_t at =
                  producer_offset<MF>(mode, head, q_block / 16 + wave, kb0 / 16, nqt, nkt, c, MF::acc_row(h, r));
              ++n.stores;
              bool ok = true;
              for (int slot = 0; slot < 2 * (K + 1); ++slot) ok = ok && slot_ok(at, slot);
              if (!ok) { ++n.bounds; continue; }
              if (owner[at] != -1) ++n.dup;
              owner[at] = code(head, my_q, key);
            }
        }
      }
    }

    // ---- consumer: taylor_attention_bwd_kv_mat_kernel<T, K, D, NS_KM, WHAT> ----
    const int nkb = (S + 63) / 64;
    const int slices_k = Plan::DB / Plan::NS_KM;
    std::vector<uint8_t> seen(static_cast<size_t>(bh) * L * S * slices_k, 0);
    for (int64_t t = 0; t < static_cast<int64_t>(nkb) * bh * slices_k; ++t) {
      int64_t head;
      int slice, kv_block;
      attn_bwd_kv_item(t, bh, slices_k, head, slice, kv_block);
      int lo, hi;
      attn_query_range(L, kv_block, causal, rg, lo, hi);
      for (int wave = 0; wave < kAttnWaves; ++wave) {
        const int kt = (kv_block / 16 + wave) < nkt - 1 ? kv_block / 16 + wave : nkt - 1;
        for (int lane = 0; lane < kWave; ++lane) {
          const int c = lane % 16, h = lane / 16;
          const int my_k = kv_block + wave * 16 + c;
          for (int qb0 = lo; qb0 < hi; qb0 += 16) {
            const int64_t at = consumer_offset(mode, head, qb0 / 16, kt, nqt, nkt, c, h);
            ++n.loads;
            if (at % 4 != 0) ++n.align;
            bool ok = true;
            for (int slot = 0; slot < 2 * (K + 1); ++slot) ok = ok && slot_ok(at, slot) && slot_ok(at + 3, slot);
            if (!ok) { ++n.bounds; continue; }
            for (int s = 0; s < 4; ++s) {
              const int q = qb0 + MF::acc_row(h, s);   // the query the kernel assigns to value s
              if (!admissible(q, my_k)) continue;      // masked to zero by the kernel
              if (owner[at + s] != code(head, q, my_k)) ++n.mismatch;
              uint8_t& mark = seen[((static_cast<size_t>(head) * L + q) * S + my_k) * slices_k + slice];
              if (mark) ++n.dup;
              mark = 1;
            }
          }
        }
      }
    }
    for (int64_t head = 0; head < bh; ++head)
      for (int q = 0; q < L; ++q)
        for (int k = 0; k < S; ++k)
          if (admissible(q, k))
            for (int sl = 0; sl < slices_k; ++sl)
              if (!seen[((static_cast<size_t>(head) * L + q) * S + k) * slices_k + sl]) ++n.uncovered;
  }
}

template <typename T, int K>
void check_degree(Mode mode, const std::vector<Shape>& shapes, Counts& n) {
  for (const Shape& sh : shapes) {
    check_case<T, K, 16>(mode, sh, n);
    check_case<T, K, 32>(mode, sh, n);
    check_case<T, K, 64>(mode, sh, n);
    check_case<T, K, 128>(mode, sh, n);
  }
}

template <typename T>
void check_all(Mode mode, const char* name, const std::vector<Shape>& shapes) {
  Counts n;
  check_degree<T, 0>(mode, shapes, n);
  check_degree<T, 1>(mode, shapes, n);
  check_degree<T, 2>(mode, shapes, n);
  check_degree<T, 3>(mode, shapes, n);
  check_degree<T, 4>(mode, shapes, n);
  check_degree<T, 5>(mode, shapes, n);
  check_degree<T, 6>(mode, shapes, n);
  check_degree<T, 7>(mode, shapes, n);
  check_degree<T, 8>(mode, shapes, n);
  std::printf("%s cases=%ld stores=%ld loads=%ld bounds=%ld dup=%ld align=%ld mismatch=%ld uncovered=%ld\n", name,
              n.cases, n.stores, n.loads, n.bounds, n.dup, n.align, n.mismatch, n.uncovered);
}

}  // namespace

int main() {
  std::vector<Shape> shapes;
  const int lengths[][2] = {{1, 1}, {15, 17}, {16, 16}, {64, 64}, {33, 70}, {70, 33}, {150, 150}, {129, 200}};
  for (const auto& ls : lengths)
    for (int mask = 0; mask < 4; ++mask) {
      if (mask == 1 && ls[0] != ls[1]) continue;   // causal is square here, as in the tests
      shapes.push_back(Shape{2, ls[0], ls[1], mask});
    }
  check_all<float>(kCurrent, "current", shapes);
  check_all<double>(kCurrentDouble, "current-double", shapes);
  check_all<double>(kOldDouble, "old-double", shapes);
  return 0;
}
