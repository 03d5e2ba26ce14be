/*
 * MLX CPU argpartition — TEST INFRASTRUCTURE ONLY (part of the CPU oracle).
 *
 * The reference routes with argpartition(p, kth = E - k) (crates/model-serving/src/
 * qwen3_5_moe/model/routing.rs:27-42, through mlx_argpartition_axis,
 * crates/runtime-integration/src/mlx_operations.rs:364-373).  MLX 0.32.1's CPU backend (not
 * vendored: third-party/pins/mlx-v0.32.1.cmake) fills an index vector 0..n-1 and calls
 * std::nth_element on it with the comparator (value, index):
 *   comp(a, b) = v[a] < v[b] || (v[a] == v[b] && a < b)
 * so the selected set is the top-k of that total order and the order inside the slice is the
 * one the C++ library's nth_element leaves.  This file calls the host's libstdc++
 * std::nth_element itself with that comparator (values compared as floats, as MLX compares
 * bfloat16), so the slice order is the library's by construction, not a restatement.
 * NaN values are outside the contract (p = softmax output).
 */
#include <algorithm>
#include <cstdint>
#include <cstring>

extern "C" {

/* idx[0..n) = the index vector after std::nth_element(idx, idx + kth, idx + n, comp) over the
 * bf16 values v[0..n).  0 <= kth <= n. */
void orc_argpartition_bf16(const uint16_t *v, int32_t n, int32_t kth, uint32_t *idx) {
  for (int32_t i = 0; i < n; ++i) idx[i] = (uint32_t)i;
  if (n <= 0 || kth >= n) return;
  auto value = [v](uint32_t a) {
    const uint32_t u = (uint32_t)v[a] << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
  };
  std::nth_element(idx, idx + kth, idx + n, [&](uint32_t a, uint32_t b) {
    const float va = value(a), vb = value(b);
    return va < vb || (va == vb && a < b);
  });
}

/* Adversarial rows for the selection's heap fallback: runs std::nth_element(idx, idx + kth,
 * idx + n) with a comparator that decides its answers lazily (McIlroy's "gas" adversary:
 * undecided items compare above every decided one; comparing two undecided items fixes the
 * current pivot candidate to the next smallest rank), then gives the still-undecided items the
 * remaining ranks in index order.  ranks[i] is a permutation of 0..n-1 consistent with every
 * answer given, so std::nth_element on these ranks makes the same choices again: a run of
 * unbalanced partitions that ends in the heap selection once n is large enough. */
void orc_adversarial_ranks(int32_t n, int32_t kth, int32_t *ranks) {
  const int32_t gas = n;
  for (int32_t i = 0; i < n; ++i) ranks[i] = gas;
  int32_t solid = 0, cand = -1;
  uint32_t *idx = new uint32_t[(size_t)n + 1];
  for (int32_t i = 0; i < n; ++i) idx[i] = (uint32_t)i;
  if (n > 0 && kth < n)
    std::nth_element(idx, idx + kth, idx + n, [&](uint32_t x, uint32_t y) {
      if (ranks[x] == gas && ranks[y] == gas) {
        if ((int32_t)x == cand) ranks[x] = solid++;
        else ranks[y] = solid++;
      }
      if (ranks[x] == gas) cand = (int32_t)x;
      else if (ranks[y] == gas) cand = (int32_t)y;
      return ranks[x] < ranks[y] || (ranks[x] == ranks[y] && x < y);
    });
  for (int32_t i = 0; i < n; ++i)
    if (ranks[i] == gas) ranks[i] = solid++;
  delete[] idx;
}

}  // extern "C"
