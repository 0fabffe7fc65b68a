// Label filters restricting a search to a subset of the index, with the reference's interface
// (include/quiver/filter.h:24-102). The device path materializes a filter once per search_batch
// call as a bitmap over rows (flat) or over inverted-list positions (IVF-PQ).
#pragma once

#include <bit>
#include <cstddef>
#include <cstdint>
#include <functional>
#include <initializer_list>
#include <optional>
#include <unordered_set>
#include <utility>
#include <vector>

#include "quiver/common.h"

namespace quiver {

/// Decides which labels a search may return. contains() may run on any host thread and must not
/// call back into the index being searched.
class Filter {
 public:
  virtual ~Filter() = default;
  virtual bool contains(Label label) const = 0;
  /// Exact number of admitted labels, when cheap to know.
  virtual std::optional<std::size_t> cardinality() const { return std::nullopt; }
  /// Calls `fn` for every admitted label; false if enumeration is unsupported.
  virtual bool for_each(const std::function<void(Label)>& /*fn*/) const { return false; }
};

/// Dense bitset over labels [0, universe).
class BitsetFilter final : public Filter {
 public:
  explicit BitsetFilter(std::size_t universe) : bits_((universe + 63) / 64, 0), universe_(universe) {}

  void insert(Label label) {
    QUIVER_CHECK(label < universe_, "label outside BitsetFilter universe");
    std::uint64_t& word = bits_[label / 64];
    const std::uint64_t mask = std::uint64_t{1} << (label % 64);
    if ((word & mask) == 0) ++count_;
    word |= mask;
  }
  bool contains(Label label) const override {
    return label < universe_ && ((bits_[label / 64] >> (label % 64)) & 1u) != 0;
  }
  std::optional<std::size_t> cardinality() const override { return count_; }
  bool for_each(const std::function<void(Label)>& fn) const override {
    for (std::size_t w = 0; w < bits_.size(); ++w) {
      std::uint64_t word = bits_[w];
      while (word != 0) {
        fn(w * 64 + static_cast<unsigned>(std::countr_zero(word)));
        word &= word - 1;
      }
    }
    return true;
  }

 private:
  std::vector<std::uint64_t> bits_;
  std::size_t universe_;
  std::size_t count_ = 0;
};

/// Hash set of labels, for sparse or very large label values.
class LabelSetFilter final : public Filter {
 public:
  LabelSetFilter() = default;
  LabelSetFilter(std::initializer_list<Label> labels) : set_(labels) {}
  template <class It>
  LabelSetFilter(It first, It last) : set_(first, last) {}

  void insert(Label label) { set_.insert(label); }
  bool contains(Label label) const override { return set_.find(label) != set_.end(); }
  std::optional<std::size_t> cardinality() const override { return set_.size(); }
  bool for_each(const std::function<void(Label)>& fn) const override {
    for (Label l : set_) fn(l);
    return true;
  }

 private:
  std::unordered_set<Label> set_;
};

/// Arbitrary predicate over labels.
template <class Pred>
class PredicateFilter final : public Filter {
 public:
  explicit PredicateFilter(Pred pred) : pred_(std::move(pred)) {}
  bool contains(Label label) const override { return pred_(label); }

 private:
  Pred pred_;
};

}  // namespace quiver
