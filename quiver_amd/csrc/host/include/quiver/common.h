// Core vocabulary of the Quiver C++ API, kept name-for-name with the reference
// (include/quiver/common.h:14-76) so code written against it compiles unchanged.
#pragma once

#include <cstddef>
#include <cstdint>
#include <limits>
#include <stdexcept>
#include <string>
#include <string_view>

namespace quiver {

/// Caller-visible identifier attached to every stored vector.
using Label = std::uint64_t;
/// Dense internal row / node identifier.
using NodeId = std::uint32_t;

/// Largest supported vector dimensionality.
inline constexpr std::size_t kMaxDimension = 65536;

/// Marks result slots that could not be filled (k larger than the index or the filter admits).
inline constexpr Label kInvalidLabel = std::numeric_limits<Label>::max();

/// Distance conventions, smaller is closer: kL2 = squared Euclidean distance,
/// kInnerProduct = 1 - <q, x>, kCosine = 1 - cos(q, x) (vectors are normalized on insert and
/// query).
enum class Metric : std::uint32_t { kL2 = 0, kInnerProduct = 1, kCosine = 2 };

std::string_view to_string(Metric metric) noexcept;
/// Accepts "l2"/"euclidean", "ip"/"inner_product"/"dot", "cosine"/"cos"/"angular".
Metric parse_metric(std::string_view name);

struct Neighbor {
  float distance;
  Label label;

  friend constexpr bool operator<(const Neighbor& a, const Neighbor& b) noexcept {
    return a.distance < b.distance || (a.distance == b.distance && a.label < b.label);
  }
  friend constexpr bool operator==(const Neighbor&, const Neighbor&) noexcept = default;
};

/// How an index file is brought into memory (kept for API compatibility).
struct LoadOptions {
  bool mmap = false;
  bool verify_checksums = true;
};

/// Every recoverable failure (bad arguments, device errors) is thrown as this.
class Error : public std::runtime_error {
 public:
  using std::runtime_error::runtime_error;
};

namespace detail {
[[noreturn]] void throw_error(const std::string& message);
}  // namespace detail

}  // namespace quiver

/// Throws quiver::Error when `cond` is false; `message` is evaluated only then.
#define QUIVER_CHECK(cond, message)             \
  do {                                          \
    if (!(cond)) [[unlikely]] {                 \
      ::quiver::detail::throw_error((message)); \
    }                                           \
  } while (0)
