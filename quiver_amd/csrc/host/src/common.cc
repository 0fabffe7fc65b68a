#include <algorithm>
#include <iterator>

#include "quiver/common.h"

namespace quiver {

namespace {

struct MetricAlias {
  std::string_view name;
  Metric metric;
};

// Every spelling parse_metric accepts (include/quiver/common.h:35-36 of the reference lists
// them); the first spelling of each metric is its canonical name, which to_string returns.
constexpr MetricAlias kAliases[] = {
    {"l2", Metric::kL2},          {"euclidean", Metric::kL2},         {"ip", Metric::kInnerProduct},
    {"inner_product", Metric::kInnerProduct}, {"dot", Metric::kInnerProduct},
    {"cosine", Metric::kCosine},  {"cos", Metric::kCosine},           {"angular", Metric::kCosine},
};

}  // namespace

std::string_view to_string(Metric metric) noexcept {
  const auto* hit = std::find_if(std::begin(kAliases), std::end(kAliases),
                                 [metric](const MetricAlias& a) { return a.metric == metric; });
  return hit == std::end(kAliases) ? std::string_view("unknown") : hit->name;
}

Metric parse_metric(std::string_view name) {
  const auto* hit = std::find_if(std::begin(kAliases), std::end(kAliases),
                                 [name](const MetricAlias& a) { return a.name == name; });
  // The message is part of the API: the Python layer surfaces it as the ValueError text.
  QUIVER_CHECK(hit != std::end(kAliases),
               "unknown metric '" + std::string(name) + "' (expected l2, ip, or cosine)");
  return hit->metric;
}

[[noreturn]] void detail::throw_error(const std::string& message) { throw Error(message); }

}  // namespace quiver
