// The `.qvr` index container (format version 1), read and written bit-compatibly with the
// reference (src/internal/file_format.h:1-9, :27-58) so that an index saved by either side loads
// in the other:
//
//   offset 0     header, 64 bytes: magic "QUIVERDB", version u32 = 1, kind u32 (1 flat,
//                2 hnsw, 3 ivf-pq), endian tag u32 = 0x01020304, section count u32,
//                file size u64, CRC-32C of the section table u32, CRC-32C of the 40 header
//                bytes before this field u32, 24 reserved zero bytes
//   offset 64    section table: {tag u32 (four ASCII bytes, first byte lowest), CRC-32C u32,
//                offset u64, size u64} per section
//   ...          section payloads, each at a 64-byte aligned offset; the file is padded to the
//                aligned end of the last one
//
// Writes go to a temporary file that is synced and renamed over the target, so a reader never
// sees a partial file. Loading reads the whole file into host memory and validates every
// structural invariant (and, optionally, each section's checksum) before handing out spans.
#pragma once

#include <cstddef>
#include <cstdint>
#include <cstring>
#include <functional>
#include <memory>
#include <string>
#include <type_traits>
#include <vector>

#include "quiver/common.h"

namespace quiver::internal {

/// CRC-32C (Castagnoli, reflected polynomial 0x82F63B78), continuing from `crc` (0 to start).
std::uint32_t crc32c(const void* data, std::size_t size, std::uint32_t crc = 0) noexcept;

enum class ContainerKind : std::uint32_t { kFlat = 1, kHnsw = 2, kIvfPq = 3 };

constexpr std::uint32_t section_tag(const char (&s)[5]) noexcept {
  return static_cast<std::uint32_t>(static_cast<unsigned char>(s[0])) |
         static_cast<std::uint32_t>(static_cast<unsigned char>(s[1])) << 8 |
         static_cast<std::uint32_t>(static_cast<unsigned char>(s[2])) << 16 |
         static_cast<std::uint32_t>(static_cast<unsigned char>(s[3])) << 24;
}

/// Receives one section's bytes in order.
class SectionOut {
 public:
  virtual void put(const void* data, std::size_t size) = 0;

 protected:
  ~SectionOut() = default;
};

class ContainerWriter {
 public:
  using Producer = std::function<void(SectionOut&)>;

  explicit ContainerWriter(ContainerKind kind) : kind_(kind) {}

  /// A section of exactly `size` bytes, produced at commit time.
  void section(std::uint32_t tag, std::size_t size, Producer produce);
  /// A section backed by caller memory that stays valid until commit().
  void section_bytes(std::uint32_t tag, const void* data, std::size_t size);
  /// A section holding a copy of `value`'s bytes.
  template <typename T>
  void section_pod(std::uint32_t tag, const T& value) {
    static_assert(std::is_trivially_copyable_v<T>);
    section_copy(tag, &value, sizeof(T));
  }
  void section_copy(std::uint32_t tag, const void* data, std::size_t size);

  /// Writes the file (temporary file, fsync, rename over `path`).
  void commit(const std::string& path) const;

 private:
  struct Pending {
    std::uint32_t tag;
    std::size_t size;
    Producer produce;
    std::vector<std::byte> owned;  // payload of section_copy
  };
  ContainerKind kind_;
  std::vector<Pending> sections_;
};

class ContainerImage {
 public:
  /// Reads and validates `path`; throws quiver::Error naming the first problem found.
  static std::unique_ptr<ContainerImage> open(const std::string& path, ContainerKind kind,
                                              bool verify_checksums);

  std::size_t file_size() const noexcept { return bytes_.size(); }

  /// The payload of section `tag` (throws when absent).
  const std::byte* section(std::uint32_t tag, std::size_t* size) const;

  /// Section `tag` as exactly `count` elements of T (throws on a size mismatch).
  template <typename T>
  const T* array(std::uint32_t tag, std::size_t count) const {
    static_assert(std::is_trivially_copyable_v<T>);
    std::size_t size = 0;
    const std::byte* p = section(tag, &size);
    QUIVER_CHECK(count <= size / sizeof(T) && size == count * sizeof(T),
                 "corrupt index file '" + path_ + "': section " + tag_name(tag) + " holds " +
                     std::to_string(size) + " bytes, expected " + std::to_string(count) + " x " +
                     std::to_string(sizeof(T)));
    return reinterpret_cast<const T*>(p);
  }
  template <typename T>
  T pod(std::uint32_t tag) const {
    T value;
    std::memcpy(&value, array<T>(tag, 1), sizeof(T));
    return value;
  }

  static std::string tag_name(std::uint32_t tag);

 private:
  struct Entry {
    std::uint32_t tag, crc;
    std::uint64_t offset, size;
  };
  std::string path_;
  std::vector<std::byte> bytes_;
  std::vector<Entry> entries_;
};

}  // namespace quiver::internal
