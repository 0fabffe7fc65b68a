#include "container.h"

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <array>
#include <atomic>
#include <cerrno>
#include <cstdio>
#include <filesystem>

namespace quiver::internal {
namespace {

constexpr char kMagic[8] = {'Q', 'U', 'I', 'V', 'E', 'R', 'D', 'B'};
constexpr std::uint32_t kVersion = 1;
constexpr std::uint32_t kEndianTag = 0x01020304u;
constexpr std::size_t kHeaderBytes = 64;
constexpr std::size_t kEntryBytes = 24;
constexpr std::size_t kAlign = 64;
constexpr std::size_t kMaxSections = 64;
constexpr std::size_t kHeaderCrcOffset = 36;  // the header CRC covers bytes [0, 36)

std::size_t aligned(std::size_t x) noexcept { return (x + kAlign - 1) / kAlign * kAlign; }

std::string os_error() { return std::strerror(errno); }

// ---- CRC-32C: slicing-by-one table, or the SSE4.2 crc32 instruction when the CPU has it. ----

std::array<std::uint32_t, 256> crc_table() {
  std::array<std::uint32_t, 256> t{};
  for (std::uint32_t b = 0; b < 256; ++b) {
    std::uint32_t r = b;
    for (int i = 0; i < 8; ++i) r = (r >> 1) ^ (0x82F63B78u & (0u - (r & 1u)));
    t[b] = r;
  }
  return t;
}

std::uint32_t crc_table_update(std::uint32_t c, const unsigned char* p, std::size_t n) noexcept {
  static const std::array<std::uint32_t, 256> table = crc_table();
  while (n--) c = table[(c ^ *p++) & 0xFFu] ^ (c >> 8);
  return c;
}

__attribute__((target("sse4.2"))) std::uint32_t crc_sse42_update(std::uint32_t c, const unsigned char* p,
                                                                  std::size_t n) noexcept {
  std::uint64_t w = c;
  while (n >= 8) {
    std::uint64_t v;
    std::memcpy(&v, p, 8);
    w = __builtin_ia32_crc32di(w, v);
    p += 8;
    n -= 8;
  }
  c = static_cast<std::uint32_t>(w);
  while (n--) c = __builtin_ia32_crc32qi(c, *p++);
  return c;
}

bool cpu_has_sse42() noexcept {
  static const bool yes = [] {
    __builtin_cpu_init();
    return __builtin_cpu_supports("sse4.2") != 0;
  }();
  return yes;
}

void put_u32(unsigned char* p, std::uint32_t v) { std::memcpy(p, &v, 4); }
void put_u64(unsigned char* p, std::uint64_t v) { std::memcpy(p, &v, 8); }
std::uint32_t get_u32(const std::byte* p) {
  std::uint32_t v;
  std::memcpy(&v, p, 4);
  return v;
}
std::uint64_t get_u64(const std::byte* p) {
  std::uint64_t v;
  std::memcpy(&v, p, 8);
  return v;
}

/// An output file written sequentially through a 4 MiB buffer; removed unless released.
class OutFile final : public SectionOut {
 public:
  explicit OutFile(std::string path) : path_(std::move(path)) {
    fd_ = ::open(path_.c_str(), O_WRONLY | O_CREAT | O_TRUNC | O_CLOEXEC, 0644);
    QUIVER_CHECK(fd_ >= 0, "cannot create '" + path_ + "': " + os_error());
    buf_.reserve(kBuffer);
  }
  ~OutFile() {
    if (fd_ >= 0) ::close(fd_);
    if (!released_) std::remove(path_.c_str());
  }

  void put(const void* data, std::size_t size) override {
    crc_ = crc32c(data, size, crc_);
    count_ += size;
    const auto* p = static_cast<const unsigned char*>(data);
    if (buf_.size() + size > kBuffer) drain();
    if (size >= kBuffer) {
      raw_write(p, size);
    } else {
      buf_.insert(buf_.end(), p, p + size);
    }
  }

  /// Starts a section: resets the running CRC and byte count.
  void begin() {
    crc_ = 0;
    count_ = 0;
  }
  std::uint32_t crc() const noexcept { return crc_; }
  std::size_t count() const noexcept { return count_; }

  void pad_to(std::size_t offset) {
    static const unsigned char zeros[kAlign] = {};
    QUIVER_CHECK(offset >= pos_ + buf_.size(), "internal error: section layout");
    std::size_t gap = offset - (pos_ + buf_.size());
    while (gap > 0) {
      const std::size_t n = std::min(gap, kAlign);
      buf_.insert(buf_.end(), zeros, zeros + n);
      gap -= n;
    }
  }

  std::size_t position() const noexcept { return pos_ + buf_.size(); }

  void write_at(std::size_t offset, const void* data, std::size_t size) {
    drain();
    const auto* p = static_cast<const unsigned char*>(data);
    while (size > 0) {
      const ssize_t w = ::pwrite(fd_, p, size, static_cast<off_t>(offset));
      if (w < 0 && errno == EINTR) continue;
      QUIVER_CHECK(w > 0, "write to '" + path_ + "' failed: " + os_error());
      p += w;
      size -= static_cast<std::size_t>(w);
      offset += static_cast<std::size_t>(w);
    }
  }

  void finish() {
    drain();
    QUIVER_CHECK(::fsync(fd_) == 0, "fsync of '" + path_ + "' failed: " + os_error());
    QUIVER_CHECK(::close(fd_) == 0, "close of '" + path_ + "' failed: " + os_error());
    fd_ = -1;
  }
  void release() noexcept { released_ = true; }
  const std::string& path() const noexcept { return path_; }

 private:
  static constexpr std::size_t kBuffer = std::size_t{4} << 20;

  void drain() {
    if (buf_.empty()) return;
    raw_write(buf_.data(), buf_.size());
    buf_.clear();
  }
  void raw_write(const unsigned char* p, std::size_t size) {
    while (size > 0) {
      const ssize_t w = ::pwrite(fd_, p, size, static_cast<off_t>(pos_));
      if (w < 0 && errno == EINTR) continue;
      QUIVER_CHECK(w > 0, "write to '" + path_ + "' failed: " + os_error());
      p += w;
      size -= static_cast<std::size_t>(w);
      pos_ += static_cast<std::size_t>(w);
    }
  }

  std::string path_;
  int fd_ = -1;
  bool released_ = false;
  std::vector<unsigned char> buf_;
  std::size_t pos_ = 0;
  std::uint32_t crc_ = 0;
  std::size_t count_ = 0;
};

}  // namespace

std::uint32_t crc32c(const void* data, std::size_t size, std::uint32_t crc) noexcept {
  const auto* p = static_cast<const unsigned char*>(data);
  const std::uint32_t c = ~crc;
  return ~(cpu_has_sse42() ? crc_sse42_update(c, p, size) : crc_table_update(c, p, size));
}

void ContainerWriter::section(std::uint32_t tag, std::size_t size, Producer produce) {
  for (const Pending& s : sections_) {
    QUIVER_CHECK(s.tag != tag, "duplicate section " + ContainerImage::tag_name(tag));
  }
  QUIVER_CHECK(sections_.size() < kMaxSections, "too many sections");
  sections_.push_back({tag, size, std::move(produce), {}});
}

void ContainerWriter::section_bytes(std::uint32_t tag, const void* data, std::size_t size) {
  section(tag, size, [data, size](SectionOut& out) {
    if (size > 0) out.put(data, size);
  });
}

void ContainerWriter::section_copy(std::uint32_t tag, const void* data, std::size_t size) {
  section(tag, size, nullptr);
  const auto* p = static_cast<const std::byte*>(data);
  sections_.back().owned.assign(p, p + size);
}

void ContainerWriter::commit(const std::string& path) const {
  static std::atomic<std::uint64_t> serial{0};
  OutFile out(path + ".tmp." + std::to_string(::getpid()) + "." + std::to_string(serial.fetch_add(1)));

  const std::size_t n = sections_.size();
  std::vector<unsigned char> table(n * kEntryBytes, 0);
  std::size_t offset = aligned(kHeaderBytes + table.size());
  for (std::size_t i = 0; i < n; ++i) {
    const Pending& s = sections_[i];
    out.pad_to(offset);
    out.begin();
    if (s.produce) {
      s.produce(out);
    } else if (!s.owned.empty()) {
      out.put(s.owned.data(), s.owned.size());
    }
    QUIVER_CHECK(out.count() == s.size, "internal error: section " + ContainerImage::tag_name(s.tag) +
                                            " produced " + std::to_string(out.count()) + " of " +
                                            std::to_string(s.size) + " bytes");
    unsigned char* e = table.data() + i * kEntryBytes;
    put_u32(e, s.tag);
    put_u32(e + 4, out.crc());
    put_u64(e + 8, offset);
    put_u64(e + 16, s.size);
    offset = aligned(offset + s.size);
  }
  out.pad_to(offset);

  unsigned char header[kHeaderBytes] = {};
  std::memcpy(header, kMagic, 8);
  put_u32(header + 8, kVersion);
  put_u32(header + 12, static_cast<std::uint32_t>(kind_));
  put_u32(header + 16, kEndianTag);
  put_u32(header + 20, static_cast<std::uint32_t>(n));
  put_u64(header + 24, offset);
  put_u32(header + 32, crc32c(table.data(), table.size()));
  put_u32(header + kHeaderCrcOffset, crc32c(header, kHeaderCrcOffset));
  if (!table.empty()) out.write_at(kHeaderBytes, table.data(), table.size());
  out.write_at(0, header, kHeaderBytes);
  out.finish();
  QUIVER_CHECK(std::rename(out.path().c_str(), path.c_str()) == 0,
               "cannot rename '" + out.path() + "' to '" + path + "': " + os_error());
  out.release();
  // Make the rename durable (best effort).
  std::filesystem::path dir = std::filesystem::path(path).parent_path();
  if (dir.empty()) dir = ".";
  const int dfd = ::open(dir.c_str(), O_RDONLY | O_CLOEXEC);
  if (dfd >= 0) {
    (void)::fsync(dfd);
    ::close(dfd);
  }
}

std::string ContainerImage::tag_name(std::uint32_t tag) {
  std::string s = "'....'";
  for (int i = 0; i < 4; ++i) {
    const unsigned c = (tag >> (8 * i)) & 0xFFu;
    s[static_cast<std::size_t>(i) + 1] = (c >= 32 && c < 127) ? static_cast<char>(c) : '?';
  }
  return s;
}

std::unique_ptr<ContainerImage> ContainerImage::open(const std::string& path, ContainerKind kind,
                                                     bool verify_checksums) {
  auto img = std::unique_ptr<ContainerImage>(new ContainerImage());
  img->path_ = path;
  {
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    QUIVER_CHECK(fd >= 0, "cannot open '" + path + "': " + os_error());
    struct Closer {
      int fd;
      ~Closer() { ::close(fd); }
    } closer{fd};
    struct stat st {};
    QUIVER_CHECK(::fstat(fd, &st) == 0 && S_ISREG(st.st_mode), "'" + path + "' is not a regular file");
    const auto size = static_cast<std::size_t>(st.st_size);
    QUIVER_CHECK(size >= kHeaderBytes, "'" + path + "' is too small to be a Quiver index");
    img->bytes_.resize(size);
    std::size_t got = 0;
    while (got < size) {
      const ssize_t r = ::pread(fd, img->bytes_.data() + got, size - got, static_cast<off_t>(got));
      if (r < 0 && errno == EINTR) continue;
      QUIVER_CHECK(r > 0, "read of '" + path + "' failed: " + (r == 0 ? std::string("unexpected end") : os_error()));
      got += static_cast<std::size_t>(r);
    }
  }
  const std::byte* b = img->bytes_.data();
  const std::size_t size = img->bytes_.size();
  const std::string bad = "corrupt index file '" + path + "': ";
  QUIVER_CHECK(std::memcmp(b, kMagic, 8) == 0, "'" + path + "' is not a Quiver index (bad magic)");
  QUIVER_CHECK(get_u32(b + 16) == kEndianTag, bad + "written on a machine with different endianness");
  QUIVER_CHECK(get_u32(b + kHeaderCrcOffset) == crc32c(b, kHeaderCrcOffset), bad + "header checksum mismatch");
  QUIVER_CHECK(get_u32(b + 8) == kVersion, "'" + path + "' uses format version " + std::to_string(get_u32(b + 8)) +
                                               "; this build reads version " + std::to_string(kVersion));
  QUIVER_CHECK(get_u32(b + 12) == static_cast<std::uint32_t>(kind), "'" + path + "' holds a different index type");
  QUIVER_CHECK(get_u64(b + 24) == size, bad + "truncated or padded (size " + std::to_string(size) +
                                            ", header says " + std::to_string(get_u64(b + 24)) + ")");
  const std::uint32_t n = get_u32(b + 20);
  QUIVER_CHECK(n <= kMaxSections, bad + "too many sections");
  const std::size_t table_end = kHeaderBytes + std::size_t{n} * kEntryBytes;
  QUIVER_CHECK(table_end <= size, bad + "section table out of bounds");
  QUIVER_CHECK(get_u32(b + 32) == crc32c(b + kHeaderBytes, table_end - kHeaderBytes),
               bad + "section table checksum mismatch");
  img->entries_.resize(n);
  for (std::uint32_t i = 0; i < n; ++i) {
    const std::byte* e = b + kHeaderBytes + std::size_t{i} * kEntryBytes;
    Entry& s = img->entries_[i];
    s = Entry{get_u32(e), get_u32(e + 4), get_u64(e + 8), get_u64(e + 16)};
    const std::string name = tag_name(s.tag);
    QUIVER_CHECK(s.offset % kAlign == 0, bad + "misaligned section " + name);
    QUIVER_CHECK(s.offset >= table_end && s.offset <= size && s.size <= size - s.offset,
                 bad + "section " + name + " out of bounds");
    for (std::uint32_t j = 0; j < i; ++j) {
      QUIVER_CHECK(img->entries_[j].tag != s.tag, bad + "duplicate section " + name);
    }
    if (verify_checksums) {
      QUIVER_CHECK(crc32c(b + s.offset, s.size) == s.crc, bad + "checksum mismatch in section " + name);
    }
  }
  std::vector<Entry> sorted = img->entries_;
  std::sort(sorted.begin(), sorted.end(), [](const Entry& x, const Entry& y) { return x.offset < y.offset; });
  for (std::size_t i = 1; i < sorted.size(); ++i) {
    QUIVER_CHECK(sorted[i - 1].offset + sorted[i - 1].size <= sorted[i].offset, bad + "overlapping sections");
  }
  return img;
}

const std::byte* ContainerImage::section(std::uint32_t tag, std::size_t* size) const {
  for (const Entry& e : entries_) {
    if (e.tag == tag) {
      *size = static_cast<std::size_t>(e.size);
      return bytes_.data() + e.offset;
    }
  }
  detail::throw_error("corrupt index file '" + path_ + "': missing section " + tag_name(tag));
}

}  // namespace quiver::internal
