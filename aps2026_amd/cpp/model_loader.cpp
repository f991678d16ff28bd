// ModelLoader (declared in include/model_loader.h).
//
// The file format and the error messages are the reference's
// (src/model_loader.cu:14-53 of the reference): a u32 entry count, then per
// entry u32 name length, the name, u32 rank, rank x u32 extents, u64 byte
// offset and u64 byte count, all little-endian, fp32 data at the offsets.
//
// This implementation reads through positional reads (pread) on a file
// descriptor, never through stream state.  The index is parsed from a
// window that is refilled from the file as the cursor advances; every field
// is checked against the file's size before it is taken, so a short file is
// reported as "truncated model.bin" wherever the index ends.  A tensor's
// byte range is checked against the file size before it is read ("truncated
// tensor: <name>"), and the data lands straight in the Tensor's host storage
// before the upload that keeps weights resident on the device.
#include "../../include/model_loader.h"

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstring>
#include <memory>
#include <stdexcept>

namespace {

// An open file descriptor, closed on scope exit.
class File {
public:
    explicit File(const std::string& path) : fd_(::open(path.c_str(), O_RDONLY | O_CLOEXEC)) {}
    ~File() {
        if (fd_ >= 0) ::close(fd_);
    }
    File(const File&) = delete;
    File& operator=(const File&) = delete;
    bool ok() const { return fd_ >= 0; }
    std::uint64_t bytes() const {
        struct stat st {};
        return ::fstat(fd_, &st) == 0 ? static_cast<std::uint64_t>(st.st_size) : 0;
    }
    // Reads exactly n bytes at `offset`; false on a short read or an error.
    bool read_at(void* dst, std::uint64_t n, std::uint64_t offset) const {
        char* out = static_cast<char*>(dst);
        while (n) {
            const ssize_t got = ::pread(fd_, out, n, static_cast<off_t>(offset));
            if (got < 0 && errno == EINTR) continue;
            if (got <= 0) return false;
            out += got;
            n -= static_cast<std::uint64_t>(got);
            offset += static_cast<std::uint64_t>(got);
        }
        return true;
    }

private:
    int fd_;
};

// Sequential little-endian fields of the index, read through a 64 KB window.
class IndexCursor {
public:
    IndexCursor(const File& f, std::uint64_t file_bytes) : file_(f), end_(file_bytes) {}

    template <typename T>
    T field() {
        T v;
        take(&v, sizeof(T));
        return v;
    }
    std::string text(std::uint32_t n) {
        std::string s(n, '\0');
        take(&s[0], n);
        return s;
    }

private:
    void take(void* dst, std::uint64_t n) {
        if (n > end_ - pos_) throw std::runtime_error("truncated model.bin");
        char* out = static_cast<char*>(dst);
        while (n) {
            if (pos_ < win_at_ || pos_ >= win_at_ + win_len_) refill();
            const std::uint64_t in_win = win_at_ + win_len_ - pos_;
            const std::uint64_t c = n < in_win ? n : in_win;
            std::memcpy(out, window_ + (pos_ - win_at_), c);
            out += c;
            n -= c;
            pos_ += c;
        }
    }
    void refill() {
        const std::uint64_t left = end_ - pos_;
        win_len_ = left < sizeof(window_) ? left : sizeof(window_);
        win_at_ = pos_;
        if (!file_.read_at(window_, win_len_, win_at_)) throw std::runtime_error("truncated model.bin");
    }

    const File& file_;
    std::uint64_t end_;
    std::uint64_t pos_ = 0, win_at_ = 0, win_len_ = 0;
    char window_[64 * 1024];
};

}  // namespace

ModelLoader::ModelLoader(const std::string& path) : path_(path) {
    File f(path_);
    if (!f.ok()) throw std::runtime_error("cannot open model: " + path_);
    const std::uint64_t file_bytes = f.bytes();
    auto cursor = std::make_unique<IndexCursor>(f, file_bytes);  // the window is too large for the stack
    const std::uint32_t entries = cursor->field<std::uint32_t>();
    for (std::uint32_t i = 0; i < entries; ++i) {
        const std::uint32_t name_len = cursor->field<std::uint32_t>();
        std::string name = cursor->text(name_len);
        Entry entry;
        entry.shape.resize(cursor->field<std::uint32_t>());
        for (std::size_t& extent : entry.shape) extent = cursor->field<std::uint32_t>();
        entry.offset = cursor->field<std::uint64_t>();
        entry.bytes = cursor->field<std::uint64_t>();
        // a repeated name keeps its first entry (the reference's map emplace)
        entries_.insert({std::move(name), std::move(entry)});
    }
}

Tensor ModelLoader::load(const std::string& name) const {
    const auto found = entries_.find(name);
    if (found == entries_.end()) throw std::runtime_error("missing tensor: " + name);
    const Entry& entry = found->second;
    std::uint64_t count = 1;
    for (std::size_t extent : entry.shape) count *= extent;
    if (entry.bytes != count * sizeof(float)) throw std::runtime_error("tensor is not float32: " + name);
    File f(path_);
    if (!f.ok()) throw std::runtime_error("cannot reopen model: " + path_);
    const std::uint64_t file_bytes = f.bytes();
    if (entry.offset > file_bytes || entry.bytes > file_bytes - entry.offset)
        throw std::runtime_error("truncated tensor: " + name);
    Tensor out(entry.shape);
    if (entry.bytes && !f.read_at(out.data(), entry.bytes, entry.offset))
        throw std::runtime_error("truncated tensor: " + name);
    out.prepare_cuda();  // weights stay resident on the device
    return out;
}
