// ModelLoader (declared in include/model_loader.h).  Reference:
// src/model_loader.cu:14-53 -- the index layout, the checks and their
// messages.  The index is read through one buffered stream; a tensor is read
// straight into the Tensor's host storage and then uploaded (prepare_cuda).
#include "../../include/model_loader.h"

#include <fstream>
#include <stdexcept>

namespace {

template <typename T>
T read_field(std::ifstream& f) {
    T v{};
    f.read(reinterpret_cast<char*>(&v), sizeof(T));
    if (!f) throw std::runtime_error("truncated model.bin");
    return v;
}

}  // namespace

ModelLoader::ModelLoader(const std::string& path) : path_(path) {
    std::ifstream f(path_, std::ios::binary);
    if (!f) throw std::runtime_error("cannot open model: " + path_);
    const std::uint32_t count = read_field<std::uint32_t>(f);
    for (std::uint32_t i = 0; i < count; ++i) {
        const std::uint32_t name_len = read_field<std::uint32_t>(f);
        std::string name(name_len, '\0');
        f.read(&name[0], name_len);
        if (!f) throw std::runtime_error("truncated model.bin");
        Entry e;
        const std::uint32_t ndim = read_field<std::uint32_t>(f);
        e.shape.resize(ndim);
        for (std::uint32_t d = 0; d < ndim; ++d) e.shape[d] = read_field<std::uint32_t>(f);
        e.offset = read_field<std::uint64_t>(f);
        e.bytes = read_field<std::uint64_t>(f);
        entries_.emplace(std::move(name), std::move(e));  // first entry of a name wins, as in the reference
    }
}

Tensor ModelLoader::load(const std::string& name) const {
    const auto it = entries_.find(name);
    if (it == entries_.end()) throw std::runtime_error("missing tensor: " + name);
    const Entry& e = it->second;
    std::size_t elements = 1;
    for (std::size_t d : e.shape) elements *= d;
    if (e.bytes != elements * sizeof(float)) throw std::runtime_error("tensor is not float32: " + name);
    Tensor out(e.shape);
    std::ifstream f(path_, std::ios::binary);
    if (!f) throw std::runtime_error("cannot reopen model: " + path_);
    f.seekg(static_cast<std::streamoff>(e.offset));
    f.read(reinterpret_cast<char*>(out.data()), static_cast<std::streamsize>(e.bytes));
    if (!f) throw std::runtime_error("truncated tensor: " + name);
    out.prepare_cuda();  // weights stay resident on the device
    return out;
}
