// Tensor storage: a dense fp32 array with a host copy and a device copy kept
// lazily in step (declared in include/tensor.h).
//
// The observable rules are the reference's Tensor (include/tensor.h:8-61 of
// the reference): cuda_data() gives a readable device copy, uploading a stale
// one; cuda_data_write() makes the device copy the only current one; host
// accessors download a stale host copy, and the non-const ones make the host
// copy the only current one.  The messages of its exceptions are kept
// ("Tensor dimension", "Tensor index", "Tensor rank mismatch", "reshape
// changes tensor size", "tensor has no valid storage").
//
// This implementation tracks the current copies as a bit mask, treats a host
// copy that was never materialised as zeros (no host allocation for tensors
// that only ever live on the device), copies a device-resident tensor on the
// device (stream-ordered, no round trip through the host), and implements
// every assignment through copy/move construction and swap.  Device memory is
// stream-ordered on the legacy default stream, where every op of this
// library's C++ layer runs.
#include "../../include/tensor.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <stdexcept>
#include <string>
#include <utility>

namespace {

void device_call(hipError_t err, const char* what) {
    if (err != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(err));
}

std::size_t element_count(const std::vector<std::size_t>& shape) {
    std::size_t n = 1;
    for (std::size_t d : shape) n *= d;
    return n;
}

}  // namespace

Tensor::Tensor(std::vector<std::size_t> shape) : shape_(std::move(shape)), numel_(element_count(shape_)) {}

Tensor::~Tensor() { release_device(); }

Tensor::Tensor(const Tensor& other) : shape_(other.shape_), numel_(other.numel_) {
    if (other.fresh_ & kOnHost) {
        host_ = other.host_;  // possibly empty: zeros, as in `other`
        fresh_ = kOnHost;
    } else if (numel_) {
        device_call(hipMemcpyAsync(device_buffer(), other.dev_, numel_ * sizeof(float), hipMemcpyDeviceToDevice,
                                   nullptr),
                    "hipMemcpyAsync tensor D2D");
        fresh_ = kOnDevice;
    }
}

Tensor& Tensor::operator=(const Tensor& other) {
    if (this != &other) {
        Tensor copy(other);
        swap(copy);
    }
    return *this;
}

Tensor::Tensor(Tensor&& other) noexcept { swap(other); }

Tensor& Tensor::operator=(Tensor&& other) noexcept {
    if (this != &other) {
        Tensor taken(std::move(other));
        swap(taken);  // `taken` now owns the old storage and frees it
    }
    return *this;
}

void Tensor::swap(Tensor& other) noexcept {
    shape_.swap(other.shape_);
    std::swap(numel_, other.numel_);
    host_.swap(other.host_);
    std::swap(dev_, other.dev_);
    std::swap(fresh_, other.fresh_);
    std::swap(bf16_, other.bf16_);
    std::swap(bf16_bytes_, other.bf16_bytes_);
}

void Tensor::release_device() noexcept {
    if (dev_) (void)hipFreeAsync(dev_, nullptr);
    if (bf16_) (void)hipFreeAsync(bf16_, nullptr);
    dev_ = nullptr;
    bf16_ = nullptr;
    bf16_bytes_ = 0;
    fresh_ &= ~kOnDevice;
    if (!fresh_) fresh_ = kOnHost;  // nothing current left: the values are gone, zeros stand in
}

float* Tensor::device_buffer() const {
    if (!dev_ && numel_)
        device_call(hipMallocAsync(reinterpret_cast<void**>(&dev_), numel_ * sizeof(float), nullptr),
                    "hipMallocAsync tensor");
    return dev_;
}

float* Tensor::host_current() const {
    if (fresh_ & kOnHost) {
        if (host_.size() != numel_) host_.assign(numel_, 0.0f);
        return host_.data();
    }
    if (!dev_) throw std::runtime_error("tensor has no valid storage");
    host_.resize(numel_);
    // blocking copy on the legacy default stream: ordered after every kernel
    // that wrote the device copy
    device_call(hipMemcpy(host_.data(), dev_, numel_ * sizeof(float), hipMemcpyDeviceToHost), "hipMemcpy tensor D2H");
    fresh_ |= kOnHost;
    return host_.data();
}

float* Tensor::host_for_write() {
    float* p = host_current();
    fresh_ = kOnHost;
    return p;
}

void Tensor::prepare_cuda() const {
    if (!numel_ || (fresh_ & kOnDevice)) return;
    float* d = device_buffer();
    if (host_.empty())  // an unmaterialised host copy: zeros
        device_call(hipMemsetAsync(d, 0, numel_ * sizeof(float), nullptr), "hipMemsetAsync tensor");
    else
        device_call(hipMemcpy(d, host_.data(), numel_ * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy tensor H2D");
    fresh_ |= kOnDevice;
}

const float* Tensor::cuda_data() const {
    prepare_cuda();
    return dev_;
}

float* Tensor::cuda_data_write() {
    float* d = device_buffer();
    fresh_ = kOnDevice;
    return d;
}

void Tensor::sync_cuda_to_host() const { (void)host_current(); }

void Tensor::prepare_cuda_bf16_weight(bool with_low_residual) const {
    if (shape_.size() != 2) throw std::invalid_argument("BF16 packing requires a matrix");
    if (bf16_) return;
    const std::size_t bytes =
        aps_linear_tc_packed_bytes(static_cast<int32_t>(shape_[0]), static_cast<int32_t>(shape_[1]));
    if (bytes == 0 || shape_[0] % 4 != 0) return;   // a shape the split kernel does not take: fp32 stays
    void* p = nullptr;
    device_call(hipMallocAsync(&p, bytes, nullptr), "hipMallocAsync BF16 weight");
    const int rc = aps_linear_tc_prepare(cuda_data(), static_cast<int32_t>(shape_[0]), static_cast<int32_t>(shape_[1]),
                                         p, bytes, nullptr);
    if (rc) {
        (void)hipFreeAsync(p, nullptr);
        throw std::runtime_error(std::string("prepare_cuda_bf16_weight: ") + aps_moe_last_error());
    }
    if (!with_low_residual)
        device_call(hipMemsetAsync(static_cast<char*>(p) + bytes / 2, 0, bytes / 2, nullptr), "hipMemsetAsync BF16 lo");
    bf16_ = p;
    bf16_bytes_ = bytes;
    // As the reference (src/tensor.cu:168-175), the fp32 device copy goes once
    // packed: the matmuls read the bf16 images, and a later cuda_data() uploads
    // the host copy again.  The free is queued after the packing on the same
    // stream.  A weight whose only current copy is on the device keeps it.
    if ((fresh_ & kOnHost) && dev_) {
        device_call(hipFreeAsync(dev_, nullptr), "hipFreeAsync packed FP32 weight");
        dev_ = nullptr;
        fresh_ &= ~kOnDevice;
    }
}

float* Tensor::data() { return host_for_write(); }
const float* Tensor::data() const { return host_current(); }
float& Tensor::operator[](std::size_t i) { return host_for_write()[i]; }
const float& Tensor::operator[](std::size_t i) const { return host_current()[i]; }

std::size_t Tensor::size(std::size_t dim) const {
    if (dim >= shape_.size()) throw std::out_of_range("Tensor dimension");
    return shape_[dim];
}

// Row-major offset of an n-index, each index checked against its extent.
std::size_t Tensor::flat_index(const std::size_t* idx, std::size_t n) const {
    if (n != shape_.size()) throw std::invalid_argument("Tensor rank mismatch");
    std::size_t off = 0;
    for (std::size_t d = 0; d < n; ++d) {
        if (idx[d] >= shape_[d]) throw std::out_of_range("Tensor index");
        off = off * shape_[d] + idx[d];
    }
    return off;
}

float& Tensor::at(std::size_t i) {
    const std::size_t ix[] = {i};
    return host_for_write()[flat_index(ix, 1)];
}
float& Tensor::at(std::size_t i, std::size_t j) {
    const std::size_t ix[] = {i, j};
    return host_for_write()[flat_index(ix, 2)];
}
float& Tensor::at(std::size_t i, std::size_t j, std::size_t k) {
    const std::size_t ix[] = {i, j, k};
    return host_for_write()[flat_index(ix, 3)];
}
float& Tensor::at(std::size_t i, std::size_t j, std::size_t k, std::size_t l) {
    const std::size_t ix[] = {i, j, k, l};
    return host_for_write()[flat_index(ix, 4)];
}
const float& Tensor::at(std::size_t i) const {
    const std::size_t ix[] = {i};
    return host_current()[flat_index(ix, 1)];
}
const float& Tensor::at(std::size_t i, std::size_t j) const {
    const std::size_t ix[] = {i, j};
    return host_current()[flat_index(ix, 2)];
}
const float& Tensor::at(std::size_t i, std::size_t j, std::size_t k) const {
    const std::size_t ix[] = {i, j, k};
    return host_current()[flat_index(ix, 3)];
}
const float& Tensor::at(std::size_t i, std::size_t j, std::size_t k, std::size_t l) const {
    const std::size_t ix[] = {i, j, k, l};
    return host_current()[flat_index(ix, 4)];
}

void Tensor::reshape(std::vector<std::size_t> shape) {
    if (element_count(shape) != numel_) throw std::invalid_argument("reshape changes tensor size");
    shape_ = std::move(shape);
}

void Tensor::fill(float value) {
    host_.assign(numel_, value);
    fresh_ = kOnHost;
}
