// C++ tensor and the MoE tensor ops, over the C ABI of include/aps_moe.h.
//
// Mirrors the reference's Tensor (include/tensor.h:8-61) and the tensor_ops
// entry points the MoE path calls (include/tensor.h:72, 142-147): same
// names, signatures, argument meaning and exception types/messages, so a
// caller of the reference compiles against this header unchanged for this
// path.  Tensors are dense fp32, row-major, with a host copy and a device
// copy (HIP) that are synchronised lazily, as in the reference:
//   * cuda_data()        device pointer for reading; uploads a stale copy;
//   * cuda_data_write()  device pointer for writing; the device copy becomes
//                        the valid one and the host copy is refreshed on the
//                        next host access;
//   * data() / at() / operator[] (non-const) make the host copy the valid one.
// Device memory is stream-ordered on the legacy default stream, where every
// op below runs (the reference's ordering: all of its work is on stream 0).
#pragma once

#include <cstddef>
#include <cstdint>
#include <vector>

#include "aps_moe.h"

class Tensor {
public:
    Tensor() = default;
    explicit Tensor(std::vector<std::size_t> shape);
    ~Tensor();
    Tensor(const Tensor& other);
    Tensor& operator=(const Tensor& other);
    Tensor(Tensor&& other) noexcept;
    Tensor& operator=(Tensor&& other) noexcept;

    std::size_t ndim() const { return shape_.size(); }
    std::size_t size() const { return numel_; }
    std::size_t size(std::size_t dim) const;
    const std::vector<std::size_t>& shape() const { return shape_; }

    float* data();
    const float* data() const;
    float& operator[](std::size_t i);
    const float& operator[](std::size_t i) const;

    float& at(std::size_t i);
    float& at(std::size_t i, std::size_t j);
    float& at(std::size_t i, std::size_t j, std::size_t k);
    float& at(std::size_t i, std::size_t j, std::size_t k, std::size_t l);
    const float& at(std::size_t i) const;
    const float& at(std::size_t i, std::size_t j) const;
    const float& at(std::size_t i, std::size_t j, std::size_t k) const;
    const float& at(std::size_t i, std::size_t j, std::size_t k, std::size_t l) const;

    void reshape(std::vector<std::size_t> shape);
    void fill(float value);
    void zero() { fill(0.0f); }
    void prepare_cuda() const;
    const float* cuda_data() const;
    float* cuda_data_write();
    void sync_cuda_to_host() const;
    // The split-bf16 weight copy of the reference's tensor-core Linear
    // (reference include/tensor.h:41-46, src/tensor.cu:149-177): packs this
    // [out][in] matrix into bf16 hi = bf16(w) and lo = bf16(w - hi) tile
    // images (lo left zero without with_low_residual); matmul_transposed_gpu
    // and matmul_transposed_bias_gpu then run the split products
    // (aps_linear_tc; all four terms when built with USE_TC_ALL).  Matrices
    // whose in % 64 != 0 or out % 4 != 0 keep the fp32 path (no copy is
    // made), as the reference's dispatch falls back for shapes its kernel
    // does not take.  The fp32 device copy is kept.
    void prepare_cuda_bf16_weight(bool with_low_residual) const;
    const void* cuda_bf16_weight_hi() const { return bf16_; }
    const void* cuda_bf16_weight_lo() const {
        return bf16_ ? static_cast<const char*>(bf16_) + bf16_bytes_ / 2 : nullptr;
    }
    bool has_cuda_bf16_weight() const { return bf16_ != nullptr; }

private:
    // Which copies hold the current values: a bit mask of kOnHost / kOnDevice.
    // A host copy that was never materialised (host_ empty while kOnHost is
    // set) stands for all zeros, so a fresh tensor costs no host memory until
    // the host reads it, and a device-written one never allocates it at all.
    enum : unsigned { kOnHost = 1u, kOnDevice = 2u };
    std::vector<std::size_t> shape_;
    std::size_t numel_ = 0;
    mutable std::vector<float> host_;
    mutable float* dev_ = nullptr;
    mutable unsigned fresh_ = kOnHost;
    mutable void* bf16_ = nullptr;        // hi images, then lo images (aps_linear_tc_prepare)
    mutable std::size_t bf16_bytes_ = 0;

    std::size_t flat_index(const std::size_t* idx, std::size_t n) const;
    float* host_current() const;      // host copy brought up to date
    float* host_for_write();          // ... and made the only current copy
    float* device_buffer() const;     // allocated on first use, stream-ordered
    void release_device() noexcept;
    void swap(Tensor& other) noexcept;
};

namespace tensor_ops {

// c[m][n] = a[m][k] . b[n][k]^T on the GPU, one fp32 FMA chain per output,
// k ascending (the reference's k_matmul_transposed_narrow for the router
// shape, src/tensor.cu:2943-3006, and k_matmul_transposed_8x8 for the
// others, :715-800).  The router shape (n <= 64, k % 256 == 0) runs the
// router kernel; other shapes need k % 16 == 0 and n % 4 == 0.  Mismatched
// shapes throw std::invalid_argument("matmul_transposed_gpu shape") as the
// reference does; unsupported ones throw std::invalid_argument naming the
// limit.
void matmul_transposed_gpu(const Tensor& a, const Tensor& b, Tensor& c);

// c = a . b^T + bias (reference include/tensor.h, src/tensor.cu:3120-3143):
// one fp32 FMA chain per output over k ascending, then the bias.  Throws
// std::invalid_argument("matmul_transposed_bias_gpu shape") as the reference
// does; this build needs k % 16 == 0 and n % 4 == 0.
void matmul_transposed_bias_gpu(const Tensor& a, const Tensor& b, const Tensor& bias, Tensor& c);

// out = silu(a . gate_weight^T) * (a . up_weight^T) (reference
// include/tensor.h:75-76, src/tensor.cu:3146-3170): each product one fp32
// FMA chain per output over k ascending, then the reference's SiLU-mul
// (exp in double).  Throws std::invalid_argument("matmul_pair_silu_gpu
// shape") as the reference does.
void matmul_pair_silu_gpu(const Tensor& a, const Tensor& gate_weight, const Tensor& up_weight, Tensor& out);

// first_out = a . first_weight^T + first_bias and the same for second
// (reference include/tensor.h:77-81, src/tensor.cu:3172-3234: the k/v
// projections sharing their input).  Throws
// std::invalid_argument("matmul_pair_bias_gpu shape").
void matmul_pair_bias_gpu(const Tensor& a, const Tensor& first_weight, const Tensor& first_bias, Tensor& first_out,
                          const Tensor& second_weight, const Tensor& second_bias, Tensor& second_out);

// Elementwise ops of the reference (include/tensor.h:82-85,
// src/tensor.cu:3236-3260, 277-281): x = 0; a += b ("add shape");
// a += bias per last-dimension column ("bias shape"); out = silu(gate) * up
// ("silu_mul shape").
void zero_gpu(Tensor& x);
void add_inplace_gpu(Tensor& a, const Tensor& b);
void add_bias_inplace_gpu(Tensor& a, const Tensor& bias);
void silu_mul_gpu(const Tensor& gate, const Tensor& up, Tensor& out);

// RoPE and GQA-4 attention over packed sequences (reference
// include/tensor.h:91-98, src/tensor.cu:3296-3340): the rows of q/k/v are
// the sequences of seq_lens one after another; a row's position restarts at
// 0 with its sequence and its keys are the earlier rows of its own sequence
// (the last SLIDING_WINDOW of them).  The per-row segment table is
// uploaded once per distinct seq_lens and cached, as the reference's
// packed_meta.  attention_gpu throws std::invalid_argument("attention_gpu
// expects GQA-4") unless q_heads == 4 kv_heads (the reference's fallback
// kernel for other ratios is not provided); a seq_lens total different from
// the row count throws std::invalid_argument("packed sequence lengths").
void apply_rope_gpu(Tensor& q, Tensor& k, const std::vector<std::size_t>& seq_lens, std::size_t q_heads,
                    std::size_t kv_heads, std::size_t head_dim, float theta);
void attention_gpu(const Tensor& q, const Tensor& k, const Tensor& v, Tensor& out,
                   const std::vector<std::size_t>& seq_lens, std::size_t q_heads, std::size_t kv_heads,
                   std::size_t head_dim);

// Registers the 16 experts' w1 / w2 / w3 (nn.Linear layout: w1, w3 [F][H],
// w2 [H][F]) and returns a 1-based handle.  Throws
// std::invalid_argument("MoE weight table size") unless each table has
// apss26::NUM_EXPERTS entries (reference src/tensor.cu:2757-2788).  The
// default computes in fp32 with the reference's accumulation order; the
// overload selects bf16 MFMA compute (APS_DTYPE_BF16).
std::size_t register_moe_weights_gpu(const std::vector<const Tensor*>& w1,
                                     const std::vector<const Tensor*>& w2,
                                     const std::vector<const Tensor*>& w3);
std::size_t register_moe_weights_gpu(const std::vector<const Tensor*>& w1,
                                     const std::vector<const Tensor*>& w2,
                                     const std::vector<const Tensor*>& w3, aps_dtype compute);

// out = MoE block of x [rows][H] given router logits [rows][16] and a
// registered handle (reference src/tensor.cu:2790-2928).  Allocates `out`
// as [rows][H].  Throws std::invalid_argument("grouped MoE shape or handle")
// for a router of the wrong shape or an invalid handle.
void moe_forward_grouped_gpu(const Tensor& x, const Tensor& router, std::size_t weights_handle, Tensor& out);

// y = LayerNorm(x) over the last dimension (reference include/tensor.h:86-87,
// src/tensor.cu:3262-3280): both row sums serial in ascending order, as the
// reference GPU kernel.  y must already have x's size.  Throws
// std::invalid_argument("layer norm shape") for mismatched sizes; this
// build needs the last dimension to be a multiple of 256.
void layer_norm_gpu(const Tensor& x, const Tensor& weight, const Tensor& bias, float eps, Tensor& y);

// x += residual, then y = LayerNorm(x) (reference include/tensor.h:88-90,
// src/tensor.cu:3282-3295).  Throws std::invalid_argument("add layer norm
// shape") for mismatched sizes.
void add_layer_norm_gpu(Tensor& x, const Tensor& residual, const Tensor& weight, const Tensor& bias, float eps,
                        Tensor& y);

// out[i][:] = x[rows[i]][:] over the last dimension of x (reference
// include/tensor.h:115-116, src/tensor.cu:3379-3386): the index list is
// uploaded through a blocking copy on the default stream, then one HIP
// gather kernel.  out must hold rows.size() rows.  An index past the end of
// x throws std::invalid_argument("gather_rows_gpu row index"), and a wrong
// out size std::invalid_argument("gather_rows_gpu shape") (the reference
// does not check either).
void gather_rows_gpu(const Tensor& x, const std::vector<std::size_t>& rows, Tensor& out);

// A row-index map uploaded to the device once and reused across many
// gathers (reference include/tensor.h:119-137).
class RowIndexBuffer {
public:
    RowIndexBuffer() = default;
    explicit RowIndexBuffer(const std::vector<std::size_t>& rows);
    ~RowIndexBuffer();
    RowIndexBuffer(const RowIndexBuffer&) = delete;
    RowIndexBuffer& operator=(const RowIndexBuffer&) = delete;
    RowIndexBuffer(RowIndexBuffer&& other) noexcept;
    RowIndexBuffer& operator=(RowIndexBuffer&& other) noexcept;
    // `size` entries left for the caller to fill on the device (through
    // mutable_data()), each at most max_row.
    static RowIndexBuffer allocate(std::size_t size, std::size_t max_row);
    const std::uint32_t* data() const { return ptr_; }
    std::uint32_t* mutable_data() { return ptr_; }
    std::size_t size() const { return size_; }
    bool empty() const { return size_ == 0; }
    std::size_t max_row() const { return max_row_; }  // largest index (0 when empty)

private:
    std::uint32_t* ptr_ = nullptr;
    std::size_t size_ = 0;
    std::size_t max_row_ = 0;
};

// The same gather from a device-resident index map (reference
// include/tensor.h:138, src/tensor.cu:3420-3426); same checks as above.
void gather_rows_gpu(const Tensor& x, const RowIndexBuffer& rows, Tensor& out);

// RoPE in place on q [rows][q_heads * head_dim] and k [rows][kv_heads *
// head_dim] at the device positions row_pos[rows] (reference
// include/tensor.h:100-103, src/tensor.cu:3342-3359): the cos/sin tables of
// max_seq positions are built on the host once per (head_dim, theta) and
// kept on the device, grown when a larger max_seq arrives.  Positions must
// be < max_seq: the positions are device data this function does not read,
// so a row past the table is left unchanged rather than reported
// (PhiAttention checks its expansion's positions before the call).
void apply_rope_tree_gpu(Tensor& q, Tensor& k, const std::uint32_t* row_pos, std::size_t rows, std::size_t max_seq,
                         std::size_t q_heads, std::size_t kv_heads, std::size_t head_dim, float theta);

// Attention of each row over its ancestor chain anc[row][0 .. row_pos[row]]
// (device arrays; the last SLIDING_WINDOW keys), GQA-4, head_dim 128
// (reference include/tensor.h:109-114, src/tensor.cu:3361-3377).  Throws
// std::invalid_argument("attention_tree_gpu expects GQA-4") as the
// reference does; out must hold rows x q_heads x head_dim values.
// Positions must be < anc_stride and ancestors < rows: the kernel clamps
// device values outside those ranges for memory safety only (PhiAttention
// checks its expansion first).
void attention_tree_gpu(const Tensor& q, const Tensor& k, const Tensor& v, Tensor& out, const std::uint32_t* row_pos,
                        const std::uint32_t* anc, std::size_t anc_stride, std::size_t rows, std::size_t max_seq,
                        std::size_t q_heads, std::size_t kv_heads, std::size_t head_dim);

}  // namespace tensor_ops
