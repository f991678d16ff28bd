// tensor_ops over the C ABI (declared in include/tensor.h; the Tensor class
// itself is in tensor_storage.cpp).
//
// Reference behaviour mirrored: register_moe_weights_gpu
// (src/tensor.cu:2757-2788), moe_forward_grouped_gpu (src/tensor.cu:2790-2928),
// the other tensor_ops launchers named at each function, and the error
// conventions of check_cuda (src/tensor.cu:370-374).
#include "../../include/tensor.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <deque>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>

#include "../../include/config.h"

namespace {

void hip_check(hipError_t err, const char* what) {
    if (err != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(err));
}

// A non-zero status from the C ABI: argument errors become
// std::invalid_argument, device errors std::runtime_error, each carrying the
// library's message.
[[noreturn]] void throw_status(int rc, const char* op) {
    const std::string msg = std::string(op) + ": " + aps_moe_last_error();
    if (rc == APS_ERR_HIP) throw std::runtime_error(msg);
    throw std::invalid_argument(msg);
}

// Grow-only device workspace for the forward calls, ordered on the default
// stream like the reference's moe_scratch (src/tensor.cu:1227-1291).
struct Workspace {
    std::mutex mu;
    void* ptr = nullptr;
    std::size_t bytes = 0;
    void* get(std::size_t need) {
        if (need <= bytes) return ptr;
        if (ptr) hip_check(hipFreeAsync(ptr, nullptr), "hipFreeAsync workspace");
        ptr = nullptr;
        bytes = 0;
        hip_check(hipMallocAsync(&ptr, need, nullptr), "hipMallocAsync workspace");
        bytes = need;
        return ptr;
    }
};

Workspace& workspace() {
    static Workspace* w = new Workspace();  // lives for the process, like the reference's scratch
    return *w;
}

// The split-bf16 Linear (a weight with a bf16 copy, Tensor::
// prepare_cuda_bf16_weight): x split once into hi / lo rows in a grow-only
// buffer of its own, then aps_linear_tc; four terms when built with
// USE_TC_ALL (reference src/tensor.cu:566-568).
void linear_tc(const float* da, const Tensor& b, const float* dbias, std::size_t m, std::size_t k, std::size_t n,
               float* dc, const char* op) {
#ifdef USE_TC_ALL
    constexpr int kAllTerms = 1;
#else
    constexpr int kAllTerms = 0;
#endif
    static Workspace* split = new Workspace();
    std::lock_guard<std::mutex> lock(split->mu);
    void* xs = split->get(m * k * 2 * sizeof(std::uint16_t));
    int rc = aps_linear_tc_split(da, static_cast<int64_t>(m), static_cast<int32_t>(k), xs, nullptr);
    if (!rc)
        rc = aps_linear_tc(xs, static_cast<int64_t>(m), static_cast<int32_t>(k), b.cuda_bf16_weight_hi(), dbias,
                           static_cast<int32_t>(n), kAllTerms, dc, nullptr);
    if (rc) throw_status(rc, op);
}

}  // namespace

// ---- tensor_ops ------------------------------------------------------------

namespace tensor_ops {

void matmul_transposed_gpu(const Tensor& a, const Tensor& b, Tensor& c) {
    const std::size_t k = a.size(a.ndim() - 1);
    const std::size_t m = a.size() / k;
    const std::size_t n = b.size(0);
    if (b.size(1) != k || c.size(0) != m || c.size(1) != n)
        throw std::invalid_argument("matmul_transposed_gpu shape");
    const float* da = a.cuda_data();
    if (b.has_cuda_bf16_weight()) {   // the reference's USE_TC branch (src/tensor.cu:3042-3055)
        linear_tc(da, b, nullptr, m, k, n, c.cuda_data_write(), "matmul_transposed_gpu");
        return;
    }
    const float* db = b.cuda_data();
    if (n <= 64 && k % 256 == 0) {  // the router shape: the router kernel
        const int rc = aps_router_logits(da, APS_DTYPE_F32, db, static_cast<int64_t>(m), static_cast<int32_t>(k),
                                         static_cast<int32_t>(n), c.cuda_data_write(), nullptr);
        if (rc) throw_status(rc, "matmul_transposed_gpu");
        return;
    }
    const int rc = aps_linear(da, db, nullptr, static_cast<int64_t>(m), static_cast<int32_t>(k),
                              static_cast<int32_t>(n), c.cuda_data_write(), nullptr);
    if (rc) throw_status(rc, "matmul_transposed_gpu");
}

void matmul_transposed_bias_gpu(const Tensor& a, const Tensor& b, const Tensor& bias, Tensor& c) {
    const std::size_t k = a.size(a.ndim() - 1);
    const std::size_t m = a.size() / k;
    const std::size_t n = b.size(0);
    if (b.size(1) != k || c.size(0) != m || c.size(1) != n || bias.size() != n)
        throw std::invalid_argument("matmul_transposed_bias_gpu shape");
    if (b.has_cuda_bf16_weight()) {   // the product, then the bias (reference src/tensor.cu:3121-3142)
        linear_tc(a.cuda_data(), b, bias.cuda_data(), m, k, n, c.cuda_data_write(), "matmul_transposed_bias_gpu");
        return;
    }
    const int rc = aps_linear(a.cuda_data(), b.cuda_data(), bias.cuda_data(), static_cast<int64_t>(m),
                              static_cast<int32_t>(k), static_cast<int32_t>(n), c.cuda_data_write(), nullptr);
    if (rc) throw_status(rc, "matmul_transposed_bias_gpu");
}

void layer_norm_gpu(const Tensor& x, const Tensor& weight, const Tensor& bias, float eps, Tensor& y) {
    const std::size_t h = x.size(x.ndim() - 1);
    const std::size_t rows = x.size() / h;
    if (weight.size() != h || bias.size() != h || y.size() != x.size())
        throw std::invalid_argument("layer norm shape");
    if (h % 256 != 0) throw std::invalid_argument("layer_norm_gpu: this build needs the last dimension % 256 == 0");
    const float* dx = x.cuda_data();
    const int rc = aps_layer_norm(dx, weight.cuda_data(), bias.cuda_data(), static_cast<int64_t>(rows),
                                  static_cast<int32_t>(h), eps, y.cuda_data_write(), nullptr);
    if (rc) throw_status(rc, "layer_norm_gpu");
}

void add_layer_norm_gpu(Tensor& x, const Tensor& residual, const Tensor& weight, const Tensor& bias, float eps,
                        Tensor& y) {
    const std::size_t h = x.size(x.ndim() - 1);
    const std::size_t rows = x.size() / h;
    if (residual.size() != x.size() || weight.size() != h || bias.size() != h || y.size() != x.size())
        throw std::invalid_argument("add layer norm shape");
    if (h % 256 != 0)
        throw std::invalid_argument("add_layer_norm_gpu: this build needs the last dimension % 256 == 0");
    x.cuda_data();  // upload if the host copy is the valid one, then write in place
    const int rc = aps_add_layer_norm(x.cuda_data_write(), residual.cuda_data(), weight.cuda_data(),
                                      bias.cuda_data(), static_cast<int64_t>(rows), static_cast<int32_t>(h), eps,
                                      y.cuda_data_write(), nullptr);
    if (rc) throw_status(rc, "add_layer_norm_gpu");
}

std::size_t register_moe_weights_gpu(const std::vector<const Tensor*>& w1, const std::vector<const Tensor*>& w2,
                                     const std::vector<const Tensor*>& w3, aps_dtype compute) {
    if (w1.size() != apss26::NUM_EXPERTS || w2.size() != apss26::NUM_EXPERTS || w3.size() != apss26::NUM_EXPERTS)
        throw std::invalid_argument("MoE weight table size");
    const std::size_t E = w1.size();
    const std::size_t F = w1[0]->size(0), H = w1[0]->size(1);
    std::vector<const void*> p1(E), p2(E), p3(E);
    for (std::size_t e = 0; e < E; ++e) {
        if (w1[e]->size(0) != F || w1[e]->size(1) != H || w3[e]->size(0) != F || w3[e]->size(1) != H ||
            w2[e]->size(0) != H || w2[e]->size(1) != F)
            throw std::invalid_argument("MoE weight table size");
        p1[e] = w1[e]->cuda_data();
        p2[e] = w2[e]->cuda_data();
        p3[e] = w3[e]->cuda_data();
    }
    aps_moe_weights_desc d{};
    d.num_experts = static_cast<int32_t>(E);
    d.hidden = static_cast<int32_t>(H);
    d.ffn = static_cast<int32_t>(F);
    d.src_dtype = APS_DTYPE_F32;
    d.compute_dtype = compute;
    d.w1 = p1.data();
    d.w3 = p3.data();
    d.w2 = p2.data();
    uint64_t handle = 0;
    const int rc = aps_moe_weights_register(&d, nullptr, &handle);
    if (rc) throw_status(rc, "register_moe_weights_gpu");
    return static_cast<std::size_t>(handle);
}

std::size_t register_moe_weights_gpu(const std::vector<const Tensor*>& w1, const std::vector<const Tensor*>& w2,
                                     const std::vector<const Tensor*>& w3) {
    return register_moe_weights_gpu(w1, w2, w3, APS_DTYPE_F32);
}

void moe_forward_grouped_gpu(const Tensor& x, const Tensor& router, std::size_t weights_handle, Tensor& out) {
    const std::size_t rows = x.size(0), h = x.size(1);
    aps_moe_ws_layout L{};
    if (router.ndim() != 2 || router.size(0) != rows || router.size(1) != apss26::NUM_EXPERTS ||
        weights_handle == 0 || aps_moe_workspace_layout(weights_handle, static_cast<int64_t>(rows), &L) != APS_OK)
        throw std::invalid_argument("grouped MoE shape or handle");
    out = Tensor({rows, h});
    if (rows == 0) return;
    const float* dx = x.cuda_data();
    const float* dr = router.cuda_data();
    float* dout = out.cuda_data_write();
    Workspace& ws = workspace();
    std::lock_guard<std::mutex> lk(ws.mu);
    void* buf = ws.get(L.total_bytes);
    const int rc = aps_moe_forward_grouped(weights_handle, dx, APS_DTYPE_F32, dr, static_cast<int64_t>(rows), dout,
                                           APS_DTYPE_F32, buf, L.total_bytes, nullptr);
    if (rc) throw_status(rc, "moe_forward_grouped_gpu");
}

}  // namespace tensor_ops

// ---- dense FFN (used by PhiMLP) ---------------------------------------------

namespace aps_cpp_detail {

// PhiMoE::forward's GPU branch as one aps_moe_forward call: router logits,
// routing, dispatch, expert FFN and combine over fp32 x [rows][H] into a new
// out [rows][H].  Throws as moe_forward_grouped_gpu does.
void moe_forward_fused(std::size_t handle, const Tensor& x, const Tensor& gate, Tensor& out) {
    const std::size_t rows = x.size(0), h = x.size(x.ndim() - 1);
    aps_moe_ws_layout L{};
    if (x.ndim() != 2 || gate.ndim() != 2 || gate.size(0) != apss26::NUM_EXPERTS || gate.size(1) != h ||
        handle == 0 || aps_moe_workspace_layout(handle, static_cast<int64_t>(rows), &L) != APS_OK)
        throw std::invalid_argument("grouped MoE shape or handle");
    out = Tensor({rows, h});
    if (rows == 0) return;
    const float* dx = x.cuda_data();
    const float* dg = gate.cuda_data();
    float* dout = out.cuda_data_write();
    Workspace& ws = workspace();
    std::lock_guard<std::mutex> lk(ws.mu);
    void* buf = ws.get(L.total_bytes);
    const int rc = aps_moe_forward(handle, dx, APS_DTYPE_F32, dg, static_cast<int64_t>(rows), dout, APS_DTYPE_F32, buf,
                                   L.total_bytes, nullptr);
    if (rc) throw_status(rc, "PhiMoE::forward");
}

void mlp_forward_gpu(std::size_t handle, const Tensor& x, std::size_t rows, Tensor& out) {
    const std::size_t need = aps_mlp_workspace_size(handle, static_cast<int64_t>(rows));
    const float* dx = x.cuda_data();
    float* dout = out.cuda_data_write();
    Workspace& ws = workspace();
    std::lock_guard<std::mutex> lk(ws.mu);
    void* buf = ws.get(need ? need : 1);
    const int rc = aps_mlp_forward(handle, dx, APS_DTYPE_F32, static_cast<int64_t>(rows), dout, buf, need, nullptr);
    if (rc) throw_status(rc, "PhiMLP::forward");
}

std::size_t register_dense(const Tensor& w1, const Tensor& w2, const Tensor& w3) {
    const void* p1 = w1.cuda_data();
    const void* p2 = w2.cuda_data();
    const void* p3 = w3.cuda_data();
    aps_moe_weights_desc d{};
    d.num_experts = 1;
    d.hidden = static_cast<int32_t>(w1.size(1));
    d.ffn = static_cast<int32_t>(w1.size(0));
    d.src_dtype = APS_DTYPE_F32;
    d.compute_dtype = APS_DTYPE_F32;
    d.w1 = &p1;
    d.w3 = &p3;
    d.w2 = &p2;
    uint64_t handle = 0;
    const int rc = aps_moe_weights_register(&d, nullptr, &handle);
    if (rc) throw_status(rc, "PhiMLP weights");
    return static_cast<std::size_t>(handle);
}

}  // namespace aps_cpp_detail

// ---- row gather (reference src/tensor.cu:3379-3426) ------------------------

namespace {

// Grow-only device staging buffer of the std::vector overload, as the
// reference's device_rows: the blocking upload on the default stream orders
// it after every earlier gather that read it.
struct RowStaging {
    std::mutex mu;
    std::uint32_t* ptr = nullptr;
    std::size_t cap = 0;
};
RowStaging g_rows;

std::vector<std::uint32_t> compact_rows(const std::vector<std::size_t>& rows, std::size_t* max_row) {
    std::vector<std::uint32_t> c(rows.size());
    std::size_t mx = 0;
    for (std::size_t i = 0; i < rows.size(); ++i) {
        if (rows[i] > 0xFFFFFFFFull) throw std::invalid_argument("gather_rows_gpu row index");
        c[i] = static_cast<std::uint32_t>(rows[i]);
        mx = std::max(mx, rows[i]);
    }
    *max_row = mx;
    return c;
}

void gather_common(const Tensor& x, const std::uint32_t* drows, std::size_t count, std::size_t max_row, Tensor& out) {
    if (count == 0) return;
    const std::size_t h = x.ndim() ? x.size(x.ndim() - 1) : 0;
    const std::size_t x_rows = h ? x.size() / h : 0;
    if (out.size() != count * h) throw std::invalid_argument("gather_rows_gpu shape");
    if (max_row >= x_rows) throw std::invalid_argument("gather_rows_gpu row index");
    const int rc = aps_gather_rows(x.cuda_data(), static_cast<int64_t>(x_rows), static_cast<int64_t>(h), drows,
                                   static_cast<int64_t>(count), out.cuda_data_write(), nullptr);
    if (rc) throw_status(rc, "gather_rows_gpu");
}

}  // namespace

namespace tensor_ops {

void gather_rows_gpu(const Tensor& x, const std::vector<std::size_t>& rows, Tensor& out) {
    if (rows.empty()) return;
    std::size_t max_row = 0;
    const std::vector<std::uint32_t> c = compact_rows(rows, &max_row);
    std::lock_guard<std::mutex> lock(g_rows.mu);
    if (g_rows.cap < c.size()) {
        if (g_rows.ptr) hip_check(hipFree(g_rows.ptr), "hipFree row staging");
        g_rows.ptr = nullptr;
        g_rows.cap = 0;
        hip_check(hipMalloc(&g_rows.ptr, c.size() * sizeof(std::uint32_t)), "hipMalloc row staging");
        g_rows.cap = c.size();
    }
    hip_check(hipMemcpy(g_rows.ptr, c.data(), c.size() * sizeof(std::uint32_t), hipMemcpyHostToDevice),
              "copy row indices");
    gather_common(x, g_rows.ptr, c.size(), max_row, out);
}

RowIndexBuffer::RowIndexBuffer(const std::vector<std::size_t>& rows) : size_(rows.size()) {
    if (size_ == 0) return;
    const std::vector<std::uint32_t> c = compact_rows(rows, &max_row_);
    hip_check(hipMalloc(&ptr_, size_ * sizeof(std::uint32_t)), "hipMalloc RowIndexBuffer");
    hip_check(hipMemcpy(ptr_, c.data(), size_ * sizeof(std::uint32_t), hipMemcpyHostToDevice),
              "copy RowIndexBuffer");
}

RowIndexBuffer RowIndexBuffer::allocate(std::size_t size, std::size_t max_row) {
    if (max_row > 0xFFFFFFFFull) throw std::invalid_argument("RowIndexBuffer row index");
    RowIndexBuffer b;
    if (size == 0) return b;
    hip_check(hipMalloc(&b.ptr_, size * sizeof(std::uint32_t)), "hipMalloc RowIndexBuffer");
    b.size_ = size;
    b.max_row_ = max_row;
    return b;
}

RowIndexBuffer::~RowIndexBuffer() {
    if (ptr_) (void)hipFree(ptr_);
}

RowIndexBuffer::RowIndexBuffer(RowIndexBuffer&& other) noexcept
    : ptr_(other.ptr_), size_(other.size_), max_row_(other.max_row_) {
    other.ptr_ = nullptr;
    other.size_ = 0;
    other.max_row_ = 0;
}

RowIndexBuffer& RowIndexBuffer::operator=(RowIndexBuffer&& other) noexcept {
    if (this != &other) {
        if (ptr_) (void)hipFree(ptr_);
        ptr_ = other.ptr_;
        size_ = other.size_;
        max_row_ = other.max_row_;
        other.ptr_ = nullptr;
        other.size_ = 0;
        other.max_row_ = 0;
    }
    return *this;
}

void gather_rows_gpu(const Tensor& x, const RowIndexBuffer& rows, Tensor& out) {
    if (rows.empty()) return;
    gather_common(x, rows.data(), rows.size(), rows.max_row(), out);
}

}  // namespace tensor_ops

// ---- tree attention (reference src/tensor.cu:2703-2735, 3342-3377) ----------

namespace {

// Device RoPE tables, one set per (device, head_dim, theta), grown on demand
// (the reference keeps one static table).
struct RopeTables {
    std::mutex mu;
    struct Entry {
        int dev;
        std::size_t half;
        float theta;
        std::size_t max_seq;
        float* cosv;
        float* sinv;
    };
    std::vector<Entry> entries;
};
RopeTables g_rope;

RopeTables::Entry rope_tables(std::size_t max_seq, std::size_t head_dim, float theta) {
    int dev = 0;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    std::lock_guard<std::mutex> lock(g_rope.mu);
    RopeTables::Entry* e = nullptr;
    for (auto& x : g_rope.entries)
        if (x.dev == dev && x.half == head_dim / 2 && x.theta == theta) e = &x;
    if (e && e->max_seq >= max_seq) return *e;
    const std::size_t half = head_dim / 2, n = max_seq * half;
    std::vector<float> c(n ? n : 1), s(n ? n : 1);
    const int rc = aps_rope_table(static_cast<int64_t>(max_seq), static_cast<int32_t>(head_dim), theta, c.data(),
                                  s.data());
    if (rc) throw_status(rc, "apply_rope_tree_gpu");
    float *dc = nullptr, *ds = nullptr;
    hip_check(hipMalloc(&dc, c.size() * sizeof(float)), "hipMalloc rope cosine");
    hip_check(hipMalloc(&ds, s.size() * sizeof(float)), "hipMalloc rope sine");
    hip_check(hipMemcpy(dc, c.data(), c.size() * sizeof(float), hipMemcpyHostToDevice), "copy rope cosine");
    hip_check(hipMemcpy(ds, s.data(), s.size() * sizeof(float), hipMemcpyHostToDevice), "copy rope sine");
    if (e) {
        // the old tables may still be read by queued kernels: the legacy
        // default stream orders this free after them
        hip_check(hipDeviceSynchronize(), "rope table resize");
        (void)hipFree(e->cosv);
        (void)hipFree(e->sinv);
        e->cosv = dc;
        e->sinv = ds;
        e->max_seq = max_seq;
        return *e;
    }
    g_rope.entries.push_back({dev, half, theta, max_seq, dc, ds});
    return g_rope.entries.back();
}

}  // namespace

namespace tensor_ops {

void apply_rope_tree_gpu(Tensor& q, Tensor& k, const std::uint32_t* row_pos, std::size_t rows, std::size_t max_seq,
                         std::size_t q_heads, std::size_t kv_heads, std::size_t head_dim, float theta) {
    if (q.size() != rows * q_heads * head_dim || k.size() != rows * kv_heads * head_dim || head_dim % 2 != 0)
        throw std::invalid_argument("apply_rope_tree_gpu shape");
    if (rows == 0) return;
    const RopeTables::Entry t = rope_tables(max_seq, head_dim, theta);
    q.cuda_data();
    k.cuda_data();
    const int rc = aps_rope_tree(q.cuda_data_write(), k.cuda_data_write(), row_pos, static_cast<int64_t>(rows),
                                 static_cast<int32_t>(q_heads), static_cast<int32_t>(kv_heads),
                                 static_cast<int32_t>(head_dim), t.cosv, t.sinv, static_cast<int64_t>(t.max_seq),
                                 nullptr);
    if (rc) throw_status(rc, "apply_rope_tree_gpu");
}

void attention_tree_gpu(const Tensor& q, const Tensor& k, const Tensor& v, Tensor& out, const std::uint32_t* row_pos,
                        const std::uint32_t* anc, std::size_t anc_stride, std::size_t rows, std::size_t max_seq,
                        std::size_t q_heads, std::size_t kv_heads, std::size_t head_dim) {
    if (q_heads != 4 * kv_heads) throw std::invalid_argument("attention_tree_gpu expects GQA-4");
    if (q.size() != rows * q_heads * head_dim || k.size() != rows * kv_heads * head_dim ||
        v.size() != k.size() || out.size() != q.size())
        throw std::invalid_argument("attention_tree_gpu shape");
    (void)max_seq;  // the window is SLIDING_WINDOW; the ancestor stride bounds the chains
    if (rows == 0) return;
    const int rc = aps_attention_tree(q.cuda_data(), k.cuda_data(), v.cuda_data(), out.cuda_data_write(), row_pos, anc,
                                      static_cast<int64_t>(anc_stride), static_cast<int64_t>(rows),
                                      static_cast<int32_t>(q_heads), static_cast<int32_t>(kv_heads),
                                      static_cast<int32_t>(head_dim), static_cast<int32_t>(apss26::SLIDING_WINDOW),
                                      nullptr);
    if (rc) throw_status(rc, "attention_tree_gpu");
}

}  // namespace tensor_ops

// ---- elementwise ops, paired projections (reference src/tensor.cu:3146-3260) -

namespace tensor_ops {

void zero_gpu(Tensor& x) {
    const int rc = aps_zero(x.cuda_data_write(), static_cast<int64_t>(x.size()), nullptr);
    if (rc) throw_status(rc, "zero_gpu");
}

void add_inplace_gpu(Tensor& a, const Tensor& b) {
    if (a.size() != b.size()) throw std::invalid_argument("add shape");
    if (!a.size()) return;
    a.cuda_data();  // upload a stale device copy before writing in place
    const int rc = aps_add_inplace(a.cuda_data_write(), b.cuda_data(), static_cast<int64_t>(a.size()), nullptr);
    if (rc) throw_status(rc, "add_inplace_gpu");
}

void add_bias_inplace_gpu(Tensor& a, const Tensor& bias) {
    if (bias.ndim() != 1 || a.ndim() == 0 || a.size(a.ndim() - 1) != bias.size(0) || bias.size(0) == 0)
        throw std::invalid_argument("bias shape");
    if (!a.size()) return;
    a.cuda_data();
    const int rc = aps_add_bias_inplace(a.cuda_data_write(), bias.cuda_data(), static_cast<int64_t>(a.size()),
                                        static_cast<int32_t>(bias.size(0)), nullptr);
    if (rc) throw_status(rc, "add_bias_inplace_gpu");
}

void silu_mul_gpu(const Tensor& gate, const Tensor& up, Tensor& out) {
    if (gate.size() != up.size() || out.size() != gate.size()) throw std::invalid_argument("silu_mul shape");
    if (!gate.size()) return;
    const float* g = gate.cuda_data();
    const float* u = up.cuda_data();
    const int rc = aps_silu_mul(g, u, out.cuda_data_write(), static_cast<int64_t>(gate.size()), nullptr);
    if (rc) throw_status(rc, "silu_mul_gpu");
}

void matmul_pair_silu_gpu(const Tensor& a, const Tensor& gate_weight, const Tensor& up_weight, Tensor& out) {
    const std::size_t k = a.size(a.ndim() - 1);
    const std::size_t m = a.size() / k;
    const std::size_t n = gate_weight.size(0);
    if (gate_weight.size(1) != k || up_weight.size(0) != n || up_weight.size(1) != k || out.size(0) != m ||
        out.size(1) != n)
        throw std::invalid_argument("matmul_pair_silu_gpu shape");
    // the two products as single fp32 chains, then the SiLU-mul: the
    // reference kernel's arithmetic per output, in three launches
    Tensor g({m, n}), u({m, n});
    matmul_transposed_gpu(a, gate_weight, g);
    matmul_transposed_gpu(a, up_weight, u);
    silu_mul_gpu(g, u, out);
}

void matmul_pair_bias_gpu(const Tensor& a, const Tensor& first_weight, const Tensor& first_bias, Tensor& first_out,
                          const Tensor& second_weight, const Tensor& second_bias, Tensor& second_out) {
    const std::size_t k = a.size(a.ndim() - 1);
    const std::size_t m = a.size() / k;
    const std::size_t n = first_weight.size(0);
    if (first_weight.size(1) != k || second_weight.size(0) != n || second_weight.size(1) != k ||
        first_bias.size() != n || second_bias.size() != n || first_out.size(0) != m || first_out.size(1) != n ||
        second_out.size(0) != m || second_out.size(1) != n)
        throw std::invalid_argument("matmul_pair_bias_gpu shape");
    if (first_weight.has_cuda_bf16_weight() || second_weight.has_cuda_bf16_weight()) {
        // the split-bf16 Linear (USE_TC) per output
        matmul_transposed_bias_gpu(a, first_weight, first_bias, first_out);
        matmul_transposed_bias_gpu(a, second_weight, second_bias, second_out);
        return;
    }
    if (k % 16 != 0 || n % 4 != 0) {
        // shapes the one-grid kernel does not take: each output on its own
        // (aps_linear's general kernel, the same chains)
        matmul_transposed_bias_gpu(a, first_weight, first_bias, first_out);
        matmul_transposed_bias_gpu(a, second_weight, second_bias, second_out);
        return;
    }
    // both outputs in one grid (their column blocks share it)
    const float* ws[2] = {first_weight.cuda_data(), second_weight.cuda_data()};
    const float* bs[2] = {first_bias.cuda_data(), second_bias.cuda_data()};
    float* ys[2] = {first_out.cuda_data_write(), second_out.cuda_data_write()};
    const std::int32_t ns[2] = {static_cast<std::int32_t>(n), static_cast<std::int32_t>(n)};
    const int rc = aps_linear_multi(a.cuda_data(), static_cast<std::int64_t>(m), static_cast<std::int32_t>(k), 2, ws,
                                    bs, ns, ys, nullptr);
    if (rc) throw_status(rc, "matmul_pair_bias_gpu");
}

}  // namespace tensor_ops

// ---- packed-sequence RoPE and attention (reference src/tensor.cu:3296-3340) ---

namespace {

// Per-row segment start and position of a packed batch, on the device,
// cached per seq_lens (the reference's packed_meta keeps the last one; this
// keeps a few, since a prefill alternates between the same two or three).
// Entries are shared: a caller holds its entry until its launches are
// queued, so evicting it from the cache (another thread, a ninth seq_lens)
// never frees arrays a launch is about to use; the last holder frees them
// after the device has finished its queued work.
struct PackedSegments {
    std::vector<std::size_t> lens;
    std::size_t rows = 0, max_seq = 0;
    int dev = 0;
    std::uint32_t* offset = nullptr;  // [rows]
    std::uint32_t* pos = nullptr;     // [rows]
    PackedSegments() = default;
    PackedSegments(const PackedSegments&) = delete;
    PackedSegments& operator=(const PackedSegments&) = delete;
    ~PackedSegments() {
        if (!offset && !pos) return;
        int cur = 0;
        (void)hipGetDevice(&cur);
        if (cur != dev) (void)hipSetDevice(dev);
        (void)hipDeviceSynchronize();
        (void)hipFree(offset);
        (void)hipFree(pos);
        if (cur != dev) (void)hipSetDevice(cur);
    }
};
std::mutex g_seg_mu;
// never destroyed: its entries call into HIP, which may be gone at exit
std::deque<std::shared_ptr<const PackedSegments>>& g_segs = *new std::deque<std::shared_ptr<const PackedSegments>>();

std::shared_ptr<const PackedSegments> packed_segments(const std::vector<std::size_t>& seq_lens) {
    int dev = 0;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    std::lock_guard<std::mutex> lock(g_seg_mu);
    for (const auto& e : g_segs)
        if (e->dev == dev && e->lens == seq_lens) return e;
    auto entry = std::make_shared<PackedSegments>();
    PackedSegments& s = *entry;
    s.lens = seq_lens;
    s.dev = dev;
    std::vector<std::uint32_t> off, pos;
    for (std::size_t len : seq_lens) {
        if (s.rows + len > 0xFFFFFFFFull) throw std::invalid_argument("packed sequence lengths");
        for (std::size_t p = 0; p < len; ++p) {
            off.push_back(static_cast<std::uint32_t>(s.rows));
            pos.push_back(static_cast<std::uint32_t>(p));
        }
        s.rows += len;
        s.max_seq = std::max(s.max_seq, len);
    }
    if (s.rows) {
        hip_check(hipMalloc(&s.offset, s.rows * sizeof(std::uint32_t)), "hipMalloc segment offsets");
        hip_check(hipMalloc(&s.pos, s.rows * sizeof(std::uint32_t)), "hipMalloc segment positions");
        hip_check(hipMemcpy(s.offset, off.data(), s.rows * sizeof(std::uint32_t), hipMemcpyHostToDevice),
                  "copy segment offsets");
        hip_check(hipMemcpy(s.pos, pos.data(), s.rows * sizeof(std::uint32_t), hipMemcpyHostToDevice),
                  "copy segment positions");
    }
    if (g_segs.size() == 8) g_segs.pop_front();  // keep the cache small; holders keep their entry alive
    g_segs.push_back(entry);
    return entry;
}

}  // namespace

namespace tensor_ops {

void apply_rope_gpu(Tensor& q, Tensor& k, const std::vector<std::size_t>& seq_lens, std::size_t q_heads,
                    std::size_t kv_heads, std::size_t head_dim, float theta) {
    const std::size_t rows = head_dim && q_heads ? q.size() / (q_heads * head_dim) : 0;
    if (q.size() != rows * q_heads * head_dim || k.size() != rows * kv_heads * head_dim || head_dim % 2 != 0)
        throw std::invalid_argument("apply_rope_gpu shape");
    const auto seg = packed_segments(seq_lens);
    if (seg->rows != rows) throw std::invalid_argument("packed sequence lengths");
    if (rows == 0) return;
    // positions restart per sequence, so the longest sequence bounds the table
    apply_rope_tree_gpu(q, k, seg->pos, rows, seg->max_seq, q_heads, kv_heads, head_dim, theta);
}

void attention_gpu(const Tensor& q, const Tensor& k, const Tensor& v, Tensor& out,
                   const std::vector<std::size_t>& seq_lens, std::size_t q_heads, std::size_t kv_heads,
                   std::size_t head_dim) {
    // GQA-4 takes the grouped kernel, other layouts the generic one (as the
    // reference's attention_gpu, src/tensor.cu:3316-3340)
    if (kv_heads == 0 || q_heads % kv_heads != 0) throw std::invalid_argument("attention_gpu shape");
    const std::size_t rows = head_dim && q_heads ? q.size() / (q_heads * head_dim) : 0;
    if (q.size() != rows * q_heads * head_dim || k.size() != rows * kv_heads * head_dim || v.size() != k.size() ||
        out.size() != q.size())
        throw std::invalid_argument("attention_gpu shape");
    const auto seg = packed_segments(seq_lens);
    if (seg->rows != rows) throw std::invalid_argument("packed sequence lengths");
    if (rows == 0) return;
    const int rc = aps_attention_packed(q.cuda_data(), k.cuda_data(), v.cuda_data(), out.cuda_data_write(),
                                        seg->offset, seg->pos, static_cast<int64_t>(seg->max_seq),
                                        static_cast<int64_t>(rows), static_cast<int32_t>(q_heads),
                                        static_cast<int32_t>(kv_heads), static_cast<int32_t>(head_dim),
                                        static_cast<int32_t>(apss26::SLIDING_WINDOW), nullptr);
    if (rc) throw_status(rc, "attention_gpu");
}

}  // namespace tensor_ops
