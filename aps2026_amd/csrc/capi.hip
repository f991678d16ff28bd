// C ABI of the MoE engine (declared in include/aps_moe.h).
//
// Host-side replacement of the reference's launch layer for this path:
// register_moe_weights_gpu / moe_forward_grouped_gpu (src/tensor.cu:2757-2928)
// and the router call of PhiMoE::forward (src/layer.cu:113-121).  Differences
// by design:
//  * weights are packed once into kernel-native layouts owned by the library
//    (the reference keeps pointers to the caller's fp32 tensors);
//  * all scratch comes from a caller-provided workspace, so a forward call
//    performs no allocation and no host synchronisation;
//  * errors are status codes plus a thread-local message instead of C++
//    exceptions crossing the ABI.
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/aps_moe.h"
#include "common.hpp"

namespace {

thread_local std::string g_error;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_error = buf;
    return code;
}

int hip_fail(hipError_t err, const char* what) {
    return fail(APS_ERR_HIP, "%s: %s", what, hipGetErrorString(err));
}

#define APS_HIP(call, what)                                 \
    do {                                                    \
        hipError_t err_ = (call);                           \
        if (err_ != hipSuccess) return hip_fail(err_, what); \
    } while (0)

struct WeightSet {
    int device = 0;
    int E = 0, H = 0, F = 0;
    int compute = APS_DTYPE_F32;
    // bf16 path
    aps::bf16_t* w13 = nullptr;  // tile images [E][F/64][H/64][128][64]
    aps::bf16_t* w2b = nullptr;  // tile images [E][H/128][F/64][128][64]
    // f32 path
    float* w1 = nullptr;         // [E][F][H]
    float* w3 = nullptr;         // [E][F][H]
    float* w2 = nullptr;         // [E][H][F]
    // fp8 path
    uint8_t* q13 = nullptr;      // e4m3 tile images [E][F/64][H/128][128][128]
    uint8_t* q2 = nullptr;       // e4m3 tile images [E][H/128][Kp/128][128][128]
    float* s1 = nullptr;         // [E][F] per-channel scales of w1
    float* s3 = nullptr;         // [E][F]
    float* s2 = nullptr;         // [E][H]
    ~WeightSet() {
        int cur = 0;
        (void)hipGetDevice(&cur);
        if (cur != device) (void)hipSetDevice(device);
        for (void* p : {static_cast<void*>(w13), static_cast<void*>(w2b), static_cast<void*>(w1),
                        static_cast<void*>(w3), static_cast<void*>(w2), static_cast<void*>(q13),
                        static_cast<void*>(q2), static_cast<void*>(s1), static_cast<void*>(s3),
                        static_cast<void*>(s2)})
            if (p) (void)hipFree(p);
        if (cur != device) (void)hipSetDevice(cur);
    }
};

std::mutex g_mu;
std::vector<std::unique_ptr<WeightSet>> g_sets;  // handle h -> g_sets[h-1]

WeightSet* lookup(uint64_t handle) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (handle == 0 || handle > g_sets.size()) return nullptr;
    return g_sets[handle - 1].get();
}

constexpr size_t kAlign = 256;
size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

size_t kpad128(int n) { return (static_cast<size_t>(n) + 127) / 128 * 128; }

void make_layout(const WeightSet& w, int64_t rows, aps_moe_ws_layout* L) {
    std::memset(L, 0, sizeof(*L));
    const size_t T = static_cast<size_t>(rows);
    const size_t E = static_cast<size_t>(w.E);
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t at = off;
        off = align_up(off + bytes);
        return at;
    };
    const size_t elt = w.compute == APS_DTYPE_F32 ? 4 : 2;
    L->logits = take(T * E * 4);
    L->routes = take(T * 2);
    L->tile_counts = take(static_cast<size_t>(aps::ceil_div(rows, aps::kTileTokens)) * E * 4);
    L->counts = take(E * 4);
    L->offsets = take((E + 1) * 4);
    L->assignment_rows = take(2 * T * 4);
    L->route_positions = take(2 * T * 4);
    L->act = take(2 * T * static_cast<size_t>(w.F) * elt);
    L->y = take(2 * T * static_cast<size_t>(w.H) * elt);
    L->act_scale = 0;
    L->actq = 0;
    L->xq = 0;
    L->xq_scale = 0;
    // the fused forward's folded combine: the slot-0 histogram and the
    // dispatch's slot-ordered lists
    L->tile_counts0 = take(static_cast<size_t>(aps::ceil_div(rows, aps::kTileTokens)) * E * 4);
    L->slot1 = take(E * 4);
    L->slot_rows = take(2 * T * 4);
    L->slot_tokens = take(2 * T * 4);
    if (w.compute == APS_DTYPE_BF16) {
        // bf16 copy of x for the fused entry points when x arrives as fp32:
        // written by the router, last read by the w1||w3 GEMM, so it shares
        // the bytes of y (first written by the w2 GEMM, after it); nothing is
        // reserved for it, whatever the dtype of x
        L->xq = L->y;
    } else if (w.compute == APS_DTYPE_E4M3) {
        L->xq = take(T * static_cast<size_t>(w.H));
        L->xq_scale = take(T * 4);
        L->actq = take(2 * T * static_cast<size_t>(kpad128(w.F)));
        L->act_scale = take(2 * T * 4);
    }
    L->total_bytes = off;
}

int check_device(const WeightSet& w) {
    int cur = 0;
    APS_HIP(hipGetDevice(&cur), "hipGetDevice");
    if (cur != w.device)
        return fail(APS_ERR_ARG, "weight set lives on device %d but device %d is current", w.device, cur);
    return APS_OK;
}

// The two grouped GEMMs of the expert FFN over a filled routing plan
// (offsets, assignment_rows).  Shared by every entry point that runs them.
int run_ffn_up(const WeightSet& w, const void* x, int64_t rows, const uint32_t* offsets,
               const uint32_t* arows, void* act, hipStream_t s) {
    if (w.compute == APS_DTYPE_F32)
        APS_HIP(aps::launch_ffn_up_f32(static_cast<const float*>(x), offsets, arows, w.w1, w.w3,
                                       static_cast<float*>(act), rows, w.H, w.F, w.E, s),
                "ffn_up_f32 launch");
    else
        APS_HIP(aps::launch_ffn_up_bf16(static_cast<const aps::bf16_t*>(x), offsets, arows, w.w13,
                                        static_cast<aps::bf16_t*>(act), rows, w.H, w.F, w.E, s),
                "ffn_up_bf16 launch");
    return APS_OK;
}

int run_ffn_down(const WeightSet& w, const void* act, int64_t rows, const uint32_t* offsets, void* y,
                 hipStream_t s) {
    if (w.compute == APS_DTYPE_F32)
        APS_HIP(aps::launch_ffn_down_f32(static_cast<const float*>(act), offsets, w.w2,
                                         static_cast<float*>(y), rows, w.H, w.F, w.E, s),
                "ffn_down_f32 launch");
    else
        APS_HIP(aps::launch_ffn_down_bf16(static_cast<const aps::bf16_t*>(act), offsets, w.w2b,
                                          static_cast<aps::bf16_t*>(y), rows, w.H, w.F, w.E, s),
                "ffn_down_bf16 launch");
    return APS_OK;
}

int run_ffn(const WeightSet& w, const void* x, int64_t rows, const uint32_t* offsets,
            const uint32_t* arows, void* act, void* y, hipStream_t s) {
    if (int rc = run_ffn_up(w, x, rows, offsets, arows, act, s)) return rc;
    return run_ffn_down(w, act, rows, offsets, y, s);
}

// The fp8 path quantises x and the activations per row inside the fused
// entry points, so its staged GEMMs are not exposed on their own.
int check_not_fp8(const WeightSet& w, const char* what) {
    if (w.compute == APS_DTYPE_E4M3)
        return fail(APS_ERR_DTYPE, "%s: fp8 weight sets run through aps_moe_forward / aps_moe_forward_grouped", what);
    return APS_OK;
}

int check_x_dtype(const WeightSet& w, int32_t x_dtype) {
    const int want = w.compute == APS_DTYPE_F32 ? APS_DTYPE_F32 : APS_DTYPE_BF16;  // fp8 sets quantise bf16 x
    if (x_dtype != want)
        return fail(APS_ERR_DTYPE, "x dtype %d does not match the weight set (expects %d)", x_dtype, want);
    return APS_OK;
}

// Routing (from `logits`; nullptr when the router kernel already wrote the
// routes and tile histogram into the workspace), dispatch, FFN and combine.
// The fp8 path with bf16 output folds the combine into the w2 GEMM when the
// router wrote the slot-0 histogram (aps_moe_forward): no y round trip.
bool fold_combine(const WeightSet& w, int64_t rows, int32_t out_dtype) {
    return w.compute == APS_DTYPE_E4M3 && out_dtype == APS_DTYPE_BF16 && aps::ffn_down_fold_fits(rows, w.H, w.F);
}

// xq_ready: the router has written the fp8 codes and scales of x (fp8 path).
int grouped_from_logits(const WeightSet& w, const void* x, bool x_is_f32, const float* logits, int64_t rows,
                        void* out, int32_t out_dtype, char* ws, const aps_moe_ws_layout& L,
                        hipStream_t s, bool fold = false, bool xq_ready = false) {
    auto* routes = reinterpret_cast<uint8_t*>(ws + L.routes);
    auto* tiles = reinterpret_cast<uint32_t*>(ws + L.tile_counts);
    auto* counts = reinterpret_cast<uint32_t*>(ws + L.counts);
    auto* offsets = reinterpret_cast<uint32_t*>(ws + L.offsets);
    auto* arows = reinterpret_cast<uint32_t*>(ws + L.assignment_rows);
    auto* rpos = reinterpret_cast<uint32_t*>(ws + L.route_positions);
    if (x_is_f32 && w.compute == APS_DTYPE_BF16) {
        auto* xb = reinterpret_cast<aps::bf16_t*>(ws + L.xq);
        APS_HIP(aps::launch_to_bf16(static_cast<const float*>(x), xb, rows * w.H, s), "x to bf16 launch");
        x = xb;
    }
    if (logits) APS_HIP(aps::launch_route_top2(logits, rows, w.E, routes, tiles, s), "route_top2 launch");
    auto* tiles0 = reinterpret_cast<uint32_t*>(ws + L.tile_counts0);
    auto* slot1 = reinterpret_cast<uint32_t*>(ws + L.slot1);
    auto* srows = reinterpret_cast<uint32_t*>(ws + L.slot_rows);
    auto* stoks = reinterpret_cast<uint32_t*>(ws + L.slot_tokens);
    if (fold)
        APS_HIP(aps::launch_dispatch_scatter(routes, tiles, rows, w.E, counts, offsets, arows, rpos, nullptr, s,
                                             tiles0, slot1, srows, stoks),
                "dispatch launch");
    else
        APS_HIP(aps::launch_dispatch_scatter(routes, tiles, rows, w.E, counts, offsets, arows, rpos, nullptr, s),
                "dispatch launch");
    if (w.compute == APS_DTYPE_E4M3) {
        auto* xq = reinterpret_cast<uint8_t*>(ws + L.xq);
        auto* xs = reinterpret_cast<float*>(ws + L.xq_scale);
        auto* act = reinterpret_cast<aps::bf16_t*>(ws + L.act);
        auto* actq = reinterpret_cast<uint8_t*>(ws + L.actq);
        auto* as = reinterpret_cast<float*>(ws + L.act_scale);
        const int64_t kp = static_cast<int64_t>(kpad128(w.F));
        if (!xq_ready)
            APS_HIP(aps::launch_quant_rows_e4m3(static_cast<const aps::bf16_t*>(x), w.H, w.H, xq, w.H, xs, rows, s),
                    "quantise x launch");
        APS_HIP(aps::launch_ffn_up_fp8(xq, xs, offsets, arows, w.q13, w.s1, w.s3, act, rows, w.H, w.F, w.E, s),
                "ffn_up_fp8 launch");
        APS_HIP(aps::launch_quant_rows_e4m3(act, w.F, w.F, actq, kp, as, 2 * rows, s), "quantise act launch");
        if (fold) {
            // slot-0 rows to y's bytes as [rows][H] by token, then slot-1 rows
            // combined with them straight into out
            APS_HIP(aps::launch_ffn_down_fold_fp8(actq, as, offsets, slot1, srows, stoks, w.q2, w.s2,
                                                  reinterpret_cast<aps::bf16_t*>(ws + L.y),
                                                  static_cast<aps::bf16_t*>(out), rows, w.H, w.F, w.E, s),
                    "ffn_down_fold_fp8 launch");
            return APS_OK;
        }
        APS_HIP(aps::launch_ffn_down_fp8(actq, as, offsets, w.q2, w.s2, reinterpret_cast<aps::bf16_t*>(ws + L.y),
                                         rows, w.H, w.F, w.E, s),
                "ffn_down_fp8 launch");
    } else {
        int rc = run_ffn(w, x, rows, offsets, arows, ws + L.act, ws + L.y, s);
        if (rc) return rc;
    }
    APS_HIP(aps::launch_combine(ws + L.y, w.compute != APS_DTYPE_F32, rpos, rows, w.H, out,
                                out_dtype == APS_DTYPE_BF16, s),
            "combine launch");
    return APS_OK;
}

}  // namespace

extern "C" {

const char* aps_moe_last_error(void) { return g_error.c_str(); }
int aps_moe_abi_version(void) { return APS_MOE_ABI_VERSION; }

int aps_moe_weights_register(const aps_moe_weights_desc* d, void* stream, uint64_t* handle_out) {
    if (!d || !handle_out) return fail(APS_ERR_ARG, "register: NULL descriptor or handle pointer");
    *handle_out = 0;
    // reference: "MoE weight table size" (src/tensor.cu:2761-2764).  One
    // expert is a dense FFN (aps_mlp_forward); routing needs two or more.
    if (d->num_experts < 1 || d->num_experts > aps::kMaxExperts)
        return fail(APS_ERR_SHAPE, "MoE weight table size: %d experts (1..%d supported)",
                    d->num_experts, aps::kMaxExperts);
    if (d->hidden <= 0 || d->ffn <= 0 || d->hidden % 256 != 0 || d->ffn % 64 != 0)
        return fail(APS_ERR_SHAPE, "hidden %d must be a multiple of 256 and ffn %d of 64",
                    d->hidden, d->ffn);
    if (!d->w1 || !d->w3 || !d->w2) return fail(APS_ERR_ARG, "register: NULL weight table");
    for (int e = 0; e < d->num_experts; ++e)
        if (!d->w1[e] || !d->w3[e] || !d->w2[e])
            return fail(APS_ERR_ARG, "register: NULL weight pointer for expert %d", e);
    if (d->compute_dtype == APS_DTYPE_F32) {
        if (d->src_dtype != APS_DTYPE_F32)
            return fail(APS_ERR_DTYPE, "fp32 compute needs fp32 source weights");
    } else if (d->compute_dtype == APS_DTYPE_BF16) {
        if (d->src_dtype != APS_DTYPE_F32 && d->src_dtype != APS_DTYPE_BF16)
            return fail(APS_ERR_DTYPE, "bf16 compute needs fp32 or bf16 source weights");
    } else if (d->compute_dtype == APS_DTYPE_E4M3) {
        if (d->src_dtype != APS_DTYPE_E4M3)
            return fail(APS_ERR_DTYPE, "fp8 compute needs e4m3 source weights with per-channel scales");
        if (!d->w1_scale || !d->w3_scale || !d->w2_scale)
            return fail(APS_ERR_ARG, "register: NULL fp8 scale table");
        for (int e = 0; e < d->num_experts; ++e)
            if (!d->w1_scale[e] || !d->w3_scale[e] || !d->w2_scale[e])
                return fail(APS_ERR_ARG, "register: NULL fp8 scale pointer for expert %d", e);
    } else {
        return fail(APS_ERR_DTYPE, "compute dtype %d not supported", d->compute_dtype);
    }

    auto w = std::make_unique<WeightSet>();
    APS_HIP(hipGetDevice(&w->device), "hipGetDevice");
    w->E = d->num_experts;
    w->H = d->hidden;
    w->F = d->ffn;
    w->compute = d->compute_dtype;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const size_t fh = static_cast<size_t>(w->F) * w->H;
    const size_t n = fh * w->E;
    if (w->compute == APS_DTYPE_F32) {
        APS_HIP(hipMalloc(&w->w1, n * 4), "hipMalloc w1");
        APS_HIP(hipMalloc(&w->w3, n * 4), "hipMalloc w3");
        APS_HIP(hipMalloc(&w->w2, n * 4), "hipMalloc w2");
        for (int e = 0; e < w->E; ++e) {
            APS_HIP(hipMemcpyAsync(w->w1 + e * fh, d->w1[e], fh * 4, hipMemcpyDeviceToDevice, s), "copy w1");
            APS_HIP(hipMemcpyAsync(w->w3 + e * fh, d->w3[e], fh * 4, hipMemcpyDeviceToDevice, s), "copy w3");
            APS_HIP(hipMemcpyAsync(w->w2 + e * fh, d->w2[e], fh * 4, hipMemcpyDeviceToDevice, s), "copy w2");
        }
    } else if (w->compute == APS_DTYPE_E4M3) {
        const size_t kp = kpad128(w->F);
        APS_HIP(hipMalloc(&w->q13, 2 * n), "hipMalloc w13 fp8");
        APS_HIP(hipMalloc(&w->q2, static_cast<size_t>(w->E) * w->H * kp), "hipMalloc w2 fp8");
        APS_HIP(hipMalloc(&w->s1, static_cast<size_t>(w->E) * w->F * 4), "hipMalloc s1");
        APS_HIP(hipMalloc(&w->s3, static_cast<size_t>(w->E) * w->F * 4), "hipMalloc s3");
        APS_HIP(hipMalloc(&w->s2, static_cast<size_t>(w->E) * w->H * 4), "hipMalloc s2");
        for (int e = 0; e < w->E; ++e) {
            APS_HIP(hipMemcpyAsync(w->s1 + static_cast<size_t>(e) * w->F, d->w1_scale[e], w->F * 4u,
                                   hipMemcpyDeviceToDevice, s), "copy s1");
            APS_HIP(hipMemcpyAsync(w->s3 + static_cast<size_t>(e) * w->F, d->w3_scale[e], w->F * 4u,
                                   hipMemcpyDeviceToDevice, s), "copy s3");
            APS_HIP(hipMemcpyAsync(w->s2 + static_cast<size_t>(e) * w->H, d->w2_scale[e], w->H * 4u,
                                   hipMemcpyDeviceToDevice, s), "copy s2");
        }
        APS_HIP(aps::launch_pack_w13_e4m3(d->w1, d->w3, w->q13, w->E, w->F, w->H, s), "pack w1/w3 fp8");
        APS_HIP(aps::launch_pack_w2_e4m3(d->w2, w->q2, w->E, w->F, w->H, s), "pack w2 fp8");
    } else {
        const bool src_bf16 = d->src_dtype == APS_DTYPE_BF16;
        APS_HIP(hipMalloc(&w->w13, 2 * n * 2), "hipMalloc w13");
        APS_HIP(hipMalloc(&w->w2b, n * 2), "hipMalloc w2");
        APS_HIP(aps::launch_pack_w13_bf16(d->w1, d->w3, src_bf16, w->w13, w->E, w->F, w->H, s),
                "pack w1/w3");
        APS_HIP(aps::launch_pack_w2_bf16(d->w2, src_bf16, w->w2b, w->E, w->F, w->H, s), "pack w2");
    }
    APS_HIP(hipStreamSynchronize(s), "register: synchronize");
    std::lock_guard<std::mutex> lk(g_mu);
    g_sets.push_back(std::move(w));
    *handle_out = g_sets.size();
    return APS_OK;
}

int aps_moe_weights_release(uint64_t handle) {
    std::unique_ptr<WeightSet> victim;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        if (handle == 0 || handle > g_sets.size() || !g_sets[handle - 1])
            return fail(APS_ERR_HANDLE, "release: invalid handle %llu", (unsigned long long)handle);
        victim = std::move(g_sets[handle - 1]);
    }
    (void)hipDeviceSynchronize();  // the set may still be in use by queued work
    return APS_OK;
}

int aps_moe_workspace_layout(uint64_t handle, int64_t rows, aps_moe_ws_layout* out) {
    const WeightSet* w = lookup(handle);
    if (!w) return fail(APS_ERR_HANDLE, "grouped MoE shape or handle: invalid handle %llu",
                        (unsigned long long)handle);
    if (!out) return fail(APS_ERR_ARG, "workspace_layout: NULL output");
    if (rows < 0 || rows > (int64_t(1) << 30)) return fail(APS_ERR_SHAPE, "rows %lld out of range", (long long)rows);
    make_layout(*w, rows, out);
    return APS_OK;
}

size_t aps_moe_dispatch_workspace_size(int64_t rows, int32_t num_experts) {
    if (rows < 0 || num_experts <= 0) return 0;
    // tile histogram, then the clamped-id counter
    return static_cast<size_t>(aps::ceil_div(rows, aps::kTileTokens)) * num_experts * 4 + 4;
}

int aps_router_logits(const void* x, int32_t x_dtype, const float* gate, int64_t rows,
                      int32_t hidden, int32_t num_experts, float* logits, void* stream) {
    if (rows < 0 || hidden <= 0 || hidden % 256 != 0 || num_experts <= 0 || num_experts > aps::kMaxExperts)
        return fail(APS_ERR_SHAPE, "matmul_transposed_gpu shape: rows %lld hidden %d experts %d",
                    (long long)rows, hidden, num_experts);
    if (x_dtype != APS_DTYPE_F32 && x_dtype != APS_DTYPE_BF16)
        return fail(APS_ERR_DTYPE, "router x dtype %d not supported", x_dtype);
    if (rows > 0 && (!x || !gate || !logits)) return fail(APS_ERR_ARG, "router: NULL pointer");
    APS_HIP(aps::launch_router(x, x_dtype == APS_DTYPE_BF16, gate, rows, hidden, num_experts, logits, nullptr,
                               nullptr, nullptr, nullptr, nullptr, nullptr, static_cast<hipStream_t>(stream)),
            "router_logits launch");
    return APS_OK;
}

int aps_moe_route_top2(const float* logits, int64_t rows, int32_t num_experts, uint8_t* routes,
                       void* stream) {
    if (rows < 0 || num_experts < 2 || num_experts > aps::kMaxExperts)
        return fail(APS_ERR_SHAPE, "route_top2: rows %lld experts %d", (long long)rows, num_experts);
    if (rows > 0 && (!logits || !routes)) return fail(APS_ERR_ARG, "route_top2: NULL pointer");
    APS_HIP(aps::launch_route_top2(logits, rows, num_experts, routes, nullptr,
                                   static_cast<hipStream_t>(stream)),
            "route_top2 launch");
    return APS_OK;
}

int aps_moe_dispatch(const uint8_t* routes, int64_t rows, int32_t num_experts, uint32_t* counts,
                     uint32_t* offsets, uint32_t* assignment_rows, uint32_t* route_positions,
                     void* scratch, size_t scratch_bytes, void* stream) {
    if (rows < 0 || num_experts < 2 || num_experts > aps::kMaxExperts)
        return fail(APS_ERR_SHAPE, "dispatch: rows %lld experts %d", (long long)rows, num_experts);
    if (!counts || !offsets) return fail(APS_ERR_ARG, "dispatch: NULL counts/offsets");
    if (rows > 0 && (!routes || !assignment_rows || !route_positions))
        return fail(APS_ERR_ARG, "dispatch: NULL pointer");
    const size_t need = aps_moe_dispatch_workspace_size(rows, num_experts);
    if (need && (!scratch || scratch_bytes < need))
        return fail(APS_ERR_WORKSPACE, "dispatch: scratch %zu bytes, need %zu", scratch_bytes, need);
    hipStream_t s = static_cast<hipStream_t>(stream);
    auto* tiles = static_cast<uint32_t*>(scratch);
    auto* status = reinterpret_cast<uint32_t*>(static_cast<char*>(scratch) + need - 4);
    APS_HIP(aps::launch_tile_hist(routes, rows, num_experts, tiles, status, s), "tile_hist launch");
    APS_HIP(aps::launch_dispatch_scatter(routes, tiles, rows, num_experts, counts, offsets,
                                         assignment_rows, route_positions, status, s),
            "dispatch launch");
    return APS_OK;
}

int aps_moe_expert_ffn(uint64_t handle, const void* x, int32_t x_dtype, int64_t rows,
                       const uint32_t* offsets, const uint32_t* assignment_rows, void* act,
                       float* act_scale, void* y_perm, void* stream) {
    (void)act_scale;
    const WeightSet* w = lookup(handle);
    if (!w) return fail(APS_ERR_HANDLE, "grouped MoE shape or handle: invalid handle %llu",
                        (unsigned long long)handle);
    if (int rc = check_device(*w)) return rc;
    if (int rc = check_not_fp8(*w, "expert_ffn")) return rc;
    if (rows < 0) return fail(APS_ERR_SHAPE, "expert_ffn: rows %lld", (long long)rows);
    if (int rc = check_x_dtype(*w, x_dtype)) return rc;
    if (rows > 0 && (!x || !offsets || !assignment_rows || !act || !y_perm))
        return fail(APS_ERR_ARG, "expert_ffn: NULL pointer");
    return run_ffn(*w, x, rows, offsets, assignment_rows, act, y_perm, static_cast<hipStream_t>(stream));
}

int aps_moe_ffn_up(uint64_t handle, const void* x, int32_t x_dtype, int64_t rows,
                   const uint32_t* offsets, const uint32_t* assignment_rows, void* act,
                   float* act_scale, void* stream) {
    (void)act_scale;
    const WeightSet* w = lookup(handle);
    if (!w) return fail(APS_ERR_HANDLE, "grouped MoE shape or handle: invalid handle %llu",
                        (unsigned long long)handle);
    if (int rc = check_device(*w)) return rc;
    if (int rc = check_not_fp8(*w, "ffn_up")) return rc;
    if (rows < 0) return fail(APS_ERR_SHAPE, "ffn_up: rows %lld", (long long)rows);
    if (int rc = check_x_dtype(*w, x_dtype)) return rc;
    if (rows > 0 && (!x || !offsets || !assignment_rows || !act)) return fail(APS_ERR_ARG, "ffn_up: NULL pointer");
    return run_ffn_up(*w, x, rows, offsets, assignment_rows, act, static_cast<hipStream_t>(stream));
}

int aps_moe_ffn_down(uint64_t handle, const void* act, const float* act_scale, int64_t rows,
                     const uint32_t* offsets, void* y_perm, void* stream) {
    (void)act_scale;
    const WeightSet* w = lookup(handle);
    if (!w) return fail(APS_ERR_HANDLE, "grouped MoE shape or handle: invalid handle %llu",
                        (unsigned long long)handle);
    if (int rc = check_device(*w)) return rc;
    if (int rc = check_not_fp8(*w, "ffn_down")) return rc;
    if (rows < 0) return fail(APS_ERR_SHAPE, "ffn_down: rows %lld", (long long)rows);
    if (rows > 0 && (!act || !offsets || !y_perm)) return fail(APS_ERR_ARG, "ffn_down: NULL pointer");
    return run_ffn_down(*w, act, rows, offsets, y_perm, static_cast<hipStream_t>(stream));
}

int aps_quantise_rows_e4m3(const void* src, int64_t src_stride, int32_t n, uint8_t* dst, int64_t dst_stride,
                           float* scale, int64_t rows, void* stream) {
    if (rows < 0 || n <= 0 || n % 8 != 0 || dst_stride < n || dst_stride % 8 != 0 || dst_stride > 8192 ||
        src_stride < n || src_stride % 8 != 0)
        return fail(APS_ERR_SHAPE, "quantise_rows_e4m3: rows %lld n %d strides %lld/%lld", (long long)rows, n,
                    (long long)src_stride, (long long)dst_stride);
    if (rows > 0 && (!src || !dst || !scale)) return fail(APS_ERR_ARG, "quantise_rows_e4m3: NULL pointer");
    if (rows > 0 && (reinterpret_cast<uintptr_t>(src) & 15u))
        return fail(APS_ERR_ARG, "quantise_rows_e4m3: src must be 16-byte aligned");
    APS_HIP(aps::launch_quant_rows_e4m3(static_cast<const aps::bf16_t*>(src), src_stride, n, dst, dst_stride, scale,
                                        rows, static_cast<hipStream_t>(stream)),
            "quantise_rows_e4m3 launch");
    return APS_OK;
}

static int fp8_set(uint64_t handle, const WeightSet** out, const char* what) {
    const WeightSet* w = lookup(handle);
    if (!w) return fail(APS_ERR_HANDLE, "grouped MoE shape or handle: invalid handle %llu",
                        (unsigned long long)handle);
    if (int rc = check_device(*w)) return rc;
    if (w->compute != APS_DTYPE_E4M3) return fail(APS_ERR_DTYPE, "%s: weight set is not fp8", what);
    *out = w;
    return APS_OK;
}

int aps_moe_ffn_up_fp8(uint64_t handle, const uint8_t* xq, const float* x_scale, int64_t rows,
                       const uint32_t* offsets, const uint32_t* assignment_rows, void* act, void* stream) {
    const WeightSet* w = nullptr;
    if (int rc = fp8_set(handle, &w, "ffn_up_fp8")) return rc;
    if (rows < 0) return fail(APS_ERR_SHAPE, "ffn_up_fp8: rows %lld", (long long)rows);
    if (rows > 0 && (!xq || !x_scale || !offsets || !assignment_rows || !act))
        return fail(APS_ERR_ARG, "ffn_up_fp8: NULL pointer");
    APS_HIP(aps::launch_ffn_up_fp8(xq, x_scale, offsets, assignment_rows, w->q13, w->s1, w->s3,
                                   static_cast<aps::bf16_t*>(act), rows, w->H, w->F, w->E,
                                   static_cast<hipStream_t>(stream)),
            "ffn_up_fp8 launch");
    return APS_OK;
}

int aps_moe_ffn_down_fp8(uint64_t handle, const uint8_t* actq, const float* act_scale, int64_t rows,
                         const uint32_t* offsets, void* y_perm, void* stream) {
    const WeightSet* w = nullptr;
    if (int rc = fp8_set(handle, &w, "ffn_down_fp8")) return rc;
    if (rows < 0) return fail(APS_ERR_SHAPE, "ffn_down_fp8: rows %lld", (long long)rows);
    if (rows > 0 && (!actq || !act_scale || !offsets || !y_perm)) return fail(APS_ERR_ARG, "ffn_down_fp8: NULL pointer");
    APS_HIP(aps::launch_ffn_down_fp8(actq, act_scale, offsets, w->q2, w->s2, static_cast<aps::bf16_t*>(y_perm),
                                     rows, w->H, w->F, w->E, static_cast<hipStream_t>(stream)),
            "ffn_down_fp8 launch");
    return APS_OK;
}

int aps_moe_combine(const void* y_perm, int32_t y_dtype, const uint32_t* route_positions,
                    int64_t rows, int32_t hidden, void* out, int32_t out_dtype, void* stream) {
    if (rows < 0 || hidden <= 0 || hidden % 8 != 0)
        return fail(APS_ERR_SHAPE, "combine: rows %lld hidden %d", (long long)rows, hidden);
    if ((y_dtype != APS_DTYPE_F32 && y_dtype != APS_DTYPE_BF16) ||
        (out_dtype != APS_DTYPE_F32 && out_dtype != APS_DTYPE_BF16))
        return fail(APS_ERR_DTYPE, "combine: y dtype %d / out dtype %d", y_dtype, out_dtype);
    if (rows > 0 && (!y_perm || !route_positions || !out)) return fail(APS_ERR_ARG, "combine: NULL pointer");
    APS_HIP(aps::launch_combine(y_perm, y_dtype == APS_DTYPE_BF16, route_positions, rows, hidden, out,
                                out_dtype == APS_DTYPE_BF16, static_cast<hipStream_t>(stream)),
            "combine launch");
    return APS_OK;
}

static int layer_norm_common(float* x, const float* residual, const float* weight, const float* bias,
                             int64_t rows, int32_t hidden, float eps, float* y, void* stream, const char* what) {
    if (rows < 0 || hidden <= 0 || hidden % 256 != 0)
        return fail(APS_ERR_SHAPE, "%s shape: rows %lld hidden %d (hidden must be a multiple of 256)", what,
                    (long long)rows, hidden);
    if (rows > 0 && (!x || !weight || !bias || !y)) return fail(APS_ERR_ARG, "%s: NULL pointer", what);
    if (residual == nullptr && std::strcmp(what, "add layer norm") == 0)
        return fail(APS_ERR_ARG, "%s: NULL residual", what);
    const bool aligned = ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(residual) |
                           reinterpret_cast<uintptr_t>(weight) | reinterpret_cast<uintptr_t>(bias) |
                           reinterpret_cast<uintptr_t>(y)) & 15u) == 0;
    if (!aligned) return fail(APS_ERR_ARG, "%s: arrays must be 16-byte aligned", what);
    if (rows > 0 && (y == x || (residual && y == residual)))
        return fail(APS_ERR_ARG, "%s: y must not alias x or the residual", what);
    APS_HIP(aps::launch_layer_norm(x, residual, weight, bias, y, rows, hidden, eps, static_cast<hipStream_t>(stream)),
            "layer norm launch");
    return APS_OK;
}

int aps_layer_norm(const float* x, const float* weight, const float* bias, int64_t rows, int32_t hidden, float eps,
                   float* y, void* stream) {
    return layer_norm_common(const_cast<float*>(x), nullptr, weight, bias, rows, hidden, eps, y, stream,
                             "layer norm");
}

int aps_add_layer_norm(float* x, const float* residual, const float* weight, const float* bias, int64_t rows,
                       int32_t hidden, float eps, float* y, void* stream) {
    return layer_norm_common(x, residual, weight, bias, rows, hidden, eps, y, stream, "add layer norm");
}

int aps_gather_rows(const float* x, int64_t x_rows, int64_t hidden, const uint32_t* rows, int64_t count, float* out,
                    void* stream) {
    if (x_rows < 0 || hidden < 0 || count < 0)
        return fail(APS_ERR_SHAPE, "gather rows shape: x_rows %lld hidden %lld count %lld", (long long)x_rows,
                    (long long)hidden, (long long)count);
    if (count == 0 || hidden == 0) return APS_OK;
    if (!rows || !out || (x_rows > 0 && !x)) return fail(APS_ERR_ARG, "gather rows: NULL pointer");
    if (count * ((hidden + 1023) / 1024) > 0x7FFFFFFF)
        return fail(APS_ERR_SHAPE, "gather rows shape: %lld rows of %lld values is past the grid limit",
                    (long long)count, (long long)hidden);
    APS_HIP(aps::launch_gather_rows(x, x_rows, hidden, rows, count, out, static_cast<hipStream_t>(stream)),
            "gather rows launch");
    return APS_OK;
}

int aps_prefix_dedup(const int32_t* ids, const int64_t* seq_offsets, int64_t batch, int64_t vocab_size,
                     int64_t max_positions, uint32_t* token_node, uint32_t* node_token, uint32_t* node_depth,
                     uint32_t* node_anc, int64_t anc_stride, int64_t* nodes) {
    // reference src/model.cu:47-49: an empty batch is a std::runtime_error
    if (batch <= 0) return fail(APS_ERR_SHAPE, "generate received an empty input batch");
    if (!seq_offsets || !nodes) return fail(APS_ERR_ARG, "prefix dedup: NULL pointer");
    if (seq_offsets[batch] > 0 && (!ids || !token_node || !node_token || !node_depth))
        return fail(APS_ERR_ARG, "prefix dedup: NULL pointer");
    std::string err;
    const int rc = aps::prefix_dedup(ids, seq_offsets, batch, vocab_size, max_positions, token_node, node_token,
                                     node_depth, node_anc, anc_stride, nodes, err);
    if (rc == 1) return fail(APS_ERR_ARG, "%s", err.c_str());
    if (rc != 0) return fail(APS_ERR_SHAPE, "prefix dedup: %s", err.c_str());
    return APS_OK;
}

int aps_prefix_ancestors(const uint32_t* node_parent, const uint32_t* node_depth, const uint32_t* run_start,
                         int64_t nodes, int64_t anc_stride, uint32_t* node_anc, void* stream) {
    if (nodes < 0 || anc_stride <= 0 || nodes > 0xFFFFFFFFll || anc_stride > (1ll << 24) ||
        nodes > (1ll << 38) / anc_stride)
        return fail(APS_ERR_SHAPE, "prefix ancestors: nodes %lld stride %lld", (long long)nodes, (long long)anc_stride);
    if (nodes == 0) return APS_OK;
    if (!node_parent || !node_depth || !run_start || !node_anc) return fail(APS_ERR_ARG, "prefix ancestors: NULL pointer");
    APS_HIP(aps::launch_prefix_ancestors(node_parent, node_depth, run_start, nodes, anc_stride, node_anc,
                                         static_cast<hipStream_t>(stream)),
            "prefix ancestors launch");
    return APS_OK;
}

int aps_linear(const float* x, const float* weight, const float* bias, int64_t rows, int32_t in_features,
               int32_t out_features, float* y, void* stream) {
    if (rows < 0 || in_features <= 0 || out_features <= 0)
        return fail(APS_ERR_SHAPE, "linear shape: rows %lld in %d out %d", (long long)rows, in_features,
                    out_features);
    if (rows == 0) return APS_OK;
    if (!x || !weight || !y) return fail(APS_ERR_ARG, "linear: NULL pointer");
    const uintptr_t addr_bits = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(weight) |
                                reinterpret_cast<uintptr_t>(bias) | reinterpret_cast<uintptr_t>(y);
    if ((addr_bits & 3u) != 0) return fail(APS_ERR_ARG, "linear: arrays must be 4-byte aligned");
    if (y == x) return fail(APS_ERR_ARG, "linear: y must not alias x");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    // in % 16, out % 4 and 16-byte alignment take the vector / matrix-core
    // kernels; any other shape the SIMT kernel (same chains, same bits)
    if (in_features % 16 == 0 && out_features % 4 == 0 && (addr_bits & 15u) == 0 && (rows + 63) / 64 <= 65535)
        APS_HIP(aps::launch_linear_f32(x, weight, bias, y, rows, in_features, out_features, s), "linear launch");
    else
        APS_HIP(aps::launch_linear_any_f32(x, weight, bias, y, rows, in_features, out_features, s),
                "linear launch");
    return APS_OK;
}

int aps_linear_multi(const float* x, int64_t rows, int32_t in_features, int32_t count, const float* const* weights,
                     const float* const* biases, const int32_t* out_features, float* const* ys, void* stream) {
    if (count < 1 || count > 3 || !out_features) return fail(APS_ERR_SHAPE, "linear multi: count %d (1..3)", count);
    if (rows < 0 || in_features <= 0 || in_features % 16 != 0 || (rows + 63) / 64 > 65535)
        return fail(APS_ERR_SHAPE, "linear multi shape: rows %lld in %d (multiple of 16)", (long long)rows,
                    in_features);
    for (int32_t j = 0; j < count; ++j)
        if (out_features[j] <= 0 || out_features[j] % 4 != 0)
            return fail(APS_ERR_SHAPE, "linear multi: out %d of output %d (multiple of 4)", out_features[j], j);
    if (rows == 0) return APS_OK;
    if (!x || !weights || !ys) return fail(APS_ERR_ARG, "linear multi: NULL pointer");
    const float* ws[3] = {};
    const float* bs[3] = {};
    bool fits = aps::linear_mfma_fits(rows, in_features, out_features[0]);
    for (int32_t j = 0; j < count; ++j) {
        ws[j] = weights[j];
        bs[j] = biases ? biases[j] : nullptr;
        if (!ws[j] || !ys[j]) return fail(APS_ERR_ARG, "linear multi: NULL pointer (output %d)", j);
        if (((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(ws[j]) | reinterpret_cast<uintptr_t>(bs[j]) |
              reinterpret_cast<uintptr_t>(ys[j])) & 15u) != 0)
            return fail(APS_ERR_ARG, "linear multi: arrays must be 16-byte aligned");
        if (ys[j] == x) return fail(APS_ERR_ARG, "linear multi: output %d aliases x", j);
        for (int32_t i = 0; i < j; ++i)
            if (ys[i] == ys[j]) return fail(APS_ERR_ARG, "linear multi: outputs %d and %d are the same array", i, j);
        fits = fits && aps::linear_mfma_fits(rows, in_features, out_features[j]);
    }
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (fits) {
        APS_HIP(aps::launch_linear_mfma_multi(x, rows, in_features, count, ws, bs, ys, out_features, s),
                "linear multi launch");
    } else {
        for (int32_t j = 0; j < count; ++j)
            APS_HIP(aps::launch_linear_f32(x, ws[j], bs[j], ys[j], rows, in_features, out_features[j], s),
                    "linear multi launch");
    }
    return APS_OK;
}

size_t aps_linear_tc_packed_bytes(int32_t out_features, int32_t in_features) {
    if (out_features <= 0 || in_features <= 0 || in_features % 64 != 0) return 0;
    return static_cast<size_t>(aps::linear_tc_packed_elems(out_features, in_features)) * sizeof(uint16_t);
}

int aps_linear_tc_prepare(const float* weight, int32_t out_features, int32_t in_features, void* packed,
                          size_t packed_bytes, void* stream) {
    if (out_features <= 0 || in_features <= 0 || in_features % 64 != 0 || out_features % 4 != 0)
        return fail(APS_ERR_SHAPE, "split-bf16 weight shape: out %d (multiple of 4) in %d (multiple of 64)",
                    out_features, in_features);
    if (!weight || !packed) return fail(APS_ERR_ARG, "split-bf16 prepare: NULL pointer");
    const size_t need = aps_linear_tc_packed_bytes(out_features, in_features);
    if (packed_bytes < need)
        return fail(APS_ERR_ARG, "split-bf16 prepare: packed buffer %zu bytes, needs %zu", packed_bytes, need);
    if (((reinterpret_cast<uintptr_t>(weight) | reinterpret_cast<uintptr_t>(packed)) & 15u) != 0)
        return fail(APS_ERR_ARG, "split-bf16 prepare: arrays must be 16-byte aligned");
    APS_HIP(aps::launch_linear_tc_prepare(weight, out_features, in_features, static_cast<uint16_t*>(packed),
                                          static_cast<hipStream_t>(stream)),
            "split-bf16 prepare launch");
    return APS_OK;
}

int aps_linear_tc_split(const float* x, int64_t rows, int32_t in_features, void* x_split, void* stream) {
    if (rows < 0 || in_features <= 0 || in_features % 64 != 0)
        return fail(APS_ERR_SHAPE, "split-bf16 input shape: rows %lld in %d (multiple of 64)", (long long)rows,
                    in_features);
    if (rows == 0) return APS_OK;
    if (!x || !x_split) return fail(APS_ERR_ARG, "split-bf16 split: NULL pointer");
    if (((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(x_split)) & 15u) != 0)
        return fail(APS_ERR_ARG, "split-bf16 split: arrays must be 16-byte aligned");
    const int64_t n = rows * in_features;
    uint16_t* hi = static_cast<uint16_t*>(x_split);
    APS_HIP(aps::launch_split_bf16(x, n, hi, hi + n, static_cast<hipStream_t>(stream)), "split-bf16 split launch");
    return APS_OK;
}

int aps_linear_tc(const void* x_split, int64_t rows, int32_t in_features, const void* packed, const float* bias,
                  int32_t out_features, int32_t all_terms, float* y, void* stream) {
    if (rows < 0 || in_features <= 0 || in_features % 64 != 0 || out_features <= 0 || out_features % 4 != 0 ||
        (rows + 127) / 128 > 65535)
        return fail(APS_ERR_SHAPE, "split-bf16 linear shape: rows %lld in %d (multiple of 64) out %d (multiple of 4)",
                    (long long)rows, in_features, out_features);
    if (rows == 0) return APS_OK;
    if (!x_split || !packed || !y) return fail(APS_ERR_ARG, "split-bf16 linear: NULL pointer");
    if (((reinterpret_cast<uintptr_t>(x_split) | reinterpret_cast<uintptr_t>(packed) |
          reinterpret_cast<uintptr_t>(bias) | reinterpret_cast<uintptr_t>(y)) & 15u) != 0)
        return fail(APS_ERR_ARG, "split-bf16 linear: arrays must be 16-byte aligned");
    const int64_t n = rows * in_features;
    const uint16_t* hi = static_cast<const uint16_t*>(x_split);
    APS_HIP(aps::launch_linear_tc(hi, hi + n, static_cast<const uint16_t*>(packed), bias, y, rows, in_features,
                                  out_features, all_terms != 0, static_cast<hipStream_t>(stream)),
            "split-bf16 linear launch");
    return APS_OK;
}

int aps_linear_tc_multi(const void* x_split, int64_t rows, int32_t in_features, int32_t count,
                        const void* const* packed, const float* const* biases, const int32_t* out_features,
                        int32_t all_terms, float* const* ys, void* stream) {
    if (count < 1 || count > 3 || !out_features)
        return fail(APS_ERR_SHAPE, "split-bf16 linear multi: count %d (1..3)", count);
    if (rows < 0 || in_features <= 0 || in_features % 64 != 0 || (rows + 127) / 128 > 65535)
        return fail(APS_ERR_SHAPE, "split-bf16 linear multi shape: rows %lld in %d (multiple of 64)",
                    (long long)rows, in_features);
    for (int32_t j = 0; j < count; ++j)
        if (out_features[j] <= 0 || out_features[j] % 4 != 0)
            return fail(APS_ERR_SHAPE, "split-bf16 linear multi: out %d of output %d (multiple of 4)",
                        out_features[j], j);
    if (rows == 0) return APS_OK;
    if (!x_split || !packed || !ys) return fail(APS_ERR_ARG, "split-bf16 linear multi: NULL pointer");
    const uint16_t* pk[3] = {};
    const float* bs[3] = {};
    for (int32_t j = 0; j < count; ++j) {
        pk[j] = static_cast<const uint16_t*>(packed[j]);
        bs[j] = biases ? biases[j] : nullptr;
        if (!pk[j] || !ys[j]) return fail(APS_ERR_ARG, "split-bf16 linear multi: NULL pointer (output %d)", j);
        if (((reinterpret_cast<uintptr_t>(pk[j]) | reinterpret_cast<uintptr_t>(bs[j]) |
              reinterpret_cast<uintptr_t>(ys[j]) | reinterpret_cast<uintptr_t>(x_split)) & 15u) != 0)
            return fail(APS_ERR_ARG, "split-bf16 linear multi: arrays must be 16-byte aligned");
        for (int32_t i = 0; i < j; ++i)
            if (ys[i] == ys[j])
                return fail(APS_ERR_ARG, "split-bf16 linear multi: outputs %d and %d are the same array", i, j);
    }
    const int64_t n = rows * in_features;
    const uint16_t* hi = static_cast<const uint16_t*>(x_split);
    APS_HIP(aps::launch_linear_tc_multi(hi, hi + n, count, pk, bs, ys, out_features, rows, in_features,
                                        all_terms != 0, static_cast<hipStream_t>(stream)),
            "split-bf16 linear multi launch");
    return APS_OK;
}

int aps_rope_table(int64_t max_seq, int32_t head_dim, float theta, float* cos_out, float* sin_out) {
    if (max_seq < 0 || head_dim <= 0 || head_dim % 2 != 0)
        return fail(APS_ERR_SHAPE, "rope table shape: max_seq %lld head_dim %d", (long long)max_seq, head_dim);
    if (max_seq > 0 && (!cos_out || !sin_out)) return fail(APS_ERR_ARG, "rope table: NULL pointer");
    // reference src/tensor.cu:2716-2725: float arithmetic through powf / cosf / sinf
    const int32_t half = head_dim / 2;
    for (int64_t p = 0; p < max_seq; ++p)
        for (int32_t j = 0; j < half; ++j) {
            const float ex = (-2.0f * static_cast<float>(j)) / static_cast<float>(head_dim);
            const float inv = powf(theta, ex);
            const float ang = static_cast<float>(p) * inv;
            cos_out[p * half + j] = cosf(ang);
            sin_out[p * half + j] = sinf(ang);
        }
    return APS_OK;
}

int aps_rope_tree(float* q, float* k, const uint32_t* row_pos, int64_t rows, int32_t q_heads, int32_t kv_heads,
                  int32_t head_dim, const float* cos_table, const float* sin_table, int64_t max_seq, void* stream) {
    if (rows < 0 || q_heads <= 0 || kv_heads <= 0 || head_dim <= 0 || head_dim % 2 != 0 || max_seq < 0)
        return fail(APS_ERR_SHAPE, "rope shape: rows %lld heads %d/%d head_dim %d", (long long)rows, q_heads,
                    kv_heads, head_dim);
    if (rows == 0) return APS_OK;
    if (!q || !k || !row_pos || !cos_table || !sin_table) return fail(APS_ERR_ARG, "rope: NULL pointer");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    APS_HIP(aps::launch_rope_tree(q, row_pos, rows, q_heads, head_dim, cos_table, sin_table, max_seq, s),
            "rope launch");
    APS_HIP(aps::launch_rope_tree(k, row_pos, rows, kv_heads, head_dim, cos_table, sin_table, max_seq, s),
            "rope launch");
    return APS_OK;
}

int aps_attention_tree(const float* q, const float* k, const float* v, float* out, const uint32_t* row_pos,
                       const uint32_t* anc, int64_t anc_stride, int64_t rows, int32_t q_heads, int32_t kv_heads,
                       int32_t head_dim, int32_t window, void* stream) {
    // reference src/tensor.cu:3367-3368: "attention_tree_gpu expects GQA-4"
    if (kv_heads <= 0 || q_heads != 4 * kv_heads)
        return fail(APS_ERR_SHAPE, "attention_tree_gpu expects GQA-4");
    if (rows < 0 || head_dim != 128 || anc_stride <= 0 || window <= 0)
        return fail(APS_ERR_SHAPE, "attention tree shape: rows %lld head_dim %d (128 only) anc_stride %lld window %d",
                    (long long)rows, head_dim, (long long)anc_stride, window);
    if ((anc_stride < window ? anc_stride : window) > aps::kAttnMaxWindow)
        return fail(APS_ERR_SHAPE, "attention tree: a window of %lld keys exceeds the %d that fit in LDS",
                    (long long)(anc_stride < window ? anc_stride : window), aps::kAttnMaxWindow);
    if (rows == 0) return APS_OK;
    if (!q || !k || !v || !out || !row_pos || !anc) return fail(APS_ERR_ARG, "attention tree: NULL pointer");
    if ((reinterpret_cast<uintptr_t>(k) & 15u) != 0) return fail(APS_ERR_ARG, "attention tree: k must be 16-byte aligned");
    APS_HIP(aps::launch_attention_tree(q, k, v, out, row_pos, anc, anc_stride, rows, q_heads, kv_heads, head_dim,
                                       window, false, static_cast<hipStream_t>(stream)),
            "attention tree launch");
    return APS_OK;
}

int aps_attention_packed(const float* q, const float* k, const float* v, float* out, const uint32_t* seg_offset,
                         const uint32_t* seg_pos, int64_t max_seq, int64_t rows, int32_t q_heads, int32_t kv_heads,
                         int32_t head_dim, int32_t window, void* stream) {
    if (kv_heads <= 0 || q_heads <= 0 || q_heads % kv_heads != 0)
        return fail(APS_ERR_SHAPE, "attention heads: %d query heads over %d KV heads", q_heads, kv_heads);
    if (q_heads != 4 * kv_heads) {
        // other head layouts: the reference's generic kernel (k_attention)
        if (rows < 0 || head_dim <= 0 || head_dim > 128 || max_seq <= 0 || window <= 0)
            return fail(APS_ERR_SHAPE, "attention shape: rows %lld head_dim %d (1..128) max_seq %lld window %d",
                        (long long)rows, head_dim, (long long)max_seq, window);
        if ((max_seq < window ? max_seq : window) > aps::kAttnMaxWindow)
            return fail(APS_ERR_SHAPE, "attention: a window of %lld keys exceeds the %d that fit in LDS",
                        (long long)(max_seq < window ? max_seq : window), aps::kAttnMaxWindow);
        if (rows * q_heads > 0x7FFFFFFFll)
            return fail(APS_ERR_SHAPE, "attention: %lld rows x %d heads", (long long)rows, q_heads);
        if (rows == 0) return APS_OK;
        if (!q || !k || !v || !out || !seg_offset || !seg_pos) return fail(APS_ERR_ARG, "attention: NULL pointer");
        APS_HIP(aps::launch_attention_any(q, k, v, out, seg_offset, seg_pos, max_seq, rows, q_heads, kv_heads,
                                          head_dim, window, static_cast<hipStream_t>(stream)),
                "attention launch");
        return APS_OK;
    }
    if (rows < 0 || head_dim != 128 || max_seq <= 0 || window <= 0)
        return fail(APS_ERR_SHAPE, "attention shape: rows %lld head_dim %d (128 only) max_seq %lld window %d",
                    (long long)rows, head_dim, (long long)max_seq, window);
    if ((max_seq < window ? max_seq : window) > aps::kAttnMaxWindow)
        return fail(APS_ERR_SHAPE, "attention: a window of %lld keys exceeds the %d that fit in LDS",
                    (long long)(max_seq < window ? max_seq : window), aps::kAttnMaxWindow);
    if (rows == 0) return APS_OK;
    if (!q || !k || !v || !out || !seg_offset || !seg_pos) return fail(APS_ERR_ARG, "attention: NULL pointer");
    if ((reinterpret_cast<uintptr_t>(k) & 15u) != 0) return fail(APS_ERR_ARG, "attention: k must be 16-byte aligned");
    APS_HIP(aps::launch_attention_tree(q, k, v, out, seg_pos, seg_offset, max_seq, rows, q_heads, kv_heads, head_dim,
                                       window, true, static_cast<hipStream_t>(stream)),
            "attention launch");
    return APS_OK;
}

int aps_add_inplace(float* a, const float* b, int64_t n, void* stream) {
    if (n < 0) return fail(APS_ERR_SHAPE, "add shape: %lld elements", (long long)n);
    if (n > 0 && (!a || !b)) return fail(APS_ERR_ARG, "add: NULL pointer");
    APS_HIP(aps::launch_add_inplace(a, b, n, static_cast<hipStream_t>(stream)), "add launch");
    return APS_OK;
}

int aps_add_bias_inplace(float* a, const float* bias, int64_t n, int32_t h, void* stream) {
    if (n < 0 || h <= 0 || n % h != 0)
        return fail(APS_ERR_SHAPE, "bias shape: %lld elements, bias of %d", (long long)n, h);
    if (n > 0 && (!a || !bias)) return fail(APS_ERR_ARG, "add bias: NULL pointer");
    APS_HIP(aps::launch_add_bias(a, bias, n, h, static_cast<hipStream_t>(stream)), "add bias launch");
    return APS_OK;
}

int aps_silu_mul(const float* gate, const float* up, float* out, int64_t n, void* stream) {
    if (n < 0) return fail(APS_ERR_SHAPE, "silu_mul shape: %lld elements", (long long)n);
    if (n > 0 && (!gate || !up || !out)) return fail(APS_ERR_ARG, "silu_mul: NULL pointer");
    APS_HIP(aps::launch_silu_mul(gate, up, out, n, static_cast<hipStream_t>(stream)), "silu_mul launch");
    return APS_OK;
}

int aps_zero(float* x, int64_t n, void* stream) {
    if (n < 0) return fail(APS_ERR_SHAPE, "zero shape: %lld elements", (long long)n);
    if (n > 0 && !x) return fail(APS_ERR_ARG, "zero: NULL pointer");
    APS_HIP(aps::launch_zero(x, n, static_cast<hipStream_t>(stream)), "zero launch");
    return APS_OK;
}

static int forward_common(uint64_t handle, const void* x, int32_t x_dtype, int64_t rows, void* out,
                          int32_t out_dtype, void* workspace, size_t workspace_bytes,
                          const WeightSet** w_out, aps_moe_ws_layout* L) {
    const WeightSet* w = lookup(handle);
    // reference: "grouped MoE shape or handle" (src/tensor.cu:2793-2797)
    if (!w) return fail(APS_ERR_HANDLE, "grouped MoE shape or handle: invalid handle %llu",
                        (unsigned long long)handle);
    if (int rc = check_device(*w)) return rc;
    if (rows < 0 || rows > (int64_t(1) << 30))
        return fail(APS_ERR_SHAPE, "grouped MoE shape or handle: rows %lld", (long long)rows);
    if (w->E < 2) return fail(APS_ERR_SHAPE, "grouped MoE shape or handle: top-2 routing needs 2+ experts");
    // fp32 x is accepted with bf16 weights: the router reads it exactly and
    // the FFN gets a bf16 copy in the workspace.
    const bool f32_into_bf16 = w->compute == APS_DTYPE_BF16 && x_dtype == APS_DTYPE_F32;
    if (!f32_into_bf16)
        if (int rc = check_x_dtype(*w, x_dtype)) return rc;
    if (f32_into_bf16 && rows > 0 && (reinterpret_cast<uintptr_t>(x) & 15u))
        return fail(APS_ERR_ARG, "forward: fp32 x must be 16-byte aligned");
    if (out_dtype != APS_DTYPE_F32 && out_dtype != APS_DTYPE_BF16)
        return fail(APS_ERR_DTYPE, "out dtype %d not supported", out_dtype);
    make_layout(*w, rows, L);
    if (rows > 0) {
        if (!x || !out) return fail(APS_ERR_ARG, "forward: NULL x or out");
        if (!workspace || workspace_bytes < L->total_bytes)
            return fail(APS_ERR_WORKSPACE, "workspace %zu bytes, need %zu", workspace_bytes, L->total_bytes);
    }
    *w_out = w;
    return APS_OK;
}

int aps_moe_forward_grouped(uint64_t handle, const void* x, int32_t x_dtype,
                            const float* router_logits, int64_t rows, void* out, int32_t out_dtype,
                            void* workspace, size_t workspace_bytes, void* stream) {
    const WeightSet* w = nullptr;
    aps_moe_ws_layout L;
    if (int rc = forward_common(handle, x, x_dtype, rows, out, out_dtype, workspace, workspace_bytes, &w, &L))
        return rc;
    if (rows == 0) return APS_OK;
    if (!router_logits) return fail(APS_ERR_ARG, "forward_grouped: NULL router logits");
    return grouped_from_logits(*w, x, x_dtype == APS_DTYPE_F32, router_logits, rows, out, out_dtype,
                               static_cast<char*>(workspace), L, static_cast<hipStream_t>(stream));
}

int aps_moe_forward(uint64_t handle, const void* x, int32_t x_dtype, const float* gate, int64_t rows,
                    void* out, int32_t out_dtype, void* workspace, size_t workspace_bytes, void* stream) {
    const WeightSet* w = nullptr;
    aps_moe_ws_layout L;
    if (int rc = forward_common(handle, x, x_dtype, rows, out, out_dtype, workspace, workspace_bytes, &w, &L))
        return rc;
    if (rows == 0) return APS_OK;
    if (!gate) return fail(APS_ERR_ARG, "forward: NULL gate");
    char* ws = static_cast<char*>(workspace);
    hipStream_t s = static_cast<hipStream_t>(stream);
    // logits, routes and the tile histogram in one kernel (and, for fp32 x
    // with a bf16 weight set, the FFN's bf16 copy of x); the grouped path
    // then starts at the dispatch
    float* logits = reinterpret_cast<float*>(ws + L.logits);
    auto* routes = reinterpret_cast<uint8_t*>(ws + L.routes);
    auto* tiles = reinterpret_cast<uint32_t*>(ws + L.tile_counts);
    const bool copy = x_dtype == APS_DTYPE_F32 && w->compute == APS_DTYPE_BF16;
    auto* xb = copy ? reinterpret_cast<aps::bf16_t*>(ws + L.xq) : nullptr;
    const bool fold = fold_combine(*w, rows, out_dtype);
    auto* tiles0 = fold ? reinterpret_cast<uint32_t*>(ws + L.tile_counts0) : nullptr;
    // fp8 weights with bf16 x: the router also writes x's e4m3 codes and row
    // scales (x read once for both)
    const bool xq_in_router = w->compute == APS_DTYPE_E4M3 && x_dtype == APS_DTYPE_BF16 &&
                              aps::router_quantises_x(w->H, w->E);
    auto* xq = xq_in_router ? reinterpret_cast<uint8_t*>(ws + L.xq) : nullptr;
    auto* xqs = xq_in_router ? reinterpret_cast<float*>(ws + L.xq_scale) : nullptr;
    APS_HIP(aps::launch_router(x, x_dtype == APS_DTYPE_BF16, gate, rows, w->H, w->E, logits, routes, tiles, tiles0,
                               xb, xq, xqs, s),
            "router launch");
    if (copy) return grouped_from_logits(*w, xb, false, nullptr, rows, out, out_dtype, ws, L, s, fold);
    return grouped_from_logits(*w, x, x_dtype == APS_DTYPE_F32, nullptr, rows, out, out_dtype, ws, L, s, fold,
                               xq_in_router);
}

// ---- allocation-free forward --------------------------------------------
//
// aps_moe_forward with its workspace in a static device array instead of a
// caller buffer, for callers that cannot allocate (code under HIP graph
// capture, serving loops).  Each device holds its own copy of `scratch` for
// the life of the process; its address is looked up once per device (with
// that device current) and kept, since the host-side name is not a device
// address.  The forward path writes every workspace byte it reads, so the
// previous call's contents never matter; calls that overlap on one device
// share the array and race.
namespace {

constexpr size_t kStaticScratchBytes = size_t(96) << 20;  // 96 MiB per device
static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices] = {};

int static_scratch(void** out) {
    int dev = 0;
    APS_HIP(hipGetDevice(&dev), "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) return fail(APS_ERR_ARG, "forward_noalloc: device %d out of range", dev);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_dev[dev]) {
        void* p = nullptr;
        APS_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress scratch");
        if (!p) return fail(APS_ERR_HIP, "hipGetSymbolAddress scratch: null address");
        g_scratch_dev[dev] = p;
    }
    *out = g_scratch_dev[dev];
    return APS_OK;
}

}  // namespace

size_t aps_moe_noalloc_scratch_bytes(void) { return kStaticScratchBytes; }

int aps_moe_forward_noalloc(uint64_t handle, const void* x, int32_t x_dtype, const float* gate, int64_t rows,
                            void* out, int32_t out_dtype, void* stream) {
    aps_moe_ws_layout L;
    if (int rc = aps_moe_workspace_layout(handle, rows, &L)) return rc;
    if (L.total_bytes > kStaticScratchBytes)
        return fail(APS_ERR_WORKSPACE,
                    "forward_noalloc: %lld rows need %zu bytes of scratch, the static scratch holds %zu "
                    "(use aps_moe_forward with a workspace)",
                    (long long)rows, L.total_bytes, kStaticScratchBytes);
    void* ws = nullptr;
    if (int rc = static_scratch(&ws)) return rc;
    return aps_moe_forward(handle, x, x_dtype, gate, rows, out, out_dtype, ws, kStaticScratchBytes, stream);
}

// Dense FFN of a single-expert weight set: offsets {0, rows} and the
// identity assignment in the workspace, then the two grouped GEMMs with
// y_perm = out (position p is row p).
static size_t mlp_layout(const WeightSet& w, int64_t rows, size_t* arows, size_t* act) {
    size_t off = align_up(2 * sizeof(uint32_t));
    *arows = off;
    off = align_up(off + static_cast<size_t>(rows) * 4);
    *act = off;
    const size_t elt = w.compute == APS_DTYPE_F32 ? 4 : 2;
    return align_up(off + static_cast<size_t>(rows) * w.F * elt);
}

size_t aps_mlp_workspace_size(uint64_t handle, int64_t rows) {
    const WeightSet* w = lookup(handle);
    if (!w || rows < 0) return 0;
    size_t a, b;
    return mlp_layout(*w, rows, &a, &b);
}

int aps_mlp_forward(uint64_t handle, const void* x, int32_t x_dtype, int64_t rows, void* out,
                    void* workspace, size_t workspace_bytes, void* stream) {
    const WeightSet* w = lookup(handle);
    if (!w) return fail(APS_ERR_HANDLE, "mlp: invalid handle %llu", (unsigned long long)handle);
    if (int rc = check_device(*w)) return rc;
    if (w->E != 1) return fail(APS_ERR_SHAPE, "mlp: weight set has %d experts, a dense FFN has 1", w->E);
    if (int rc = check_not_fp8(*w, "mlp")) return rc;
    if (rows < 0 || rows > (int64_t(1) << 30)) return fail(APS_ERR_SHAPE, "mlp: rows %lld", (long long)rows);
    if (int rc = check_x_dtype(*w, x_dtype)) return rc;
    if (rows == 0) return APS_OK;
    size_t arows_off, act_off;
    const size_t need = mlp_layout(*w, rows, &arows_off, &act_off);
    if (!x || !out) return fail(APS_ERR_ARG, "mlp: NULL x or out");
    if (!workspace || workspace_bytes < need)
        return fail(APS_ERR_WORKSPACE, "mlp: workspace %zu bytes, need %zu", workspace_bytes, need);
    char* ws = static_cast<char*>(workspace);
    hipStream_t s = static_cast<hipStream_t>(stream);
    auto* offsets = reinterpret_cast<uint32_t*>(ws);
    auto* arows = reinterpret_cast<uint32_t*>(ws + arows_off);
    APS_HIP(aps::launch_dense_plan(offsets, arows, rows, s), "dense plan launch");
    return run_ffn(*w, x, rows, offsets, arows, ws + act_off, out, s);
}

}  // extern "C"
