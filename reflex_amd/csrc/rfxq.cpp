// Host side of librfxq: the C ABI declared in include/rfxq.h.
//
// Mirrors the reference's matmul dispatch for quantized-resident weights
// (src/model/kernels.rs: gemv_to :1463, gemv :1826, gemv_q4k :2110,
// gemv_q6k :1972, gemv_q8_0 :1874, gemm :2197, gemm_quant_mma :2262,
// quant_expert_weight :2656, moe_gather/moe_scatter_add :2722-2790;
// src/model/dense.rs: expert_gemv/expert_gemm :1086-1115, moe_ffn_grouped
// :1509-1559; src/moe.rs:47-98 route_top_k_with_norm): the same preconditions
// and error kinds, checked on the host before any launch, and the kernels of
// the embedded gfx950 code object resolved by name (src/aot.rs:113-160).
#include "../../include/rfxq.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>
#include <cerrno>

#include "gguf.hpp"
#include "scratch.hpp"


extern "C" const unsigned char rfxq_code_object[];
extern "C" const unsigned char rfxq_code_object_end[];

namespace {

// ------------------------------------------------------------------ errors

thread_local std::string g_err;
thread_local int g_code = RFXQ_OK;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    g_code = code;
    return code;
}

int ok() {
    g_err.clear();
    g_code = RFXQ_OK;
    return RFXQ_OK;
}

#define HIPCHK(expr, what)                                                                        \
    do {                                                                                          \
        hipError_t e_ = (expr);                                                                   \
        if (e_ != hipSuccess) return fail(RFXQ_ERR_GPU, "%s: %s", (what), hipGetErrorString(e_)); \
    } while (0)

// ------------------------------------------------------------------ descriptors (device layout)

struct GemvDesc {
    const void* w;
    const float* x;
    float* y;
    uint32_t k, n, type, lpr_log2;
    uint32_t pad[4];
};
constexpr uint32_t kGemvInline = 4;
#ifndef RFXQ_GEMV_RING
#define RFXQ_GEMV_RING 2
#endif
// the GEMV kernel's static LDS: per wave RFXQ_GEMV_RING slots of 4 KB
constexpr uint32_t kGemvRingLds = RFXQ_GEMV_RING * 16384u;
struct GemvRange {
    uint32_t d0, it0, d1, it1;
};
struct GemvArgs {
    const GemvDesc* table;
    const GemvRange* ranges;
    uint32_t ndesc, part_floats;
    uint32_t iters_each, pad;
    GemvDesc inl[kGemvInline];
};
static_assert(sizeof(GemvDesc) == 56, "GemvDesc layout");

struct MmqDesc {
    const void* w;
    const int8_t* xq;
    const uint32_t* xds;
    const int32_t* rows;
    float* y;
    uint32_t m, n, k, type;
    uint32_t ldq, ldy, tiles_m, tiles_n;
    uint32_t splits, sb_per_split, wg_begin;
    uint32_t gu_pair;  // gate/up pair with silu(gate) * up stored (Q4_K f16 tiles)
    union {
        int32_t* dots_out;
        const uint8_t* w_up;
    };
    const float* xrs;
};
constexpr uint32_t kMmqInline = 2;
constexpr uint32_t mmqh_pair_bn = 128;  // columns of a gate/up pair tile (mmqh.hpp)
struct MmqArgs {
    const MmqDesc* table;
    uint32_t ndesc, pad;
    MmqDesc inl[kMmqInline];
};
static_assert(sizeof(MmqDesc) == 104, "MmqDesc layout");
// rfxq_splitk_reduce_multi's arguments (mmq.hpp)
struct ReduceItem {
    const float* ws;
    float* y;
    uint32_t n, splits, wg_begin, wgs;
};
constexpr uint32_t REDUCE_INLINE = 32;
struct ReduceArgs {
    uint32_t count, pad;
    ReduceItem items[REDUCE_INLINE];
};
static_assert(sizeof(ReduceItem) == 32 && sizeof(ReduceArgs) == 8 + 32 * 32, "ReduceArgs layout");

constexpr uint32_t kMmqBM = 128, kMmqBN = 128;

constexpr uint32_t kMaxLds = 65536;    // dynamic LDS per GEMV workgroup (plus its 32 KB weight ring)
constexpr uint32_t kMaxGemvK = 16384;  // x staged in LDS: k*2 + k/4 bytes <= 36 KB
constexpr uint32_t kMoeGemvRows = 4;   // moe_ffn_grouped: up to this many tokens run as GEMVs
constexpr uint32_t kRouteMaxE = 1024;     // rfxq_moe_route: experts per token
constexpr uint32_t kDecRouteMaxE = 256;  // moe_decode.hpp: experts of the one-wave router
constexpr uint32_t kPlanMaxPairs = 16384;  // rfxq_moe_plan: routed pairs sorted in LDS
constexpr uint32_t kNormRowsPerWg = 4;  // rows per rfxq_rmsnorm_q8_1 workgroup (the kernel's constant)

// ------------------------------------------------------------------ per-device module

struct Ctx {
    int device = -1;
    int cus = 256;
    hipModule_t mod = nullptr;
    hipFunction_t gemv = nullptr, quant = nullptr, quant_multi = nullptr, reduce = nullptr, reduce_multi = nullptr;
    hipFunction_t mmq[3] = {}, dots[3] = {}, mmq64[3] = {};
    hipFunction_t mmqh[3][3] = {};  // [Q4_K, Q6_K, Q8_0][128-row, 32-row, 64-row tiles]
    hipFunction_t mmqh_mix_m32 = nullptr;  // 32-row tiles, Q4_K or Q6_K per descriptor
    hipFunction_t act_f16 = nullptr, act_f16_multi = nullptr, act_f16_wg = nullptr, act_f16_multi_wg = nullptr;
    hipFunction_t deq[3][2] = {};
    hipFunction_t gather = nullptr, scatter = nullptr, silu = nullptr, combine = nullptr;
    hipFunction_t rms_q = nullptr, silu_q = nullptr, moe_route = nullptr, moe_route_w = nullptr, moe_plan = nullptr;
    // MoE decode kernels: [Q4_K, Q6_K, Q8_0][4, 8, 16, 32 lanes per row]
    hipFunction_t moe_dec_gu[3][4] = {}, moe_dec_dn[3][4] = {};
    void* ws = nullptr;
    uint64_t ws_bytes = 0;
    void* scratch = nullptr;  // this device's fixed scratch array (rfxq_gemm_no_alloc)
    hipError_t scratch_err = hipSuccess;  // why `scratch` is NULL on a loaded device
    // device area for per-call descriptor tables (grow-only, separate from ws)
    void* tab = nullptr;
    uint64_t tab_bytes = 0;
    // pinned host staging for stream-ordered table uploads: a ring of buffers,
    // each reused once the copy that last read it has completed
    struct Stage {
        void* host = nullptr;
        size_t bytes = 0;
        hipEvent_t done = nullptr;
        bool pending = false;
    };
    Stage stage[4];
    uint32_t stage_next = 0;
    std::mutex mu;                // guards ws / tab growth
    std::vector<void*> retired;  // replaced areas: kept until the process ends
};

std::mutex g_mu;
std::map<int, std::unique_ptr<Ctx>> g_ctx;

uint64_t align256(uint64_t v) { return (v + 255u) & ~(uint64_t)255u; }

int type_index(uint32_t ty) { return ty == RFXQ_TYPE_Q4_K ? 0 : ty == RFXQ_TYPE_Q6_K ? 1 : 2; }

int load_ctx(int device, Ctx** out) {
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_ctx.find(device);
    if (it != g_ctx.end()) {
        *out = it->second.get();
        return RFXQ_OK;
    }
    auto c = std::make_unique<Ctx>();
    c->device = device;
    hipDeviceProp_t prop;
    HIPCHK(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(RFXQ_ERR_GPU, "device %d is %s; this build's kernels are gfx950 only", device, prop.gcnArchName);
    c->cus = prop.multiProcessorCount;
    HIPCHK(hipModuleLoadData(&c->mod, rfxq_code_object), "hipModuleLoadData(embedded gfx950 code object)");
    struct {
        hipFunction_t* f;
        const char* name;
    } fns[] = {
        {&c->gemv, "rfxq_gemv"},
        {&c->quant_multi, "rfxq_quantize_q8_1_multi"},
        {&c->quant, "rfxq_quantize_q8_1"},
        {&c->reduce, "rfxq_splitk_reduce"},
        {&c->reduce_multi, "rfxq_splitk_reduce_multi"},
        {&c->mmq[0], "rfxq_mmq_q4k"},
        {&c->mmq[1], "rfxq_mmq_q6k"},
        {&c->mmq[2], "rfxq_mmq_q8_0"},
        {&c->mmq64[0], "rfxq_mmq_q4k_m64"},
        {&c->mmq64[1], "rfxq_mmq_q6k_m64"},
        {&c->mmq64[2], "rfxq_mmq_q8_0_m64"},
        {&c->dots[0], "rfxq_mmq_dots_q4k"},
        {&c->dots[1], "rfxq_mmq_dots_q6k"},
        {&c->dots[2], "rfxq_mmq_dots_q8_0"},
        {&c->mmqh[0][0], "rfxq_mmqh_q4k"},
        {&c->mmqh[1][0], "rfxq_mmqh_q6k"},
        {&c->mmqh[0][1], "rfxq_mmqh_q4k_m32"},
        {&c->mmqh[1][1], "rfxq_mmqh_q6k_m32"},
        {&c->mmqh[0][2], "rfxq_mmqh_q4k_m64"},
        {&c->mmqh[1][2], "rfxq_mmqh_q6k_m64"},
        {&c->mmqh[2][0], "rfxq_mmqh_q8_0"},
        {&c->mmqh[2][1], "rfxq_mmqh_q8_0_m32"},
        {&c->mmqh[2][2], "rfxq_mmqh_q8_0_m64"},
        {&c->mmqh_mix_m32, "rfxq_mmqh_mix_m32"},
        {&c->act_f16, "rfxq_act_f16"},
        {&c->act_f16_multi, "rfxq_act_f16_multi"},
        {&c->act_f16_wg, "rfxq_act_f16_wg"},
        {&c->act_f16_multi_wg, "rfxq_act_f16_multi_wg"},
        {&c->deq[0][0], "rfxq_dequant_q4k_f32"},
        {&c->deq[0][1], "rfxq_dequant_q4k_f16"},
        {&c->deq[1][0], "rfxq_dequant_q6k_f32"},
        {&c->deq[1][1], "rfxq_dequant_q6k_f16"},
        {&c->deq[2][0], "rfxq_dequant_q8_0_f32"},
        {&c->deq[2][1], "rfxq_dequant_q8_0_f16"},
        {&c->gather, "rfxq_moe_gather"},
        {&c->scatter, "rfxq_moe_scatter_add"},
        {&c->silu, "rfxq_silu_and_mul"},
        {&c->rms_q, "rfxq_rmsnorm_q8_1"},
        {&c->silu_q, "rfxq_silu_and_mul_q8_1"},
        {&c->moe_route, "rfxq_moe_route"},
        {&c->moe_route_w, "rfxq_moe_route_w"},
        {&c->moe_plan, "rfxq_moe_plan"},
        {&c->combine, "rfxq_moe_combine"},
    };
    for (auto& f : fns) {
        hipError_t e = hipModuleGetFunction(f.f, c->mod, f.name);
        if (e != hipSuccess)
            return fail(RFXQ_ERR_GPU, "hipModuleGetFunction(%s): %s", f.name, hipGetErrorString(e));
    }
    static const char* const kDecTy[3] = {"q4k", "q6k", "q8_0"};
    for (int t = 0; t < 3; t++)
        for (int l = 0; l < 4; l++)
            for (int g = 0; g < 2; g++) {
                char name[64];
                std::snprintf(name, sizeof name, "rfxq_moe_dec_%s_%s_%d", g ? "down" : "gu", kDecTy[t], 4 << l);
                hipFunction_t* f = g ? &c->moe_dec_dn[t][l] : &c->moe_dec_gu[t][l];
                hipError_t e = hipModuleGetFunction(f, c->mod, name);
                if (e != hipSuccess)
                    return fail(RFXQ_ERR_GPU, "hipModuleGetFunction(%s): %s", name, hipGetErrorString(e));
            }
    // the fixed scratch of rfxq_gemm_no_alloc, resolved now (the device is
    // current); a failure disables only that entry point, which reports it
    c->scratch_err = rfxq_scratch::setup(device, &c->scratch);
    if (c->scratch_err != hipSuccess) c->scratch = nullptr;
    *out = c.get();
    g_ctx[device] = std::move(c);
    return RFXQ_OK;
}

// true if `stream` is capturing a graph
bool capturing(hipStream_t stream) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(stream, &st) == hipSuccess && st != hipStreamCaptureStatusNone;
}

// Grow-only device areas shared by a device's calls (the workspace and the
// per-call tables). A grown area replaces the old one, which stays allocated
// until the process ends: launches still in flight and graphs captured
// earlier may hold its address, so no area is ever freed and growth never
// waits for the device. Growth is refused while `stream` captures a graph (run
// the call once before capturing, or pass a caller workspace). Calls that use
// an area without a caller workspace must be ordered on one stream.
int grow_area(Ctx* c, void** area, uint64_t* size, uint64_t bytes, uint64_t min_bytes, hipStream_t stream,
              const char* what, void** out) {
    std::lock_guard<std::mutex> lk(c->mu);
    if (bytes > *size) {
        if (capturing(stream))
            return fail(RFXQ_ERR_INVALID_INPUT,
                        "%s: needs %llu bytes (has %llu) while the stream captures a graph; run the call once "
                        "before capturing or pass a workspace",
                        what, (unsigned long long)bytes, (unsigned long long)*size);
        const uint64_t sz = std::max<uint64_t>({bytes, 2u * *size, min_bytes});
        void* p = nullptr;
        hipError_t e = hipMalloc(&p, sz);
        if (e != hipSuccess)
            return fail(RFXQ_ERR_OUT_OF_MEMORY, "%s alloc of %llu bytes: %s", what, (unsigned long long)sz,
                        hipGetErrorString(e));
        if (*area) c->retired.push_back(*area);
        *area = p;
        *size = sz;
    }
    *out = *area;
    return RFXQ_OK;
}

int ctx_tables(Ctx* c, uint64_t bytes, void** out, hipStream_t stream) {
    return grow_area(c, &c->tab, &c->tab_bytes, bytes, 64u << 10, stream, "table area", out);
}

// Stream-ordered upload of `bytes` from host memory to `dst` through a pinned
// staging buffer: returns once the data is staged, without waiting for the
// stream (the reference's per-expert pageable copies synchronise).
int stage_upload(Ctx* c, void* dst, const void* src, size_t bytes, hipStream_t stream) {
    if (bytes == 0) return RFXQ_OK;
    // a captured copy would replay from a staging buffer that later calls reuse
    if (capturing(stream))
        return fail(RFXQ_ERR_INVALID_INPUT,
                    "per-call tables cannot be captured into a graph; use a plan (rfxq_gemv_plan_create / "
                    "rfxq_gemm_plan_create) or the device-routed MoE entry point");
    Ctx::Stage& s = c->stage[c->stage_next];
    c->stage_next = (c->stage_next + 1u) % 4u;
    if (s.pending) {
        HIPCHK(hipEventSynchronize(s.done), "staging buffer reuse");
        s.pending = false;
    }
    if (!s.done) HIPCHK(hipEventCreateWithFlags(&s.done, hipEventDisableTiming), "hipEventCreate");
    if (bytes > s.bytes) {
        if (s.host) HIPCHK(hipHostFree(s.host), "hipHostFree");
        s.host = nullptr;
        s.bytes = 0;
        const size_t sz = std::max<size_t>(bytes, 64u << 10);
        hipError_t e = hipHostMalloc(&s.host, sz, hipHostMallocDefault);
        if (e != hipSuccess) return fail(RFXQ_ERR_OUT_OF_MEMORY, "pinned staging alloc: %s", hipGetErrorString(e));
        s.bytes = sz;
    }
    std::memcpy(s.host, src, bytes);
    HIPCHK(hipMemcpyAsync(dst, s.host, bytes, hipMemcpyHostToDevice, stream), "table upload");
    HIPCHK(hipEventRecord(s.done, stream), "hipEventRecord");
    s.pending = true;
    return RFXQ_OK;
}

int current_ctx(Ctx** out) {
    int dev = 0;
    HIPCHK(hipGetDevice(&dev), "hipGetDevice");
    return load_ctx(dev, out);
}

// Per-device scratch for calls without a caller workspace (the reference
// allocates per call, alloc_out kernels.rs:1001); see grow_area.
int ctx_workspace(Ctx* c, uint64_t bytes, void** out, hipStream_t stream) {
    return grow_area(c, &c->ws, &c->ws_bytes, bytes, 1u << 20, stream, "workspace", out);
}

int launch(hipFunction_t f, uint32_t grid, uint32_t lds, hipStream_t stream, void* args, size_t args_size,
           const char* what, uint32_t threads = 256) {
    void* cfg[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, args, HIP_LAUNCH_PARAM_BUFFER_SIZE, &args_size,
                   HIP_LAUNCH_PARAM_END};
    HIPCHK(hipModuleLaunchKernel(f, grid, 1, 1, threads, 1, 1, lds, stream, nullptr, cfg), what);
    return RFXQ_OK;
}

// ------------------------------------------------------------------ shapes

bool block_dims(uint32_t ty, uint32_t* qk, uint32_t* bb) {
    switch (ty) {
        case RFXQ_TYPE_F32: *qk = 1; *bb = 4; return true;
        case RFXQ_TYPE_F16: *qk = 1; *bb = 2; return true;
        case RFXQ_TYPE_Q8_0: *qk = 32; *bb = 34; return true;
        case RFXQ_TYPE_Q8_1: *qk = 32; *bb = 36; return true;
        case RFXQ_TYPE_Q4_K: *qk = 256; *bb = 144; return true;
        case RFXQ_TYPE_Q6_K: *qk = 256; *bb = 210; return true;
        default: {
            uint64_t q, b;  // every other type of the GGUF block table
            if (!gguf::block_dims(ty, &q, &b)) return false;
            *qk = (uint32_t)q;
            *bb = (uint32_t)b;
            return true;
        }
    }
}

bool is_kernel_type(uint32_t ty) {
    return ty == RFXQ_TYPE_Q4_K || ty == RFXQ_TYPE_Q6_K || ty == RFXQ_TYPE_Q8_0;
}

const char* type_name(uint32_t ty) {
    return ty == RFXQ_TYPE_Q4_K ? "Q4K" : ty == RFXQ_TYPE_Q6_K ? "Q6K" : ty == RFXQ_TYPE_Q8_0 ? "Q8_0" : "?";
}

uint64_t row_bytes(uint32_t ty, uint32_t k) {
    uint32_t qk = 1, bb = 1;
    block_dims(ty, &qk, &bb);
    return (uint64_t)(k / qk) * bb;
}

// The 2-D weight preconditions every kernel shares (kernels.rs:2118-2130).
int check_weight(const rfxq_weight* w, const char* what) {
    if (!w) return fail(RFXQ_ERR_INVALID_INPUT, "%s: weight is NULL", what);
    if (!is_kernel_type(w->ggml_type))
        return fail(RFXQ_ERR_GGUF, "%s: no quantized kernel for ggml_type=%u", what, w->ggml_type);
    if (w->expert_count != 0)
        return fail(RFXQ_ERR_OTHER, "%s: 3-D per-expert weight; slice it with rfxq_quant_expert_weight", what);
    const uint32_t qk = w->ggml_type == RFXQ_TYPE_Q8_0 ? 32u : 256u;
    if (w->in_features == 0 || w->in_features % qk != 0)
        return fail(RFXQ_ERR_OTHER, "%s: in_features=%u (must be a multiple of %u)", what, w->in_features, qk);
    if (w->out_features == 0) return fail(RFXQ_ERR_OTHER, "%s: out_features=0", what);
    const uint64_t need = row_bytes(w->ggml_type, w->in_features) * w->out_features;
    if (w->len < need)
        return fail(RFXQ_ERR_OTHER, "%s: %s weight of %llu bytes, shape [%u, %u] needs %llu", what,
                    type_name(w->ggml_type), (unsigned long long)w->len, w->in_features, w->out_features,
                    (unsigned long long)need);
    if (!w->data) return fail(RFXQ_ERR_INVALID_INPUT, "%s: weight data is NULL", what);
    const uintptr_t a = reinterpret_cast<uintptr_t>(w->data);
    if (w->ggml_type == RFXQ_TYPE_Q4_K ? (a % 16u) != 0 : (a % 2u) != 0)
        return fail(RFXQ_ERR_OTHER, "%s: %s weight data at %p is not %u-byte aligned", what,
                    type_name(w->ggml_type), w->data, w->ggml_type == RFXQ_TYPE_Q4_K ? 16u : 2u);
    return RFXQ_OK;
}

// ------------------------------------------------------------------ options

// The prefill path's switches (rfxq_options), read from the environment once,
// on first use, with the reference's strict parsing
// (QuantMmaKernels::from_env, src/model/kernels.rs:747-802; quant_fused_max_rows,
// :4180-4194): an invalid value is an RFXQ_ERR_INVALID_INPUT error, with the
// reference's message, from every call that needs the options.
struct Options {
    rfxq_options o;
    int code = RFXQ_OK;
    std::string msg;
};

// Rust's `str::parse::<usize>`: an optional '+', then decimal digits only;
// values beyond 32 bits saturate (they act as "no limit" here)
bool parse_usize(const char* v, uint32_t* out) {
    if (*v == '+') v++;
    if (!*v) return false;
    uint64_t x = 0;
    for (; *v; v++) {
        if (*v < '0' || *v > '9') return false;
        x = std::min<uint64_t>(x * 10u + (uint64_t)(*v - '0'), 0xFFFFFFFFull);
    }
    *out = (uint32_t)x;
    return true;
}

Options load_options() {
    Options O;
    rfxq_options& o = O.o;
    o.quant_mma = 1;
    o.mmq_f16 = 1;
    o.fused_max_rows = 16;
    auto env = [](const char* name) -> const char* {
        const char* v = std::getenv(name);
        return v && *v ? v : nullptr;  // unset and "" both take the default
    };
    auto bad = [&](const char* name, const char* want, const char* v) {
        if (O.code != RFXQ_OK) return;  // the first bad variable is reported
        char buf[320];
        std::snprintf(buf, sizeof buf, "%s must be %s, got \"%s\"", name, want, v);
        O.code = RFXQ_ERR_INVALID_INPUT;
        O.msg = buf;
    };
    if (const char* v = env("REFLEX_QUANT_MMA")) {
        if (!std::strcmp(v, "0")) o.quant_mma = 0;
        else if (std::strcmp(v, "1")) bad("REFLEX_QUANT_MMA", "1 (the default) or 0", v);
    }
    if (const char* v = env("REFLEX_QUANT_MMA_SPLITS")) {
        if (!parse_usize(v, &o.quant_mma_splits) || o.quant_mma_splits == 0) {
            o.quant_mma_splits = 0;
            bad("REFLEX_QUANT_MMA_SPLITS", "a positive integer", v);
        }
    }
    if (const char* v = env("REFLEX_QUANT_MMA_MAX_ROWS")) {
        if (!parse_usize(v, &o.quant_mma_max_rows)) {
            o.quant_mma_max_rows = 0;
            bad("REFLEX_QUANT_MMA_MAX_ROWS", "a non-negative integer", v);
        }
    }
    if (const char* v = env("REFLEX_QUANT_MMA_TILE")) {
        if (!std::strcmp(v, "64")) o.quant_mma_tile = 64;
        else if (!std::strcmp(v, "128")) o.quant_mma_tile = 128;
        else bad("REFLEX_QUANT_MMA_TILE", "64 or 128", v);
    }
    // this build's switch, parsed like REFLEX_QUANT_MMA
    if (const char* v = env("REFLEX_MMQ_F16")) {
        if (!std::strcmp(v, "0")) o.mmq_f16 = 0;
        else if (std::strcmp(v, "1")) bad("REFLEX_MMQ_F16", "1 (the default) or 0", v);
    }
    // the reference keeps its default for a value that does not parse
    // (quant_fused_max_rows, kernels.rs:4186-4194)
    if (const char* v = env("REFLEX_QUANT_FUSED_MAX_ROWS")) {
        if (!parse_usize(v, &o.fused_max_rows)) o.fused_max_rows = 16;
    }
    return O;
}

// the process's options: the environment's on first use, rfxq_set_options' after
std::mutex g_opt_mu;
Options& options_locked() {
    static Options O = load_options();
    return O;
}

// the options, or the environment's parse error
int get_options(rfxq_options* out) {
    Options O;
    {
        std::lock_guard<std::mutex> lk(g_opt_mu);
        O = options_locked();
    }
    if (O.code != RFXQ_OK) return fail(O.code, "%s", O.msg.c_str());
    *out = O.o;
    return RFXQ_OK;
}

// a snapshot of the options of a call that already checked them (get_options)
rfxq_options opt() {
    std::lock_guard<std::mutex> lk(g_opt_mu);
    return options_locked().o;
}
bool options_ok() {
    std::lock_guard<std::mutex> lk(g_opt_mu);
    return options_locked().code == RFXQ_OK;
}

int check_options(const rfxq_options& o) {
    if (o.quant_mma != 0 && o.quant_mma != 1)
        return fail(RFXQ_ERR_INVALID_INPUT, "quant_mma must be 0 or 1, got %d", o.quant_mma);
    if (o.quant_mma_tile != 0 && o.quant_mma_tile != 64 && o.quant_mma_tile != 128)
        return fail(RFXQ_ERR_INVALID_INPUT, "quant_mma_tile must be 0, 64 or 128, got %u", o.quant_mma_tile);
    if (o.mmq_f16 != 0 && o.mmq_f16 != 1)
        return fail(RFXQ_ERR_INVALID_INPUT, "mmq_f16 must be 0 or 1, got %d", o.mmq_f16);
    return RFXQ_OK;
}

// ------------------------------------------------------------------ GEMV planning

// One GEMV of a launch: its descriptor and how its rows split into row
// iterations (4 * 64 / LPR rows: one lane group per wave and row).
struct GemvItem {
    GemvDesc d;
    uint32_t iters, rows_iter;
    uint64_t iter_bytes;
    bool passes;  // several units per lane: row partials in LDS
};

void gemv_shape(GemvItem* it, uint32_t k);

int make_gemv_item(const float* x, const rfxq_weight* w, float* y, GemvItem* it) {
    if (int rc = check_weight(w, "gemv")) return rc;
    const uint32_t k = w->in_features, n = w->out_features;
    // buffer offsets are 32-bit and 0xFFFFF000 marks "past the end"
    if (row_bytes(w->ggml_type, k) * n >= 0xFFFFF000ull - 4096u)
        return fail(RFXQ_ERR_OTHER, "gemv: weight of %llu bytes exceeds the 4 GiB buffer-offset range",
                    (unsigned long long)(row_bytes(w->ggml_type, k) * n));
    if (k > kMaxGemvK) return fail(RFXQ_ERR_OTHER, "gemv: in_features=%u exceeds %u", k, kMaxGemvK);
    if (!x || !y) return fail(RFXQ_ERR_INVALID_INPUT, "gemv: x or y is NULL");
    if (reinterpret_cast<uintptr_t>(x) % 16u) return fail(RFXQ_ERR_OTHER, "gemv: x is not 16-byte aligned");
    if (reinterpret_cast<uintptr_t>(y) % 4u) return fail(RFXQ_ERR_OTHER, "gemv: y is not 4-byte aligned");
    if (w->ggml_type == RFXQ_TYPE_Q8_0 && (k / 32u) % 4u)
        // Q8_0 with k/32 not a multiple of 4: not supported by the lane mapping
        return fail(RFXQ_ERR_OTHER, "gemv: %s in_features=%u needs k/32 %% 4 == 0", type_name(w->ggml_type), k);
    std::memset(it, 0, sizeof *it);
    GemvDesc* d = &it->d;
    d->w = w->data;
    d->x = x;
    d->y = y;
    d->n = n;
    d->type = w->ggml_type;
    gemv_shape(it, k);
    return RFXQ_OK;
}

// K, lanes per row (the most units per lane group up to 64 lanes that divide
// the row's units; at least 4) and the iteration sizes of an item.
void gemv_shape(GemvItem* it, uint32_t k) {
    GemvDesc* d = &it->d;
    const uint32_t units = d->type == RFXQ_TYPE_Q8_0 ? k / 32u : k / 64u;
    uint32_t lpr_log2 = 0;
    while (lpr_log2 < 6u && (units % (2u << lpr_log2)) == 0) lpr_log2++;
    if (lpr_log2 < 2) lpr_log2 = 2;  // >= 4 lanes per row (units is always a multiple of 4 here)
    d->k = k;
    d->lpr_log2 = lpr_log2;
    it->rows_iter = 256u >> lpr_log2;
    it->iters = (d->n + it->rows_iter - 1u) / it->rows_iter;
    it->iter_bytes = row_bytes(d->type, k) * it->rows_iter;
    it->passes = (units >> lpr_log2) > 1u;
}

// Workgroups of a launch: about 128 KB of weights
// each, so the x staging is amortised and each wave's load ring reaches a
// steady state; launches too small for 2 workgroups per CU at that size use
// smaller ranges (down to one iteration). A launch with more workgroups than
// the chip holds at once (CUs x workgroups per CU, set by the LDS of the
// widest x) runs as exactly one wave of resident workgroups with larger
// ranges: ranges are byte-balanced, so any further wave would be partial and
// leave most CUs idle while it runs (measured on a 139 MB launch: 34.6 us
// against 44.0 us with 1062 workgroups). Only launches of more than 512 KB
// per resident workgroup take whole waves of workgroups instead.
uint32_t gemv_grid(const Ctx* c, const GemvItem* v, size_t n) {
    uint64_t total_iters = 0, total_bytes = 0;
    uint32_t kmax = 0;
    for (size_t i = 0; i < n; i++) {
        const GemvItem& it = v[i];
        total_iters += it.iters;
        total_bytes += it.iters * it.iter_bytes;
        kmax = std::max(kmax, it.d.k);
    }
    const uint64_t kb = 128u;
    uint64_t g = (total_bytes + kb * 1024u - 1u) / (kb * 1024u);
    g = std::max<uint64_t>(g, 2u * (uint32_t)c->cus);
    // LDS per workgroup: the 32 KB weight ring, x and its sums, and up to 4 KB of row results
    const uint32_t occ = std::min<uint32_t>(4u, (160u * 1024u) / (kGemvRingLds + kmax * 2u + kmax / 4u + 4096u));
    const uint64_t slots = (uint64_t)std::max(1, c->cus) * std::max(1u, occ);
    if (g > slots) {
        const uint64_t waves = (total_bytes + slots * 512u * 1024u - 1u) / (slots * 512u * 1024u);
        g = slots * std::max<uint64_t>(1u, waves);
    }
    return (uint32_t)std::max<uint64_t>(1u, std::min<uint64_t>(g, total_iters));
}
uint32_t gemv_grid(const Ctx* c, const std::vector<GemvItem>& v) { return gemv_grid(c, v.data(), v.size()); }

// LDS bytes for a launch whose workgroups hold at most `max_iters` iterations
// of one GEMV: a row buffer (results and several-pass partials; a multiple of
// 4 floats so x stays 16-byte aligned), then x (f16) and x sums.
int gemv_lds(const std::vector<GemvItem>& v, const std::vector<uint32_t>& max_iters, uint32_t* part_floats,
             uint32_t* lds) {
    uint32_t part = 0, kmax = 0;
    for (size_t i = 0; i < v.size(); i++) {
        part = std::max(part, max_iters[i] * v[i].rows_iter);
        kmax = std::max(kmax, v[i].d.k);
    }
    part = (std::max(part, 4u) + 3u) & ~3u;  // at least 4: the x staging keeps the waves' maxima there
    *part_floats = part;
    *lds = part * 4u + kmax * 2u + kmax / 4u;
    if (*lds > kMaxLds) return fail(RFXQ_ERR_OTHER, "gemv: launch needs %u bytes of LDS", *lds);
    return RFXQ_OK;
}

// One launch whose workgroups split the iterations evenly by count (no
// range table): over up to kGemvInline descriptors passed inline (`table`
// NULL), or over a table the device writes (in the order of `v`, whose
// shapes it shares).
// (No host allocation: rfxq_gemm_no_alloc launches through here.)
int gemv_launch_counted(Ctx* c, const GemvItem* v, size_t n, const GemvDesc* table, hipStream_t stream) {
    if (!table && n > kGemvInline) return fail(RFXQ_ERR_OTHER, "gemv: %zu inline descriptors", n);
    uint64_t total = 0;
    for (size_t i = 0; i < n; i++) total += v[i].iters;
    const uint32_t grid = gemv_grid(c, v, n);
    const uint32_t per_wg = (uint32_t)((total + grid - 1u) / grid);  // no range holds more iterations
    // LDS as gemv_lds, each workgroup holding at most per_wg iterations of a GEMV
    uint32_t part = 0, kmax = 0;
    for (size_t i = 0; i < n; i++) {
        part = std::max(part, std::min(per_wg, v[i].iters) * v[i].rows_iter);
        kmax = std::max(kmax, v[i].d.k);
    }
    GemvArgs a;
    std::memset(&a, 0, sizeof a);
    a.part_floats = (std::max(part, 4u) + 3u) & ~3u;
    const uint32_t lds = a.part_floats * 4u + kmax * 2u + kmax / 4u;
    if (lds > kMaxLds) return fail(RFXQ_ERR_OTHER, "gemv: launch needs %u bytes of LDS", lds);
    a.ndesc = (uint32_t)n;
    a.table = table;
    // one iteration count for every descriptor: the kernel need not read them
    a.iters_each = n ? v[0].iters : 0u;
    for (size_t i = 0; i < n; i++)
        if (v[i].iters != a.iters_each) a.iters_each = 0u;
    if (!table)
        for (size_t i = 0; i < n; i++) a.inl[i] = v[i].d;
    return launch(c->gemv, grid, lds, stream, &a, sizeof a, "rfxq_gemv launch");
}
int gemv_launch_counted(Ctx* c, const std::vector<GemvItem>& v, const GemvDesc* table, hipStream_t stream) {
    return gemv_launch_counted(c, v.data(), v.size(), table, stream);
}

int gemv_launch_inline(Ctx* c, const std::vector<GemvItem>& v, hipStream_t stream) {
    return gemv_launch_counted(c, v, nullptr, stream);
}

void gemv_split_bytes(const std::vector<GemvItem>& v, uint32_t grid, std::vector<GemvRange>* ranges,
                      std::vector<uint32_t>* max_iters);

// One launch over any number of GEMVs: descriptors and byte-balanced ranges
// uploaded (stream-ordered) into the context's table area at byte `at`
int gemv_launch_table(Ctx* c, const std::vector<GemvItem>& v, uint64_t at, hipStream_t stream) {
    const uint32_t grid = gemv_grid(c, v);
    std::vector<GemvRange> ranges;
    std::vector<uint32_t> max_iters;
    gemv_split_bytes(v, grid, &ranges, &max_iters);
    GemvArgs a;
    std::memset(&a, 0, sizeof a);
    uint32_t lds;
    if (int rc = gemv_lds(v, max_iters, &a.part_floats, &lds)) return rc;
    const size_t tb = align256(sizeof(GemvDesc) * v.size()), rb = sizeof(GemvRange) * ranges.size();
    std::vector<uint8_t> host(tb + rb, 0);
    for (size_t i = 0; i < v.size(); i++) std::memcpy(host.data() + i * sizeof(GemvDesc), &v[i].d, sizeof(GemvDesc));
    std::memcpy(host.data() + tb, ranges.data(), rb);
    void* area;
    if (int rc = ctx_tables(c, at + host.size(), &area, stream)) return rc;
    uint8_t* dst = static_cast<uint8_t*>(area) + at;
    if (int rc = stage_upload(c, dst, host.data(), host.size(), stream)) return rc;
    a.ndesc = (uint32_t)v.size();
    a.table = reinterpret_cast<const GemvDesc*>(dst);
    a.ranges = reinterpret_cast<const GemvRange*>(dst + tb);
    if (v.size() <= kGemvInline)
        for (size_t i = 0; i < v.size(); i++) a.inl[i] = v[i].d;
    return launch(c->gemv, grid, lds, stream, &a, sizeof a, "rfxq_gemv launch");
}

int gemv_items(Ctx* c, const rfxq_gemv_item* items, uint32_t count, hipStream_t stream) {
    if (count > kGemvInline) {  // one launch over a descriptor table
        std::vector<GemvItem> v(count);
        for (uint32_t j = 0; j < count; j++)
            if (int rc = make_gemv_item(items[j].x, items[j].w, items[j].y, &v[j])) return rc;
        return gemv_launch_table(c, v, 0, stream);
    }
    for (uint32_t i0 = 0; i0 < count; i0 += kGemvInline) {
        const uint32_t cnt = std::min<uint32_t>(kGemvInline, count - i0);
        std::vector<GemvItem> v(cnt);
        for (uint32_t j = 0; j < cnt; j++) {
            const rfxq_gemv_item& it = items[i0 + j];
            if (int rc = make_gemv_item(it.x, it.w, it.y, &v[j])) return rc;
        }
        if (int rc = gemv_launch_inline(c, v, stream)) return rc;
    }
    return RFXQ_OK;
}

// A plan's ranges, balanced by cost: workgroup g starts at the first
// iteration (in descriptor order) whose start lies at or after g/grid of the
// launch's cost; the last range ends at the end of the last descriptor. An
// iteration costs its weight bytes, times kGemvLongCost for a GEMV whose x
// exceeds kGemvLongK elements and whose rows take several passes (its x
// staging and passes make its bytes slower), and no range runs into such a
// GEMV from the one before it: the descriptors split into segments at each
// one's start, each segment gets workgroups in proportion to its cost
// (largest remainders) and balances them within itself. (The 8B layer's
// down projection, K = 14336: 32.9 us by bytes; 28.1 us this way, and
// 27.8-28.3 us for any cost factor from 1.2 to 2.0. A workgroup that ran the
// end of up and the start of down staged both x's and finished last; without
// the segments the measured time jumped between 28 and 35 us with the
// position of that boundary.)
constexpr uint32_t kGemvLongK = 4096;
constexpr double kGemvLongCost = 1.5;
uint64_t gemv_iter_cost(const GemvItem& it) {
    return it.d.k > kGemvLongK && it.passes ? (uint64_t)((double)it.iter_bytes * kGemvLongCost) : it.iter_bytes;
}

void gemv_split_bytes(const std::vector<GemvItem>& v, uint32_t grid, std::vector<GemvRange>* ranges,
                      std::vector<uint32_t>* max_iters) {
    // segments [seg[s], seg[s + 1]) of descriptors and their costs
    std::vector<uint32_t> seg{0u};
    for (uint32_t d = 1; d < v.size(); d++)
        if (gemv_iter_cost(v[d]) != v[d].iter_bytes) seg.push_back(d);
    seg.push_back((uint32_t)v.size());
    const uint32_t ns = (uint32_t)seg.size() - 1u;
    std::vector<uint64_t> scost(ns, 0);
    uint64_t total = 0;
    for (uint32_t s2 = 0; s2 < ns; s2++) {
        for (uint32_t d = seg[s2]; d < seg[s2 + 1u]; d++) scost[s2] += v[d].iters * gemv_iter_cost(v[d]);
        total += scost[s2];
    }
    // workgroups per segment: proportional, at least one, largest remainders
    std::vector<uint32_t> sg(ns, 1u);
    if (grid > ns) {
        std::vector<std::pair<double, uint32_t>> rem;
        uint32_t used = 0;
        for (uint32_t s2 = 0; s2 < ns; s2++) {
            const double want = total ? (double)(grid - ns) * (double)scost[s2] / (double)total : 0.0;
            sg[s2] += (uint32_t)want;
            used += (uint32_t)want;
            rem.push_back({want - (double)(uint32_t)want, s2});
        }
        std::sort(rem.begin(), rem.end(), [](const auto& a, const auto& b) { return a.first > b.first; });
        for (uint32_t r = 0; used < grid - ns; r++, used++) sg[rem[r % ns].second]++;
    }
    std::vector<std::pair<uint32_t, uint32_t>> start(grid + 1u);
    uint32_t g = 0;
    for (uint32_t s2 = 0; s2 < ns && g < grid; s2++) {
        const uint32_t g0 = g, gn = std::min(sg[s2], grid - g0);
        uint64_t pos = 0;
        for (uint32_t d = seg[s2]; d < seg[s2 + 1u] && g < g0 + gn; d++) {
            const uint64_t c = gemv_iter_cost(v[d]);
            for (uint32_t i = 0; i < v[d].iters && g < g0 + gn; i++) {
                while (g < g0 + gn && pos >= (scost[s2] * (g - g0) + gn - 1u) / gn) start[g++] = {d, i};
                pos += c;
            }
        }
        // workgroups the segment could not fill (fewer iterations): empty
        // ranges at its end
        const uint32_t dl = seg[s2 + 1u] - 1u;
        while (g < g0 + gn) start[g++] = {dl, v[dl].iters};
    }
    while (g < grid) start[g++] = {(uint32_t)v.size() - 1u, v.back().iters};  // empty tail ranges
    start[grid] = {(uint32_t)v.size() - 1u, v.back().iters};
    ranges->resize(grid);
    max_iters->assign(v.size(), 0u);
    for (uint32_t w = 0; w < grid; w++) {
        GemvRange r{start[w].first, start[w].second, start[w + 1u].first, start[w + 1u].second};
        // an end at iteration 0 of a descriptor is the end of the one before
        while (r.d1 > r.d0 && r.it1 == 0u) {
            r.d1--;
            r.it1 = v[r.d1].iters;
        }
        (*ranges)[w] = r;
        for (uint32_t d = r.d0; d <= r.d1; d++) {
            const uint32_t a = d == r.d0 ? r.it0 : 0u, b = d == r.d1 ? r.it1 : v[d].iters;
            if (b > a) (*max_iters)[d] = std::max((*max_iters)[d], b - a);
        }
    }
}

// ------------------------------------------------------------------ MMQ planning

// Prefill GEMMs run on the f16-activation kernels (rfxq_mmqh_q4k / _q6k /
// _q8_0: f16 activations scaled per row, weights as f16 operands, f32
// accumulation in the matrix core) unless REFLEX_MMQ_F16=0 selects the int8
// MMQ kernels (Q8_1 activations, per-32 int32 block dots). The int8 format's
// own error exceeds the 1e-3 bound at some shapes, so the default never falls
// back to it: a GEMM the f16 kernels cannot run takes the GEMV path.
constexpr uint32_t kMmqThreads = 256;  // every MMQ kernel's workgroup
bool mmq_f16() { return opt().mmq_f16 != 0; }

// The f16 kernels run any Q4_K, Q6_K or Q8_0 GEMM with k a multiple of 256:
// their buffer resources start at the tile (weights at its first column,
// activations at its first row), so offsets fit in 32 bits for any size. A
// gathered GEMM (MoE expert groups: `gather_src` source rows, 0 = not
// gathered) addresses every source row from the buffer start, so its f16
// activations must stay below the limit.
bool f16_capable(uint32_t ty, uint64_t k, uint64_t gather_src) {
    if (ty != RFXQ_TYPE_Q4_K && ty != RFXQ_TYPE_Q6_K && ty != RFXQ_TYPE_Q8_0) return false;
    if (k == 0 || k % 256u) return false;
    const uint64_t lim = 0xF0000000ull;
    return gather_src * k * 2u < lim;
}

// an f16 kernel for a gathered GEMM of `src_rows` source rows in f16 mode
bool f16_kernel(const rfxq_weight* w, uint32_t src_rows) {
    return mmq_f16() && f16_capable(w->ggml_type, w->in_features, src_rows);
}

// weight columns per workgroup tile: 256 on the f16 kernels, 128 on the int8 ones
uint32_t tile_bn(bool f16) { return f16 ? 256u : 128u; }

// How a GEMM of `rows` rows runs (Model::gemm's choice between the fused GEMV,
// the MMA kernel and its split-K, kernels.rs:628-713 quant_mma_splits /
// block_rows / max_rows and :2144-2169, re-derived for MI355X):
// - one GEMV per row (PATH_GEMV_ROWS) for a single row, with the MMA path off
//   (REFLEX_QUANT_MMA=0), above REFLEX_QUANT_MMA_MAX_ROWS, with in_features
//   not a multiple of 256, and up to REFLEX_QUANT_FUSED_MAX_ROWS rows
//   (default 16) on the int8 path, up to kGemvRowsMax of them on the f16
//   path (a GEMV per row re-reads the weights, cheaper than the few-row
//   tiles' launch pair below 5 rows);
// - otherwise the f16-activation kernels (PATH_MMQ_F16: Q4_K, Q6_K and Q8_0,
//   the default): 32-row tiles up to 32 rows (the fused
//   few-row form: each weight read once for all rows), 64-row tiles up to
//   64, 128-row tiles above,
//   or the int8 kernels (PATH_MMQ_INT8; 64-row tiles with
//   REFLEX_QUANT_MMA_TILE=64);
// - split-K: none once the tiles cover half the CUs (each CU holds two
//   workgroups; a split costs a partials round trip and a reduce launch),
//   else the smallest split (at least two super-blocks; one with 32-row
//   tiles) whose workgroups all fit in two per CU (split_sb);
//   REFLEX_QUANT_MMA_SPLITS forces the count.
enum : uint32_t { PATH_GEMV_ROWS = RFXQ_PATH_GEMV_ROWS, PATH_MMQ_INT8 = RFXQ_PATH_MMQ_INT8, PATH_MMQ_F16 = RFXQ_PATH_MMQ_F16 };
constexpr uint32_t kGemvRowsMax = 4;
constexpr uint64_t kGemvReread = 56ull << 20;  // bytes of weight re-reads above which few rows take tiles

// Super-blocks per split-K workgroup for the GEMMs of one launch (their
// tile counts and super-blocks per row): the fewest, at least min_sb, whose
// workgroups (tiles x ceil(nsb / W) per GEMM) fit in `budget`, so that the
// launch runs as one wave of workgroups. (With the splits rounded up
// instead, the 8B layer's v + down launch made 544 workgroups for 512
// places: a second wave of 32 that started when the first v workgroups
// ended and finished well after the rest.)
uint32_t split_sb(const std::vector<std::pair<uint32_t, uint32_t>>& tiles_nsb, uint32_t min_sb, uint32_t budget) {
    uint32_t max_nsb = 1;
    for (const auto& t : tiles_nsb) max_nsb = std::max(max_nsb, t.second);
    for (uint32_t w = std::max(1u, min_sb); w < max_nsb; w++) {
        uint64_t total = 0;
        for (const auto& t : tiles_nsb) total += (uint64_t)t.first * ((t.second + w - 1u) / w);
        if (total <= budget) return w;
    }
    return max_nsb;
}


// Row tile of the f16 kernels for a GEMM (or an expert group averaging
// `rows`): weights are read once per tile, so the smallest tile that holds
// the rows (32 or 64 rows: weight-stream bound, more workgroups per CU), 128
// above
uint32_t f16_tile_m(uint32_t rows) { return rows <= 32u ? 32u : rows <= 64u ? 64u : kMmqBM; }

// Row tile of one grouped MoE GEMM, `pairs` routed rows over `experts`
// groups, `tiles_n` column tiles per expert: f16 kernels 32-row tiles up to
// 12 rows per expert on average, 128 above 64; in between 64 or 128,
// whichever runs the launch's tiles (estimated from the average) in fewer
// waves of resident workgroups (64-row tiles: 3 per CU for Q4_K, 2 for
// Q6_K; 128-row tiles: 2 per CU), 128 on a tie. Config 5 (32 rows per expert
// on average): gate + up, 768 tiles, stay at 64 rows (88 us against 105 us
// at 128, which needs 2 waves), and the down projection, 1024 tiles and 2
// waves either way, takes 128 (60 us against 67 us). int8 kernels: 64-row
// tiles up to 48 rows on average.
uint32_t moe_tile_m(uint32_t pairs, uint32_t experts, bool f16, uint32_t ty, uint32_t tiles_n, uint32_t cus) {
    if (!experts) return kMmqBM;
    const uint32_t avg = (pairs + experts - 1u) / experts;
    if (!f16) return avg <= 48u ? 64u : kMmqBM;
    if (avg <= 12u) return 32u;
    if (avg > 64u) return kMmqBM;
    auto waves = [&](uint32_t bm, uint32_t per_cu) {
        const uint64_t tiles = (uint64_t)experts * ((avg + bm - 1u) / bm) * tiles_n;
        const uint64_t slots = (uint64_t)std::max(1u, cus) * per_cu;
        return (tiles + slots - 1u) / slots;
    };
    return waves(64u, ty == RFXQ_TYPE_Q6_K ? 2u : 3u) < waves(kMmqBM, 2u) ? 64u : kMmqBM;
}

// Row tile of a GEMM of 256 rows or more launched alone (not in a grouped
// launch, whose workgroups are counted over all its GEMMs; fewer rows keep
// the tile that holds them) that is too small to occupy half
// the CUs even at its largest split (nsb / 2 splits of 128- or 64-row
// tiles): smaller row tiles, down to 32. Config 1's 1024 x 1024 Q8_0 matrix
// at 512 rows has 16 tiles of 128 rows (32 workgroups with two splits) and
// 64 of 32 rows (256 workgroups with four one-super-block splits).
uint32_t small_gemm_tile_m(uint32_t tile_m, uint32_t rows, uint32_t n, uint32_t nsb, uint32_t cus) {
    const uint64_t tn = (n + 255u) / 256u;
    while (tile_m > 32u && (uint64_t)((rows + tile_m - 1u) / tile_m) * tn * std::max(1u, nsb / 2u) * 2u <
                               std::max(cus, 1u))
        tile_m /= 2u;
    return tile_m;
}

// raw bytes of a weight matrix
uint64_t gemm_weight_bytes(uint32_t ty, uint32_t k, uint32_t n) {
    return ty == RFXQ_TYPE_Q8_0 ? (uint64_t)n * (k / 32u) * 34u : (uint64_t)n * (k / 256u) * (ty == RFXQ_TYPE_Q6_K ? 210u : 144u);
}

rfxq_gemm_policy gemm_policy(uint32_t ty, uint32_t k, uint32_t n, uint32_t rows, uint32_t cus, const rfxq_options& o,
                             bool alone = true, uint64_t group_bytes = 0) {
    rfxq_gemm_policy p;
    std::memset(&p, 0, sizeof p);
    p.splits = 1;
    const bool f16 = o.mmq_f16 && f16_capable(ty, k, 0);
    // f16 path: up to kGemvRowsMax rows run as GEMVs, except 3+ rows whose
    // re-reads of the weights ((rows - 1) x their bytes: this GEMM's alone,
    // or `group_bytes`, a grouped launch's, so that all of its GEMMs take one
    // path) would reach kGemvReread (56 MiB): they read them once on 32-row tiles (an
    // 8B layer at 3 / 4 rows: 78 us on tiles against 84-87 / 90-109 us as
    // GEMVs or mixed; a 0.6B layer, 9 MB, stays faster as GEMVs at 2-4 rows)
    const uint64_t wbytes = group_bytes ? group_bytes : gemm_weight_bytes(ty, k, n);
    const bool few_gemv = rows <= kGemvRowsMax && (rows <= 2u || (uint64_t)(rows - 1u) * wbytes < kGemvReread);
    const bool gemv = rows <= 1 || !o.quant_mma || (o.quant_mma_max_rows && rows > o.quant_mma_max_rows) ||
                      (rows <= o.fused_max_rows && (!f16 || few_gemv)) || k % 256u != 0 ||
                      (o.mmq_f16 && !f16);
    if (gemv) {
        p.path = PATH_GEMV_ROWS;
        return p;
    }
    p.path = f16 ? PATH_MMQ_F16 : PATH_MMQ_INT8;
    p.tile_m = f16 ? f16_tile_m(rows) : o.quant_mma_tile == 64 ? 64u : kMmqBM;
    p.tile_n = tile_bn(f16);
    const uint32_t nsb = k / 256u;
    if (f16 && alone && !o.quant_mma_splits && rows >= 256u) p.tile_m = small_gemm_tile_m(p.tile_m, rows, n, nsb, cus);
    const uint32_t tiles = ((rows + p.tile_m - 1u) / p.tile_m) * ((n + p.tile_n - 1u) / p.tile_n);
    uint32_t splits = 1;
    if (o.quant_mma_splits) splits = o.quant_mma_splits;
    else if (2u * tiles < std::max(cus, 1u)) {
        // 32-row tiles stream weights (few rows): splits down to one super-block
        const uint32_t w = split_sb({{tiles, nsb}}, p.tile_m == 32u ? 1u : 2u, 2u * std::max(cus, 1u));
        splits = (nsb + w - 1u) / w;
    }
    splits = std::min(std::max(1u, splits), nsb);
    p.sb_per_split = (nsb + splits - 1u) / splits;
    p.splits = (nsb + p.sb_per_split - 1u) / p.sb_per_split;
    return p;
}

// One activation in the layouts its GEMMs read, each 256-byte aligned:
// int8 (xq [rows][k], xds [rows][k/32] = d | s << 16) and f16 (xh [rows][k],
// xsx [rows][k/256][16] f16 block sums, xrs [rows] f32 row scales).
struct ActLayout {
    uint64_t xq = 0, xds = 0, xh = 0, xsx = 0, xrs = 0, total = 0;
};

ActLayout act_layout_sel(uint32_t rows, uint32_t k, bool i8, bool h) {
    ActLayout L;
    uint64_t o = 0;
    if (i8) {
        L.xq = o;
        o += align256((uint64_t)rows * k);
        L.xds = o;
        o += align256((uint64_t)rows * (k / 32u) * 4u);
    }
    if (h) {
        L.xh = o;
        o += align256((uint64_t)rows * k * 2u);
        L.xsx = o;
        o += align256((uint64_t)rows * (k / 256u) * 32u);
        L.xrs = o;
        o += align256((uint64_t)rows * 4u);
    }
    L.total = o;
    return L;
}

// the public activation buffer (rfxq_act_q8_1_size): every layout
ActLayout act_layout(uint32_t rows, uint32_t k) { return act_layout_sel(rows, k, true, true); }

// the descriptor fields of a GEMM reading activation layouts L at `base`
void act_desc(MmqDesc* d, const uint8_t* base, const ActLayout& L, bool f16, uint32_t k) {
    if (f16) {
        d->xq = reinterpret_cast<const int8_t*>(base + L.xh);
        d->xds = reinterpret_cast<const uint32_t*>(base + L.xsx);
        d->xrs = reinterpret_cast<const float*>(base + L.xrs);
        d->ldq = 2u * k;
    } else {
        d->xq = reinterpret_cast<const int8_t*>(base + L.xq);
        d->xds = reinterpret_cast<const uint32_t*>(base + L.xds);
        d->xrs = nullptr;
        d->ldq = k;
    }
}

uint32_t quant_grid(uint64_t blocks) {
    const uint64_t waves = (blocks + 7u) / 8u;
    return (uint32_t)std::min<uint64_t>(std::max<uint64_t>((waves + 3u) / 4u, 1u), 8192u);
}

// int8 layout of x (rfxq_quantize_q8_1); `src_rows` gathers rows
int launch_quant(Ctx* c, const float* x, uint32_t ldx, const int32_t* src_rows, uint32_t rows, uint32_t k,
                 int8_t* xq, uint32_t* xds, hipStream_t stream) {
    struct {
        const float* x;
        uint32_t ldx, pad0;
        const int32_t* src_rows;
        uint32_t rows, k;
        int8_t* xq;
        uint32_t ldq, pad1;
        uint32_t* xds;
    } a = {x, ldx, 0, src_rows, rows, k, xq, k, 0, xds};
    return launch(c->quant, quant_grid((uint64_t)rows * (k / 32u)), 0, stream, &a, sizeof a,
                  "rfxq_quantize_q8_1 launch");
}

// f16 layout of x (rfxq_act_f16): one wave per row
// f16 activation kernels: a row per wave (rfxq_act_f16[_multi], 4 rows per
// workgroup) for at least 128 rows of at most 4096 values, else a row per
// workgroup (rfxq_act_f16[_multi]_wg: few rows, or rows too long for one
// wave's registers)
bool act_f16_wave(uint32_t rows, uint32_t k) { return k <= 4096u && rows >= 128u; }
uint32_t act_f16_grid(uint32_t rows, bool wave) {
    return wave ? std::min<uint32_t>((rows + 3u) / 4u, 4096u) : std::min<uint32_t>(rows, 16384u);
}

int launch_act_f16(Ctx* c, const float* x, uint32_t ldx, const int32_t* src_rows, uint32_t rows, uint32_t k,
                   uint8_t* base, const ActLayout& L, hipStream_t stream) {
    struct {
        const float* x;
        uint32_t ldx, pad0;
        const int32_t* src_rows;
        uint32_t rows, k;
        uint16_t* xh;
        uint16_t* xsx;
        float* xrs;
    } a = {x, ldx, 0, src_rows, rows, k, reinterpret_cast<uint16_t*>(base + L.xh),
           reinterpret_cast<uint16_t*>(base + L.xsx), reinterpret_cast<float*>(base + L.xrs)};
    // (one activation: the row-per-wave kernel only once its grid fills the
    // chip; 512 rows of 2048 take 6 us as 512 workgroups against 9.6 us as 128)
    const bool wave = act_f16_wave(rows, k) && rows >= 1024u;
    return launch(wave ? c->act_f16 : c->act_f16_wg, act_f16_grid(rows, wave), 0, stream, &a, sizeof a,
                  "rfxq_act_f16 launch");
}

// the activation layouts of L at `base` from x
int launch_act(Ctx* c, const float* x, uint32_t rows, uint32_t k, uint8_t* base, const ActLayout& L, bool i8,
               bool h, hipStream_t stream) {
    if (i8)
        if (int rc = launch_quant(c, x, k, nullptr, rows, k, reinterpret_cast<int8_t*>(base + L.xq),
                                  reinterpret_cast<uint32_t*>(base + L.xds), stream))
            return rc;
    if (h)
        if (int rc = launch_act_f16(c, x, k, nullptr, rows, k, base, L, stream)) return rc;
    return RFXQ_OK;
}

// SiLU(gate) * up of rows x k written straight into the layouts of L at
// `base` (rfxq_silu_and_mul_q8_1 without its f32 output): one launch instead
// of rfxq_silu_and_mul and the layout pass, the same values
int launch_silu_act(Ctx* c, const float* gate, const float* up, uint32_t rows, uint32_t k, uint8_t* base,
                    const ActLayout& L, bool i8, bool h, hipStream_t stream) {
    struct {
        const float* gate;
        const float* up;
        uint32_t rows, k;
        int8_t* xq;
        uint32_t* xds;
        uint16_t* xh;
        uint16_t* xsx;
        float* xrs;
        float* y;
    } a = {gate,
           up,
           rows,
           k,
           i8 ? reinterpret_cast<int8_t*>(base + L.xq) : nullptr,
           i8 ? reinterpret_cast<uint32_t*>(base + L.xds) : nullptr,
           h ? reinterpret_cast<uint16_t*>(base + L.xh) : nullptr,
           h ? reinterpret_cast<uint16_t*>(base + L.xsx) : nullptr,
           h ? reinterpret_cast<float*>(base + L.xrs) : nullptr,
           nullptr};
    const uint32_t grid = i8 ? quant_grid((uint64_t)rows * (k / 32u)) : act_f16_grid(rows, act_f16_wave(rows, k));
    return launch(c->silu_q, grid, 0, stream, &a, sizeof a, "rfxq_silu_and_mul_q8_1 launch");
}

// rfxq_moe_combine: out[t,:] = sum over the token's k pairs of w * pair_out row
int launch_combine(Ctx* c, const float* pair_out, const int32_t* idx, const float* w, float* out, uint32_t tokens,
                   uint32_t k, uint32_t hidden, hipStream_t stream) {
    const bool vec = hidden % 4u == 0u && reinterpret_cast<uintptr_t>(pair_out) % 16u == 0u &&
                     reinterpret_cast<uintptr_t>(out) % 16u == 0u;
    struct {
        const float* po;
        const int32_t* idx;
        const float* w;
        float* out;
        uint32_t tokens, k, hidden, vec;
    } a = {pair_out, idx, w, out, tokens, k, hidden, vec ? 1u : 0u};
    const uint64_t blocks = vec ? std::min<uint64_t>((uint64_t)tokens * ((hidden + 1023u) / 1024u), 16384u)
                                : std::min<uint64_t>(((uint64_t)tokens * hidden + 255u) / 256u, 16384u);
    return launch(c->combine, (uint32_t)std::max<uint64_t>(blocks, 1u), 0, stream, &a, sizeof a,
                  "moe_combine launch");
}

// f16: Q4_K / Q6_K descriptors on rfxq_mmqh_q4k / _q6k (f16 activation
// layout; tile_m 32: the *_m32 kernels); int8: tile_m 64 takes rfxq_mmq_*_m64
// f16 tiles of this type and height run in the mixed-type kernel (Q4_K and
// Q6_K 32-row tiles: the same bodies, one launch for a few-row layer)
bool mix_f16(uint32_t ty, uint32_t tile_m) { return (ty == RFXQ_TYPE_Q4_K || ty == RFXQ_TYPE_Q6_K) && tile_m == 32u; }

int launch_mmq(Ctx* c, uint32_t ty, const MmqDesc* descs, uint32_t count, const MmqDesc* table, uint32_t total_wgs,
               bool dots, hipStream_t stream, bool f16 = false, uint32_t tile_m = kMmqBM) {
    const bool m64 = !f16 && tile_m == 64u;
    MmqArgs a;
    std::memset(&a, 0, sizeof a);
    a.ndesc = count;
    a.table = table;
    if (count <= kMmqInline) std::copy(descs, descs + count, a.inl);
    hipFunction_t f = dots ? c->dots[type_index(ty)] : m64 ? c->mmq64[type_index(ty)] : c->mmq[type_index(ty)];
    // f16: Q4_K and Q6_K 32-row tiles mixed in one launch, others per type
    if (f16 && !dots)
        f = mix_f16(ty, tile_m) ? c->mmqh_mix_m32 : c->mmqh[type_index(ty)][tile_m == 32u ? 1 : tile_m == 64u ? 2 : 0];
    return launch(f, total_wgs, 0, stream, &a, sizeof a, "rfxq_mmq launch", kMmqThreads);
}

int check_mmq_weight(const rfxq_weight* w, const char* what) {
    if (int rc = check_weight(w, what)) return rc;
    if (w->in_features % 256u)
        return fail(RFXQ_ERR_OTHER, "%s: in_features=%u (the MMQ path needs a multiple of 256)", what,
                    w->in_features);
    return RFXQ_OK;
}

struct GemmPlan {
    rfxq_gemm_policy pol;
    bool f16 = false;
    uint32_t tiles_m = 1, tiles_n = 1;
    ActLayout act;
    uint64_t off_part = 0, total = 0;
};

// an MMQ plan for a GEMM the policy sends to an MMQ path
GemmPlan plan_gemm(const Ctx* c, const rfxq_weight* w, uint32_t rows, const rfxq_options& o) {
    GemmPlan p;
    const uint32_t k = w->in_features, n = w->out_features;
    p.pol = gemm_policy(w->ggml_type, k, n, rows, c ? (uint32_t)c->cus : 256u, o);
    p.f16 = p.pol.path == PATH_MMQ_F16;
    if (p.pol.path == PATH_GEMV_ROWS) return p;  // no MMQ launch: tiles, layouts and workspace stay 0
    p.tiles_m = (rows + p.pol.tile_m - 1u) / p.pol.tile_m;
    p.tiles_n = (n + p.pol.tile_n - 1u) / p.pol.tile_n;
    p.act = act_layout_sel(rows, k, !p.f16, p.f16);
    p.off_part = p.act.total;
    p.total = p.off_part + (p.pol.splits > 1 ? align256((uint64_t)p.pol.splits * rows * n * 4u) : 0u);
    return p;
}

int launch_reduce(Ctx* c, const float* part, float* y, uint64_t n, uint32_t splits, hipStream_t stream) {
    struct {
        const float* ws;
        float* y;
        uint64_t n;
        uint32_t splits, pad;
    } a = {part, y, n, splits, 0};
    const uint64_t blocks = std::min<uint64_t>((n + 255u) / 256u, 8192u);
    return launch(c->reduce, (uint32_t)blocks, 0, stream, &a, sizeof a, "rfxq_splitk_reduce launch");
}

// One GEMM's MMQ launch from activation layouts (`act`, layouts p.act), then
// the split-K reduce when p splits K (partials in `part`).
int gemm_run(Ctx* c, const GemmPlan& p, const uint8_t* act, const ActLayout& L, const rfxq_weight* w,
             uint32_t rows, float* y, float* part, hipStream_t stream) {
    const uint32_t k = w->in_features, n = w->out_features;
    MmqDesc d;
    std::memset(&d, 0, sizeof d);
    d.w = w->data;
    act_desc(&d, act, L, p.f16, k);
    d.y = p.pol.splits > 1 ? part : y;
    d.m = rows;
    d.n = n;
    d.k = k;
    d.type = w->ggml_type;
    d.ldy = n;
    d.tiles_m = p.tiles_m;
    d.tiles_n = p.tiles_n;
    d.splits = p.pol.splits;
    d.sb_per_split = p.pol.sb_per_split;
    const uint32_t wgs = p.tiles_m * p.tiles_n * p.pol.splits;
    if (int rc = launch_mmq(c, w->ggml_type, &d, 1, nullptr, wgs, false, stream, p.f16, p.pol.tile_m))
        return rc;
    if (p.pol.splits > 1)
        if (int rc = launch_reduce(c, part, y, (uint64_t)rows * n, p.pol.splits, stream)) return rc;
    return RFXQ_OK;
}

int gemm_impl(Ctx* c, const float* x, const rfxq_weight* w, uint32_t rows, float* y, void* ws, uint64_t ws_bytes,
              const rfxq_options& o, hipStream_t stream) {
    const GemmPlan p = plan_gemm(c, w, rows, o);
    if (!ws) {
        if (int rc = ctx_workspace(c, p.total, &ws, stream)) return rc;
    } else if (ws_bytes < p.total) {
        return fail(RFXQ_ERR_INVALID_INPUT, "gemm: workspace of %llu bytes, needs %llu",
                    (unsigned long long)ws_bytes, (unsigned long long)p.total);
    }
    uint8_t* base = static_cast<uint8_t*>(ws);
    if (int rc = launch_act(c, x, rows, w->in_features, base, p.act, !p.f16, p.f16, stream)) return rc;
    return gemm_run(c, p, base, p.act, w, rows, y, reinterpret_cast<float*>(base + p.off_part), stream);
}

int check_act(const void* act, uint32_t rows, uint32_t k, const char* what) {
    if (!act) return fail(RFXQ_ERR_INVALID_INPUT, "%s: act is NULL", what);
    if (reinterpret_cast<uintptr_t>(act) % 256u) return fail(RFXQ_ERR_OTHER, "%s: act is not 256-byte aligned", what);
    if (rows == 0 || k == 0 || k % 256u)
        return fail(RFXQ_ERR_OTHER, "%s: rows=%u k=%u (k must be a non-zero multiple of 256)", what, rows, k);
    return RFXQ_OK;
}

// ------------------------------------------------------------------ grouped GEMMs

// GEMMs of one row count over several weights, grouped: each distinct
// activation (by address) is brought into the layouts its GEMMs read once,
// and each MMQ kernel runs as one launch over all of its GEMMs. Each GEMM
// takes the single-GEMM policy's path (gemm_policy); GEMMs on the GEMV path
// run as one GEMV per row in one table-driven launch.
// type_index + 3 * variant (0: int8, 1: int8 64-row, 2: f16, 3: f16 32-row,
// 4: f16 64-row)
constexpr uint32_t kGroupKernels = 15;
struct GemmGroup {
    struct Act {
        const float* x;
        uint32_t k;
        uint64_t off = 0;  // workspace offset of the layouts L
        ActLayout L;
        bool need_i8 = false, need_h = false;
        const uint8_t* ext = nullptr;  // a caller's activation buffer (every layout, act_layout): not quantized here
        uint8_t* base(uint8_t* ws) const { return ext ? const_cast<uint8_t*>(ext) : ws + off; }
    };
    std::vector<Act> acts;
    std::vector<MmqDesc> descs[kGroupKernels];
    std::vector<uint32_t> act_of[kGroupKernels];  // per descriptor: its activation
    uint32_t wgs[kGroupKernels] = {};
    // GEMMs split along K (a kernel with fewer tiles than two per CU):
    // partials at workspace offset `off`, reduced into y after the kernel's launch
    struct Reduce {
        uint32_t t, i;
        uint64_t off;
        float* y;
        float* part;  // bound
        uint64_t n;
        uint32_t splits;
    };
    std::vector<Reduce> reduces;
    uint64_t ws_bytes = 0;
    std::vector<rfxq_gemv_item> gemv_rows;  // GEMMs on the GEMV path, one item per row
};

bool group_f16(uint32_t g) { return g >= 6u; }
uint32_t group_tile_m(uint32_t g) {
    const uint32_t v = g / 3u;
    return v == 1u || v == 4u ? 64u : v == 3u ? 32u : kMmqBM;
}
uint32_t group_variant(bool f16, uint32_t tile_m) { return f16 ? (tile_m == 32u ? 3u : tile_m == 64u ? 4u : 2u) : (tile_m == 64u ? 1u : 0u); }
// the group (launch) of a GEMM: type_index + 3 * variant, except that the f16
// 32-row tiles of Q4_K and Q6_K share one launch (rfxq_mmqh_mix_m32)
uint32_t group_index(uint32_t ty, bool f16, uint32_t tile_m) {
    return (mix_f16(ty, tile_m) && f16 ? 0u : (uint32_t)type_index(ty)) + 3u * group_variant(f16, tile_m);
}

// `ext` (optional, one per item): the items' x are caller activation buffers
// (rfxq_act_q8_1_size layouts, already quantized): every GEMM takes an MMQ
// kernel (f16 unless REFLEX_MMQ_F16=0) and the group quantizes nothing.
int build_gemm_group(const rfxq_gemm_item* items, uint32_t count, uint32_t rows, GemmGroup* g, uint32_t cus,
                     bool ext = false) {
    if (!items || count == 0 || rows == 0) return fail(RFXQ_ERR_INVALID_INPUT, "gemm group: empty");
    rfxq_options o;
    if (int rc = get_options(&o)) return rc;
    std::vector<uint32_t> item_act(count, ~0u), item_kernel(count, 0);
    uint64_t group_bytes = 0;  // the few-row path is chosen for the group as a whole
    for (uint32_t i = 0; i < count; i++)
        if (items[i].w) group_bytes += gemm_weight_bytes(items[i].w->ggml_type, items[i].w->in_features, items[i].w->out_features);
    for (uint32_t i = 0; i < count; i++) {
        const rfxq_gemm_item& it = items[i];
        if (int rc = check_weight(it.w, "gemm group")) return rc;
        if (!it.x || !it.y) return fail(RFXQ_ERR_INVALID_INPUT, "gemm group: item %u has a NULL x or y", i);
        if (reinterpret_cast<uintptr_t>(it.x) % (ext ? 256u : 16u))
            return fail(RFXQ_ERR_OTHER, "gemm group: x of item %u is not %u-byte aligned", i, ext ? 256u : 16u);
        const uint32_t k = it.w->in_features;
        rfxq_gemm_policy pol = gemm_policy(it.w->ggml_type, k, it.w->out_features, rows, cus, o, count == 1u, group_bytes);
        if (ext) {
            if (int rc = check_act(it.x, rows, k, "gemm_q8_1 plan")) return rc;
            const bool f16 = o.mmq_f16 && f16_capable(it.w->ggml_type, k, 0);
            pol.path = f16 ? PATH_MMQ_F16 : PATH_MMQ_INT8;
            pol.tile_m = f16 ? f16_tile_m(rows) : o.quant_mma_tile == 64 ? 64u : kMmqBM;
            if (f16 && count == 1u && !o.quant_mma_splits && rows >= 256u)
                pol.tile_m = small_gemm_tile_m(pol.tile_m, rows, it.w->out_features, k / 256u, cus);
        }
        if (pol.path == PATH_GEMV_ROWS) {
            for (uint32_t r = 0; r < rows; r++)
                g->gemv_rows.push_back({it.x + (uint64_t)r * k, it.w, it.y + (uint64_t)r * it.w->out_features});
            continue;
        }
        const bool f16 = pol.path == PATH_MMQ_F16;
        item_kernel[i] = group_index(it.w->ggml_type, f16, pol.tile_m);
        size_t ai = 0;
        while (ai < g->acts.size() && g->acts[ai].x != it.x) ai++;
        if (ai == g->acts.size()) {
            GemmGroup::Act act;
            act.x = it.x;
            act.k = k;
            if (ext) act.ext = reinterpret_cast<const uint8_t*>(it.x);
            g->acts.push_back(act);
        } else if (g->acts[ai].k != k) {
            return fail(RFXQ_ERR_OTHER, "gemm group: one x used with in_features %u and %u", g->acts[ai].k, k);
        }
        item_act[i] = (uint32_t)ai;
        if (f16) g->acts[ai].need_h = true;
        else g->acts[ai].need_i8 = true;
    }
    for (auto& a : g->acts) {
        if (a.ext) {
            a.L = act_layout(rows, a.k);
            continue;
        }
        a.L = act_layout_sel(rows, a.k, a.need_i8, a.need_h);
        a.off = g->ws_bytes;
        g->ws_bytes += a.L.total;
    }
    for (uint32_t i = 0; i < count; i++) {
        if (item_act[i] == ~0u) continue;
        const rfxq_gemm_item& it = items[i];
        const uint32_t k = it.w->in_features, t = item_kernel[i];
        const GemmGroup::Act& a = g->acts[item_act[i]];
        MmqDesc d;
        std::memset(&d, 0, sizeof d);
        d.w = it.w->data;
        // offsets until the workspace is known
        act_desc(&d, reinterpret_cast<const uint8_t*>(a.off), a.L, group_f16(t), k);
        d.y = it.y;
        d.m = rows;
        d.n = it.w->out_features;
        d.k = k;
        d.type = it.w->ggml_type;
        d.ldy = d.n;
        const uint32_t bm = group_tile_m(t), bn = tile_bn(group_f16(t));
        d.tiles_m = (rows + bm - 1u) / bm;
        d.tiles_n = (d.n + bn - 1u) / bn;
        d.splits = 1;
        d.sb_per_split = k / 256u;
        d.wg_begin = g->wgs[t];
        g->wgs[t] += d.tiles_m * d.tiles_n;
        g->descs[t].push_back(d);
        g->act_of[t].push_back(item_act[i]);
    }
    // a kernel whose tiles would leave CUs idle splits K (fixed-order reduce);
    // REFLEX_QUANT_MMA_SPLITS sets the split count, as for single GEMMs
    const uint32_t forced = o.quant_mma_splits;
    bool split_small[kGroupKernels] = {};
    for (uint32_t t = 0; t < kGroupKernels; t++) {
        auto& v = g->descs[t];
        if (v.empty() || (!forced && 2u * g->wgs[t] >= cus)) continue;
        split_small[t] = true;
        // one split size for the launch, so its workgroups take alike
        std::vector<std::pair<uint32_t, uint32_t>> tn;
        for (const auto& d : v) tn.push_back({d.tiles_m * d.tiles_n, d.k / 256u});
        const uint32_t w_sb = split_sb(tn, group_tile_m(t) == 32u ? 1u : 2u, 2u * std::max(cus, 1u));
        uint32_t wg = 0;
        for (uint32_t i = 0; i < v.size(); i++) {
            MmqDesc& d = v[i];
            const uint32_t nsb = d.k / 256u;
            const uint32_t s = forced ? std::min(forced, nsb) : (nsb + w_sb - 1u) / w_sb;
            d.sb_per_split = (nsb + s - 1u) / s;
            d.splits = (nsb + d.sb_per_split - 1u) / d.sb_per_split;
            if (d.splits > 1u) {
                const uint64_t n = (uint64_t)rows * d.n;
                g->reduces.push_back({t, i, g->ws_bytes, d.y, nullptr, n, d.splits});
                g->ws_bytes += align256((uint64_t)d.splits * n * 4u);
            }
            d.wg_begin = wg;
            wg += d.tiles_m * d.tiles_n * d.splits;
        }
        g->wgs[t] = wg;
    }
    // A launch of many tiles with GEMMs of very different K (a Q8_0 layer's
    // down projection, K = 14336, among K = 4096 GEMMs): a GEMM whose tiles
    // run over 3x the launch's median super-blocks splits K to about the
    // median, and such a launch starts its longest tiles first, so that they
    // do not run alone at its end.
    for (uint32_t t = 0; t < kGroupKernels && !forced; t++) {
        auto& v = g->descs[t];
        if (v.size() < 2u || split_small[t]) continue;
        std::vector<std::pair<uint32_t, uint32_t>> by_sb;  // (super-blocks per tile, tiles)
        uint64_t all = 0;
        for (const auto& d : v) {
            by_sb.push_back({d.sb_per_split, d.tiles_m * d.tiles_n * d.splits});
            all += by_sb.back().second;
        }
        std::sort(by_sb.begin(), by_sb.end());
        uint64_t acc = 0;
        uint32_t med = by_sb.back().first;
        for (const auto& e : by_sb)
            if ((acc += e.second) * 2u >= all) {
                med = e.first;
                break;
            }
        bool changed = false;
        for (uint32_t i = 0; i < v.size(); i++) {
            MmqDesc& d = v[i];
            if (d.splits != 1u || d.sb_per_split <= 3u * med) continue;
            const uint32_t nsb = d.k / 256u, s = (nsb + med - 1u) / med;
            d.sb_per_split = (nsb + s - 1u) / s;
            d.splits = (nsb + d.sb_per_split - 1u) / d.sb_per_split;
            changed = true;
        }
        // longest tiles first (stable), descriptors and their activations
        // alike; a launch with no split keeps its order, which groups the
        // GEMMs that read one activation buffer
        if (!changed) continue;
        std::vector<uint32_t> ord(v.size());
        for (uint32_t i = 0; i < ord.size(); i++) ord[i] = i;
        std::stable_sort(ord.begin(), ord.end(),
                         [&](uint32_t a, uint32_t b) { return v[a].sb_per_split > v[b].sb_per_split; });
        std::vector<MmqDesc> nv;
        std::vector<uint32_t> na;
        for (uint32_t i : ord) {
            nv.push_back(v[i]);
            na.push_back(g->act_of[t][i]);
        }
        v.swap(nv);
        g->act_of[t].swap(na);
        uint32_t wg = 0;
        for (uint32_t i = 0; i < v.size(); i++) {
            MmqDesc& d = v[i];
            if (d.splits > 1u) {
                const uint64_t n = (uint64_t)rows * d.n;
                g->reduces.push_back({t, i, g->ws_bytes, d.y, nullptr, n, d.splits});
                g->ws_bytes += align256((uint64_t)d.splits * n * 4u);
            }
            d.wg_begin = wg;
            wg += d.tiles_m * d.tiles_n * d.splits;
        }
        g->wgs[t] = wg;
    }
    return RFXQ_OK;
}

// the MMQ launch of kernel t of a group (descriptors inline or from `table`)
int launch_group_kernel(Ctx* c, const GemmGroup& g, uint32_t t, const MmqDesc* table, hipStream_t stream) {
    const auto& v = g.descs[t];
    if (v.empty()) return RFXQ_OK;
    return launch_mmq(c, v[0].type, v.data(), (uint32_t)v.size(), table, g.wgs[t], false, stream, group_f16(t),
                      group_tile_m(t));
}

// the split-K reduces of kernel t
int run_group_reduces(Ctx* c, const GemmGroup& g, uint32_t t, hipStream_t stream) {
    // all of kernel t's reduces in launches of up to REDUCE_INLINE items
    ReduceArgs a;
    std::memset(&a, 0, sizeof a);
    uint32_t wg = 0;
    auto flush = [&]() -> int {
        if (a.count == 0) return RFXQ_OK;
        const int rc = launch(c->reduce_multi, wg, 0, stream, &a, sizeof a, "rfxq_splitk_reduce_multi launch");
        std::memset(&a, 0, sizeof a);
        wg = 0;
        return rc;
    };
    for (const auto& r : g.reduces) {
        if (r.t != t) continue;
        const uint32_t wgs = (uint32_t)std::min<uint64_t>((r.n + 255u) / 256u, 2048u);
        a.items[a.count++] = ReduceItem{r.part, r.y, (uint32_t)r.n, r.splits, wg, wgs};
        wg += wgs;
        if (a.count == REDUCE_INLINE)
            if (int rc = flush()) return rc;
    }
    return flush();
}

// workspace offsets -> addresses
void bind_gemm_group(GemmGroup* g, uint8_t* ws) {
    for (uint32_t t = 0; t < kGroupKernels; t++)
        for (size_t i = 0; i < g->descs[t].size(); i++) {
            MmqDesc& d = g->descs[t][i];
            const GemmGroup::Act& a = g->acts[g->act_of[t][i]];
            act_desc(&d, a.base(ws), a.L, group_f16(t), d.k);
        }
    for (auto& r : g->reduces) {
        r.part = reinterpret_cast<float*>(ws + r.off);
        g->descs[r.t][r.i].y = r.part;
    }
}

int run_gemm_quant(Ctx* c, const GemmGroup& g, uint8_t* ws, uint32_t rows, hipStream_t stream) {
    for (const auto& a : g.acts)
        if (!a.ext)
            if (int rc = launch_act(c, a.x, rows, a.k, ws + a.off, a.L, a.need_i8, a.need_h, stream)) return rc;
    return RFXQ_OK;
}

// ------------------------------------------------------------------ router (src/moe.rs:47-98)

int route_top_k(const float* logits, uint32_t n, uint32_t k, bool normalize, uint32_t* idx, float* w) {
    if (!logits || n == 0) return fail(RFXQ_ERR_OTHER, "route_top_k: logits must not be empty");
    if (k == 0 || k > n) return fail(RFXQ_ERR_OTHER, "route_top_k: k (%u) must be in 1..=%u (logits.len())", k, n);
    // probabilities on the stack up to kRouteStack experts (heap above)
    constexpr uint32_t kRouteStack = 1024;
    float stack_probs[kRouteStack];
    std::vector<float> heap_probs;
    float* probs = stack_probs;
    if (n > kRouteStack) {
        heap_probs.resize(n);
        probs = heap_probs.data();
    }
    float maxl = -INFINITY;
    for (uint32_t i = 0; i < n; i++) maxl = std::max(maxl, logits[i]);
    for (uint32_t i = 0; i < n; i++) probs[i] = std::exp(logits[i] - maxl);
    float sum = 0.0f;
    for (uint32_t i = 0; i < n; i++) sum += probs[i];
    if (!std::isfinite(sum) || sum <= 0.0f)
        return fail(RFXQ_ERR_OTHER, "route_top_k: softmax sum is non-finite or non-positive (%g)", (double)sum);
    for (uint32_t i = 0; i < n; i++) probs[i] = probs[i] / sum;
    // the k best in (probability descending, index ascending) order: the
    // first k of a stable sort, by insertion into a sorted list of k
    uint32_t stack_best[65];
    std::vector<uint32_t> heap_best;
    uint32_t* best = stack_best;
    if (k + 1u > 65u) {
        heap_best.resize(k + 1u);
        best = heap_best.data();
    }
    uint32_t nb = 0;
    for (uint32_t i = 0; i < n; i++) {
        const float p = probs[i];
        if (nb == k && !(p > probs[best[nb - 1u]])) continue;  // ties keep the lower index
        uint32_t pos = nb;
        while (pos > 0 && p > probs[best[pos - 1u]]) pos--;
        for (uint32_t q = nb; q > pos; q--) best[q] = best[q - 1u];
        best[pos] = i;
        if (nb < k) nb++;
    }
    float top_sum = 0.0f;
    for (uint32_t t = 0; t < k; t++) top_sum += probs[best[t]];
    if (normalize && (!std::isfinite(top_sum) || top_sum <= 0.0f))
        return fail(RFXQ_ERR_OTHER, "route_top_k: top-%u probability mass is non-finite or non-positive (%g)", k,
                    (double)top_sum);
    for (uint32_t t = 0; t < k; t++) {
        idx[t] = best[t];
        w[t] = normalize ? probs[best[t]] / top_sum : probs[best[t]];
    }
    return RFXQ_OK;
}

int expert_slice(const rfxq_weight* w, uint32_t e, rfxq_weight* out, const char* what) {
    if (!w || !out) return fail(RFXQ_ERR_INVALID_INPUT, "%s: NULL weight", what);
    if (w->expert_count == 0)
        return fail(RFXQ_ERR_OTHER, "%s: expected 3-D per-expert tensor shape, got [%u, %u]", what, w->in_features,
                    w->out_features);
    if (e >= w->expert_count || w->len % w->expert_count != 0)
        return fail(RFXQ_ERR_OTHER, "%s: expert %u of %u in a %llu-byte %s tensor", what, e, w->expert_count,
                    (unsigned long long)w->len, type_name(w->ggml_type));
    const uint64_t el = w->len / w->expert_count;
    *out = *w;
    out->expert_count = 0;
    out->data = static_cast<const uint8_t*>(w->data) + (uint64_t)e * el;
    out->len = el;
    return RFXQ_OK;
}

}  // namespace

// ====================================================================== C ABI

struct QuantDesc {  // rfxq_quantize_q8_1_multi
    const float* x;
    int8_t* xq;
    uint32_t* xds;
    uint32_t rows, k, wg_begin, wgs;
};
static_assert(sizeof(QuantDesc) == 40, "QuantDesc layout");
struct ActF16Desc {  // rfxq_act_f16_multi
    const float* x;
    uint16_t* xh;
    uint16_t* xsx;
    float* xrs;
    uint32_t rows, k, wg_begin, wgs;
};
static_assert(sizeof(ActF16Desc) == 48, "ActF16Desc layout");

struct rfxq_gemm_plan {
    int device;
    uint32_t rows;
    void* dev = nullptr;  // quantized activations, one descriptor table per weight type, the quantize table
    GemmGroup g;
    MmqDesc* table[kGroupKernels] = {};
    QuantDesc* qtable = nullptr;  // int8 layouts: one rfxq_quantize_q8_1_multi launch
    uint32_t nq = 0, qgrid = 0;
    ActF16Desc* htable = nullptr;  // f16 layouts: one rfxq_act_f16_multi launch
    uint32_t nh = 0, hgrid = 0;
    bool hwave = true;  // htable runs on rfxq_act_f16_multi (else _multi_wg)
    rfxq_gemv_plan* q8 = nullptr;  // GEMMs on the GEMV path, one item per row
};

struct rfxq_gemv_plan {
    int device;
    void* dev = nullptr;  // descriptor table, then the per-workgroup ranges
    GemvArgs args;
    uint32_t grid = 0, lds = 0;
};

extern "C" {

const char* rfxq_last_error(void) { return g_code == RFXQ_OK ? nullptr : g_err.c_str(); }

int rfxq_last_error_code(void) { return g_code; }

int rfxq_init(int device) {
    int n = 0;
    HIPCHK(hipGetDeviceCount(&n), "hipGetDeviceCount");
    if (device < 0 || device >= n) return fail(RFXQ_ERR_INVALID_INPUT, "rfxq_init: device %d of %d", device, n);
    int prev = 0;
    HIPCHK(hipGetDevice(&prev), "hipGetDevice");
    HIPCHK(hipSetDevice(device), "hipSetDevice");
    Ctx* c = nullptr;
    const int rc = load_ctx(device, &c);
    (void)hipSetDevice(prev);
    return rc ? rc : ok();
}

int rfxq_get_options(rfxq_options* out) {
    if (!out) return fail(RFXQ_ERR_INVALID_INPUT, "rfxq_get_options: NULL output");
    if (int rc = get_options(out)) return rc;
    return ok();
}

int rfxq_set_options(const rfxq_options* o) {
    if (!o) return fail(RFXQ_ERR_INVALID_INPUT, "rfxq_set_options: NULL options");
    if (int rc = check_options(*o)) return rc;
    std::lock_guard<std::mutex> lk(g_opt_mu);
    Options& O = options_locked();
    O.o = *o;
    O.code = RFXQ_OK;
    O.msg.clear();
    return ok();
}

int rfxq_gemm_policy_for(uint32_t ty, uint32_t k, uint32_t n, uint32_t rows, uint32_t cus, rfxq_gemm_policy* out) {
    if (!out) return fail(RFXQ_ERR_INVALID_INPUT, "rfxq_gemm_policy_for: NULL output");
    uint32_t qk = 0, bb = 0;
    if (!block_dims(ty, &qk, &bb) || !(ty == RFXQ_TYPE_Q4_K || ty == RFXQ_TYPE_Q6_K || ty == RFXQ_TYPE_Q8_0))
        return fail(RFXQ_ERR_GGUF, "rfxq_gemm_policy_for: ggml_type=%u has no GEMM", ty);
    if (k == 0 || n == 0 || rows == 0 || cus == 0)
        return fail(RFXQ_ERR_INVALID_INPUT, "rfxq_gemm_policy_for: zero dimension");
    rfxq_options o;
    if (int rc = get_options(&o)) return rc;
    *out = gemm_policy(ty, k, n, rows, cus, o);
    return ok();
}

int rfxq_block_dims(uint32_t ty, uint32_t* qk, uint32_t* bb) {
    if (!qk || !bb) return fail(RFXQ_ERR_INVALID_INPUT, "rfxq_block_dims: NULL output");
    if (!block_dims(ty, qk, bb))
        return fail(RFXQ_ERR_GGUF, "unknown ggml_type=%u: on-disk block size not known to this library", ty);
    return ok();
}

int rfxq_dequantize(uint32_t ty, const void* blocks, uint64_t num_blocks, void* y, int f16_out, hipStream_t stream) {
    if (!is_kernel_type(ty)) return fail(RFXQ_ERR_GGUF, "dequantize: no device dequantizer for ggml_type=%u", ty);
    if (num_blocks == 0) return ok();
    if (!blocks || !y) return fail(RFXQ_ERR_INVALID_INPUT, "dequantize: NULL pointer");
    if (num_blocks > 0xFFFFFFFFull) return fail(RFXQ_ERR_OTHER, "dequantize: too many blocks");
    if (reinterpret_cast<uintptr_t>(blocks) % 2u) return fail(RFXQ_ERR_OTHER, "dequantize: blocks not 2-byte aligned");
    Ctx* c;
    if (int rc = current_ctx(&c)) return rc;
    const uint64_t groups = ty == RFXQ_TYPE_Q8_0 ? (num_blocks + 7u) / 8u : num_blocks;
    const uint32_t grid = (uint32_t)std::min<uint64_t>(groups, 16384u);
    struct {
        const void* b;
        void* y;
        uint32_t n, pad;
    } a = {blocks, y, (uint32_t)num_blocks, 0};
    if (int rc = launch(c->deq[type_index(ty)][f16_out ? 1 : 0], grid, 0, stream, &a, sizeof a, "dequantize launch"))
        return rc;
    return ok();
}

int rfxq_gemv_to(const float* x, uint64_t x_len, const rfxq_weight* w, float* y, hipStream_t stream) {
    if (int rc = check_weight(w, "gemv_to")) return rc;
    if (x_len != w->in_features)
        return fail(RFXQ_ERR_OTHER, "gemv_to: x.len()=%llu != in_features=%u", (unsigned long long)x_len,
                    w->in_features);
    Ctx* c;
    if (int rc = current_ctx(&c)) return rc;
    rfxq_gemv_item it = {x, w, y};
    if (int rc = gemv_items(c, &it, 1, stream)) return rc;
    return ok();
}

int rfxq_gemv_rows(const float* x, uint64_t x_len, const rfxq_weight* w, uint32_t rows, float* y,
                   hipStream_t stream) {
    if (int rc = check_weight(w, "gemv_rows")) return rc;
    if (rows == 0 || x_len != (uint64_t)rows * w->in_features)
        return fail(RFXQ_ERR_OTHER, "gemv_rows: x.len()=%llu rows=%u in_features=%u (must be rows*in_features)",
                    (unsigned long long)x_len, rows, w->in_features);
    Ctx* c;
    if (int rc = current_ctx(&c)) return rc;
    std::vector<rfxq_gemv_item> items(rows);
    for (uint32_t r = 0; r < rows; r++)
        items[r] = {x + (uint64_t)r * w->in_features, w, y + (uint64_t)r * w->out_features};
    if (int rc = gemv_items(c, items.data(), rows, stream)) return rc;
    return ok();
}

int rfxq_gemv_gather(const float* x, uint64_t x_len, const rfxq_weight* w, const uint32_t* row_indices,
                     uint32_t count, float* y, hipStream_t stream) {
    if (int rc = check_weight(w, "gemv_gather")) return rc;
    if (x_len != w->in_features)
        return fail(RFXQ_ERR_OTHER, "gemv_gather: x.len()=%llu != in_features=%u", (unsigned long long)x_len,
                    w->in_features);
    if (count == 0 || !row_indices) return fail(RFXQ_ERR_OTHER, "gemv_gather: row_indices must not be empty");
    for (uint32_t j = 0; j < count; j++)
        if (row_indices[j] >= w->out_features)
            return fail(RFXQ_ERR_OTHER, "gemv_gather: row index %u out of range (out_features=%u)", row_indices[j],
                        w->out_features);
    Ctx* c;
    if (int rc = current_ctx(&c)) return rc;
    // each run of consecutive indices is one GEMV over that row slice of W
    // (rows are whole blocks, so a slice keeps the format's alignment)
    const uint64_t rb = row_bytes(w->ggml_type, w->in_features);
    std::vector<GemvItem> v;
    for (uint32_t i = 0; i < count;) {
        uint32_t j = i + 1u;
        while (j < count && row_indices[j] == row_indices[j - 1u] + 1u) j++;
        rfxq_weight slice = *w;
        slice.out_features = j - i;
        slice.data = static_cast<const uint8_t*>(w->data) + (uint64_t)row_indices[i] * rb;
        slice.len = (uint64_t)(j - i) * rb;
        GemvItem it;
        if (int rc = make_gemv_item(x, &slice, y + i, &it)) return rc;
        v.push_back(it);
        i = j;
    }
    int rc = v.size() <= kGemvInline ? gemv_launch_inline(c, v, stream) : gemv_launch_table(c, v, 0, stream);
    return rc ? rc : ok();
}

int rfxq_gemv_batch(const rfxq_gemv_item* items, uint32_t count, hipStream_t stream) {
    if (count == 0) return ok();
    if (!items) return fail(RFXQ_ERR_INVALID_INPUT, "gemv_batch: items is NULL");
    Ctx* c;
    if (int rc = current_ctx(&c)) return rc;
    // validate everything before launching anything
    for (uint32_t i = 0; i < count; i++) {
        GemvItem it;
        if (int rc = make_gemv_item(items[i].x, items[i].w, items[i].y, &it)) return rc;
    }
    if (int rc = gemv_items(c, items, count, stream)) return rc;
    return ok();
}

int rfxq_gemv_plan_create(const rfxq_gemv_item* items, uint32_t count, int device, rfxq_gemv_plan** out) {
    if (!out || !items || count == 0) return fail(RFXQ_ERR_INVALID_INPUT, "gemv_plan_create: empty plan");
    *out = nullptr;
    int prev = 0;
    HIPCHK(hipGetDevice(&prev), "hipGetDevice");
    HIPCHK(hipSetDevice(device), "hipSetDevice");
    Ctx* c = nullptr;
    int rc = load_ctx(device, &c);
    auto plan = std::make_unique<rfxq_gemv_plan>();
    plan->device = device;
    std::vector<GemvItem> v(count);
    for (uint32_t i = 0; rc == RFXQ_OK && i < count; i++) rc = make_gemv_item(items[i].x, items[i].w, items[i].y, &v[i]);
    std::vector<GemvRange> ranges;
    std::vector<uint32_t> max_iters;
    if (rc == RFXQ_OK) {
        plan->grid = gemv_grid(c, v);
        gemv_split_bytes(v, plan->grid, &ranges, &max_iters);
        std::memset(&plan->args, 0, sizeof plan->args);
        plan->args.ndesc = count;
        rc = gemv_lds(v, max_iters, &plan->args.part_floats, &plan->lds);
    }
    if (rc == RFXQ_OK) {
        const size_t tb = sizeof(GemvDesc) * count, rbytes = sizeof(GemvRange) * ranges.size();
        std::vector<uint8_t> host(tb + rbytes);
        for (uint32_t i = 0; i < count; i++) std::memcpy(host.data() + i * sizeof(GemvDesc), &v[i].d, sizeof(GemvDesc));
        std::memcpy(host.data() + tb, ranges.data(), rbytes);
        hipError_t e = hipMalloc(&plan->dev, host.size());
        if (e != hipSuccess) rc = fail(RFXQ_ERR_OUT_OF_MEMORY, "gemv_plan_create: %s", hipGetErrorString(e));
        else {
            e = hipMemcpy(plan->dev, host.data(), host.size(), hipMemcpyHostToDevice);
            if (e != hipSuccess) rc = fail(RFXQ_ERR_GPU, "gemv_plan_create upload: %s", hipGetErrorString(e));
        }
        plan->args.table = static_cast<const GemvDesc*>(plan->dev);
        plan->args.ranges = reinterpret_cast<const GemvRange*>(static_cast<const uint8_t*>(plan->dev) + tb);
        if (count <= kGemvInline)
            for (uint32_t i = 0; i < count; i++) plan->args.inl[i] = v[i].d;
    }
    (void)hipSetDevice(prev);
    if (rc != RFXQ_OK) {
        if (plan->dev) (void)hipFree(plan->dev);
        return rc;
    }
    *out = plan.release();
    return ok();
}

int rfxq_gemv_plan_run(const rfxq_gemv_plan* plan, hipStream_t stream) {
    if (!plan) return fail(RFXQ_ERR_INVALID_INPUT, "gemv_plan_run: NULL plan");
    Ctx* c;
    if (int rc = load_ctx(plan->device, &c)) return rc;
    GemvArgs a = plan->args;
    if (int rc = launch(c->gemv, plan->grid, plan->lds, stream, &a, sizeof a, "rfxq_gemv launch")) return rc;
    return ok();
}

void rfxq_gemv_plan_destroy(rfxq_gemv_plan* plan) {
    if (!plan) return;
    if (plan->dev) (void)hipFree(plan->dev);
    delete plan;
}

int rfxq_quantize_q8_1(const float* x, uint32_t rows, uint32_t k, int8_t* xq, uint32_t* xds, hipStream_t stream) {
    if (rows == 0) return ok();
    if (!x || !xq || !xds) return fail(RFXQ_ERR_INVALID_INPUT, "quantize_q8_1: NULL pointer");
    if (k == 0 || k % 32u) return fail(RFXQ_ERR_OTHER, "quantize_q8_1: k=%u (must be a multiple of 32)", k);
    if (reinterpret_cast<uintptr_t>(x) % 16u || reinterpret_cast<uintptr_t>(xq) % 4u ||
        reinterpret_cast<uintptr_t>(xds) % 4u)
        return fail(RFXQ_ERR_OTHER, "quantize_q8_1: x must be 16-byte and xq/xds 4-byte aligned");
    Ctx* c;
    if (int rc = current_ctx(&c)) return rc;
    if (int rc = launch_quant(c, x, k, nullptr, rows, k, xq, xds, stream)) return rc;
    return ok();
}

uint64_t rfxq_gemm_workspace_size(const rfxq_weight* w, uint32_t rows) {
    if (!w || rows == 0) return 0;
    Ctx* c = nullptr;
    int dev = 0;
    if (hipGetDevice(&dev) == hipSuccess) {
        std::lock_guard<std::mutex> lk(g_mu);
        auto it = g_ctx.find(dev);
        if (it != g_ctx.end()) c = it->second.get();
    }
    if (!options_ok()) return 0;
    const GemmPlan p = plan_gemm(c, w, rows, opt());
    return p.pol.path == PATH_GEMV_ROWS ? 0 : p.total;
}

int rfxq_gemm(const float* x, uint64_t x_len, const rfxq_weight* w, uint32_t rows, float* y, void* workspace,
              uint64_t workspace_bytes, hipStream_t stream) {
    if (int rc = check_weight(w, "gemm")) return rc;
    if (rows == 0 || x_len != (uint64_t)rows * w->in_features)
        return fail(RFXQ_ERR_OTHER, "gemm: x.len()=%llu != rows*in_features=%llu", (unsigned long long)x_len,
                    (unsigned long long)rows * w->in_features);
    if (!x || !y) return fail(RFXQ_ERR_INVALID_INPUT, "gemm: x or y is NULL");
    if (rows == 1) return rfxq_gemv_to(x, x_len, w, y, stream);
    rfxq_options o;
    if (int rc = get_options(&o)) return rc;
    if (gemm_policy(w->ggml_type, w->in_features, w->out_features, rows, 256u, o).path == PATH_GEMV_ROWS)
        return rfxq_gemv_rows(x, x_len, w, rows, y, stream);
    if (int rc = check_mmq_weight(w, "gemm")) return rc;
    if (reinterpret_cast<uintptr_t>(x) % 16u) return fail(RFXQ_ERR_OTHER, "gemm: x is not 16-byte aligned");
    Ctx* c;
    if (int rc = current_ctx(&c)) return rc;
    if (int rc = gemm_impl(c, x, w, rows, y, workspace, workspace_bytes, o, stream)) return rc;
    return ok();
}

int rfxq_gemm_no_alloc(const float* x, uint64_t x_len, const rfxq_weight* w, uint32_t rows, float* y,
                       hipStream_t stream) {
    if (int rc = check_weight(w, "gemm_no_alloc")) return rc;
    if (rows == 0 || x_len != (uint64_t)rows * w->in_features)
        return fail(RFXQ_ERR_OTHER, "gemm_no_alloc: x.len()=%llu != rows*in_features=%llu", (unsigned long long)x_len,
                    (unsigned long long)rows * w->in_features);
    if (!x || !y) return fail(RFXQ_ERR_INVALID_INPUT, "gemm_no_alloc: x or y is NULL");
    // the device's context and scratch exist already (rfxq_init): loading them would allocate
    int dev = 0;
    HIPCHK(hipGetDevice(&dev), "hipGetDevice");
    Ctx* c = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        auto it = g_ctx.find(dev);
        if (it != g_ctx.end()) c = it->second.get();
    }
    if (!c)
        return fail(RFXQ_ERR_INVALID_INPUT, "gemm_no_alloc: device %d is not initialised; call rfxq_init(%d) first",
                    dev, dev);
    if (!c->scratch)
        return fail(RFXQ_ERR_GPU, "gemm_no_alloc: the fixed scratch array of device %d is unavailable: %s", dev,
                    hipGetErrorString(c->scratch_err));
    rfxq_options o;
    if (int rc = get_options(&o)) return rc;
    if (rows == 1 ||
        gemm_policy(w->ggml_type, w->in_features, w->out_features, rows, 256u, o).path == PATH_GEMV_ROWS) {
        // rfxq_gemv_to / rfxq_gemv_rows: one GEMV per row, launched with inline
        // descriptors (no descriptor table to upload); per-row results do not
        // depend on how rows group into launches
        for (uint32_t r0 = 0; r0 < rows; r0 += kGemvInline) {
            const uint32_t cnt = std::min<uint32_t>(kGemvInline, rows - r0);
            GemvItem v[kGemvInline];
            for (uint32_t j = 0; j < cnt; j++)
                if (int rc = make_gemv_item(x + (uint64_t)(r0 + j) * w->in_features, w,
                                            y + (uint64_t)(r0 + j) * w->out_features, &v[j]))
                    return rc;
            if (int rc = gemv_launch_counted(c, v, cnt, nullptr, stream)) return rc;
        }
        return ok();
    }
    if (int rc = check_mmq_weight(w, "gemm_no_alloc")) return rc;
    if (reinterpret_cast<uintptr_t>(x) % 16u) return fail(RFXQ_ERR_OTHER, "gemm_no_alloc: x is not 16-byte aligned");
    const GemmPlan p = plan_gemm(c, w, rows, o);
    if (p.total > rfxq_scratch::kScratchBytes)
        return fail(RFXQ_ERR_INVALID_INPUT,
                    "gemm_no_alloc: rows=%u in_features=%u out_features=%u needs %llu bytes of scratch; the fixed "
                    "scratch holds %llu (use rfxq_gemm with a workspace)",
                    rows, w->in_features, w->out_features, (unsigned long long)p.total,
                    (unsigned long long)rfxq_scratch::kScratchBytes);
    if (int rc = gemm_impl(c, x, w, rows, y, c->scratch, rfxq_scratch::kScratchBytes, o, stream)) return rc;
    return ok();
}

int rfxq_gemm_batch(const rfxq_gemm_item* items, uint32_t count, uint32_t rows, hipStream_t stream) {
    if (count == 0) return ok();
    Ctx* c;
    if (int rc = current_ctx(&c)) return rc;
    GemmGroup g;
    if (int rc = build_gemm_group(items, count, rows, &g, (uint32_t)c->cus)) return rc;
    void* ws = nullptr;
    if (int rc = ctx_workspace(c, g.ws_bytes, &ws, stream)) return rc;
    bind_gemm_group(&g, static_cast<uint8_t*>(ws));
    if (int rc = run_gemm_quant(c, g, static_cast<uint8_t*>(ws), rows, stream)) return rc;
    // descriptors inline, kMmqInline per launch
    for (uint32_t t = 0; t < kGroupKernels; t++) {
        auto& v = g.descs[t];
        for (size_t i0 = 0; i0 < v.size(); i0 += kMmqInline) {
            const uint32_t cnt = (uint32_t)std::min<size_t>(kMmqInline, v.size() - i0);
            MmqDesc d[kMmqInline];
            uint32_t wg = 0;
            for (uint32_t j = 0; j < cnt; j++) {
                d[j] = v[i0 + j];
                d[j].wg_begin = wg;
                wg += d[j].tiles_m * d[j].tiles_n * d[j].splits;
            }
            if (int rc = launch_mmq(c, d[0].type, d, cnt, nullptr, wg, false, stream, group_f16(t), group_tile_m(t)))
                return rc;
        }
        if (int rc = run_group_reduces(c, g, t, stream)) return rc;
    }
    if (!g.gemv_rows.empty())
        if (int rc = gemv_items(c, g.gemv_rows.data(), (uint32_t)g.gemv_rows.size(), stream)) return rc;
    return ok();
}

uint64_t rfxq_act_q8_1_size(uint32_t rows, uint32_t k) {
    return rows && k && k % 256u == 0 ? act_layout(rows, k).total : 0;
}

int rfxq_quantize_act_q8_1(const float* x, uint32_t rows, uint32_t k, void* act, hipStream_t stream) {
    if (int rc = check_act(act, rows, k, "quantize_act_q8_1")) return rc;
    if (!x || reinterpret_cast<uintptr_t>(x) % 16u)
        return fail(RFXQ_ERR_OTHER, "quantize_act_q8_1: x is NULL or not 16-byte aligned");
    Ctx* c;
    if (int rc = current_ctx(&c)) return rc;
    if (int rc = launch_act(c, x, rows, k, static_cast<uint8_t*>(act), act_layout(rows, k), true, true, stream))
        return rc;
    return ok();
}

int rfxq_rmsnorm_q8_1(const float* x, const float* weight, uint32_t rows, uint32_t k, float eps, void* act, float* y,
                      hipStream_t stream) {
    if (int rc = check_act(act, rows, k, "rmsnorm_q8_1")) return rc;
    if (!x || !weight || reinterpret_cast<uintptr_t>(x) % 16u || reinterpret_cast<uintptr_t>(weight) % 16u ||
        reinterpret_cast<uintptr_t>(y) % 16u)
        return fail(RFXQ_ERR_OTHER, "rmsnorm_q8_1: x and weight must be non-NULL, x, weight and y 16-byte aligned");
    Ctx* c;
    if (int rc = current_ctx(&c)) return rc;
    const ActLayout L = act_layout(rows, k);
    uint8_t* b = static_cast<uint8_t*>(act);
    struct {
        const float* x;
        const float* g;
        uint32_t rows, k;
        float eps;
        uint32_t pad;
        int8_t* xq;
        uint32_t* xds;
        uint16_t* xh;
        uint16_t* xsx;
        float* xrs;
        float* y;
    } a = {x, weight, rows, k, eps, 0, reinterpret_cast<int8_t*>(b + L.xq), reinterpret_cast<uint32_t*>(b + L.xds),
           reinterpret_cast<uint16_t*>(b + L.xh), reinterpret_cast<uint16_t*>(b + L.xsx),
           reinterpret_cast<float*>(b + L.xrs), y};
    const uint32_t grid = (rows + kNormRowsPerWg - 1u) / kNormRowsPerWg;
    if (int rc = launch(c->rms_q, grid, 0, stream, &a, sizeof a, "rfxq_rmsnorm_q8_1 launch")) return rc;
    return ok();
}

int rfxq_silu_and_mul_q8_1(const float* gate, const float* up, uint32_t rows, uint32_t k, void* act, float* y,
                           hipStream_t stream) {
    if (int rc = check_act(act, rows, k, "silu_and_mul_q8_1")) return rc;
    if (!gate || !up || reinterpret_cast<uintptr_t>(gate) % 16u || reinterpret_cast<uintptr_t>(up) % 16u ||
        reinterpret_cast<uintptr_t>(y) % 16u)
        return fail(RFXQ_ERR_OTHER, "silu_and_mul_q8_1: gate and up must be non-NULL, gate, up and y 16-byte aligned");
    Ctx* c;
    if (int rc = current_ctx(&c)) return rc;
    const ActLayout L = act_layout(rows, k);
    uint8_t* b = static_cast<uint8_t*>(act);
    struct {
        const float* gate;
        const float* up;
        uint32_t rows, k;
        int8_t* xq;
        uint32_t* xds;
        uint16_t* xh;
        uint16_t* xsx;
        float* xrs;
        float* y;
    } a = {gate, up, rows, k, reinterpret_cast<int8_t*>(b + L.xq), reinterpret_cast<uint32_t*>(b + L.xds),
           reinterpret_cast<uint16_t*>(b + L.xh), reinterpret_cast<uint16_t*>(b + L.xsx),
           reinterpret_cast<float*>(b + L.xrs), y};
    if (int rc = launch(c->silu_q, quant_grid((uint64_t)rows * (k / 32u)), 0, stream, &a, sizeof a,
                        "rfxq_silu_and_mul_q8_1 launch"))
        return rc;
    return ok();
}

int rfxq_gemm_q8_1(const void* act, uint32_t rows, const rfxq_weight* w, float* y, void* workspace,
                   uint64_t workspace_bytes, hipStream_t stream) {
    if (int rc = check_mmq_weight(w, "gemm_q8_1")) return rc;
    const uint32_t k = w->in_features, n = w->out_features;
    if (int rc = check_act(act, rows, k, "gemm_q8_1")) return rc;
    if (!y) return fail(RFXQ_ERR_INVALID_INPUT, "gemm_q8_1: y is NULL");
    Ctx* c;
    if (int rc = current_ctx(&c)) return rc;
    rfxq_options o;
    if (int rc = get_options(&o)) return rc;
    if (gemm_policy(w->ggml_type, k, n, rows, (uint32_t)c->cus, o).path == PATH_GEMV_ROWS) {
        // a buffer holds no f32 copy for GEMVs: its few rows run on the MMQ kernel
        o.fused_max_rows = 0;
        o.quant_mma = 1;
        o.quant_mma_max_rows = 0;
    }
    // one row plans as two (same tiles): the policy sends single rows to the GEMV
    const GemmPlan p = plan_gemm(c, w, std::max(rows, 2u), o);
    float* part = nullptr;
    if (p.pol.splits > 1) {
        const uint64_t need = (uint64_t)p.pol.splits * rows * n * 4u;
        void* ws = workspace;
        if (!ws) {
            if (int rc = ctx_workspace(c, need, &ws, stream)) return rc;
        } else if (workspace_bytes < need) {
            return fail(RFXQ_ERR_INVALID_INPUT, "gemm_q8_1: workspace of %llu bytes, needs %llu",
                        (unsigned long long)workspace_bytes, (unsigned long long)need);
        }
        part = static_cast<float*>(ws);
    }
    if (int rc = gemm_run(c, p, static_cast<const uint8_t*>(act), act_layout(rows, k), w, rows, y, part, stream))
        return rc;
    return ok();
}

// the fused form of rfxq_gemm_gate_up_silu_q8_1: Q4_K gate / up on the f16 kernels
static bool gate_up_pair_ok(const rfxq_weight* gate, const rfxq_options& o) {
    return o.mmq_f16 && gate->ggml_type == RFXQ_TYPE_Q4_K && f16_capable(gate->ggml_type, gate->in_features, 0);
}

uint64_t rfxq_gemm_gate_up_silu_workspace_size(const rfxq_weight* gate, uint32_t rows) {
    if (!gate || rows == 0 || !options_ok()) return 0;
    if (gate_up_pair_ok(gate, opt())) return 0;
    // the gate and up GEMMs' outputs, then their split-K partials
    return 2u * align256((uint64_t)rows * gate->out_features * 4u) + rfxq_gemm_workspace_size(gate, std::max(rows, 2u));
}

int rfxq_gemm_gate_up_silu_q8_1(const void* act, uint32_t rows, const rfxq_weight* gate, const rfxq_weight* up,
                                void* act_out, float* y, void* workspace, uint64_t workspace_bytes,
                                hipStream_t stream) {
    if (int rc = check_mmq_weight(gate, "gemm_gate_up_silu_q8_1 gate")) return rc;
    if (int rc = check_mmq_weight(up, "gemm_gate_up_silu_q8_1 up")) return rc;
    if (gate->ggml_type != up->ggml_type || gate->in_features != up->in_features ||
        gate->out_features != up->out_features || gate->len != up->len)
        return fail(RFXQ_ERR_OTHER, "gemm_gate_up_silu_q8_1: gate and up must share a type and shape");
    const uint32_t k = gate->in_features, ffn = gate->out_features;
    if (int rc = check_act(act, rows, k, "gemm_gate_up_silu_q8_1")) return rc;
    if (int rc = check_act(act_out, rows, ffn, "gemm_gate_up_silu_q8_1 act_out")) return rc;
    if (!y || reinterpret_cast<uintptr_t>(y) % 16u)
        return fail(RFXQ_ERR_INVALID_INPUT, "gemm_gate_up_silu_q8_1: y is NULL or not 16-byte aligned");
    Ctx* c;
    if (int rc = current_ctx(&c)) return rc;
    rfxq_options o;
    if (int rc = get_options(&o)) return rc;
    if (gate_up_pair_ok(gate, o)) {
        // one launch of pair tiles (128 columns: gate in waves 0-1, up in 2-3,
        // silu(gate) * up stored), never split along K
        MmqDesc d;
        std::memset(&d, 0, sizeof d);
        d.w = gate->data;
        d.w_up = static_cast<const uint8_t*>(up->data);
        act_desc(&d, static_cast<const uint8_t*>(act), act_layout(rows, k), true, k);
        d.y = y;
        d.m = rows;
        d.n = ffn;
        d.k = k;
        d.type = gate->ggml_type;
        d.ldy = ffn;
        const uint32_t tile_m = f16_tile_m(rows);
        d.tiles_m = (rows + tile_m - 1u) / tile_m;
        d.tiles_n = (ffn + mmqh_pair_bn - 1u) / mmqh_pair_bn;
        d.splits = 1;
        d.sb_per_split = k / 256u;
        d.gu_pair = 1;
        if (int rc = launch_mmq(c, d.type, &d, 1, nullptr, d.tiles_m * d.tiles_n, false, stream, true, tile_m))
            return rc;
        return rfxq_quantize_act_q8_1(y, rows, ffn, act_out, stream);
    }
    // separate GEMMs into the workspace, then SiLU·up into y and act_out
    // (not in place: rfxq_silu_and_mul_q8_1 reads its inputs once per layout)
    const uint64_t u_bytes = align256((uint64_t)rows * ffn * 4u);
    const uint64_t need = rfxq_gemm_gate_up_silu_workspace_size(gate, rows);
    void* ws = workspace;
    if (!ws) {
        if (int rc = ctx_workspace(c, need, &ws, stream)) return rc;
    } else if (workspace_bytes < need) {
        return fail(RFXQ_ERR_INVALID_INPUT, "gemm_gate_up_silu_q8_1: workspace of %llu bytes, needs %llu",
                    (unsigned long long)workspace_bytes, (unsigned long long)need);
    }
    uint8_t* wb = static_cast<uint8_t*>(ws);
    float* g = reinterpret_cast<float*>(wb);
    float* u = reinterpret_cast<float*>(wb + u_bytes);
    uint8_t* part = wb + 2u * u_bytes;
    if (int rc = rfxq_gemm_q8_1(act, rows, gate, g, part, need - 2u * u_bytes, stream)) return rc;
    if (int rc = rfxq_gemm_q8_1(act, rows, up, u, part, need - 2u * u_bytes, stream)) return rc;
    return rfxq_silu_and_mul_q8_1(g, u, rows, ffn, act_out, y, stream);
}

int rfxq_gemm_q8_1_batch(const rfxq_gemm_q8_1_item* items, uint32_t count, uint32_t rows, hipStream_t stream) {
    if (count == 0) return ok();
    if (!items) return fail(RFXQ_ERR_INVALID_INPUT, "gemm_q8_1_batch: items is NULL");
    rfxq_options o;
    if (int rc = get_options(&o)) return rc;
    for (uint32_t i = 0; i < count; i++) {
        const rfxq_gemm_q8_1_item& it = items[i];
        if (int rc = check_mmq_weight(it.w, "gemm_q8_1_batch")) return rc;
        if (int rc = check_act(it.act, rows, it.w->in_features, "gemm_q8_1_batch")) return rc;
        if (!it.y) return fail(RFXQ_ERR_INVALID_INPUT, "gemm_q8_1_batch: item %u has a NULL y", i);
    }
    Ctx* c;
    if (int rc = current_ctx(&c)) return rc;
    // a buffer holds both layouts: f16 kernels where the weight allows them, else int8
    std::vector<MmqDesc> descs[kGroupKernels];
    for (uint32_t i = 0; i < count; i++) {
        const rfxq_gemm_q8_1_item& it = items[i];
        const uint32_t k = it.w->in_features;
        const bool f16 = o.mmq_f16 && f16_capable(it.w->ggml_type, k, 0);
        const uint32_t tile_m = f16 ? (rows <= 32u ? 32u : kMmqBM) : o.quant_mma_tile == 64u ? 64u : kMmqBM;
        const uint32_t t = group_index(it.w->ggml_type, f16, tile_m);
        MmqDesc d;
        std::memset(&d, 0, sizeof d);
        d.w = it.w->data;
        act_desc(&d, static_cast<const uint8_t*>(it.act), act_layout(rows, k), f16, k);
        d.y = it.y;
        d.m = rows;
        d.n = it.w->out_features;
        d.k = k;
        d.type = it.w->ggml_type;
        d.ldy = d.n;
        const uint32_t bm = tile_m, bn = tile_bn(f16);
        d.tiles_m = (rows + bm - 1u) / bm;
        d.tiles_n = (d.n + bn - 1u) / bn;
        d.splits = 1;
        d.sb_per_split = k / 256u;
        descs[t].push_back(d);
    }
    for (uint32_t t = 0; t < kGroupKernels; t++) {
        auto& v = descs[t];
        for (size_t i0 = 0; i0 < v.size(); i0 += kMmqInline) {
            const uint32_t cnt = (uint32_t)std::min<size_t>(kMmqInline, v.size() - i0);
            MmqDesc d[kMmqInline];
            uint32_t wg = 0;
            for (uint32_t j = 0; j < cnt; j++) {
                d[j] = v[i0 + j];
                d[j].wg_begin = wg;
                wg += d[j].tiles_m * d[j].tiles_n;
            }
            if (int rc = launch_mmq(c, d[0].type, d, cnt, nullptr, wg, false, stream, group_f16(t), group_tile_m(t)))
                return rc;
        }
    }
    return ok();
}

static int gemm_plan_create(const rfxq_gemm_item* items, uint32_t count, uint32_t rows, int device,
                            rfxq_gemm_plan** out, bool ext) {
    if (!out) return fail(RFXQ_ERR_INVALID_INPUT, "gemm_plan_create: out is NULL");
    *out = nullptr;
    int prev = 0;
    HIPCHK(hipGetDevice(&prev), "hipGetDevice");
    HIPCHK(hipSetDevice(device), "hipSetDevice");
    Ctx* c = nullptr;
    int rc = load_ctx(device, &c);
    auto plan = std::make_unique<rfxq_gemm_plan>();
    plan->device = device;
    plan->rows = rows;
    if (rc == RFXQ_OK) rc = build_gemm_group(items, count, rows, &plan->g, (uint32_t)c->cus, ext);
    uint64_t tables = 0;
    if (rc == RFXQ_OK) {
        tables = align256(plan->g.acts.size() * sizeof(QuantDesc)) + align256(plan->g.acts.size() * sizeof(ActF16Desc));
        for (const auto& v : plan->g.descs) tables += align256(v.size() * sizeof(MmqDesc));
        hipError_t e = hipMalloc(&plan->dev, std::max<uint64_t>(1u, plan->g.ws_bytes + tables));
        if (e != hipSuccess) rc = fail(RFXQ_ERR_OUT_OF_MEMORY, "gemm_plan_create: %s", hipGetErrorString(e));
    }
    if (rc == RFXQ_OK) {
        uint8_t* base = static_cast<uint8_t*>(plan->dev);
        bind_gemm_group(&plan->g, base);
        uint64_t off = plan->g.ws_bytes;
        for (uint32_t t = 0; t < kGroupKernels && rc == RFXQ_OK; t++) {
            const auto& v = plan->g.descs[t];
            plan->table[t] = reinterpret_cast<MmqDesc*>(base + off);
            if (!v.empty()) {
                hipError_t e = hipMemcpy(plan->table[t], v.data(), v.size() * sizeof(MmqDesc), hipMemcpyHostToDevice);
                if (e != hipSuccess) rc = fail(RFXQ_ERR_GPU, "gemm_plan_create upload: %s", hipGetErrorString(e));
            }
            off += align256(v.size() * sizeof(MmqDesc));
        }
        // one launch per layout kind for all activations
        std::vector<QuantDesc> q;
        std::vector<ActF16Desc> hq;
        plan->hwave = true;  // one kernel for all f16 layouts: row per wave only if every activation allows it
        for (const auto& a : plan->g.acts)
            if (!a.ext && a.need_h && !act_f16_wave(rows, a.k)) plan->hwave = false;
        for (const auto& a : plan->g.acts) {
            if (a.ext) continue;
            uint8_t* ab = base + a.off;
            if (a.need_i8) {
                const uint32_t wgs = quant_grid((uint64_t)rows * (a.k / 32u));
                q.push_back(QuantDesc{a.x, reinterpret_cast<int8_t*>(ab + a.L.xq),
                                      reinterpret_cast<uint32_t*>(ab + a.L.xds), rows, a.k, plan->qgrid, wgs});
                plan->qgrid += wgs;
            }
            if (a.need_h) {
                const uint32_t wgs = act_f16_grid(rows, plan->hwave);
                hq.push_back(ActF16Desc{a.x, reinterpret_cast<uint16_t*>(ab + a.L.xh),
                                        reinterpret_cast<uint16_t*>(ab + a.L.xsx), reinterpret_cast<float*>(ab + a.L.xrs),
                                        rows, a.k, plan->hgrid, wgs});
                plan->hgrid += wgs;
            }
        }
        plan->nq = (uint32_t)q.size();
        plan->nh = (uint32_t)hq.size();
        plan->qtable = reinterpret_cast<QuantDesc*>(base + off);
        off += align256(q.size() * sizeof(QuantDesc));
        plan->htable = reinterpret_cast<ActF16Desc*>(base + off);
        if (rc == RFXQ_OK && !q.empty()) {
            hipError_t e = hipMemcpy(plan->qtable, q.data(), q.size() * sizeof(QuantDesc), hipMemcpyHostToDevice);
            if (e != hipSuccess) rc = fail(RFXQ_ERR_GPU, "gemm_plan_create upload: %s", hipGetErrorString(e));
        }
        if (rc == RFXQ_OK && !hq.empty()) {
            hipError_t e = hipMemcpy(plan->htable, hq.data(), hq.size() * sizeof(ActF16Desc), hipMemcpyHostToDevice);
            if (e != hipSuccess) rc = fail(RFXQ_ERR_GPU, "gemm_plan_create upload: %s", hipGetErrorString(e));
        }
    }
    if (rc == RFXQ_OK && !plan->g.gemv_rows.empty())
        rc = rfxq_gemv_plan_create(plan->g.gemv_rows.data(), (uint32_t)plan->g.gemv_rows.size(), device, &plan->q8);
    (void)hipSetDevice(prev);
    if (rc != RFXQ_OK) {
        if (plan->dev) (void)hipFree(plan->dev);
        return rc;
    }
    *out = plan.release();
    return ok();
}

int rfxq_gemm_plan_create(const rfxq_gemm_item* items, uint32_t count, uint32_t rows, int device,
                          rfxq_gemm_plan** out) {
    return gemm_plan_create(items, count, rows, device, out, false);
}

int rfxq_gemm_q8_1_plan_create(const rfxq_gemm_q8_1_item* items, uint32_t count, uint32_t rows, int device,
                               rfxq_gemm_plan** out) {
    if (!items && count) return fail(RFXQ_ERR_INVALID_INPUT, "gemm_q8_1_plan_create: items is NULL");
    std::vector<rfxq_gemm_item> v(count);
    for (uint32_t i = 0; i < count; i++) v[i] = {static_cast<const float*>(items[i].act), items[i].w, items[i].y};
    return gemm_plan_create(v.data(), count, rows, device, out, true);
}

int rfxq_gemm_plan_run(const rfxq_gemm_plan* plan, hipStream_t stream) {
    if (!plan) return fail(RFXQ_ERR_INVALID_INPUT, "gemm_plan_run: NULL plan");
    Ctx* c;
    if (int rc = load_ctx(plan->device, &c)) return rc;
    if (plan->nq) {
        struct {
            const QuantDesc* table;
            uint32_t ndesc, pad;
        } qa = {plan->qtable, plan->nq, 0};
        if (int rc = launch(c->quant_multi, plan->qgrid, 0, stream, &qa, sizeof qa, "rfxq_quantize_q8_1_multi launch"))
            return rc;
    }
    if (plan->nh) {
        struct {
            const ActF16Desc* table;
            uint32_t ndesc, pad;
        } ha = {plan->htable, plan->nh, 0};
        if (int rc = launch(plan->hwave ? c->act_f16_multi : c->act_f16_multi_wg, plan->hgrid, 0, stream, &ha, sizeof ha,
                            "rfxq_act_f16_multi launch"))
            return rc;
    }
    for (uint32_t t = 0; t < kGroupKernels; t++) {
        const auto& v = plan->g.descs[t];
        if (v.empty()) continue;
        if (int rc = launch_group_kernel(c, plan->g, t, v.size() <= kMmqInline ? nullptr : plan->table[t], stream))
            return rc;
        if (int rc = run_group_reduces(c, plan->g, t, stream)) return rc;
    }
    if (plan->q8)
        if (int rc = rfxq_gemv_plan_run(plan->q8, stream)) return rc;
    return ok();
}

void rfxq_gemm_plan_destroy(rfxq_gemm_plan* plan) {
    if (!plan) return;
    rfxq_gemv_plan_destroy(plan->q8);
    if (plan->dev) (void)hipFree(plan->dev);
    delete plan;
}

int rfxq_mmq_block_dots(const int8_t* xq, const uint32_t* xds, uint32_t rows, const rfxq_weight* w, int32_t* dots,
                        hipStream_t stream) {
    if (int rc = check_mmq_weight(w, "mmq_block_dots")) return rc;
    if (!xq || !xds || !dots || rows == 0) return fail(RFXQ_ERR_INVALID_INPUT, "mmq_block_dots: bad arguments");
    Ctx* c;
    if (int rc = current_ctx(&c)) return rc;
    MmqDesc d;
    std::memset(&d, 0, sizeof d);
    d.w = w->data;
    d.xq = xq;
    d.xds = xds;
    d.m = rows;
    d.n = w->out_features;
    d.k = w->in_features;
    d.type = w->ggml_type;
    d.ldq = w->in_features;
    d.ldy = w->out_features;
    d.tiles_m = (rows + kMmqBM - 1u) / kMmqBM;
    d.tiles_n = (d.n + kMmqBN - 1u) / kMmqBN;
    d.splits = 1;
    d.sb_per_split = d.k / 256u;
    d.dots_out = dots;
    if (int rc = launch_mmq(c, w->ggml_type, &d, 1, nullptr, d.tiles_m * d.tiles_n, true, stream)) return rc;
    return ok();
}

int rfxq_route_top_k(const float* logits, uint32_t n, uint32_t k, int normalize, uint32_t* expert, float* weight) {
    if (!expert || !weight) return fail(RFXQ_ERR_INVALID_INPUT, "route_top_k: NULL output");
    if (int rc = route_top_k(logits, n, k, normalize != 0, expert, weight)) return rc;
    return ok();
}

int rfxq_quant_expert_weight(const rfxq_weight* w, uint32_t expert, rfxq_weight* out) {
    if (int rc = expert_slice(w, expert, out, "quant_expert_weight")) return rc;
    return ok();
}

int rfxq_expert_gemv(const float* x, uint64_t x_len, const rfxq_weight* w, uint32_t expert, float* y,
                     hipStream_t stream) {
    rfxq_weight ew;
    if (int rc = expert_slice(w, expert, &ew, "expert_gemv")) return rc;
    return rfxq_gemv_to(x, x_len, &ew, y, stream);
}

int rfxq_expert_gemm(const float* x, uint64_t x_len, const rfxq_weight* w, uint32_t expert, uint32_t rows, float* y,
                     void* workspace, uint64_t workspace_bytes, hipStream_t stream) {
    rfxq_weight ew;
    if (int rc = expert_slice(w, expert, &ew, "expert_gemm")) return rc;
    return rfxq_gemm(x, x_len, &ew, rows, y, workspace, workspace_bytes, stream);
}

int rfxq_moe_gather(const float* src, const uint32_t* perm_row, float* dst, uint32_t num, uint32_t hidden,
                    hipStream_t stream) {
    if (num == 0 || hidden == 0) return ok();
    if (!src || !perm_row || !dst) return fail(RFXQ_ERR_INVALID_INPUT, "moe_gather: NULL pointer");
    Ctx* c;
    if (int rc = current_ctx(&c)) return rc;
    struct {
        const float* s;
        const uint32_t* p;
        float* d;
        uint32_t num, hidden;
    } a = {src, perm_row, dst, num, hidden};
    const uint64_t blocks = std::min<uint64_t>(((uint64_t)num * hidden + 255u) / 256u, 16384u);
    if (int rc = launch(c->gather, (uint32_t)blocks, 0, stream, &a, sizeof a, "moe_gather launch")) return rc;
    return ok();
}

int rfxq_moe_scatter_add(const float* src, const uint32_t* dest_row, const float* weight, float* dst, uint32_t num,
                         uint32_t hidden, hipStream_t stream) {
    if (num == 0 || hidden == 0) return ok();
    if (!src || !dest_row || !weight || !dst) return fail(RFXQ_ERR_INVALID_INPUT, "moe_scatter_add: NULL pointer");
    Ctx* c;
    if (int rc = current_ctx(&c)) return rc;
    struct {
        const float* s;
        const uint32_t* r;
        const float* w;
        float* d;
        uint32_t num, hidden;
    } a = {src, dest_row, weight, dst, num, hidden};
    const uint64_t blocks = std::min<uint64_t>(((uint64_t)num * hidden + 255u) / 256u, 16384u);
    if (int rc = launch(c->scatter, (uint32_t)blocks, 0, stream, &a, sizeof a, "moe_scatter_add launch")) return rc;
    return ok();
}

int rfxq_silu_and_mul(const float* gate, const float* up, float* out, uint64_t n, hipStream_t stream) {
    if (n == 0) return ok();
    if (!gate || !up || !out) return fail(RFXQ_ERR_INVALID_INPUT, "silu_and_mul: NULL pointer");
    Ctx* c;
    if (int rc = current_ctx(&c)) return rc;
    struct {
        const float* g;
        const float* u;
        float* o;
        uint64_t n;
    } a = {gate, up, out, n};
    const uint64_t blocks = std::min<uint64_t>((n + 255u) / 256u, 16384u);
    if (int rc = launch(c->silu, (uint32_t)blocks, 0, stream, &a, sizeof a, "silu_and_mul launch")) return rc;
    return ok();
}

}  // extern "C"

namespace {
// rfxq_moe_route over `tokens` workgroups; with xh, each also writes its
// token's row of x (hidden values) in the f16 layout (xh, xsx, xrs)
int moe_route_launch(Ctx* c, const float* logits, uint32_t tokens, uint32_t E, uint32_t k, int normalize, float scale,
                     int32_t* idx, float* w, const float* x, uint32_t hidden, uint16_t* xh, uint16_t* xsx, float* xrs,
                     hipStream_t stream) {
    struct {
        const float* l;
        uint32_t tokens, E, k, normalize;
        float scale;
        uint32_t pad;
        int32_t* idx;
        float* w;
        const float* x;
        uint32_t hidden, pad2;
        uint16_t* xh;
        uint16_t* xsx;
        float* xrs;
    } a = {logits, tokens, E, k, normalize ? 1u : 0u, scale, 0, idx, w, x, hidden, 0, xh, xsx, xrs};
    // a wave per token (rfxq_moe_route_w) where its limits hold
    if (E <= kDecRouteMaxE && k <= 64u && (!xh || hidden <= 4096u))
        return launch(c->moe_route_w, (tokens + 3u) / 4u, 0, stream, &a, sizeof a, "rfxq_moe_route_w launch");
    return launch(c->moe_route, tokens, 0, stream, &a, sizeof a, "rfxq_moe_route launch");
}

int moe_grouped_device(const float* x, uint32_t rows, uint32_t hidden, const float* router_logits,
                       const uint32_t* host_idx, const float* host_w, uint32_t expert_count, uint32_t top_k,
                       int normalize, float weight_scale, const rfxq_weight* gate, const rfxq_weight* up,
                       const rfxq_weight* down, float* out, hipStream_t stream);
}  // namespace

extern "C" {

int rfxq_moe_ffn_grouped(const float* x, uint32_t rows, uint32_t hidden, const float* router_logits_host,
                         uint32_t expert_count, uint32_t top_k, int normalize, float weight_scale,
                         const rfxq_weight* gate, const rfxq_weight* up, const rfxq_weight* down, float* out,
                         hipStream_t stream) {
    if (!x || !out || !router_logits_host || !gate || !up || !down)
        return fail(RFXQ_ERR_INVALID_INPUT, "moe_ffn_grouped: NULL argument");
    if (rows == 0) return ok();
    if (gate->expert_count != expert_count || up->expert_count != expert_count || down->expert_count != expert_count)
        return fail(RFXQ_ERR_OTHER, "moe_ffn_grouped: expert tensors must have expert_count=%u", expert_count);
    if (gate->in_features != hidden || up->in_features != hidden || down->out_features != hidden ||
        gate->out_features != up->out_features || down->in_features != gate->out_features)
        return fail(RFXQ_ERR_OTHER, "moe_ffn_grouped: shapes gate [%u,%u] up [%u,%u] down [%u,%u] hidden %u",
                    gate->in_features, gate->out_features, up->in_features, up->out_features, down->in_features,
                    down->out_features, hidden);
    const uint32_t ffn = gate->out_features;
    rfxq_weight g0, u0, d0;
    if (int rc = expert_slice(gate, 0, &g0, "moe_ffn_grouped gate")) return rc;
    if (int rc = expert_slice(up, 0, &u0, "moe_ffn_grouped up")) return rc;
    if (int rc = expert_slice(down, 0, &d0, "moe_ffn_grouped down")) return rc;
    if (int rc = check_mmq_weight(&g0, "moe_ffn_grouped gate")) return rc;
    if (int rc = check_mmq_weight(&u0, "moe_ffn_grouped up")) return rc;
    if (int rc = check_mmq_weight(&d0, "moe_ffn_grouped down")) return rc;
    if (gate->ggml_type != up->ggml_type)
        return fail(RFXQ_ERR_OTHER, "moe_ffn_grouped: gate and up must share a type");
    if (reinterpret_cast<uintptr_t>(x) % 16u) return fail(RFXQ_ERR_OTHER, "moe_ffn_grouped: x not 16-byte aligned");
    Ctx* c;
    if (int rc = current_ctx(&c)) return rc;

    // host routing (dense.rs:1523-1530), tokens in parallel (each routes
    // alone; a failing token is routed again on this thread for the message)
    std::vector<uint32_t> ridx((uint64_t)rows * top_k);
    std::vector<float> rwts((uint64_t)rows * top_k);
    int64_t bad = -1;
#pragma omp parallel for schedule(static) if (rows >= 64)
    for (int64_t r = 0; r < (int64_t)rows; r++) {
        if (route_top_k(router_logits_host + (uint64_t)r * expert_count, expert_count, top_k, normalize != 0,
                        ridx.data() + (uint64_t)r * top_k, rwts.data() + (uint64_t)r * top_k) != RFXQ_OK) {
#pragma omp critical
            if (bad < 0 || r < bad) bad = r;
        }
    }
    if (bad >= 0)
        return route_top_k(router_logits_host + (uint64_t)bad * expert_count, expert_count, top_k, normalize != 0,
                           ridx.data() + (uint64_t)bad * top_k, rwts.data() + (uint64_t)bad * top_k);
    // grouping by expert, tokens in order (a counting sort)
    const uint32_t P = rows * top_k;
    std::vector<uint32_t> off(expert_count + 1, 0), fill(rows, 0);
    for (uint32_t q = 0; q < P; q++) off[ridx[q] + 1]++;
    for (uint32_t e = 0; e < expert_count; e++) off[e + 1] += off[e];
    std::vector<uint32_t> order(P), cur(off.begin(), off.end() - 1);
    for (uint32_t q = 0; q < P; q++) order[cur[ridx[q]]++] = q;  // pairs by expert, then token
    std::vector<int32_t> pair_row(P), comb_idx((uint64_t)rows * top_k, -1);
    std::vector<float> comb_w((uint64_t)rows * top_k, 0.0f);
    uint32_t p = 0;
    for (; p < P; p++) {
        const uint32_t q = order[p], r = q / top_k;
        pair_row[p] = (int32_t)r;
        const uint32_t slot = fill[r]++;  // the token's pairs in increasing expert order
        comb_idx[(uint64_t)r * top_k + slot] = (int32_t)p;
        comb_w[(uint64_t)r * top_k + slot] = rwts[q] * weight_scale;
    }
    off[expert_count] = p;

    // Few tokens (decode): every routed pair is a GEMV of its expert's
    // slices (gate and up in one launch, down in another): weights are read
    // once per pair at HBM rate instead of through 128-row MMQ tiles. The
    // host's routing goes up in one copy and the device plans the launches
    // (rfxq_moe_ffn_grouped_device's pipeline, same results); expert counts
    // that pipeline does not take are planned here.
    if (rows <= kMoeGemvRows && expert_count >= 4u && expert_count <= kRouteMaxE && top_k <= 64u &&
        gate->len == up->len) {
        std::vector<float> wsc(rwts.size());
        for (size_t i = 0; i < wsc.size(); i++) wsc[i] = rwts[i] * weight_scale;
        return moe_grouped_device(x, rows, hidden, nullptr, ridx.data(), wsc.data(), expert_count, top_k, normalize,
                                  weight_scale, gate, up, down, out, stream);
    }
    // f16 mode with token activations past the f16 kernels' gathered-row
    // limit: every pair runs as GEMVs too (the int8 format would miss 1e-3)
    const bool f16 = f16_kernel(&g0, rows) && f16_kernel(&u0, rows) && f16_kernel(&d0, P);
    if (rows <= kMoeGemvRows || (mmq_f16() && !f16)) {
        const uint64_t g_gate = 0;
        const uint64_t g_up = g_gate + align256((uint64_t)P * ffn * 4u);
        const uint64_t g_down = g_up + align256((uint64_t)P * ffn * 4u);
        const uint64_t g_ci = g_down + align256((uint64_t)P * hidden * 4u);
        const uint64_t g_cw = g_ci + align256((uint64_t)rows * top_k * 4u);
        const uint64_t g_total = g_cw + align256((uint64_t)rows * top_k * 4u);
        void* ws;
        if (int rc = ctx_workspace(c, g_total, &ws, stream)) return rc;
        uint8_t* B = static_cast<uint8_t*>(ws);
        float* gout = reinterpret_cast<float*>(B + g_gate);
        float* uout = reinterpret_cast<float*>(B + g_up);
        float* dout = reinterpret_cast<float*>(B + g_down);
        std::vector<rfxq_weight> gs(expert_count), us(expert_count), ds(expert_count);
        std::vector<GemvItem> gu, dn;
        for (uint32_t e = 0; e < expert_count; e++) {
            if (off[e + 1] == off[e]) continue;
            expert_slice(gate, e, &gs[e], "moe_ffn_grouped");
            expert_slice(up, e, &us[e], "moe_ffn_grouped");
            expert_slice(down, e, &ds[e], "moe_ffn_grouped");
            for (uint32_t q = off[e]; q < off[e + 1]; q++) {
                const float* xr = x + (uint64_t)pair_row[q] * hidden;
                GemvItem a, b, d;
                if (int rc = make_gemv_item(xr, &gs[e], gout + (uint64_t)q * ffn, &a)) return rc;
                if (int rc = make_gemv_item(xr, &us[e], uout + (uint64_t)q * ffn, &b)) return rc;
                if (int rc = make_gemv_item(gout + (uint64_t)q * ffn, &ds[e], dout + (uint64_t)q * hidden, &d))
                    return rc;
                gu.push_back(a);
                gu.push_back(b);
                dn.push_back(d);
            }
        }
        std::vector<uint8_t> host(g_total - g_ci, 0);
        std::memcpy(host.data(), comb_idx.data(), comb_idx.size() * 4u);
        std::memcpy(host.data() + (g_cw - g_ci), comb_w.data(), comb_w.size() * 4u);
        if (int rc = stage_upload(c, B + g_ci, host.data(), host.size(), stream)) return rc;
        if (int rc = gemv_launch_table(c, gu, 0, stream)) return rc;
        if (int rc = rfxq_silu_and_mul(gout, uout, gout, (uint64_t)P * ffn, stream)) return rc;
        if (int rc = gemv_launch_table(c, dn, 0, stream)) return rc;
        if (int rc = launch_combine(c, dout, reinterpret_cast<const int32_t*>(B + g_ci),
                                    reinterpret_cast<const float*>(B + g_cw), out, rows, top_k, hidden, stream))
            return rc;
        return ok();
    }

    // workspace layout: x and the SiLU·up rows in the layouts the expert
    // GEMMs read (f16 kernels, or int8 with REFLEX_MMQ_F16=0)
    const ActLayout Lx = act_layout_sel(rows, hidden, !f16, f16);
    const ActLayout Ls = act_layout_sel(P, ffn, !f16, f16);
    const uint64_t o_x = 0;
    const uint64_t o_gate = o_x + Lx.total;
    const uint64_t o_up = o_gate + align256((uint64_t)P * ffn * 4u);
    const uint64_t o_s = o_up + align256((uint64_t)P * ffn * 4u);
    const uint64_t o_down = o_s + Ls.total;
    const uint64_t o_tab = o_down + align256((uint64_t)P * hidden * 4u);
    // tables: pair_row[P], comb_idx[rows*k], comb_w[rows*k], descs (up to 3E)
    const uint64_t o_pr = o_tab;
    const uint64_t o_ci = o_pr + align256((uint64_t)P * 4u);
    const uint64_t o_cw = o_ci + align256((uint64_t)rows * top_k * 4u);
    const uint64_t o_desc = o_cw + align256((uint64_t)rows * top_k * 4u);
    const uint64_t total = o_desc + align256((uint64_t)3u * expert_count * sizeof(MmqDesc));
    void* ws;
    if (int rc = ctx_workspace(c, total, &ws, stream)) return rc;
    uint8_t* B = static_cast<uint8_t*>(ws);
    float* gout = reinterpret_cast<float*>(B + o_gate);
    float* uout = reinterpret_cast<float*>(B + o_up);
    float* dout = reinterpret_cast<float*>(B + o_down);
    int32_t* d_pr = reinterpret_cast<int32_t*>(B + o_pr);
    int32_t* d_ci = reinterpret_cast<int32_t*>(B + o_ci);
    float* d_cw = reinterpret_cast<float*>(B + o_cw);
    MmqDesc* d_desc = reinterpret_cast<MmqDesc*>(B + o_desc);

    // descriptor tables: [gate+up descs][down descs]; the row tile by the
    // used experts' average row count
    uint32_t used = 0;
    for (uint32_t e = 0; e < expert_count; e++) used += off[e + 1] > off[e];
    const uint32_t bn = tile_bn(f16);
    const uint32_t bm_gu = moe_tile_m(P, used, f16, gate->ggml_type, 2u * ((ffn + bn - 1u) / bn), (uint32_t)c->cus);
    const uint32_t bm_dn = moe_tile_m(P, used, f16, down->ggml_type, (hidden + bn - 1u) / bn, (uint32_t)c->cus);
    uint32_t bm = bm_gu;  // the row tile of the descriptors add() writes
    std::vector<MmqDesc> descs;
    uint32_t wg_gu = 0;
    // act: the activation layouts (rows gathered through rws, or starting at row r0)
    auto add = [&](const rfxq_weight* w, uint32_t e, const uint8_t* act, const ActLayout& L, uint32_t r0,
                   const int32_t* rws, uint32_t m, float* y, uint32_t n, uint32_t& wg) {
        rfxq_weight ew;
        expert_slice(w, e, &ew, "moe_ffn_grouped");
        MmqDesc d;
        std::memset(&d, 0, sizeof d);
        d.w = ew.data;
        act_desc(&d, act, L, f16, ew.in_features);
        if (r0) {
            d.xq += (uint64_t)r0 * d.ldq;
            d.xds = reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint8_t*>(d.xds) +
                                                      (uint64_t)r0 * (f16 ? ew.in_features / 256u * 32u
                                                                          : ew.in_features / 32u * 4u));
            if (f16) d.xrs += r0;
        }
        d.rows = rws;
        d.y = y;
        d.m = m;
        d.n = n;
        d.k = ew.in_features;
        d.type = ew.ggml_type;
        d.ldy = n;
        d.tiles_m = (m + bm - 1u) / bm;
        d.tiles_n = (n + bn - 1u) / bn;
        d.splits = 1;
        d.sb_per_split = d.k / 256u;
        d.wg_begin = wg;
        wg += d.tiles_m * d.tiles_n;
        descs.push_back(d);
    };
    // Q4_K gate / up on the f16 tiles: one gate/up pair descriptor per expert
    // (its tiles store SiLU·up into gout), then an f16 activation pass of it,
    // as the device-routed path does (RFXQ_MOE_GU_PAIR=0: separate gate and up)
    const char* gp = std::getenv("RFXQ_MOE_GU_PAIR");
    const bool gu_pair = f16 && gate->ggml_type == RFXQ_TYPE_Q4_K && !(gp && std::strcmp(gp, "0") == 0);
    for (uint32_t e = 0; e < expert_count; e++) {
        const uint32_t m = off[e + 1] - off[e];
        if (!m) continue;
        if (gu_pair) {
            const uint32_t wg0 = wg_gu;
            add(gate, e, B + o_x, Lx, 0, d_pr + off[e], m, gout + (uint64_t)off[e] * ffn, ffn, wg_gu);
            MmqDesc& d = descs.back();
            rfxq_weight ue;
            expert_slice(up, e, &ue, "moe_ffn_grouped");
            d.w_up = static_cast<const uint8_t*>(ue.data);
            d.gu_pair = 1u;
            d.tiles_n = (ffn + mmqh_pair_bn - 1u) / mmqh_pair_bn;
            wg_gu = wg0 + d.tiles_m * d.tiles_n;
        } else {
            add(gate, e, B + o_x, Lx, 0, d_pr + off[e], m, gout + (uint64_t)off[e] * ffn, ffn, wg_gu);
            add(up, e, B + o_x, Lx, 0, d_pr + off[e], m, uout + (uint64_t)off[e] * ffn, ffn, wg_gu);
        }
    }
    const uint32_t n_gu = (uint32_t)descs.size();
    uint32_t wg_dn = 0;
    bm = bm_dn;
    for (uint32_t e = 0; e < expert_count; e++) {
        const uint32_t m = off[e + 1] - off[e];
        if (!m) continue;
        add(down, e, B + o_s, Ls, off[e], nullptr, m, dout + (uint64_t)off[e] * hidden, hidden, wg_dn);
    }
    const uint32_t n_dn = (uint32_t)descs.size() - n_gu;

    // one upload of all tables (stream-ordered through pinned staging; the
    // reference copies per expert)
    std::vector<uint8_t> host(total - o_tab, 0);
    std::memcpy(host.data() + (o_pr - o_tab), pair_row.data(), (size_t)P * 4u);
    std::memcpy(host.data() + (o_ci - o_tab), comb_idx.data(), comb_idx.size() * 4u);
    std::memcpy(host.data() + (o_cw - o_tab), comb_w.data(), comb_w.size() * 4u);
    std::memcpy(host.data() + (o_desc - o_tab), descs.data(), descs.size() * sizeof(MmqDesc));
    if (int rc = stage_upload(c, B + o_tab, host.data(), host.size(), stream)) return rc;

    if (int rc = launch_act(c, x, rows, hidden, B + o_x, Lx, !f16, f16, stream)) return rc;
    if (n_gu) {
        if (int rc = launch_mmq(c, gate->ggml_type, descs.data(), n_gu, d_desc, wg_gu, false, stream, f16, bm_gu))
            return rc;
    }
    if (gu_pair) {
        if (int rc = launch_act(c, gout, P, ffn, B + o_s, Ls, false, true, stream)) return rc;
    } else if (int rc = launch_silu_act(c, gout, uout, P, ffn, B + o_s, Ls, !f16, f16, stream)) {
        return rc;
    }
    if (n_dn) {
        if (int rc = launch_mmq(c, down->ggml_type, descs.data() + n_gu, n_dn, d_desc + n_gu, wg_dn, false, stream,
                                f16, bm_dn))
            return rc;
    }
    if (int rc = launch_combine(c, dout, d_ci, d_cw, out, rows, top_k, hidden, stream)) return rc;
    return ok();
}

int rfxq_moe_route_device(const float* logits, uint32_t tokens, uint32_t expert_count, uint32_t top_k,
                          int normalize, float weight_scale, int32_t* idx, float* weights, hipStream_t stream) {
    if (tokens == 0) return ok();
    if (!logits || !idx || !weights) return fail(RFXQ_ERR_INVALID_INPUT, "moe_route_device: NULL pointer");
    if (expert_count == 0 || expert_count > kRouteMaxE)
        return fail(RFXQ_ERR_OTHER, "moe_route_device: expert_count=%u (1..=%u)", expert_count, kRouteMaxE);
    if (top_k == 0 || top_k > expert_count || top_k > 64u)
        return fail(RFXQ_ERR_OTHER, "route_top_k: k (%u) must be in 1..=%u (logits.len())", top_k,
                    std::min(expert_count, 64u));
    Ctx* c;
    if (int rc = current_ctx(&c)) return rc;
    if (int rc = moe_route_launch(c, logits, tokens, expert_count, top_k, normalize, weight_scale, idx, weights, nullptr,
                                  0, nullptr, nullptr, nullptr, stream))
        return rc;
    return ok();
}

struct MoePlanArgs {
    const int32_t* idx;
    const float* wts;
    int32_t* pair_row;
    int32_t* comb_idx;
    float* comb_w;
    MmqDesc* descs_gu;
    MmqDesc* descs_dn;
    MmqDesc tg, tu, td;
    uint64_t w_stride_gu, w_stride_dn;
    uint32_t tokens, k, E, bm_dn;
    uint32_t bm, ffn, hidden, f16;
    GemvDesc* gemv_gu;
    GemvDesc* gemv_dn;
    GemvDesc vg, vu, vd;
    const float* logits;
    uint32_t normalize;
    float scale;
    uint32_t any_order;
    uint32_t gu_pair;
};
static_assert(sizeof(MoePlanArgs) == 624, "MoePlanArgs layout");


int rfxq_moe_ffn_grouped_device(const float* x, uint32_t rows, uint32_t hidden, const float* router_logits,
                                uint32_t expert_count, uint32_t top_k, int normalize, float weight_scale,
                                const rfxq_weight* gate, const rfxq_weight* up, const rfxq_weight* down, float* out,
                                hipStream_t stream) {
    if (!router_logits) return fail(RFXQ_ERR_INVALID_INPUT, "moe_ffn_grouped_device: NULL argument");
    return moe_grouped_device(x, rows, hidden, router_logits, nullptr, nullptr, expert_count, top_k, normalize,
                              weight_scale, gate, up, down, out, stream);
}

}  // extern "C"

namespace {

// ------------------------------------------------------------------ MoE decode (two launches)

// Mirror of MoeDecArgs (moe_decode.hpp).
struct MoeDecArgs {
    const float* x;
    const float* logits;
    int32_t* idx;
    float* wts;
    const uint8_t* wg;
    const uint8_t* wu;
    const uint8_t* wd;
    uint64_t eb_gu, eb_dn;
    float* s;
    float* out;
    uint32_t tokens, E, k, hidden, ffn, normalize;
    float scale;
    uint32_t nb1, nr1;
    uint32_t nb2, nr2;
    uint32_t lds_x1, lds_x2;
    uint32_t n_inline;
    int32_t h_idx[32];
    float h_w[32];
};
constexpr uint32_t kDecInlinePairs = 32;    // moe_decode.hpp

// Lanes per row of the decode kernels: a power of two in [4, 32] dividing the
// row's units, with at least `min_units` units per lane (fewer loads in
// flight per lane below that) when the row allows; -1 if none divides.
int dec_lpr(uint32_t units, uint32_t min_units, uint32_t max_lpr) {
    int best = -1;
    for (int l = 3; l >= 0; l--) {
        const uint32_t lpr = 4u << l;
        if (lpr > max_lpr || units % lpr) continue;
        if (best < 0) best = l;  // the widest that divides
        if (units / lpr >= min_units) return l;
    }
    return best;
}

// The two-launch decode pipeline (moe_decode.hpp) when its limits hold:
// rows tokens of up to kMoeGemvRows, k <= 64, hidden and k * ffn <= 16384, at
// most kDecRouteMaxE experts when it routes,
// stacked weights below 4 GiB, row units that split over 4..32 lanes. Routing
// from `logits` (device) in the first launch, or from idx / wts already in
// device memory. s: workspace [rows][k][ffn]. Returns RFXQ_OK with *done =
// false when the shapes fall outside the limits (nothing launched).
int moe_decode_launch(Ctx* c, const float* x, uint32_t rows, uint32_t hidden, const float* logits, int32_t* idx,
                      float* wts, uint32_t E, uint32_t k, int normalize, float scale, const rfxq_weight* gate,
                      const rfxq_weight* up, const rfxq_weight* down, float* s, float* out, hipStream_t stream,
                      bool* done, const uint32_t* host_idx = nullptr, const float* host_w = nullptr) {
    *done = false;
    const uint32_t ffn = gate->out_features;
    const int tg = type_index(gate->ggml_type), td = type_index(down->ggml_type);
    auto unit_k = [](uint32_t ty) { return ty == RFXQ_TYPE_Q8_0 ? 32u : 64u; };
    const uint64_t lim = 0xF0000000ull;
    if (rows == 0 || rows > kMoeGemvRows || k == 0 || k > 64u || hidden > 16384u || (uint64_t)k * ffn > 16384u ||
        (logits && E > kDecRouteMaxE) ||
        gate->len >= lim || up->len >= lim || down->len >= lim || hidden % 256u || ffn % 256u)
        return RFXQ_OK;
    const int l1 = dec_lpr(hidden / unit_k(gate->ggml_type), 4u, 32u);
    const int l2 = dec_lpr(ffn / unit_k(down->ggml_type), 2u, std::min(32u, 256u / k));
    if (l1 < 0 || l2 < 0) return RFXQ_OK;
    MoeDecArgs a;
    std::memset(&a, 0, sizeof a);
    a.x = x;
    a.logits = logits;
    a.idx = idx;
    a.wts = wts;
    a.wg = static_cast<const uint8_t*>(gate->data);
    a.wu = static_cast<const uint8_t*>(up->data);
    a.wd = static_cast<const uint8_t*>(down->data);
    a.eb_gu = gate->len / E;
    a.eb_dn = down->len / E;
    a.s = s;
    a.out = out;
    a.tokens = rows;
    a.E = E;
    a.k = k;
    a.hidden = hidden;
    a.ffn = ffn;
    a.normalize = normalize ? 1u : 0u;
    a.scale = scale;
    const uint32_t lpr1 = 4u << l1, lpr2 = 4u << l2;
    a.nr1 = 2u * (64u / lpr1);  // waves 0-1 gate rows, 2-3 up rows
    a.nb1 = (ffn + a.nr1 - 1u) / a.nr1;
    a.nr2 = (256u / lpr2) / k;  // (row, slot) items per workgroup
    a.nb2 = (hidden + a.nr2 - 1u) / a.nr2;
    a.lds_x1 = 0u;
    a.lds_x2 = 768u;  // experts, weights, combine order
    if (host_idx) {  // the host's routing in the kernel arguments (the caller checked the count)
        a.n_inline = rows * k;
        for (uint32_t q = 0; q < rows * k; q++) {
            a.h_idx[q] = (int32_t)host_idx[q];
            a.h_w[q] = host_w[q];
        }
    }
    const uint32_t K2 = k * ffn;
    const uint32_t lds1 = a.lds_x1 + hidden * 2u + hidden / 4u + 16u + 2u * a.nr1 * 4u;
    const uint32_t lds2 = a.lds_x2 + K2 * 2u + K2 / 4u + 16u + a.nr2 * k * 4u;
    if (int rc = launch(c->moe_dec_gu[tg][l1], rows * k * a.nb1, lds1, stream, &a, sizeof a, "rfxq_moe_dec_gu launch"))
        return rc;
    if (int rc = launch(c->moe_dec_dn[td][l2], rows * a.nb2, lds2, stream, &a, sizeof a, "rfxq_moe_dec_down launch"))
        return rc;
    *done = true;
    return RFXQ_OK;
}

// The device-planned pipeline: routing on the device from `router_logits`,
// or the host's routing (`host_idx`, `host_w`: rows x top_k experts and
// weights already multiplied by weight_scale) uploaded in one copy.
int moe_grouped_device(const float* x, uint32_t rows, uint32_t hidden, const float* router_logits,
                       const uint32_t* host_idx, const float* host_w, uint32_t expert_count, uint32_t top_k,
                       int normalize, float weight_scale, const rfxq_weight* gate, const rfxq_weight* up,
                       const rfxq_weight* down, float* out, hipStream_t stream) {
    if (!x || !out || !gate || !up || !down)
        return fail(RFXQ_ERR_INVALID_INPUT, "moe_ffn_grouped_device: NULL argument");
    if (rows == 0) return ok();
    if (gate->expert_count != expert_count || up->expert_count != expert_count || down->expert_count != expert_count)
        return fail(RFXQ_ERR_OTHER, "moe_ffn_grouped: expert tensors must have expert_count=%u", expert_count);
    if (gate->in_features != hidden || up->in_features != hidden || down->out_features != hidden ||
        gate->out_features != up->out_features || down->in_features != gate->out_features)
        return fail(RFXQ_ERR_OTHER, "moe_ffn_grouped: shapes gate [%u,%u] up [%u,%u] down [%u,%u] hidden %u",
                    gate->in_features, gate->out_features, up->in_features, up->out_features, down->in_features,
                    down->out_features, hidden);
    if (expert_count < 4 || expert_count > kRouteMaxE)
        return fail(RFXQ_ERR_OTHER, "moe_ffn_grouped_device: expert_count=%u (4..=%u)", expert_count, kRouteMaxE);
    if (top_k == 0 || top_k > expert_count || top_k > 64u)
        return fail(RFXQ_ERR_OTHER, "route_top_k: k (%u) must be in 1..=%u (logits.len())", top_k,
                    std::min(expert_count, 64u));
    const uint64_t P64 = (uint64_t)rows * top_k;
    if (P64 > kPlanMaxPairs)
        return fail(RFXQ_ERR_OTHER, "moe_ffn_grouped_device: %llu routed pairs (at most %u)",
                    (unsigned long long)P64, kPlanMaxPairs);
    const uint32_t P = (uint32_t)P64, ffn = gate->out_features;
    rfxq_weight g0, u0, d0;
    if (int rc = expert_slice(gate, 0, &g0, "moe_ffn_grouped gate")) return rc;
    if (int rc = expert_slice(up, 0, &u0, "moe_ffn_grouped up")) return rc;
    if (int rc = expert_slice(down, 0, &d0, "moe_ffn_grouped down")) return rc;
    if (int rc = check_mmq_weight(&g0, "moe_ffn_grouped gate")) return rc;
    if (int rc = check_mmq_weight(&u0, "moe_ffn_grouped up")) return rc;
    if (int rc = check_mmq_weight(&d0, "moe_ffn_grouped down")) return rc;
    if (gate->ggml_type != up->ggml_type || gate->len != up->len)
        return fail(RFXQ_ERR_OTHER, "moe_ffn_grouped: gate and up must share a type and shape");
    if (reinterpret_cast<uintptr_t>(x) % 16u) return fail(RFXQ_ERR_OTHER, "moe_ffn_grouped: x not 16-byte aligned");
    Ctx* c;
    if (int rc = current_ctx(&c)) return rc;

    // workspace: quantized tokens, gate/up outputs, quantized SiLU·up, down
    // outputs, routing, grouping and descriptor tables
    const bool f16 = f16_kernel(&g0, rows) && f16_kernel(&u0, rows) && f16_kernel(&d0, P);
    if (mmq_f16() && !f16)
        return fail(RFXQ_ERR_OTHER, "moe_ffn_grouped_device: %u tokens x %u hidden exceed the f16 kernels' 4 GiB "
                    "gathered-activation range (use rfxq_moe_ffn_grouped)", rows, hidden);
    const ActLayout Lx = act_layout_sel(rows, hidden, !f16, f16);
    const ActLayout Ls = act_layout_sel(P, ffn, !f16, f16);
    const uint64_t o_x = 0;
    const uint64_t o_gate = o_x + Lx.total;
    const uint64_t o_up = o_gate + align256((uint64_t)P * ffn * 4u);
    const uint64_t o_s = o_up + align256((uint64_t)P * ffn * 4u);
    const uint64_t o_down = o_s + Ls.total;
    const uint64_t o_idx = o_down + align256((uint64_t)P * hidden * 4u);
    const uint64_t o_w = o_idx + align256((uint64_t)P * 4u);
    const uint64_t o_pr = o_w + align256((uint64_t)P * 4u);
    const uint64_t o_ci = o_pr + align256((uint64_t)P * 4u);
    const uint64_t o_cw = o_ci + align256((uint64_t)P * 4u);
    const uint64_t o_dgu = o_cw + align256((uint64_t)P * 4u);
    const uint64_t o_ddn = o_dgu + align256((uint64_t)2u * expert_count * sizeof(MmqDesc));
    // few tokens: every routed pair runs as GEMVs (as in the host-routed path)
    const bool gemv_form = rows <= kMoeGemvRows;
    const uint64_t o_vgu = o_ddn + align256((uint64_t)expert_count * sizeof(MmqDesc));
    const uint64_t o_vdn = o_vgu + (gemv_form ? align256((uint64_t)2u * P * sizeof(GemvDesc)) : 0u);
    const uint64_t total = o_vdn + (gemv_form ? align256((uint64_t)P * sizeof(GemvDesc)) : 0u);
    void* ws;
    if (int rc = ctx_workspace(c, total, &ws, stream)) return rc;
    uint8_t* B = static_cast<uint8_t*>(ws);
    float* gout = reinterpret_cast<float*>(B + o_gate);
    float* uout = reinterpret_cast<float*>(B + o_up);
    float* dout = reinterpret_cast<float*>(B + o_down);
    int32_t* d_idx = reinterpret_cast<int32_t*>(B + o_idx);
    float* d_w = reinterpret_cast<float*>(B + o_w);
    MmqDesc* d_gu = reinterpret_cast<MmqDesc*>(B + o_dgu);
    MmqDesc* d_dn = reinterpret_cast<MmqDesc*>(B + o_ddn);

    // row tiles by the average rows of the experts the pairs can reach
    const uint32_t bn = tile_bn(f16), reach = std::min(expert_count, P);
    const uint32_t bm = moe_tile_m(P, reach, f16, gate->ggml_type, 2u * ((ffn + bn - 1u) / bn), (uint32_t)c->cus);
    const uint32_t bm_dn = moe_tile_m(P, reach, f16, down->ggml_type, (hidden + bn - 1u) / bn, (uint32_t)c->cus);
    MoePlanArgs pa;
    std::memset(&pa, 0, sizeof pa);
    pa.idx = d_idx;
    pa.wts = d_w;
    pa.pair_row = reinterpret_cast<int32_t*>(B + o_pr);
    pa.comb_idx = reinterpret_cast<int32_t*>(B + o_ci);
    pa.comb_w = reinterpret_cast<float*>(B + o_cw);
    pa.descs_gu = d_gu;
    pa.descs_dn = d_dn;
    auto tmpl = [&](MmqDesc* d, const rfxq_weight* w0, const uint8_t* act, const ActLayout& L, float* y, uint32_t n,
                    uint32_t k) {
        d->w = static_cast<const uint8_t*>(w0->data);
        act_desc(d, act, L, f16, k);
        d->y = y;
        d->n = n;
        d->k = k;
        d->type = w0->ggml_type;
        d->ldy = n;
        d->tiles_n = (n + bn - 1u) / bn;
        d->splits = 1;
        d->sb_per_split = k / 256u;
    };
    tmpl(&pa.tg, &g0, B + o_x, Lx, gout, ffn, hidden);
    tmpl(&pa.tu, &u0, B + o_x, Lx, uout, ffn, hidden);
    tmpl(&pa.td, &d0, B + o_s, Ls, dout, hidden, ffn);
    pa.f16 = f16 ? 1u : 0u;
    pa.w_stride_gu = gate->len / expert_count;
    pa.w_stride_dn = down->len / expert_count;
    pa.tokens = rows;
    pa.k = top_k;
    pa.E = expert_count;
    pa.bm = bm;
    pa.bm_dn = bm_dn;
    pa.ffn = ffn;
    pa.hidden = hidden;
    pa.any_order = gemv_form ? 0u : 1u;  // (the GEMV form keeps token order within an expert)
    // Q4_K gate / up on the f16 tiles: one pair descriptor per expert whose
    // tiles store silu(gate) * up (f32, into gout), then one f16 activation
    // pass for down (RFXQ_MOE_GU_PAIR=0: gate and up GEMMs, then SiLU·up)
    const char* gp = std::getenv("RFXQ_MOE_GU_PAIR");
    const bool gu_pair = !gemv_form && f16 && gate->ggml_type == RFXQ_TYPE_Q4_K && !(gp && std::strcmp(gp, "0") == 0);
    if (gu_pair) {
        pa.gu_pair = 1u;
        pa.tg.gu_pair = 1u;
        pa.tg.tiles_n = (ffn + mmqh_pair_bn - 1u) / mmqh_pair_bn;
    }
    GemvItem ig, iu, id;
    if (gemv_form) {
        if (int rc = make_gemv_item(x, &g0, gout, &ig)) return rc;
        if (int rc = make_gemv_item(x, &u0, uout, &iu)) return rc;
        if (int rc = make_gemv_item(gout, &d0, dout, &id)) return rc;
        pa.gemv_gu = reinterpret_cast<GemvDesc*>(B + o_vgu);
        pa.gemv_dn = reinterpret_cast<GemvDesc*>(B + o_vdn);
        pa.vg = ig.d;
        pa.vu = iu.d;
        pa.vd = id.d;
    }

    if (host_idx && gemv_form && P <= kDecInlinePairs) {
        // few pairs routed on the host: the two decode launches take them in
        // their kernel arguments (no table upload) where the shapes allow
        bool done = false;
        if (int rc = moe_decode_launch(c, x, rows, hidden, nullptr, d_idx, d_w, expert_count, top_k, normalize,
                                       weight_scale, gate, up, down, gout, out, stream, &done, host_idx, host_w))
            return rc;
        if (done) return ok();
    }
    if (host_idx) {  // routed on the host
        std::vector<uint8_t> host(o_w - o_idx + (uint64_t)P * 4u, 0);
        std::memcpy(host.data(), host_idx, (uint64_t)P * 4u);
        std::memcpy(host.data() + (o_w - o_idx), host_w, (uint64_t)P * 4u);
        if (int rc = stage_upload(c, d_idx, host.data(), host.size(), stream)) return rc;
    } else if (gemv_form) {  // few tokens: the plan launch routes them too
        pa.logits = router_logits;
        pa.normalize = normalize ? 1u : 0u;
        pa.scale = weight_scale;
    } else {
        // routing, and with the f16 layout the token rows of x in the same launch
        if (int rc = moe_route_launch(c, router_logits, rows, expert_count, top_k, normalize, weight_scale, d_idx, d_w,
                                      f16 ? x : nullptr, hidden,
                                      f16 ? reinterpret_cast<uint16_t*>(B + o_x + Lx.xh) : nullptr,
                                      f16 ? reinterpret_cast<uint16_t*>(B + o_x + Lx.xsx) : nullptr,
                                      f16 ? reinterpret_cast<float*>(B + o_x + Lx.xrs) : nullptr, stream))
            return rc;
    }
    if (gemv_form) {  // two launches (moe_decode.hpp) where the shapes allow them
        bool done = false;
        if (int rc = moe_decode_launch(c, x, rows, hidden, host_idx ? nullptr : router_logits, d_idx, d_w, expert_count,
                                       top_k, normalize, weight_scale, gate, up, down, gout, out, stream, &done))
            return rc;
        if (done) return ok();
    }
    if (int rc = launch(c->moe_plan, 1, 0, stream, &pa, sizeof pa, "rfxq_moe_plan launch", 1024)) return rc;
    if (gemv_form) {
        std::vector<GemvItem> gu, dn(P, id);
        for (uint32_t q = 0; q < P; q++) {
            gu.push_back(ig);
            gu.push_back(iu);
        }
        if (int rc = gemv_launch_counted(c, gu, pa.gemv_gu, stream)) return rc;
        if (int rc = rfxq_silu_and_mul(gout, uout, gout, (uint64_t)P * ffn, stream)) return rc;
        if (int rc = gemv_launch_counted(c, dn, pa.gemv_dn, stream)) return rc;
    } else {
        // (the f16 rows came with the routing; host-routed calls convert here)
        if (int rc = launch_act(c, x, rows, hidden, B + o_x, Lx, !f16, f16 && host_idx, stream)) return rc;
        // launch grids: upper bounds on the tiles (sum over experts of
        // ceil(rows_e / bm) <= ceil(P / bm) + experts); surplus workgroups return
        const uint32_t bound_gu = (P + bm - 1u) / bm + expert_count, bound_dn = (P + bm_dn - 1u) / bm_dn + expert_count;
        const uint32_t gpe = gu_pair ? 1u : 2u;
        if (int rc = launch_mmq(c, gate->ggml_type, nullptr, gpe * expert_count, d_gu,
                                gpe * bound_gu * pa.tg.tiles_n, false, stream, f16, bm))
            return rc;
        if (gu_pair) {
            if (int rc = launch_act(c, gout, P, ffn, B + o_s, Ls, false, true, stream)) return rc;
        } else if (int rc = launch_silu_act(c, gout, uout, P, ffn, B + o_s, Ls, !f16, f16, stream)) {
            return rc;
        }
        if (int rc = launch_mmq(c, down->ggml_type, nullptr, expert_count, d_dn, bound_dn * pa.td.tiles_n, false,
                                stream, f16, bm_dn))
            return rc;
    }
    if (int rc = launch_combine(c, dout, pa.comb_idx, pa.comb_w, out, rows, top_k, hidden, stream)) return rc;
    return ok();
}

}  // namespace

extern "C" {

// ---------------------------------------------------------------- GGUF files

struct rfxq_gguf {
    int fd = -1;
    void* map = nullptr;
    size_t len = 0;
    gguf::File f;
};

int rfxq_gguf_open(const char* path, rfxq_gguf** out) {
    if (!path || !out) return fail(RFXQ_ERR_INVALID_INPUT, "gguf_open: NULL argument");
    *out = nullptr;
    const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return fail(RFXQ_ERR_IO, "opening GGUF file: %s", std::strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0) {
        const int e = errno;
        ::close(fd);
        return fail(RFXQ_ERR_IO, "stat GGUF file: %s", std::strerror(e));
    }
    auto g = std::make_unique<rfxq_gguf>();
    g->fd = fd;
    g->len = (size_t)st.st_size;
    if (g->len) {
        g->map = mmap(nullptr, g->len, PROT_READ, MAP_PRIVATE, fd, 0);
        if (g->map == MAP_FAILED) {
            const int e = errno;
            ::close(fd);
            return fail(RFXQ_ERR_IO, "mmap GGUF file: %s", std::strerror(e));
        }
    }
    g->f.data = static_cast<const uint8_t*>(g->map);
    g->f.len = g->len;
    std::string err;
    if (!g->f.parse(&err)) {
        if (g->map) munmap(g->map, g->len);
        ::close(fd);
        return fail(RFXQ_ERR_GGUF, "%s", err.c_str());
    }
    *out = g.release();
    return ok();
}

void rfxq_gguf_close(rfxq_gguf* g) {
    if (!g) return;
    if (g->map) munmap(g->map, g->len);
    if (g->fd >= 0) ::close(g->fd);
    delete g;
}

uint32_t rfxq_gguf_version(const rfxq_gguf* g) { return g ? g->f.version : 0u; }

uint64_t rfxq_gguf_tensor_count(const rfxq_gguf* g) { return g ? g->f.tensors.size() : 0u; }

int rfxq_gguf_find_tensor(const rfxq_gguf* g, const char* name, uint64_t* index) {
    if (!g || !name || !index) return fail(RFXQ_ERR_INVALID_INPUT, "gguf_find_tensor: NULL argument");
    auto it = g->f.by_name.find(name);
    if (it == g->f.by_name.end()) return fail(RFXQ_ERR_GGUF, "tensor '%s' not found in GGUF file", name);
    *index = it->second;
    return ok();
}

int rfxq_gguf_tensor_info(const rfxq_gguf* g, uint64_t index, const char** name, uint32_t* n_dims, uint64_t* dims,
                          uint32_t* ggml_type, uint64_t* offset) {
    if (!g) return fail(RFXQ_ERR_INVALID_INPUT, "gguf_tensor_info: NULL file");
    if (index >= g->f.tensors.size())
        return fail(RFXQ_ERR_INVALID_INPUT, "gguf_tensor_info: index %llu of %zu", (unsigned long long)index,
                    g->f.tensors.size());
    const gguf::Tensor& t = g->f.tensors[index];
    if (name) *name = t.name.c_str();
    if (n_dims) *n_dims = (uint32_t)t.dims.size();
    if (dims)
        for (size_t j = 0; j < 4; j++) dims[j] = j < t.dims.size() ? t.dims[j] : 1u;
    if (ggml_type) *ggml_type = t.type;
    if (offset) *offset = t.offset;
    return ok();
}

int rfxq_gguf_tensor_data(const rfxq_gguf* g, uint64_t index, const void** data, uint64_t* bytes) {
    if (!g || !data || !bytes) return fail(RFXQ_ERR_INVALID_INPUT, "gguf_tensor_data: NULL argument");
    if (index >= g->f.tensors.size()) return fail(RFXQ_ERR_INVALID_INPUT, "gguf_tensor_data: bad index");
    uint64_t start, nb;
    std::string err;
    if (!g->f.range(g->f.tensors[index], &start, &nb, &err)) return fail(RFXQ_ERR_GGUF, "%s", err.c_str());
    *data = g->f.data + start;
    *bytes = nb;
    return ok();
}

const gguf::Value* gguf_meta(const rfxq_gguf* g, const char* key) {
    if (!g || !key) return nullptr;
    auto it = g->f.meta.find(key);
    return it == g->f.meta.end() ? nullptr : &it->second;
}

int rfxq_gguf_meta_u64(const rfxq_gguf* g, const char* key, uint64_t* out) {
    const gguf::Value* v = gguf_meta(g, key);
    if (!v || !out || !v->as_u64(out))
        return fail(RFXQ_ERR_GGUF, "GGUF metadata '%s' missing or not an unsigned integer", key ? key : "");
    return ok();
}

int rfxq_gguf_meta_f64(const rfxq_gguf* g, const char* key, double* out) {
    const gguf::Value* v = gguf_meta(g, key);
    if (!v || !out || v->kind != gguf::Value::FLOAT)
        return fail(RFXQ_ERR_GGUF, "GGUF metadata '%s' missing or not a float", key ? key : "");
    *out = v->f;
    return ok();
}

int rfxq_gguf_meta_str(const rfxq_gguf* g, const char* key, const char** out) {
    const gguf::Value* v = gguf_meta(g, key);
    if (!v || !out || v->kind != gguf::Value::STR)
        return fail(RFXQ_ERR_GGUF, "GGUF metadata '%s' missing or not a string", key ? key : "");
    *out = v->s.c_str();
    return ok();
}

int rfxq_gguf_meta_array_len(const rfxq_gguf* g, const char* key, uint64_t* out) {
    const gguf::Value* v = gguf_meta(g, key);
    if (!v || !out || v->kind != gguf::Value::ARRAY)
        return fail(RFXQ_ERR_GGUF, "GGUF metadata '%s' missing or not an array", key ? key : "");
    *out = v->arr.size();
    return ok();
}

// QuantArena::for_tensors (src/model/loading.rs:266-296): every tensor at a
// 256-byte aligned offset of one allocation
uint64_t rfxq_gguf_arena_size(const rfxq_gguf* g, const uint64_t* indices, uint32_t count) {
    if (!g || (!indices && count)) return 0;
    uint64_t total = 0;
    for (uint32_t j = 0; j < count; j++) {
        uint64_t start, nb;
        std::string err;
        if (indices[j] >= g->f.tensors.size() || !g->f.range(g->f.tensors[indices[j]], &start, &nb, &err)) return 0;
        total += align256(nb);
    }
    return total;
}

int rfxq_gguf_upload(const rfxq_gguf* g, const uint64_t* indices, uint32_t count, void* arena, uint64_t arena_bytes,
                     rfxq_weight* weights, hipStream_t stream) {
    if (!g || !arena || !weights || (!indices && count))
        return fail(RFXQ_ERR_INVALID_INPUT, "gguf_upload: NULL argument");
    if (reinterpret_cast<uintptr_t>(arena) % 256u)
        return fail(RFXQ_ERR_OTHER, "gguf_upload: arena is not 256-byte aligned");
    uint64_t used = 0;
    for (uint32_t j = 0; j < count; j++) {
        if (indices[j] >= g->f.tensors.size()) return fail(RFXQ_ERR_INVALID_INPUT, "gguf_upload: bad index");
        const gguf::Tensor& t = g->f.tensors[indices[j]];
        uint64_t start, nb;
        std::string err;
        if (!g->f.range(t, &start, &nb, &err)) return fail(RFXQ_ERR_GGUF, "%s", err.c_str());
        const uint64_t end = used + align256(nb);
        if (end > arena_bytes)
            return fail(RFXQ_ERR_OTHER, "quantized weight arena overflow: need %llu bytes, have %llu",
                        (unsigned long long)end, (unsigned long long)arena_bytes);
        uint8_t* dst = static_cast<uint8_t*>(arena) + used;
        HIPCHK(hipMemcpyAsync(dst, g->f.data + start, nb, hipMemcpyHostToDevice, stream), "gguf_upload copy");
        rfxq_weight& w = weights[j];
        w.ggml_type = t.type;
        w.in_features = t.dims.empty() ? 1u : (uint32_t)t.dims[0];
        w.out_features = t.dims.size() > 1 ? (uint32_t)t.dims[1] : 1u;
        w.expert_count = t.dims.size() > 2 ? (uint32_t)t.dims[2] : 0u;
        w.data = dst;
        w.len = nb;
        used = end;
    }
    return ok();
}

}  // extern "C"
