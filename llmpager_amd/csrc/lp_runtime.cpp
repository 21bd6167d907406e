// Host side of the C ABI (include/llmpager_hip.h): device runtime, code-object
// loading, launch geometry and shape checks for the gfx950 kernels.
//
// Mirrors crates/llmpager-cuda/src/driver.rs (Cuda) and src/kernels.rs
// (Kernels) of the reference.  Kernels are loaded from .hsaco code objects
// with hipModuleLoad and launched with hipModuleLaunchKernel, each taking one
// argument block from lp_kargs.h.
#include <dlfcn.h>
#include <hip/hip_runtime_api.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/llmpager_hip.h"
#include "lp_expf.h"
#include "lp_internal.h"
#include "lp_kargs.h"

using namespace lpk;

namespace {

thread_local std::string g_err;

int fail(int code, const std::string& msg) {
    g_err = msg;
    return code;
}

}  // namespace

int lpi::set_error(int code, const std::string& msg) { return fail(code, msg); }

namespace {

int hip_fail(hipError_t e, const char* what) {
    g_err = std::string(what) + " failed: " + hipGetErrorString(e) + " (" + std::to_string((int)e) + ")";
    return (int)e;
}

#define HIPCHK(expr)                                   \
    do {                                               \
        hipError_t e_ = (expr);                        \
        if (e_ != hipSuccess) return hip_fail(e_, #expr); \
    } while (0)

enum Fn {
    kQ4Mfma,
    kQ4Valu,
    kMoeReduce,
    kSiluMul,
    kBf16Gemv,
    kAdd,
    kRouter,
    kTopk,
    kGateup,
    kDown,
    kDownWide,
    kCombine,
    kXImage,
    kTopkDispatch,
    kExpfWave,
    kResolve,
    kGemmTiles,
    kGemmGateup,
    kGemmDown,
    kDispCount,
    kDispScan,
    kDispScatter,
    kGemmRouter,
    kDispatch,
    kRouteFused,
    kRouteFused128,
    kGateupBal,
    kGateupBal8,
    kGateupBalRs,
    kGateupBalRs8,
    kGateupBalSh,
    kDownBal,
    kDownBal6,
    kDownComb,
    kDownComb16,
    kDownCombRs,
    kRmsNorm,
    kScaleAdd,
    kKvAppendF32,
    kKvAppendF16,
    kRope,
    kBf16Row,
    kMlaRope,
    kBf16GemvBatch,
    kStridedCopy,
    kAttnSplitF32,
    kAttnSplitF16,
    kAttnCombine,
    kMlaSplit,
    kMlaCombine,
    kRmsNormGemv1,
    kRmsNormGemv2,
    kRmsNormGemv4,
    kRmsNormGemv8,
    kGemvAddRmsNorm1,
    kGemvAddRmsNorm2,
    kGemvAddRmsNorm4,
    kGemvAddRmsNorm8,
    kAttnFusedG1,
    kAttnFusedG2,
    kAttnFusedG4,
    kAttnFusedG8,
    kAttnFusedG16,
    kAttnBlockG1,
    kAttnBlockG2,
    kAttnBlockG4,
    kAttnBlockG8,
    kAttnBlockG16,
    kNumFns
};

struct FnSpec {
    const char* module;
    const char* name;
};

const FnSpec kSpecs[kNumFns] = {
    {"lp_basic.hsaco", "lp_q4_gemv_mfma"}, {"lp_basic.hsaco", "lp_q4_gemv_valu"},
    {"lp_basic.hsaco", "lp_moe_reduce"},   {"lp_basic.hsaco", "lp_silu_mul"},
    {"lp_basic.hsaco", "lp_bf16_gemv"},    {"lp_basic.hsaco", "lp_add"},
    {"lp_moe.hsaco", "lp_moe_router"},     {"lp_moe.hsaco", "lp_moe_topk"},
    {"lp_moe.hsaco", "lp_moe_gateup"},
    {"lp_moe.hsaco", "lp_moe_down"},       {"lp_moe.hsaco", "lp_moe_down_wide"},
    {"lp_moe.hsaco", "lp_moe_combine"},    {"lp_moe.hsaco", "lp_moe_ximage"},
    {"lp_moe.hsaco", "lp_moe_topk_dispatch"}, {"lp_basic.hsaco", "lp_expf_wave"},
    {"lp_moe.hsaco", "lp_moe_resolve"},
    {"lp_gemm.hsaco", "lp_gemm_tiles"},    {"lp_gemm.hsaco", "lp_gemm_gateup"},
    {"lp_gemm.hsaco", "lp_gemm_down"},
    {"lp_moe.hsaco", "lp_moe_disp_count"}, {"lp_moe.hsaco", "lp_moe_disp_scan"},
    {"lp_moe.hsaco", "lp_moe_disp_scatter"}, {"lp_gemm.hsaco", "lp_gemm_router"},
    {"lp_moe.hsaco", "lp_moe_dispatch"},   {"lp_moe.hsaco", "lp_moe_route_fused"},
    {"lp_moe.hsaco", "lp_moe_route_fused128"},
    {"lp_moe.hsaco", "lp_moe_gateup_bal"},  {"lp_moe.hsaco", "lp_moe_gateup_bal8"},
    {"lp_moe.hsaco", "lp_moe_gateup_bal_rs"},  {"lp_moe.hsaco", "lp_moe_gateup_bal_rs8"},
    {"lp_moe.hsaco", "lp_moe_gateup_bal_sh"},
    {"lp_moe.hsaco", "lp_moe_down_bal"},   {"lp_moe.hsaco", "lp_moe_down_bal6"},
    {"lp_moe.hsaco", "lp_moe_down_comb"},  {"lp_moe.hsaco", "lp_moe_down_comb16"},
    {"lp_moe.hsaco", "lp_moe_down_comb_rs"},
    {"lp_attn.hsaco", "lp_rmsnorm"},       {"lp_attn.hsaco", "lp_scale_add"},
    {"lp_attn.hsaco", "lp_kv_append_f32"}, {"lp_attn.hsaco", "lp_kv_append_f16"},
    {"lp_attn.hsaco", "lp_rope"},          {"lp_attn.hsaco", "lp_bf16_row_to_f32"},
    {"lp_attn.hsaco", "lp_mla_rope"},      {"lp_attn.hsaco", "lp_bf16_gemv_batch"},
    {"lp_attn.hsaco", "lp_strided_copy"},  {"lp_attn.hsaco", "lp_attn_split_f32"},
    {"lp_attn.hsaco", "lp_attn_split_f16"}, {"lp_attn.hsaco", "lp_attn_combine"},
    {"lp_attn.hsaco", "lp_mla_split"},     {"lp_attn.hsaco", "lp_mla_combine"},
    {"lp_step.hsaco", "lp_rmsnorm_gemv_c1"}, {"lp_step.hsaco", "lp_rmsnorm_gemv_c2"},
    {"lp_step.hsaco", "lp_rmsnorm_gemv_c4"}, {"lp_step.hsaco", "lp_rmsnorm_gemv_c8"},
    {"lp_step.hsaco", "lp_gemv_add_rmsnorm_c1"}, {"lp_step.hsaco", "lp_gemv_add_rmsnorm_c2"},
    {"lp_step.hsaco", "lp_gemv_add_rmsnorm_c4"}, {"lp_step.hsaco", "lp_gemv_add_rmsnorm_c8"},
    {"lp_step.hsaco", "lp_attn_fused_g1"}, {"lp_step.hsaco", "lp_attn_fused_g2"},
    {"lp_step.hsaco", "lp_attn_fused_g4"}, {"lp_step.hsaco", "lp_attn_fused_g8"},
    {"lp_step.hsaco", "lp_attn_fused_g16"},
    {"lp_step.hsaco", "lp_attn_block_g1"}, {"lp_step.hsaco", "lp_attn_block_g2"},
    {"lp_step.hsaco", "lp_attn_block_g4"}, {"lp_step.hsaco", "lp_attn_block_g8"},
    {"lp_step.hsaco", "lp_attn_block_g16"},
};

const char* const kModules[] = {"lp_basic.hsaco", "lp_moe.hsaco", "lp_gemm.hsaco", "lp_attn.hsaco",
                                "lp_step.hsaco"};
constexpr int kNumModules = 5;

std::string library_dir() {
    Dl_info info;
    if (dladdr(reinterpret_cast<void*>(&lp_version), &info) && info.dli_fname) {
        std::string p(info.dli_fname);
        size_t cut = p.rfind('/');
        if (cut != std::string::npos) return p.substr(0, cut);
    }
    return ".";
}

uint64_t align256(uint64_t v) { return (v + 255) & ~uint64_t(255); }

// grid_1d of kernels.rs:39-41: min(ceil(n / 256), 1024), at least 1.
unsigned grid_1d(int n) {
    unsigned g = (unsigned)((n + 255) / 256);
    return std::max(1u, std::min(g, 1024u));
}

}  // namespace

struct ProfRec {
    int fn;
    hipEvent_t start, end;
};

struct lp_ctx {
    int device = 0;
    int cus = 0;
    size_t max_lds = 0;
    hipModule_t modules[kNumModules] = {};
    hipFunction_t fns[kNumFns] = {};
    // measurement (lp_profile_*)
    bool prof = false;
    std::mutex prof_mu;
    std::vector<ProfRec> prof_recs;
    std::vector<hipEvent_t> prof_pool;
    double prof_ms[kNumFns] = {};
    int64_t prof_n[kNumFns] = {};
    // arrival counters of the fused routing kernel: kSyncSlots slots of
    // kSyncWords, zero between launches.  A slot belongs to one stream (the
    // first kSyncSlots streams that route through the context get one each):
    // launches on one stream run one after another, so they may share it,
    // and launches on different streams never do.
    // A graph captured by lp_moe_stack_capture keeps a slot of its own for
    // its whole life (its kernel nodes hold the slot's address), so that
    // destroying the capture stream and routing on a stream created later
    // never shares counters with the graph's replays.
    int32_t* sync = nullptr;
    std::mutex sync_mu;
    hipStream_t sync_owner[kSyncSlots] = {};  // slot i belongs to sync_owner[i] when sync_used[i]
    bool sync_used[kSyncSlots] = {};
    bool sync_graph[kSyncSlots] = {};         // slot i belongs to a graph (sync_owner unused)
    hipStream_t cap_stream = nullptr;         // a capture in progress on this stream ...
    int cap_slot = -1;                        // ... routes through this (the graph's) slot
    bool cap_prof = false;                    // lp_graph_capture_begin: the profiling switch to restore
    int step_spin = kStepSpinMax;             // polls before lp_attn_block's wait gives up
    // decode gate/up through lp_moe_gateup_bal (LLMPAGER_HIP_GATEUP_BAL=0 at
    // lp_init turns it off, for comparison)
    bool gateup_bal = true;
};

int lpi::ctx_device(const lp_ctx* c) { return c ? c->device : -1; }

namespace {

hipEvent_t prof_event(lp_ctx* c) {
    if (!c->prof_pool.empty()) {
        hipEvent_t e = c->prof_pool.back();
        c->prof_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

// Fold completed records into the per-kernel sums (caller holds prof_mu and
// has synchronised the device).
void prof_drain(lp_ctx* c) {
    for (const ProfRec& r : c->prof_recs) {
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, r.start, r.end) == hipSuccess) {
            c->prof_ms[r.fn] += ms;
            c->prof_n[r.fn] += 1;
        }
        c->prof_pool.push_back(r.start);
        c->prof_pool.push_back(r.end);
    }
    c->prof_recs.clear();
}

}  // namespace

// hip_ext.h's launch with events attached to the dispatch (declared here:
// that header also holds templates only the HIP compiler takes).
extern "C" hipError_t hipExtModuleLaunchKernel(hipFunction_t f, uint32_t globalWorkSizeX, uint32_t globalWorkSizeY,
                                               uint32_t globalWorkSizeZ, uint32_t localWorkSizeX,
                                               uint32_t localWorkSizeY, uint32_t localWorkSizeZ,
                                               size_t sharedMemBytes, hipStream_t hStream, void** kernelParams,
                                               void** extra, hipEvent_t startEvent, hipEvent_t stopEvent,
                                               uint32_t flags);

namespace {

// Launch f; when profiling, the dispatch itself carries a start and a stop
// event (hipExtModuleLaunchKernel takes the kernel's own begin and end
// timestamps, not those of separate event packets around it).
template <typename A>
int launch(lp_ctx* c, Fn f, dim3 grid, dim3 block, size_t lds, lp_stream s, const A& args) {
    void* params[] = {const_cast<A*>(&args)};
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (c->prof) {
        std::lock_guard<std::mutex> g(c->prof_mu);
        e0 = prof_event(c);
        e1 = prof_event(c);
    }
    hipError_t e;
    if (e0 && e1) {
        e = hipExtModuleLaunchKernel(c->fns[f], grid.x * block.x, grid.y * block.y, grid.z * block.z, block.x,
                                     block.y, block.z, lds, (hipStream_t)s, params, nullptr, e0, e1, 0);
        std::lock_guard<std::mutex> g(c->prof_mu);
        if (e == hipSuccess) {
            c->prof_recs.push_back(ProfRec{(int)f, e0, e1});
        } else {
            c->prof_pool.push_back(e0);
            c->prof_pool.push_back(e1);
        }
    } else {
        if (e0 || e1) {
            std::lock_guard<std::mutex> g(c->prof_mu);
            if (e0) c->prof_pool.push_back(e0);
            if (e1) c->prof_pool.push_back(e1);
        }
        e = hipModuleLaunchKernel(c->fns[f], grid.x, grid.y, grid.z, block.x, block.y, block.z, (unsigned)lds,
                                  (hipStream_t)s, params, nullptr);
    }
    if (e != hipSuccess) return hip_fail(e, kSpecs[f].name);
    return LP_OK;
}

int check_ctx(lp_ctx* c) {
    if (!c) return fail(LP_E_INVALID, "null context");
    return LP_OK;
}

}  // namespace

extern "C" {

const char* lp_last_error(void) { return g_err.c_str(); }

const char* lp_version(void) { return "llmpager-hip 0.1.0 (gfx950)"; }

// ---- device runtime ----------------------------------------------------------

int lp_init(int device, const char* hsaco_dir, lp_ctx** out) {
    if (!out) return fail(LP_E_INVALID, "lp_init: null out");
    *out = nullptr;
    HIPCHK(hipSetDevice(device));
    lp_ctx* c = new lp_ctx();
    c->device = device;
    hipDeviceProp_t prop;
    hipError_t e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) {
        delete c;
        return hip_fail(e, "hipGetDeviceProperties");
    }
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        delete c;
        return fail(LP_E_UNSUPPORTED, std::string("device is ") + prop.gcnArchName +
                                          ", the kernels are built for gfx950 only");
    }
    c->cus = prop.multiProcessorCount;
    c->max_lds = prop.sharedMemPerBlock;
    if (const char* e = std::getenv("LLMPAGER_HIP_GATEUP_BAL")) c->gateup_bal = std::atoi(e) != 0;
    // tests only: a smaller bound on the fused step's waits, to exercise giving up
    if (const char* e = std::getenv("LLMPAGER_HIP_STEP_SPIN")) c->step_spin = std::max(1, std::min(kStepSpinMax, std::atoi(e)));
    if (const char* e = std::getenv("LLMPAGER_HIP_BAL_WAVES")) {
        // The balanced kernels run at kBalWaves waves only: a 16-wave build
        // of lp_moe_gateup_bal faulted and was never fixed, so no other
        // workgroup size is offered.
        if (std::atoi(e) != kBalWaves) {
            delete c;
            return fail(LP_E_UNSUPPORTED, "LLMPAGER_HIP_BAL_WAVES: the balanced kernels run at " +
                                              std::to_string(kBalWaves) + " waves only");
        }
    }
    const std::string dir = hsaco_dir ? std::string(hsaco_dir) : library_dir();
    for (int m = 0; m < kNumModules; ++m) {
        const std::string path = dir + "/" + kModules[m];
        e = hipModuleLoad(&c->modules[m], path.c_str());
        if (e != hipSuccess) {
            lp_destroy(c);
            return fail(LP_E_LOAD, "hipModuleLoad(" + path + "): " + hipGetErrorString(e));
        }
    }
    for (int f = 0; f < kNumFns; ++f) {
        int m = 0;
        while (m < kNumModules && strcmp(kModules[m], kSpecs[f].module) != 0) ++m;
        e = hipModuleGetFunction(&c->fns[f], c->modules[m], kSpecs[f].name);
        if (e != hipSuccess) {
            lp_destroy(c);
            return fail(LP_E_LOAD, std::string("hipModuleGetFunction(") + kSpecs[f].name +
                                       "): " + hipGetErrorString(e));
        }
    }
    {
        // the loaded code objects must take the balanced kernels' fixed
        // workgroup size (their launch bound)
        for (Fn f : {kGateupBal, kGateupBal8, kGateupBalRs, kGateupBalRs8, kGateupBalSh, kDownBal, kDownBal6, kDownComb,
                     kDownComb16, kDownCombRs}) {
            const int need = 64 * (f == kDownComb || f == kDownComb16 || f == kDownCombRs ? kCombWaves : kBalWaves);
            int mt = 0;
            if (hipFuncGetAttribute(&mt, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, c->fns[f]) != hipSuccess ||
                mt < need) {
                lp_destroy(c);
                return fail(LP_E_LOAD, std::string(kSpecs[f].name) + ": code object does not take " +
                                           std::to_string(need) + "-thread workgroups");
            }
        }
    }
    if (int r = lpi::noalloc_setup(device)) {
        lp_destroy(c);
        return r;
    }
    e = hipMalloc(reinterpret_cast<void**>(&c->sync), (size_t)kSyncSlots * kSyncWords * 4);
    if (e == hipSuccess) e = hipMemset(c->sync, 0, (size_t)kSyncSlots * kSyncWords * 4);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        lp_destroy(c);
        return hip_fail(e, "lp_init: arrival counters");
    }
    *out = c;
    return LP_OK;
}

void lp_destroy(lp_ctx* c) {
    if (!c) return;
    for (const ProfRec& r : c->prof_recs) {
        (void)hipEventDestroy(r.start);
        (void)hipEventDestroy(r.end);
    }
    for (hipEvent_t e : c->prof_pool) (void)hipEventDestroy(e);
    for (int m = 0; m < kNumModules; ++m)
        if (c->modules[m]) (void)hipModuleUnload(c->modules[m]);
    if (c->sync) {
        (void)hipDeviceSynchronize();
        (void)hipFree(c->sync);
    }
    delete c;
}

int lp_bind_thread(lp_ctx* c) {
    if (int r = check_ctx(c)) return r;
    HIPCHK(hipSetDevice(c->device));
    return LP_OK;
}

int lp_mem_info(lp_ctx* c, uint64_t* free_bytes, uint64_t* total_bytes) {
    if (int r = check_ctx(c)) return r;
    size_t f = 0, t = 0;
    HIPCHK(hipMemGetInfo(&f, &t));
    if (free_bytes) *free_bytes = f;
    if (total_bytes) *total_bytes = t;
    return LP_OK;
}

int lp_alloc_device(lp_ctx* c, size_t bytes, uint64_t* out) {
    if (int r = check_ctx(c)) return r;
    if (!out) return fail(LP_E_INVALID, "lp_alloc_device: null out");
    void* p = nullptr;
    HIPCHK(hipMalloc(&p, std::max<size_t>(bytes, 1)));
    *out = reinterpret_cast<uint64_t>(p);
    return LP_OK;
}

int lp_free_device(lp_ctx* c, uint64_t ptr) {
    if (int r = check_ctx(c)) return r;
    HIPCHK(hipFree(reinterpret_cast<void*>(ptr)));
    return LP_OK;
}

int lp_alloc_pinned(lp_ctx* c, size_t bytes, void** out) {
    if (int r = check_ctx(c)) return r;
    if (!out) return fail(LP_E_INVALID, "lp_alloc_pinned: null out");
    HIPCHK(hipHostMalloc(out, std::max<size_t>(bytes, 1), hipHostMallocDefault));
    return LP_OK;
}

int lp_free_pinned(lp_ctx* c, void* p) {
    if (int r = check_ctx(c)) return r;
    HIPCHK(hipHostFree(p));
    return LP_OK;
}

int lp_stream_create(lp_ctx* c, lp_stream* out) {
    if (int r = check_ctx(c)) return r;
    hipStream_t s;
    HIPCHK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    *out = s;
    return LP_OK;
}

int lp_stream_destroy(lp_ctx* c, lp_stream s) {
    if (int r = check_ctx(c)) return r;
    {
        // a stream that owns arrival counters gives them up once its work is
        // done, so a stream created later may take them
        std::lock_guard<std::mutex> g(c->sync_mu);
        for (int i = 0; i < kSyncSlots; ++i) {
            if (c->sync_used[i] && !c->sync_graph[i] && c->sync_owner[i] == (hipStream_t)s) {
                HIPCHK(hipStreamSynchronize((hipStream_t)s));
                c->sync_used[i] = false;
                break;
            }
        }
    }
    HIPCHK(hipStreamDestroy((hipStream_t)s));
    return LP_OK;
}

int lp_event_create(lp_ctx* c, lp_event* out) {
    if (int r = check_ctx(c)) return r;
    hipEvent_t e;
    HIPCHK(hipEventCreate(&e));
    *out = e;
    return LP_OK;
}

int lp_event_destroy(lp_ctx* c, lp_event e) {
    if (int r = check_ctx(c)) return r;
    HIPCHK(hipEventDestroy((hipEvent_t)e));
    return LP_OK;
}

int lp_htod_async(lp_ctx* c, uint64_t dst, const void* src, size_t bytes, lp_stream s) {
    if (int r = check_ctx(c)) return r;
    HIPCHK(hipMemcpyAsync(reinterpret_cast<void*>(dst), src, bytes, hipMemcpyHostToDevice,
                          (hipStream_t)s));
    return LP_OK;
}

int lp_dtoh_async(lp_ctx* c, void* dst, uint64_t src, size_t bytes, lp_stream s) {
    if (int r = check_ctx(c)) return r;
    HIPCHK(hipMemcpyAsync(dst, reinterpret_cast<const void*>(src), bytes, hipMemcpyDeviceToHost,
                          (hipStream_t)s));
    return LP_OK;
}

int lp_dtod_async(lp_ctx* c, uint64_t dst, uint64_t src, size_t bytes, lp_stream s) {
    if (int r = check_ctx(c)) return r;
    HIPCHK(hipMemcpyAsync(reinterpret_cast<void*>(dst), reinterpret_cast<const void*>(src), bytes,
                          hipMemcpyDeviceToDevice, (hipStream_t)s));
    return LP_OK;
}

int lp_memset_async(lp_ctx* c, uint64_t dst, int value, size_t bytes, lp_stream s) {
    if (int r = check_ctx(c)) return r;
    HIPCHK(hipMemsetAsync(reinterpret_cast<void*>(dst), value, bytes, (hipStream_t)s));
    return LP_OK;
}

int lp_record_event(lp_ctx* c, lp_event e, lp_stream s) {
    if (int r = check_ctx(c)) return r;
    HIPCHK(hipEventRecord((hipEvent_t)e, (hipStream_t)s));
    return LP_OK;
}

int lp_sync_event(lp_ctx* c, lp_event e) {
    if (int r = check_ctx(c)) return r;
    HIPCHK(hipEventSynchronize((hipEvent_t)e));
    return LP_OK;
}

int lp_event_done(lp_ctx* c, lp_event e) {
    if (int r = check_ctx(c)) return r;
    hipError_t q = hipEventQuery((hipEvent_t)e);
    if (q == hipSuccess) return 1;
    if (q == hipErrorNotReady) return 0;
    return hip_fail(q, "hipEventQuery");
}

int lp_event_elapsed_ms(lp_ctx* c, lp_event a, lp_event b, float* ms) {
    if (int r = check_ctx(c)) return r;
    HIPCHK(hipEventElapsedTime(ms, (hipEvent_t)a, (hipEvent_t)b));
    return LP_OK;
}

int lp_stream_wait_event(lp_ctx* c, lp_stream s, lp_event e) {
    if (int r = check_ctx(c)) return r;
    HIPCHK(hipStreamWaitEvent((hipStream_t)s, (hipEvent_t)e, 0));
    return LP_OK;
}

int lp_sync_stream(lp_ctx* c, lp_stream s) {
    if (int r = check_ctx(c)) return r;
    HIPCHK(hipStreamSynchronize((hipStream_t)s));
    return LP_OK;
}

int lp_sync(lp_ctx* c) {
    if (int r = check_ctx(c)) return r;
    HIPCHK(hipDeviceSynchronize());
    return LP_OK;
}

// ---- 1:1 launchers --------------------------------------------------------------

static int q4_gemv_common(lp_ctx* c, uint64_t blobs, uint64_t region_off, uint64_t x, int x_stride,
                          uint64_t y, int rows, int cols, int group, int experts, lp_stream s,
                          bool direct) {
    if (int r = check_ctx(c)) return r;
    if (rows <= 0 || cols <= 0 || experts <= 0 || group <= 0 || group % 8 != 0 || cols % group != 0)
        return fail(LP_E_INVALID, "q4 gemv: need group % 8 == 0 and cols % group == 0 (quant.rs:44-46)");
    Q4GemvBatchArgs a{};
    a.blobs = direct ? 0 : blobs;
    a.region_off = region_off;
    a.x = x;
    a.x_stride = x_stride;
    a.y = y;
    a.rows = rows;
    a.cols = cols;
    a.group = group;
    a.experts = experts;
    // The MFMA tile needs 32-column sub-groups (a power-of-two number of them
    // under one scale), 16-byte aligned nibble rows and x, and one LDS
    // fragment pair.
    const uint64_t data_off = region_off + (uint64_t)rows * (cols / group) * 2;
    const bool aligned = (data_off % 16 == 0) && (x % 16 == 0) && ((uint64_t)x_stride * 4 % 16 == 0);
    const bool pow2 = group % 32 == 0 && ((group / 32) & (group / 32 - 1)) == 0;
    const size_t frag = (size_t)frag_lds_bytes(cols, 1);
    if (pow2 && aligned && frag <= c->max_lds) {
        const int tiles = (rows + kTileRows - 1) / kTileRows;
        const int waves = std::min(4, tiles);
        const unsigned gx = (unsigned)((tiles + waves - 1) / waves);
        return launch(c, kQ4Mfma, dim3(gx, experts), dim3(64 * waves), frag, s, a);
    }
    return launch(c, kQ4Valu, dim3((rows + 3) / 4, experts), dim3(256), 0, s, a);
}

int lp_q4_gemv_batch(lp_ctx* c, uint64_t blobs, uint64_t region_off, uint64_t x, int x_stride,
                     uint64_t y, int rows, int cols, int group, int experts, lp_stream s) {
    return q4_gemv_common(c, blobs, region_off, x, x_stride, y, rows, cols, group, experts, s, false);
}

int lp_q4_gemv(lp_ctx* c, uint64_t blob, uint64_t x, uint64_t y, int rows, int cols, int group,
               lp_stream s) {
    return q4_gemv_common(c, 0, blob, x, 0, y, rows, cols, group, 1, s, true);
}

int lp_moe_reduce(lp_ctx* c, uint64_t eouts, uint64_t wts, uint64_t out, int experts, int n,
                  lp_stream s) {
    if (int r = check_ctx(c)) return r;
    if (n < 0 || experts < 0) return fail(LP_E_INVALID, "moe_reduce: negative size");
    MoeReduceArgs a{eouts, wts, out, experts, n};
    return launch(c, kMoeReduce, dim3(grid_1d(n)), dim3(256), 0, s, a);
}

int lp_silu_mul(lp_ctx* c, uint64_t gate, uint64_t up, uint64_t out, int n, lp_stream s) {
    if (int r = check_ctx(c)) return r;
    if (n < 0) return fail(LP_E_INVALID, "silu_mul: negative size");
    SiluMulArgs a{gate, up, out, n, 0};
    return launch(c, kSiluMul, dim3(grid_1d(n)), dim3(256), 0, s, a);
}

int lp_bf16_gemv(lp_ctx* c, uint64_t w, uint64_t x, uint64_t y, int rows, int cols, lp_stream s) {
    if (int r = check_ctx(c)) return r;
    if (rows <= 0 || cols <= 0) return fail(LP_E_INVALID, "bf16_gemv: empty shape");
    if (cols % 8 == 0 && (w % 16 != 0 || x % 16 != 0))
        return fail(LP_E_UNSUPPORTED, "bf16_gemv: w and x must be 16-byte aligned");
    Bf16GemvArgs a{w, x, y, rows, cols};
    return launch(c, kBf16Gemv, dim3((rows + 3) / 4), dim3(256), 0, s, a);
}

int lp_add(lp_ctx* c, uint64_t pa, uint64_t pb, int n, lp_stream s) {
    if (int r = check_ctx(c)) return r;
    if (n < 0) return fail(LP_E_INVALID, "add: negative size");
    AddArgs a{pa, pb, n, 0};
    return launch(c, kAdd, dim3(grid_1d(n)), dim3(256), 0, s, a);
}

// ---- the rest of the decode step (decode.cu) and MLA (mla.cu) ----------------------

int lp_rmsnorm(lp_ctx* c, uint64_t x, uint64_t w, uint64_t y, int rows, int n, float eps, lp_stream s) {
    if (int r = check_ctx(c)) return r;
    if (rows < 0 || n <= 0) return fail(LP_E_INVALID, "rmsnorm: bad shape");
    if (rows == 0) return LP_OK;
    RmsNormArgs a{x, w, y, n, eps};
    return launch(c, kRmsNorm, dim3((unsigned)rows), dim3(256), 0, s, a);
}

int lp_scale_add(lp_ctx* c, uint64_t pa, uint64_t pb, float sc, int n, lp_stream s) {
    if (int r = check_ctx(c)) return r;
    if (n < 0) return fail(LP_E_INVALID, "scale_add: negative size");
    ScaleAddArgs a{pa, pb, sc, n};
    return launch(c, kScaleAdd, dim3(grid_1d(n)), dim3(256), 0, s, a);
}

int lp_kv_append(lp_ctx* c, uint64_t k, uint64_t v, uint64_t kcache, uint64_t vcache, int kv_heads,
                 int head_dim, int pos, int max_seq, int f16, lp_stream s) {
    if (int r = check_ctx(c)) return r;
    if (kv_heads <= 0 || head_dim <= 0 || pos < 0 || pos >= max_seq)
        return fail(LP_E_INVALID, "kv_append: need 0 <= pos < max_seq and a non-empty head");
    KvAppendArgs a{k, v, kcache, vcache, kv_heads, head_dim, pos, max_seq};
    return launch(c, f16 ? kKvAppendF16 : kKvAppendF32, dim3(grid_1d(kv_heads * head_dim)), dim3(256), 0, s, a);
}

int lp_rope(lp_ctx* c, uint64_t x, int heads, int head_dim, int pos, float base, lp_stream s) {
    if (int r = check_ctx(c)) return r;
    if (heads <= 0 || head_dim <= 0 || head_dim % 2) return fail(LP_E_INVALID, "rope: head_dim must be even");
    RopeArgs a{x, heads, head_dim, pos, base};
    return launch(c, kRope, dim3(grid_1d(heads * head_dim / 2)), dim3(256), 0, s, a);
}

int lp_bf16_row(lp_ctx* c, uint64_t table, int row, int n, uint64_t out, lp_stream s) {
    if (int r = check_ctx(c)) return r;
    if (row < 0 || n < 0) return fail(LP_E_INVALID, "bf16_row: bad row or size");
    RowArgs a{table, out, row, n};
    return launch(c, kBf16Row, dim3(grid_1d(n)), dim3(256), 0, s, a);
}

int lp_mla_rope(lp_ctx* c, uint64_t x, int n_vecs, int stride, int offset, int half, int pos,
                uint64_t inv_freq, float mscale, lp_stream s) {
    if (int r = check_ctx(c)) return r;
    if (n_vecs < 0 || half < 0 || offset < 0 || offset + 2 * half > stride)
        return fail(LP_E_INVALID, "mla_rope: the rope slice must lie inside each vector");
    MlaRopeArgs a{x, inv_freq, n_vecs, stride, offset, half, pos, mscale};
    return launch(c, kMlaRope, dim3(grid_1d(n_vecs * half)), dim3(256), 0, s, a);
}

int lp_bf16_gemv_batch(lp_ctx* c, uint64_t w, uint64_t w_stride, uint64_t x, int x_stride, uint64_t y,
                       int y_stride, int rows, int cols, int batch, lp_stream s) {
    if (int r = check_ctx(c)) return r;
    if (rows <= 0 || cols <= 0 || batch <= 0 || x_stride < 0 || y_stride < 0)
        return fail(LP_E_INVALID, "bf16_gemv_batch: bad shape");
    Bf16GemvBatchArgs a{w, w_stride, x, y, x_stride, y_stride, rows, cols, batch, 0};
    return launch(c, kBf16GemvBatch, dim3((unsigned)((rows + 3) / 4), (unsigned)batch), dim3(256), 0, s, a);
}

int lp_strided_copy(lp_ctx* c, uint64_t src, int src_stride, int src_off, uint64_t dst, int dst_stride,
                    int dst_off, int n_vecs, int n, lp_stream s) {
    if (int r = check_ctx(c)) return r;
    if (n_vecs < 0 || n < 0) return fail(LP_E_INVALID, "strided_copy: negative size");
    StridedCopyArgs a{src, dst, src_stride, src_off, dst_stride, dst_off, n_vecs, n};
    return launch(c, kStridedCopy, dim3(grid_1d(n_vecs * n)), dim3(256), 0, s, a);
}

// Split decode attention: splits so that the grid fills the chip, each split
// at most kAttnSpanMax positions (and at least 32), the partial records in
// the caller's scratch [heads, max_seq] (splits * (out_dim + 2) floats per
// head); one split writes the output directly.
static int attn_launch(lp_ctx* c, AttnArgs a, int max_seq, lp_stream s) {
    if (a.seq_len < 1 || a.seq_len > max_seq) return fail(LP_E_INVALID, "attention: need 1 <= seq_len <= max_seq");
    if (a.dot_dim < 1 || a.dot_dim > 1024 || a.out_dim < 1 || a.out_dim > a.row_stride || a.dot_dim > a.row_stride)
        return fail(LP_E_UNSUPPORTED, "attention: dims must be 1..1024 and fit a cache row");
    const int by_span = (a.seq_len + kAttnSpanMax - 1) / kAttnSpanMax;
    const int by_scratch = max_seq / (a.out_dim + 2);
    int splits = std::max(1, (2 * c->cus + a.heads - 1) / a.heads);
    splits = std::min(splits, std::max(1, (a.seq_len + 31) / 32));
    splits = std::min(splits, std::max(1, by_scratch));
    splits = std::max(splits, by_span);
    if (splits > 1 && splits > by_scratch)
        return fail(LP_E_UNSUPPORTED, "attention: the scratch cannot hold the split records");
    a.span = (a.seq_len + splits - 1) / splits;
    a.splits = (a.seq_len + a.span - 1) / a.span;
    a.scratch_stride = max_seq;
    if (int r = launch(c, a.f16 ? kAttnSplitF16 : kAttnSplitF32, dim3((unsigned)a.heads, (unsigned)a.splits),
                       dim3(256), 0, s, a))
        return r;
    if (a.splits == 1) return LP_OK;
    return launch(c, kAttnCombine, dim3((unsigned)a.heads), dim3(256), 0, s, a);
}

int lp_attn_decode(lp_ctx* c, uint64_t q, uint64_t kcache, uint64_t vcache, uint64_t out, uint64_t scratch,
                   int heads, int kv_heads, int head_dim, int seq_len, int max_seq, float scale, int f16,
                   lp_stream s) {
    if (int r = check_ctx(c)) return r;
    if (heads <= 0 || kv_heads <= 0 || heads % kv_heads)
        return fail(LP_E_INVALID, "attn_decode: heads must be a multiple of kv_heads");
    AttnArgs a{};
    a.q = q;
    a.k = kcache;
    a.v = vcache;
    a.out = out;
    a.scratch = scratch;
    a.kv_stride = (uint64_t)max_seq * head_dim;
    a.heads = heads;
    a.group = heads / kv_heads;
    a.dot_dim = a.out_dim = a.row_stride = head_dim;
    a.seq_len = seq_len;
    a.scale = scale;
    a.f16 = f16 != 0;
    return attn_launch(c, a, max_seq, s);
}

int lp_mla_attn_decode(lp_ctx* c, uint64_t q, uint64_t cache, uint64_t ctx, uint64_t scratch, int heads,
                       int qk_dim, int c_dim, int seq_len, int max_seq, float scale, lp_stream s) {
    if (int r = check_ctx(c)) return r;
    if (heads <= 0 || c_dim > qk_dim) return fail(LP_E_INVALID, "mla_attn_decode: need heads >= 1, c_dim <= qk_dim");
    AttnArgs a{};
    a.q = q;
    a.k = a.v = cache;
    a.out = ctx;
    a.scratch = scratch;
    a.kv_stride = 0;  // one cache shared by every head (MQA)
    a.heads = heads;
    a.group = heads;
    a.dot_dim = qk_dim;
    a.out_dim = c_dim;
    a.row_stride = qk_dim;
    a.seq_len = seq_len;
    a.scale = scale;
    return attn_launch(c, a, max_seq, s);
}

// The batched MLA decode's split plan: about one workgroup per CU over the
// batch, each split a whole number of 64-row chunks.
static void mla_plan(const lp_ctx* c, int batch, int max_seq, int* splits, int* span) {
    const int chunks = std::max(1, (max_seq + kMlaRows - 1) / kMlaRows);
    int sp = std::max(1, std::min({chunks, (c->cus + batch - 1) / batch, kMlaMaxSplits}));
    const int per = (chunks + sp - 1) / sp;
    *span = per * kMlaRows;
    *splits = (max_seq + *span - 1) / *span;
}

uint64_t lp_mla_batch_ws_bytes(lp_ctx* c, int batch, int c_dim, int max_seq) {
    if (!c || batch <= 0 || c_dim <= 0 || max_seq <= 0) return 0;
    int splits, span;
    mla_plan(c, batch, max_seq, &splits, &span);
    return (uint64_t)batch * splits * mla_part_floats(c_dim) * 4;
}

int lp_mla_attn_decode_batch(lp_ctx* c, uint64_t q, uint64_t cache, uint64_t cache_stride, uint64_t seq_lens,
                             uint64_t ctx_out, uint64_t workspace, int batch, int heads, int qk_dim, int c_dim,
                             int max_seq, float scale, lp_stream s) {
    if (int r = check_ctx(c)) return r;
    const int steps = qk_dim / 32;
    const bool steps_ok = qk_dim % 32 == 0 && (steps == 3 || steps == 4 || steps == 6 || steps == 8 || steps == 12 ||
                                               steps == 16 || steps == 18 || steps == 20);
    if (batch <= 0 || heads <= 0 || heads > 16 || !steps_ok || c_dim <= 0 || c_dim % 64 || c_dim > kMlaMaxC ||
        c_dim > qk_dim || max_seq <= 0)
        return fail(LP_E_UNSUPPORTED, "mla_attn_decode_batch: heads <= 16, qk_dim = 32 x {3,4,6,8,12,16,18,20}, "
                                      "c_dim a multiple of 64 up to 512 and <= qk_dim");
    if ((uint64_t)max_seq * qk_dim * 2 >= (1ull << 31) || cache % 16 || cache_stride % 16 || q % 16)
        return fail(LP_E_UNSUPPORTED, "mla_attn_decode_batch: q and the caches must be 16-byte aligned, "
                                      "each cache under 2 GiB");
    const size_t lds = (size_t)mla_lds_bytes(qk_dim, c_dim);
    if (lds > c->max_lds) return fail(LP_E_UNSUPPORTED, "mla_attn_decode_batch: LDS");
    MlaBatchArgs a{};
    a.q = q;
    a.cache = cache;
    a.cache_stride = cache_stride;
    a.seq_lens = seq_lens;
    a.ctx = ctx_out;
    a.part = workspace;
    a.batch = batch;
    a.heads = heads;
    a.qk_dim = qk_dim;
    a.c_dim = c_dim;
    a.scale = scale;
    a.max_seq = max_seq;
    mla_plan(c, batch, max_seq, &a.splits, &a.span);
    if (int r = launch(c, kMlaSplit, dim3((unsigned)a.splits, (unsigned)batch), dim3(256), lds, s, a)) return r;
    return launch(c, kMlaCombine, dim3((unsigned)heads, (unsigned)batch, (unsigned)(c_dim / 64)), dim3(256), 0, s,
                  a);
}

// ---- the fused decode step (lp_step.hip) ------------------------------------------

static int sync_slot(lp_ctx* c, lp_stream s);

static uint64_t sync_words(lp_ctx* c, int slot) {
    return reinterpret_cast<uint64_t>(c->sync) + (uint64_t)slot * kSyncWords * 4;
}

// the 8-column chunks per lane of a fused GEMV: 1, 2, 4 or 8 (cols <= 4096)
static int gemv_cpl(int cols) {
    const int cpl = (cols + 511) / 512;
    return cpl <= 1 ? 1 : cpl <= 2 ? 2 : cpl <= 4 ? 4 : 8;
}

static int gemv_index(int cpl) { return cpl == 1 ? 0 : cpl == 2 ? 1 : cpl == 4 ? 2 : 3; }

int lp_rmsnorm_gemv(lp_ctx* c, uint64_t x, uint64_t ln, float eps, int cols, uint64_t w0, int rows0, uint64_t y0,
                    uint64_t w1, int rows1, uint64_t y1, uint64_t w2, int rows2, uint64_t y2, lp_stream s) {
    if (int r = check_ctx(c)) return r;
    if (cols <= 0 || rows0 <= 0 || rows1 < 0 || rows2 < 0 || (rows2 > 0 && rows1 == 0))
        return fail(LP_E_INVALID, "rmsnorm_gemv: empty shape");
    if (cols % 8 || cols > kFusedGemvMaxCols)
        return fail(LP_E_UNSUPPORTED, "rmsnorm_gemv: cols must be a multiple of 8, at most " +
                                          std::to_string(kFusedGemvMaxCols));
    if (x % 16 || w0 % 16 || (rows1 && w1 % 16) || (rows2 && w2 % 16))
        return fail(LP_E_UNSUPPORTED, "rmsnorm_gemv: x and the matrices must be 16-byte aligned");
    if ((ln && ln % 16) || !x || !w0 || !y0 || (rows1 && (!w1 || !y1)) || (rows2 && (!w2 || !y2)))
        return fail(LP_E_INVALID, "rmsnorm_gemv: null or misaligned pointer");
    const long total = (long)rows0 + rows1 + rows2;
    if (total > (long)INT32_MAX - 8) return fail(LP_E_UNSUPPORTED, "rmsnorm_gemv: too many rows");
    RmsNormGemvArgs a{};
    a.x = x;
    a.ln = ln;
    a.w0 = w0, a.w1 = w1, a.w2 = w2;
    a.y0 = y0, a.y1 = y1, a.y2 = y2;
    a.rows0 = rows0, a.rows1 = rows1, a.rows2 = rows2;
    a.cols = cols;
    a.eps = eps;
    const Fn f = (Fn)(kRmsNormGemv1 + gemv_index(gemv_cpl(cols)));
    constexpr int rpb = 4 * kFusedGemvRowsPerWave;
    return launch(c, f, dim3((unsigned)((total + rpb - 1) / rpb)), dim3(256), 0, s, a);
}

int lp_gemv_add_rmsnorm(lp_ctx* c, uint64_t w, uint64_t x, int rows, int cols, uint64_t h, uint64_t ln, float eps,
                        uint64_t hn, lp_stream s) {
    if (int r = check_ctx(c)) return r;
    if (rows <= 0 || cols <= 0) return fail(LP_E_INVALID, "gemv_add_rmsnorm: empty shape");
    if (rows > kFusedGemvMaxRows)
        return fail(LP_E_UNSUPPORTED, "gemv_add_rmsnorm: at most " + std::to_string(kFusedGemvMaxRows) + " rows");
    if (cols % 8 || cols > kFusedGemvMaxCols)
        return fail(LP_E_UNSUPPORTED, "gemv_add_rmsnorm: cols must be a multiple of 8, at most " +
                                          std::to_string(kFusedGemvMaxCols));
    if (!w || !x || !h || !ln || !hn || w % 16 || x % 16)
        return fail(LP_E_INVALID, "gemv_add_rmsnorm: null pointer, or w / x not 16-byte aligned");
    const int slot = sync_slot(c, s);
    if (slot < 0)
        return fail(LP_E_UNSUPPORTED, "gemv_add_rmsnorm: more than " + std::to_string(kSyncSlots) +
                                          " streams use this context's arrival counters");
    GemvAddRmsNormArgs a{};
    a.w = w, a.x = x, a.h = h, a.ln = ln, a.hn = hn;
    a.sync = sync_words(c, slot);
    a.rows = rows, a.cols = cols;
    a.eps = eps;
    const Fn f = (Fn)(kGemvAddRmsNorm1 + gemv_index(gemv_cpl(cols)));
    constexpr int rpb = 4 * kFusedGemvRowsPerWave;
    return launch(c, f, dim3((unsigned)((rows + rpb - 1) / rpb)), dim3(256), 0, s, a);
}

// Checks and plans lp_attn_fused: splits of whole 64-position chunks, at
// most kAttnFusedMaxSplits and as many as the scratch holds records for; the
// stream's counter slot when there is more than one split (or `counters`).
static int attn_fused_plan(lp_ctx* c, uint64_t q, uint64_t k, uint64_t v, uint64_t q_norm, uint64_t k_norm,
                           float eps, float rope_base, uint64_t kcache, uint64_t vcache, uint64_t out,
                           uint64_t scratch, int heads, int kv_heads, int head_dim, int pos, int max_seq, float scale,
                           bool counters, lp_stream s, AttnFusedArgs& a, int& gi) {
    if (heads <= 0 || kv_heads <= 0 || heads % kv_heads)
        return fail(LP_E_INVALID, "attn_fused: heads must be a multiple of kv_heads");
    const int group = heads / kv_heads;
    if (head_dim != 128 || kv_heads > kAttnFusedMaxKvHeads || group > 16 || (group & (group - 1)))
        return fail(LP_E_UNSUPPORTED, "attn_fused: head_dim 128, at most " + std::to_string(kAttnFusedMaxKvHeads) +
                                          " kv heads, 1, 2, 4, 8 or 16 query heads per kv head");
    if (pos < 0 || pos >= max_seq) return fail(LP_E_INVALID, "attn_fused: need 0 <= pos < max_seq");
    // buffer offsets reach 63 rows past the last position (int32 bytes)
    if ((uint64_t)(max_seq + 64) * head_dim * 2 >= (1ull << 31))
        return fail(LP_E_UNSUPPORTED, "attn_fused: each kv head's cache must be under 2 GiB");
    if (!q || !k || !v || !kcache || !vcache || !out || kcache % 16 || vcache % 16 || q % 4 || k % 4 || v % 4)
        return fail(LP_E_INVALID, "attn_fused: null pointer, or caches not 16-byte aligned");
    const int chunks = (pos + 64) / 64;
    // records are read 16 bytes at a time: each head's row of the scratch
    // starts at a multiple of 4 floats
    const int stride = max_seq & ~3;
    const int by_scratch = stride / kAttnFusedRec;
    int splits = std::min(chunks, std::min(kAttnFusedMaxSplits, by_scratch));
    if (splits < 1) splits = 1;
    const int cps = (chunks + splits - 1) / splits;
    splits = (chunks + cps - 1) / cps;
    if (splits > 1 && (!scratch || scratch % 16))
        return fail(LP_E_INVALID, "attn_fused: the scratch must be 16-byte aligned");
    a = AttnFusedArgs{};
    a.q = q, a.k = k, a.v = v, a.q_norm = q_norm, a.k_norm = k_norm;
    a.kcache = kcache, a.vcache = vcache, a.out = out, a.scratch = scratch;
    a.kv_heads = kv_heads, a.pos = pos, a.max_seq = max_seq, a.splits = splits, a.cps = cps;
    a.scratch_stride = stride;
    a.eps = eps, a.rope_base = rope_base, a.scale = scale;
    if (splits > 1 || counters) {
        const int slot = sync_slot(c, s);
        if (slot < 0)
            return fail(LP_E_UNSUPPORTED, "attn_fused: more than " + std::to_string(kSyncSlots) +
                                              " streams use this context's arrival counters");
        a.sync = sync_words(c, slot);
    }
    gi = group == 1 ? 0 : group == 2 ? 1 : group == 4 ? 2 : group == 8 ? 3 : 4;
    return LP_OK;
}

int lp_attn_fused(lp_ctx* c, uint64_t q, uint64_t k, uint64_t v, uint64_t q_norm, uint64_t k_norm, float eps,
                  float rope_base, uint64_t kcache, uint64_t vcache, uint64_t out, uint64_t scratch, int heads,
                  int kv_heads, int head_dim, int pos, int max_seq, float scale, lp_stream s) {
    if (int r = check_ctx(c)) return r;
    AttnFusedArgs a;
    int gi = 0;
    if (int r = attn_fused_plan(c, q, k, v, q_norm, k_norm, eps, rope_base, kcache, vcache, out, scratch, heads,
                                kv_heads, head_dim, pos, max_seq, scale, false, s, a, gi))
        return r;
    return launch(c, (Fn)(kAttnFusedG1 + gi), dim3((unsigned)a.splits, (unsigned)kv_heads), dim3(256), 0, s, a);
}

int lp_attn_block(lp_ctx* c, uint64_t q, uint64_t k, uint64_t v, uint64_t q_norm, uint64_t k_norm, float eps,
                  float rope_base, uint64_t kcache, uint64_t vcache, uint64_t att, uint64_t scratch, int heads,
                  int kv_heads, int head_dim, int pos, int max_seq, float scale, uint64_t wo, uint64_t h,
                  uint64_t post_ln, uint64_t hn, int hidden, lp_stream s) {
    if (int r = check_ctx(c)) return r;
    const int cols = heads * head_dim;
    if (hidden <= 0 || hidden > kFusedGemvMaxRows || cols > kFusedGemvMaxCols)
        return fail(LP_E_UNSUPPORTED, "attn_block: hidden and heads x head_dim at most " +
                                          std::to_string(kFusedGemvMaxRows));
    if (!wo || !h || !post_ln || !hn || wo % 16)
        return fail(LP_E_INVALID, "attn_block: null pointer, or W_o not 16-byte aligned");
    AttnBlockArgs b{};
    int gi = 0;
    if (int r = attn_fused_plan(c, q, k, v, q_norm, k_norm, eps, rope_base, kcache, vcache, att, scratch, heads,
                                kv_heads, head_dim, pos, max_seq, scale, true, s, b.at, gi))
        return r;
    b.wo = wo, b.h = h, b.ln = post_ln, b.hn = hn;
    b.rows = hidden, b.cols = cols;
    b.n_attn = b.at.splits * kv_heads;
    b.spin_max = c->step_spin;
    const unsigned n_o = (unsigned)((hidden + 4 * kBlockRowsPerWave - 1) / (4 * kBlockRowsPerWave));
    return launch(c, (Fn)(kAttnBlockG1 + gi), dim3((unsigned)b.n_attn + n_o), dim3(256), 0, s, b);
}

// ---- fused MoE layer --------------------------------------------------------------

// Prefill: the grouped GEMM takes over from the decode kernels once routed
// experts average kGemmMinPairsPerExpert (token, pick) pairs.
static bool use_gemm(const lp_moe_layer_desc* d, int T) {
    const long pairs = (long)T * d->top_k;
    return pairs >= (long)kGemmMinPairsPerExpert * std::min<long>(d->experts, pairs) &&
           act_chunks(d->inter) <= kGemmMaxChunks;
}

// The images of x a layer's expert kernels read: fp16 images for the prefill
// GEMM, digit images for the grouped kernels (every shared MLP included).
static int image_kinds(const lp_moe_layer_desc* d, int T) {
    const bool gemm = use_gemm(d, T);
    return (gemm ? kImgF16 : 0) | (!gemm || d->shared_blob ? kImgDigits : 0);
}

static int gemm_max_tiles(const lp_moe_layer_desc* d, int T) {
    const int pairs = T * d->top_k;
    return pairs / kGemmBM + std::min(d->experts, pairs) + 1;
}

// Workgroups of a GEMM launch: a multiple of kXcds covering every possible
// (tile, row block) item; the kernel maps them XCD by XCD onto the live ones.
static unsigned gemm_grid(const GemmArgs& gm) {
    const long items = (long)gm.max_tiles * gm.nblocks;
    return (unsigned)((items + kXcds - 1) / kXcds * kXcds);
}

int lp_moe_ws_layout_get(const lp_moe_layer_desc* d, int T, lp_moe_ws_layout* out) {
    if (!d || !out || T <= 0) return fail(LP_E_INVALID, "ws layout: bad arguments");
    const uint64_t E = (uint64_t)d->experts, k = (uint64_t)d->top_k, H = (uint64_t)d->hidden,
                   I = (uint64_t)d->inter, t = (uint64_t)T;
    uint64_t o = 0;
    auto take = [&](uint64_t bytes) {
        uint64_t at = o;
        o = align256(o + bytes);
        return at;
    };
    out->logits = take(t * E * 4);
    out->ids = take(t * k * 4);
    out->wts = take(t * k * 4);
    out->cnt = take(t * 4);
    out->gs = take((E + 1) * 4);
    out->perm = take(t * k * 4);
    out->inv = take(t * k * 4);
    out->uniq = take(E * 4);
    out->meta = take(64);
    out->et = take(E * sizeof(ExpertEntry));
    // the prefill GEMM writes act as fp16 images (actimg), their chunk exponents here
    out->act = take(use_gemm(d, T) ? t * k * (uint64_t)act_chunks((int)I) * 4 : t * k * I * 4);
    out->y = take(t * k * H * 4);
    out->xf = take(use_gemm(d, T) ? t * (uint64_t)himage_bytes((int)H) : 0);
    out->xd = take(t * (uint64_t)dimage_bytes((int)H));
    const bool sh = d->shared_blob != 0;
    const uint64_t Is = sh ? (uint64_t)d->shared_inter : 0;
    out->sh_et = take(sh ? (uint64_t)shared_entries(T) * sizeof(ExpertEntry) : 0);
    out->sh_perm = take(sh ? t * 4 : 0);
    out->sh_act = take(t * Is * 4);
    out->sh_y = take(sh ? t * H * 4 : 0);
    const bool gemm = use_gemm(d, T);
    out->tiles = take(gemm ? (uint64_t)gemm_max_tiles(d, T) * 4 : 0);
    out->actimg = take(gemm ? t * k * (uint64_t)himage_bytes((int)I) : 0);
    out->xexp = take(t * 4);
    out->disp = take(T > kTopkDispatchMaxT ? (2 * ((t + kDispTok - 1) / kDispTok) + 1) * E * 4 : 0);
    out->total = o;
    return LP_OK;
}

// The layer descriptor and T as the kernels assume them (no device state).
static int check_desc_shape(const lp_moe_layer_desc* d, int T) {
    if (!d) return fail(LP_E_INVALID, "null layer descriptor");
    if (T <= 0) return fail(LP_E_INVALID, "T must be >= 1");
    if (d->experts <= 0 || d->experts > kMaxExperts)
        return fail(LP_E_UNSUPPORTED, "experts must be in 1..1024");
    if (d->top_k <= 0 || d->top_k > kMaxTopK) return fail(LP_E_UNSUPPORTED, "top_k must be in 1..16");
    if (d->hidden <= 0 || d->inter <= 0 || d->hidden % 32 || d->inter % 32)
        return fail(LP_E_UNSUPPORTED, "hidden and inter must be multiples of 32");
    if (d->group <= 0 || d->group % 32 || ((d->group / 32) & (d->group / 32 - 1)) || d->group > 128 ||
        d->hidden % d->group || d->inter % d->group)
        return fail(LP_E_UNSUPPORTED, "group must be 32, 64 or 128 and divide hidden and inter");
    if (d->gating != LP_GATING_SOFTMAX && d->gating != LP_GATING_SIGMOID)
        return fail(LP_E_INVALID, "unknown gating");
    if (d->gating == LP_GATING_SIGMOID && !d->router_bias)
        return fail(LP_E_INVALID, "sigmoid gating needs router_bias");
    const uint64_t gpr_h = (uint64_t)d->hidden / d->group, gpr_i = (uint64_t)d->inter / d->group;
    const uint64_t gd = d->gate_off + (uint64_t)d->inter * gpr_h * 2;
    const uint64_t ud = d->up_off + (uint64_t)d->inter * gpr_h * 2;
    const uint64_t dd = d->down_off + (uint64_t)d->hidden * gpr_i * 2;
    if (gd % 16 || ud % 16 || dd % 16 || d->arena_base % 16 || d->slot_span % 16)
        return fail(LP_E_UNSUPPORTED, "q4 nibble rows must be 16-byte aligned in every slot");
    if (!d->router_w || !d->slot_table || !d->arena_base)
        return fail(LP_E_INVALID, "router_w, slot_table and arena_base are required");
    if (d->shared_blob) {
        const int Is = d->shared_inter, gs = d->shared_group;
        if (Is <= 0 || Is % 32) return fail(LP_E_UNSUPPORTED, "shared_inter must be a multiple of 32");
        if (gs <= 0 || gs % 32 || ((gs / 32) & (gs / 32 - 1)) || gs > 128 || d->hidden % gs || Is % gs)
            return fail(LP_E_UNSUPPORTED, "shared_group must be 32, 64 or 128 and divide hidden and shared_inter");
        const uint64_t sgd = d->sh_gate_off + (uint64_t)Is * (d->hidden / gs) * 2;
        const uint64_t sud = d->sh_up_off + (uint64_t)Is * (d->hidden / gs) * 2;
        const uint64_t sdd = d->sh_down_off + (uint64_t)d->hidden * (Is / gs) * 2;
        if ((d->shared_blob | sgd | sud | sdd) % 16)
            return fail(LP_E_UNSUPPORTED, "shared MLP nibble rows must be 16-byte aligned");
    }
    return LP_OK;
}

static int check_desc(lp_ctx* c, const lp_moe_layer_desc* d, int T) {
    if (int r = check_ctx(c)) return r;
    return check_desc_shape(d, T);
}

static void fill_views(const lp_moe_layer_desc* d, uint64_t ws, int T, LayerView* L, Workspace* W) {
    *L = LayerView{};
    L->router_w = d->router_w;
    L->router_bias = d->router_bias;
    L->slot_table = d->slot_table;
    L->arena_base = d->arena_base;
    L->slot_span = d->slot_span;
    L->gate_off = d->gate_off;
    L->up_off = d->up_off;
    L->down_off = d->down_off;
    L->hidden = d->hidden;
    L->inter = d->inter;
    L->experts = d->experts;
    L->top_k = d->top_k;
    L->group = d->group;
    L->gating = d->gating;
    L->renorm = d->renorm;
    L->routed_scaling = d->routed_scaling;
    L->min_weight = d->min_weight;
    L->shared_blob = d->shared_blob;
    L->shared_inter = d->shared_inter;
    L->shared_group = d->shared_group;
    L->sh_gate_off = d->sh_gate_off;
    L->sh_up_off = d->sh_up_off;
    L->sh_down_off = d->sh_down_off;
    lp_moe_ws_layout lay;
    lp_moe_ws_layout_get(d, T, &lay);
    W->logits = ws + lay.logits;
    W->ids = ws + lay.ids;
    W->wts = ws + lay.wts;
    W->cnt = ws + lay.cnt;
    W->gs = ws + lay.gs;
    W->perm = ws + lay.perm;
    W->inv = ws + lay.inv;
    W->uniq = ws + lay.uniq;
    W->meta = ws + lay.meta;
    W->et = ws + lay.et;
    W->act = ws + lay.act;
    W->y = ws + lay.y;
    W->xf = ws + lay.xf;
    W->xd = ws + lay.xd;
    W->sh_et = ws + lay.sh_et;
    W->sh_perm = ws + lay.sh_perm;
    W->sh_act = ws + lay.sh_act;
    W->sh_y = ws + lay.sh_y;
    W->tiles = ws + lay.tiles;
    W->actimg = ws + lay.actimg;
    W->xexp = ws + lay.xexp;
    W->disp = ws + lay.disp;
}

// The stream's slot of arrival counters (taken on its first use), or -1
// when every slot belongs to another stream.
static int sync_slot(lp_ctx* c, lp_stream s) {
    std::lock_guard<std::mutex> g(c->sync_mu);
    const hipStream_t hs = (hipStream_t)s;
    if (c->cap_slot >= 0 && c->cap_stream == hs) return c->cap_slot;
    int free_slot = -1;
    for (int i = 0; i < kSyncSlots; ++i) {
        if (c->sync_used[i] && !c->sync_graph[i] && c->sync_owner[i] == hs) return i;
        if (!c->sync_used[i] && free_slot < 0) free_slot = i;
    }
    if (free_slot >= 0) {
        c->sync_used[free_slot] = true;
        c->sync_owner[free_slot] = hs;
    }
    return free_slot;
}

// A workspace the kernels may write lp_moe_ws_layout's parts of layer d at,
// for T tokens: not null, 256-byte aligned like every part, and at least the
// layout's total bytes long (the kernels write up to its end unchecked).
static int check_ws(const lp_moe_layer_desc* d, int T, uint64_t ws, uint64_t ws_bytes) {
    if (ws == 0) return fail(LP_E_INVALID, "null workspace");
    if (ws % 256) return fail(LP_E_UNSUPPORTED, "the workspace must be 256-byte aligned");
    lp_moe_ws_layout lay;
    if (int r = lp_moe_ws_layout_get(d, T, &lay)) return r;
    if (ws_bytes < lay.total)
        return fail(LP_E_INVALID, "workspace of " + std::to_string(ws_bytes) + " bytes; this layer needs " +
                                      std::to_string(lay.total) + " for T = " + std::to_string(T));
    return LP_OK;
}

static int route_tail(lp_ctx* c, const RouteArgs& ra, lp_stream s) {
    const int T = ra.T;
    // up to kTopkFusedMaxT tokens: one workgroup does both (one token per
    // wave); more: the top-k spread over workgroups, then one dispatch
    // workgroup or, past kTopkDispatchMaxT, the three-launch dispatch
    if (T <= kTopkFusedMaxT) return launch(c, kTopkDispatch, dim3(1), dim3(1024), 0, s, ra);
    if (int r = launch(c, kTopk, dim3((unsigned)((T + 3) / 4)), dim3(256), 0, s, ra)) return r;
    if (T <= kTopkDispatchMaxT) return launch(c, kDispatch, dim3(1), dim3(256), 0, s, ra);
    const unsigned nb = (unsigned)((T + kDispTok - 1) / kDispTok);
    if (int r = launch(c, kDispCount, dim3(nb), dim3(kDispTok), 0, s, ra)) return r;
    if (int r = launch(c, kDispScan, dim3(1), dim3(1024), 0, s, ra)) return r;
    return launch(c, kDispScatter, dim3(nb), dim3(kDispTok), 0, s, ra);
}

int lp_moe_workspace_check(const lp_moe_layer_desc* layers, int n_layers, int T, uint64_t ws, uint64_t ws_bytes) {
    if (!layers || n_layers <= 0) return fail(LP_E_INVALID, "no layers");
    for (int l = 0; l < n_layers; ++l) {
        int r = check_desc_shape(&layers[l], T);
        if (!r) r = check_ws(&layers[l], T, ws, ws_bytes);
        if (r) return n_layers > 1 ? fail(r, "layer " + std::to_string(l) + ": " + g_err) : r;
    }
    return LP_OK;
}

int lp_moe_route(lp_ctx* c, const lp_moe_layer_desc* d, uint64_t x, int T, uint64_t ws, uint64_t ws_bytes,
                 lp_stream s) {
    if (int r = check_desc(c, d, T)) return r;
    if (int r = check_ws(d, T, ws, ws_bytes)) return r;
    if (x % 16) return fail(LP_E_UNSUPPORTED, "x must be 16-byte aligned");
    RouteArgs ra{};
    fill_views(d, ws, T, &ra.L, &ra.W);
    ra.x = x;
    ra.T = T;
    ra.make_xf = image_kinds(d, T);
    if (T > kTopkDispatchMaxT) {
        // large batch: the MFMA router, then the images of x on their own
        dim3 g((unsigned)((T + 15) / 16), (unsigned)((d->experts + 31) / 32));
        if (int r = launch(c, kGemmRouter, g, dim3(256), 0, s, ra)) return r;
        if (int r = launch(c, kXImage, dim3((unsigned)((T + 3) / 4)), dim3(256), 0, s, ra)) return r;
        return route_tail(c, ra, s);
    }
    if (d->hidden * 4 > kRouteXLds) {
        // token rows too wide for the fused kernel's staging: router, then top-k + dispatch
        dim3 g((unsigned)((d->experts + 3) / 4), (unsigned)((T + kRouterTokBlock - 1) / kRouterTokBlock));
        if (int r = launch(c, kRouter, g, dim3(256), 0, s, ra)) return r;
        return route_tail(c, ra, s);
    }
    // decode-sized batch: logits, top-k and dispatch in one launch
    const int slot = sync_slot(c, s);
    if (slot < 0)
        return fail(LP_E_UNSUPPORTED, "lp_moe_route: more than " + std::to_string(kSyncSlots) +
                                          " streams have routed through this context");
    ra.sync = reinterpret_cast<uint64_t>(c->sync) + (uint64_t)slot * kSyncWords * 4;
    // one block of up to kRouterTokBlock tokens, else blocks of
    // kRouteTokBlockMulti: twice the workgroups, each staging half the rows
    ra.tok_block = T <= kRouterTokBlock ? kRouterTokBlock : kRouteTokBlockMulti;
    dim3 g((unsigned)((d->experts + 8 * kRouteEPW - 1) / (8 * kRouteEPW)),
           (unsigned)((T + ra.tok_block - 1) / ra.tok_block));
    return launch(c, d->experts <= 128 ? kRouteFused128 : kRouteFused, g, dim3(512), 0, s, ra);
}

int lp_moe_route_logits(lp_ctx* c, const lp_moe_layer_desc* d, uint64_t logits, int T,
                        uint64_t ws, uint64_t ws_bytes, lp_stream s) {
    if (int r = check_desc(c, d, T)) return r;
    if (int r = check_ws(d, T, ws, ws_bytes)) return r;
    RouteArgs ra{};
    fill_views(d, ws, T, &ra.L, &ra.W);
    ra.T = T;
    if (logits != ra.W.logits)
        HIPCHK(hipMemcpyAsync(reinterpret_cast<void*>(ra.W.logits), reinterpret_cast<void*>(logits),
                              (size_t)T * d->experts * 4, hipMemcpyDeviceToDevice, (hipStream_t)s));
    return route_tail(c, ra, s);
}

static int tile_steps_host(int cols) { return ((cols >> 5) + 3) >> 2; }

// Whether lp_moe_gateup_bal takes the gate/up of ga's routed experts: one
// chunk of K, an expert table it can hold, no more token groups (up to
// kBalToks = 4 tokens of one expert each) than CUs, and its LDS.
static bool gateup_balanced(const lp_ctx* c, const GroupedArgs& ga, int maxu) {
    const int H = ga.L.hidden, pairs = ga.T * ga.L.top_k;
    const int maxv = std::min(pairs, (pairs + (kBalToks - 1) * maxu) / kBalToks);
    const int nw = tile_steps_host(H) > 8 ? 16 : 8;
    // with the shared MLP's entries (one token group each): at most the
    // grid's worth of units of the shorter width per workgroup, so that a
    // range still touches at most two blocks
    const int nsh = ga.sh_maxu;
    const long R = (ga.L.inter + 7) / 8, Rs = nsh ? (ga.L.shared_inter + 7) / 8 : R;
    const bool units_ok = (long)maxv * R + (long)nsh * Rs <= (long)c->cus * std::min(R, Rs);
    return tile_steps_host(H) <= kGateupChunk && maxu + nsh <= kBalMaxU && maxv <= c->cus && units_ok &&
           (size_t)bal_lds_bytes(H, nw, kBalWaves) <= c->max_lds && ga.L.slot_span < (1ull << 31) &&
           (uint64_t)pairs * ga.L.inter * 4 < (1ull << 31) &&
           (uint64_t)ga.T * (nsh ? ga.L.shared_inter : 0) * 4 < (1ull << 31);
}

// Whether lp_moe_down_bal(6) takes the down projection of ga's routed
// experts: at most 8 steps of K with scales in LDS windows, and what
// gateup_balanced asks of the table and the grid.  Below 32 (token, pick)
// pairs the one-shot kernel is faster: too few units to share.
static bool down_balanced(const lp_ctx* c, const GroupedArgs& ga, int maxu) {
    const int I = ga.L.inter, pairs = ga.T * ga.L.top_k;
    const int maxv = std::min(pairs, (pairs + (kBalToks - 1) * maxu) / kBalToks);
    return pairs >= 32 && tile_steps_host(I) <= 8 && scales_in_lds(ga.L.group, I) && maxu <= kBalMaxU &&
           maxv <= c->cus &&
           (size_t)bal_lds_bytes(I, 8 * kDownBalTiles, kBalWaves) <= c->max_lds &&
           (uint64_t)pairs * ga.L.hidden * 4 < (1ull << 31);
}

// The grouped down projection of ga's entries (maxu): balanced for routed
// decode batches when it can, else the one-shot kernels.
static int grouped_down(lp_ctx* c, const GroupedArgs& ga0, int maxu, bool routed, lp_stream s) {
    GroupedArgs ga = ga0;
    ga.maxu = maxu;
    ga.sh_maxu = 0;
    const int H = ga.L.hidden, I = ga.L.inter, cap = ga.pairs_cap;
    // Waves per workgroup: the most that still give every CU two workgroups
    // (routed) or one (the shared MLP: its few entries' act rows, staged by
    // each workgroup, cost more than the lost occupancy: a config-5 layer of
    // 16 tokens took 98.9 us with 2 waves, 102.2 with 1 and 100.0 with 4).
    const long want = routed ? 2L * c->cus : (long)c->cus;
    auto pick_w = [&](int rows, int tw) {
        for (int w = 4; w > 1; w >>= 1)
            if ((long)maxu * ((rows + kTileRows * w * tw - 1) / (kTileRows * w * tw)) >= want)
                return w;
        return 1;
    };
    const int steps = tile_steps_host(I);
    if (routed && c->gateup_bal && down_balanced(c, ga, maxu)) {
        return launch(c, steps == 6 ? kDownBal6 : kDownBal, dim3((unsigned)c->cus), dim3(64 * kBalWaves),
                      (size_t)bal_lds_bytes(I, 8 * kDownBalTiles, kBalWaves), s, ga);
    }
    const Fn f = steps <= kDownChunk ? kDown : kDownWide;
    const int tw = steps <= kDownChunk ? 2 : 1;
    const int w = pick_w(H, tw);
    const int chunks = (H + kTileRows * w * tw - 1) / (kTileRows * w * tw);
    const int ns = steps <= kDownChunk ? kDownChunk : kDownWideChunk;
    const int win = steps <= kDownWideChunk && scales_in_lds(ga.L.group, I) ? scale_window_lds(w, tw, ns) : 0;
    return launch(c, f, dim3((unsigned)(maxu * chunks)), dim3(64 * w), (size_t)(frag_lds_bytes(I, cap) + win),
                  s, ga);
}

// Grouped gate/up (+ SiLU) and down over the work items of ga's expert table
// (maxu entries): workgroup width chosen so that there are about two work
// items per CU, down with two tiles per wave when the inner size allows.
// `routed`: the routed experts (the balanced down may take them; the
// balanced gate/up takes the shared MLP too, as ceil(T / 4) one-group
// entries of one blob, whose weight rows neighbouring workgroups of one XCD
// read together).
// sh_maxu > 0 (routed only): the balanced gate/up also takes the shared
// MLP's entries when it can; *sh_done says whether it did.
static int grouped_ffn(lp_ctx* c, const GroupedArgs& ga0, int maxu, bool routed, lp_stream s,
                       bool with_down = true, int sh_maxu = 0, bool* sh_done = nullptr) {
    GroupedArgs ga = ga0;
    ga.maxu = maxu;
    ga.sh_maxu = 0;
    if (sh_done) *sh_done = false;
    // (the 16-step form with scales in LDS windows only: its own kernel)
    if (sh_maxu > 0 && c->gateup_bal && tile_steps_host(ga.L.hidden) > 8 && scales_in_lds(ga.L.group, ga.L.hidden)) {
        GroupedArgs gs = ga;
        gs.sh_maxu = sh_maxu;
        if (gateup_balanced(c, gs, maxu)) ga.sh_maxu = sh_maxu;
    }
    const int H = ga.L.hidden, I = ga.L.inter, cap = ga.pairs_cap;
    auto pick_w = [&](int rows, int tw) {
        for (int w = 4; w > 1; w >>= 1)
            if ((long)maxu * ((rows + kTileRows * w * tw - 1) / (kTileRows * w * tw)) >= 2L * c->cus)
                return w;
        return 1;
    };
    if (c->gateup_bal && gateup_balanced(c, ga, maxu)) {
        const bool t16 = tile_steps_host(H) > 8;
        const int nw = t16 ? 16 : 8;
        const Fn f = ga.sh_maxu ? kGateupBalSh
                     : scales_in_lds(ga.L.group, H) ? (t16 ? kGateupBal : kGateupBal8)
                                                    : (t16 ? kGateupBalRs : kGateupBalRs8);
        if (int r = launch(c, f, dim3((unsigned)c->cus), dim3(64 * kBalWaves),
                           (size_t)bal_lds_bytes(H, nw, kBalWaves), s, ga))
            return r;
        if (sh_done) *sh_done = ga.sh_maxu > 0;
        ga.sh_maxu = 0;
    } else {
        const int w = pick_w(I, 1);
        const int chunks = (I + kTileRows * w - 1) / (kTileRows * w);
        const int win = tile_steps_host(H) <= kGateupChunk && scales_in_lds(ga.L.group, H)
                            ? scale_window_lds(w, 2, kGateupChunk) : 0;
        if (int r = launch(c, kGateup, dim3((unsigned)(maxu * chunks)), dim3(64 * w),
                           (size_t)(frag_lds_bytes(H, cap) + win), s, ga))
            return r;
    }
    if (!with_down) return 0;
    return grouped_down(c, ga0, maxu, routed, s);
}

// LDS of lp_moe_down_comb(16, _rs): the picks' fragment pairs, their row
// sums (kCombWaves x 16 floats), then (scales in LDS windows) a window per
// wave (6, 8 or 16 steps wide: tile steps 6, 7..8, 9..16).
static int comb_lds(int inter, int steps, bool sl) {
    const int ns = steps == 6 ? 6 : steps <= 8 ? 8 : 16;
    const int win = sl ? 64 * 2 * ((ns + 7) / 8 * 8) : 0;
    return ((frag_lds_bytes(inter, kCombWaves) + 15) & ~15) + kCombWaves * 64 + kCombWaves * win;
}

// ... with the shared MLP's down fused in: its fragment pair and the two
// halves' row sums after the routed part.
static int comb_sh_lds(int inter, int steps, bool sl, int shared_inter) {
    return comb_lds(inter, steps, sl) + ((frag_lds_bytes(shared_inter, 1) + 15) & ~15) + kCombShWaves * 64;
}

// The shared MLP through the grouped kernels: its own width, group and
// regions, an expert table of consecutive token groups (written by dispatch).
static int shared_ffn(lp_ctx* c, const lp_moe_layer_desc* d, const GroupedArgs& ga, int T, lp_stream s,
                      bool with_down = true, bool with_gateup = true) {
    GroupedArgs gs = ga;
    gs.L.inter = d->shared_inter;
    gs.L.group = d->shared_group;
    gs.L.gate_off = d->sh_gate_off;
    gs.L.up_off = d->sh_up_off;
    gs.L.down_off = d->sh_down_off;
    gs.L.top_k = 1;
    gs.W.et = ga.W.sh_et;
    gs.W.perm = ga.W.sh_perm;
    gs.W.act = ga.W.sh_act;
    gs.W.y = ga.W.sh_y;
    if (!with_gateup) {
        // gate/up already done with the routed experts': the down alone
        if (!with_down) return 0;
        return grouped_down(c, gs, shared_entries(T), false, s);
    }
    return grouped_ffn(c, gs, shared_entries(T), false, s, with_down);
}

// The grouped expert kernels and the combine; the fragment images of x are
// written first unless the router kernel of lp_moe_forward already did.
// wave_n > 0: only the routed experts uniq[wave_u0, wave_u0 + wave_n) (one
// wave of a paged union), the shared MLP only when wave_shared.
static int experts_impl(lp_ctx* c, const lp_moe_layer_desc* d0, uint64_t x, uint64_t h, int T,
                        uint64_t ws, uint64_t ws_bytes, lp_stream s, bool have_images, int wave_u0 = 0,
                        int wave_n = 0, bool wave_shared = true) {
    if (int r = check_desc(c, d0, T)) return r;
    if (int r = check_ws(d0, T, ws, ws_bytes)) return r;
    if (x % 16) return fail(LP_E_UNSUPPORTED, "x must be 16-byte aligned");
    if (h % 16) return fail(LP_E_UNSUPPORTED, "h must be 16-byte aligned");
    const bool wave = wave_n > 0;
    lp_moe_layer_desc dw = *d0;
    if (wave && !wave_shared) dw.shared_blob = 0;
    const lp_moe_layer_desc* d = &dw;
    if (!have_images) {
        RouteArgs ra{};
        fill_views(d, ws, T, &ra.L, &ra.W);
        ra.x = x;
        ra.T = T;
        ra.make_xf = image_kinds(d, T);
        if (int r = launch(c, kXImage, dim3((unsigned)((T + 3) / 4)), dim3(256), 0, s, ra)) return r;
    }
    GroupedArgs ga{};
    fill_views(d, ws, T, &ga.L, &ga.W);
    ga.x = x;
    ga.h = h;
    ga.T = T;
    // the routed experts this call computes: every entry, or one wave's
    const int maxu_all = std::min(T * d->top_k, d->experts);
    if (wave) {
        ga.W.et += (uint64_t)wave_u0 * sizeof(ExpertEntry);
        ga.wave_u0 = wave_u0;
        ga.wave_n = wave_n;
    }
    const int maxu = wave ? wave_n : maxu_all;
    const int H = d->hidden;
    const int Is = d->shared_blob ? d->shared_inter : 0;
    // Token pairs staged at once: enough for T tokens on one expert, bounded
    // by kMaxPairs and by the LDS the fragments (and at most the largest
    // scale windows) need.
    int cap = std::min(kMaxPairs, (T + 1) / 2);
    auto lds_for = [&](int p) {
        return (size_t)std::max({frag_lds_bytes(H, p), frag_lds_bytes(d->inter, p), frag_lds_bytes(std::max(Is, 32), p)}) +
               (size_t)scale_window_lds(4, 2, kGateupChunk);
    };
    while (cap > 1 && lds_for(cap) > c->max_lds) --cap;
    if (lds_for(1) > c->max_lds)
        return fail(LP_E_UNSUPPORTED, "hidden/inter too large for one LDS fragment pair");
    ga.pairs_cap = cap;
    bool sh_gu = false;  // the shared MLP's gate/up done by the routed launch
    if (!wave && use_gemm(d, T)) {
        if ((size_t)kGemmLds > c->max_lds) return fail(LP_E_UNSUPPORTED, "GEMM stages exceed the LDS");
        // the GEMM loads address images and weights as 32-bit offsets from a base
        const uint64_t img_span = std::max((uint64_t)T * himage_bytes(d->hidden),
                                           (uint64_t)T * d->top_k * himage_bytes(d->inter));
        if (img_span >= (1ull << 32) || d->slot_span >= (1ull << 32))
            return fail(LP_E_UNSUPPORTED, "prefill GEMM: activation images or expert slots of 4 GiB or more");
        GemmArgs gm{};
        gm.L = ga.L;
        gm.W = ga.W;
        gm.T = T;
        gm.tiles = ga.W.tiles;
        gm.max_tiles = gemm_max_tiles(d, T);
        if (int r = launch(c, kGemmTiles, dim3(1), dim3(256), 0, s, gm)) return r;
        // gate/up writes act as the down GEMM's fp16 images (+ chunk exponents in W.act)
        gm.a_img = ga.W.xf;
        gm.out = ga.W.actimg;
        gm.nblocks = act_chunks(d->inter);
        if (int r = launch(c, kGemmGateup, dim3(gemm_grid(gm)), dim3(kGemmWaves * 64), 0, s, gm))
            return r;
        gm.a_img = ga.W.actimg;
        gm.out = ga.W.y;
        gm.nblocks = (d->hidden + kGemmBN - 1) / kGemmBN;
        if (int r = launch(c, kGemmDown, dim3(gemm_grid(gm)), dim3(kGemmWaves * 64), 0, s, gm))
            return r;
    } else {
        // one token: down and combine in one launch (after the shared MLP,
        // whose row it adds)
        const int Si = tile_steps_host(d->inter);
        const bool sl = scales_in_lds(d->group, d->inter);
        const bool comb = !wave && T == 1 && d->top_k <= kCombWaves && Si <= 16 &&
                          (size_t)comb_lds(d->inter, Si, sl) <= c->max_lds;
        // the shared MLP's gate/up rides on the routed balanced launch when
        // the groups agree (sh_gu: it did)
        const int shm = !wave && d->shared_blob && d->shared_group == d->group ? shared_entries(T) : 0;
        if (int r = grouped_ffn(c, ga, maxu, true, s, !comb, shm, &sh_gu)) return r;
        if (comb) {
            const Fn f = !sl ? kDownCombRs : Si <= 8 ? kDownComb : kDownComb16;
            // the shared MLP's down on the comb kernel's idle waves: per-lane
            // scales, the routed group, at most 2 x 16 steps, the LDS
            size_t lds = (size_t)comb_lds(d->inter, Si, sl);
            const size_t lds_sh = (size_t)comb_sh_lds(d->inter, Si, sl, d->shared_inter);
            const bool fuse = d->shared_blob && f == kDownCombRs && d->top_k <= kCombWaves - kCombShWaves &&
                              d->shared_group == d->group && tile_steps_host(d->shared_inter) <= 32 &&
                              lds_sh <= c->max_lds;
            if (d->shared_blob)
                if (int r = shared_ffn(c, d, ga, T, s, !fuse, !sh_gu)) return r;
            ga.maxu = std::min(d->top_k, d->experts);
            ga.sh_fused = fuse ? 1 : 0;
            if (fuse) lds = lds_sh;
            return launch(c, f, dim3((unsigned)((d->hidden + kTileRows - 1) / kTileRows)), dim3(64 * kCombWaves),
                          lds, s, ga);
        }
    }
    if (d->shared_blob)
        if (int r = shared_ffn(c, d, ga, T, s, true, !sh_gu)) return r;
    return launch(c, kCombine, dim3((unsigned)((d->hidden + 1023) / 1024), (unsigned)T), dim3(256), 0,
                  s, ga);
}

int lp_moe_resolve(lp_ctx* c, const lp_moe_layer_desc* d, int T, uint64_t ws, uint64_t ws_bytes, lp_stream s) {
    if (int r = check_desc(c, d, T)) return r;
    if (int r = check_ws(d, T, ws, ws_bytes)) return r;
    RouteArgs ra{};
    fill_views(d, ws, T, &ra.L, &ra.W);
    ra.T = T;
    return launch(c, kResolve, dim3(1), dim3(256), 0, s, ra);
}

int lp_moe_experts(lp_ctx* c, const lp_moe_layer_desc* d, uint64_t x, uint64_t h, int T,
                   uint64_t ws, uint64_t ws_bytes, lp_stream s) {
    return experts_impl(c, d, x, h, T, ws, ws_bytes, s, false);
}

int lp_moe_experts_wave(lp_ctx* c, const lp_moe_layer_desc* d, uint64_t x, uint64_t h, int T, uint64_t ws,
                        uint64_t ws_bytes, int u_first, int u_count, int with_shared, lp_stream s) {
    if (int r = check_desc(c, d, T)) return r;
    if (u_first < 0 || u_count <= 0 || u_first + u_count > std::min(T * d->top_k, d->experts))
        return fail(LP_E_INVALID, "lp_moe_experts_wave: the wave must be a non-empty range of the unique list");
    if (T > kTopkDispatchMaxT || use_gemm(d, T))
        return fail(LP_E_UNSUPPORTED, "lp_moe_experts_wave: decode batches only (at most 64 tokens, the grouped "
                                      "kernels' workspace)");
    if (x == h) return fail(LP_E_INVALID, "lp_moe_experts_wave: x must not be h (every wave reads the same x)");
    return experts_impl(c, d, x, h, T, ws, ws_bytes, s, false, u_first, u_count, with_shared != 0);
}

int lp_moe_forward(lp_ctx* c, const lp_moe_layer_desc* d, uint64_t x, uint64_t h, int T,
                   uint64_t ws, uint64_t ws_bytes, lp_stream s) {
    if (int r = lp_moe_route(c, d, x, T, ws, ws_bytes, s)) return r;
    return experts_impl(c, d, x, h, T, ws, ws_bytes, s, true);
}

int lp_moe_stack_forward(lp_ctx* c, const lp_moe_layer_desc* layers, int n_layers, uint64_t h, int T,
                         uint64_t ws, uint64_t ws_bytes, lp_stream s) {
    if (int r = check_ctx(c)) return r;
    // every layer's shape and workspace need are checked before the first
    // launch, so a bad descriptor part-way down the stack leaves h untouched
    if (int r = lp_moe_workspace_check(layers, n_layers, T, ws, ws_bytes))
        return fail(r, "lp_moe_stack_forward: " + g_err);
    for (int l = 0; l < n_layers; ++l)
        if (int r = lp_moe_forward(c, &layers[l], h, h, T, ws, ws_bytes, s)) return r;
    return LP_OK;
}

struct lp_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    lp_ctx* ctx = nullptr;
    int slot = -1;  // the graph's own arrival-counter slot, freed with it
};

// A slot of arrival counters for a graph about to be captured on s (the
// routing launches of the capture use it); -1 when none is free.
static int graph_slot_take(lp_ctx* c, lp_stream s) {
    std::lock_guard<std::mutex> g(c->sync_mu);
    for (int i = 0; i < kSyncSlots; ++i) {
        if (!c->sync_used[i]) {
            c->sync_used[i] = true;
            c->sync_graph[i] = true;
            c->sync_owner[i] = nullptr;
            c->cap_stream = (hipStream_t)s;
            c->cap_slot = i;
            return i;
        }
    }
    return -1;
}

static void graph_slot_free(lp_ctx* c, int slot) {
    std::lock_guard<std::mutex> g(c->sync_mu);
    if (slot < 0 || slot >= kSyncSlots) return;
    c->sync_used[slot] = false;
    c->sync_graph[slot] = false;
}

static void capture_end(lp_ctx* c) {
    std::lock_guard<std::mutex> g(c->sync_mu);
    c->cap_stream = nullptr;
    c->cap_slot = -1;
}

int lp_moe_stack_capture(lp_ctx* c, const lp_moe_layer_desc* layers, int n_layers, uint64_t h, int T,
                         uint64_t ws, uint64_t ws_bytes, lp_stream s, lp_graph** out) {
    if (int r = check_ctx(c)) return r;
    if (!out) return fail(LP_E_INVALID, "lp_moe_stack_capture: null out");
    *out = nullptr;
    if (!s) return fail(LP_E_INVALID, "lp_moe_stack_capture: the null stream cannot be captured");
    if (int r = lp_moe_workspace_check(layers, n_layers, T, ws, ws_bytes))
        return fail(r, "lp_moe_stack_capture: " + g_err);
    {
        std::lock_guard<std::mutex> g(c->sync_mu);
        if (c->cap_slot >= 0)
            return fail(LP_E_INVALID, "lp_moe_stack_capture: a capture is in progress (inside one, use "
                                      "lp_moe_stack_forward)");
    }
    // the graph's own arrival counters (routing in the captured launches)
    const int slot = graph_slot_take(c, s);
    if (slot < 0)
        return fail(LP_E_UNSUPPORTED, "lp_moe_stack_capture: every slot of arrival counters is taken (" +
                                          std::to_string(kSyncSlots) + " streams and graphs)");
    // no profiling events inside the graph
    const bool prof = c->prof;
    c->prof = false;
    const hipError_t be = hipStreamBeginCapture((hipStream_t)s, hipStreamCaptureModeThreadLocal);
    if (be != hipSuccess) {
        c->prof = prof;
        capture_end(c);
        graph_slot_free(c, slot);
        return hip_fail(be, "hipStreamBeginCapture");
    }
    const int r = lp_moe_stack_forward(c, layers, n_layers, h, T, ws, ws_bytes, s);
    const std::string err = g_err;
    hipGraph_t g = nullptr;
    const hipError_t e = hipStreamEndCapture((hipStream_t)s, &g);
    c->prof = prof;
    capture_end(c);
    if (r != LP_OK || e != hipSuccess) {
        if (g) (void)hipGraphDestroy(g);
        graph_slot_free(c, slot);
        return r != LP_OK ? fail(r, err) : hip_fail(e, "hipStreamEndCapture");
    }
    lp_graph* G = new lp_graph();
    G->graph = g;
    G->ctx = c;
    G->slot = slot;
    const hipError_t ie = hipGraphInstantiate(&G->exec, g, nullptr, nullptr, 0);
    if (ie != hipSuccess) {
        lp_graph_destroy(G);
        return hip_fail(ie, "hipGraphInstantiate");
    }
    *out = G;
    return LP_OK;
}

// The general capture: whatever the library launches on s between begin
// and end (1:1 kernels, fused layers, stacks) becomes one graph, which owns
// a routing counter slot as lp_moe_stack_capture's graphs do.
int lp_graph_capture_begin(lp_ctx* c, lp_stream s) {
    if (int r = check_ctx(c)) return r;
    if (!s) return fail(LP_E_INVALID, "lp_graph_capture_begin: the null stream cannot be captured");
    {
        std::lock_guard<std::mutex> g(c->sync_mu);
        if (c->cap_slot >= 0) return fail(LP_E_INVALID, "lp_graph_capture_begin: a capture is already in progress");
    }
    const int slot = graph_slot_take(c, s);
    if (slot < 0)
        return fail(LP_E_UNSUPPORTED, "lp_graph_capture_begin: every slot of arrival counters is taken (" +
                                          std::to_string(kSyncSlots) + " streams and graphs)");
    c->cap_prof = c->prof;
    c->prof = false;  // no profiling events inside the graph
    const hipError_t e = hipStreamBeginCapture((hipStream_t)s, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) {
        c->prof = c->cap_prof;
        capture_end(c);
        graph_slot_free(c, slot);
        return hip_fail(e, "hipStreamBeginCapture");
    }
    return LP_OK;
}

int lp_graph_capture_end(lp_ctx* c, lp_stream s, lp_graph** out) {
    if (int r = check_ctx(c)) return r;
    if (!out) return fail(LP_E_INVALID, "lp_graph_capture_end: null out");
    *out = nullptr;
    int slot;
    {
        std::lock_guard<std::mutex> g(c->sync_mu);
        if (c->cap_slot < 0 || c->cap_stream != (hipStream_t)s)
            return fail(LP_E_INVALID, "lp_graph_capture_end: no capture in progress on this stream");
        slot = c->cap_slot;
    }
    hipGraph_t g = nullptr;
    const hipError_t e = hipStreamEndCapture((hipStream_t)s, &g);
    c->prof = c->cap_prof;
    capture_end(c);
    if (e != hipSuccess) {
        if (g) (void)hipGraphDestroy(g);
        graph_slot_free(c, slot);
        return hip_fail(e, "hipStreamEndCapture");
    }
    lp_graph* G = new lp_graph();
    G->graph = g;
    G->ctx = c;
    G->slot = slot;
    const hipError_t ie = hipGraphInstantiate(&G->exec, g, nullptr, nullptr, 0);
    if (ie != hipSuccess) {
        lp_graph_destroy(G);
        return hip_fail(ie, "hipGraphInstantiate");
    }
    *out = G;
    return LP_OK;
}

int lp_graph_launch(lp_ctx* c, lp_graph* g, lp_stream s) {
    if (int r = check_ctx(c)) return r;
    if (!g || !g->exec) return fail(LP_E_INVALID, "lp_graph_launch: null graph");
    HIPCHK(hipGraphLaunch(g->exec, (hipStream_t)s));
    return LP_OK;
}

void lp_graph_destroy(lp_graph* g) {
    if (!g) return;
    if (g->exec) {
        // replays still in flight hold the graph's counters
        (void)hipDeviceSynchronize();
        (void)hipGraphExecDestroy(g->exec);
    }
    if (g->graph) (void)hipGraphDestroy(g->graph);
    if (g->ctx) graph_slot_free(g->ctx, g->slot);
    delete g;
}

int lp_moe_status_sync(lp_ctx* c, uint64_t ws, uint64_t ws_bytes, const lp_moe_layer_desc* d, int T, lp_stream s,
                       int32_t* unique_count, int32_t* error_flags) {
    if (int r = check_ctx(c)) return r;
    if (int r = check_desc_shape(d, T)) return r;
    if (int r = check_ws(d, T, ws, ws_bytes)) return r;
    lp_moe_ws_layout lay;
    if (int r = lp_moe_ws_layout_get(d, T, &lay)) return r;
    int32_t meta[2] = {0, 0};
    HIPCHK(hipMemcpyAsync(meta, reinterpret_cast<void*>(ws + lay.meta), 8, hipMemcpyDeviceToHost,
                          (hipStream_t)s));
    HIPCHK(hipStreamSynchronize((hipStream_t)s));
    if (unique_count) *unique_count = meta[0];
    if (error_flags) *error_flags = meta[1];
    return LP_OK;
}

int lp_step_errors_sync(lp_ctx* c, int32_t* timeouts) {
    if (int r = check_ctx(c)) return r;
    HIPCHK(hipDeviceSynchronize());
    std::lock_guard<std::mutex> g(c->sync_mu);
    int32_t total = 0;
    for (int i = 0; i < kSyncSlots; ++i) {
        int32_t* w = c->sync + (size_t)i * kSyncWords + kStepSyncErr;
        int32_t v = 0;
        HIPCHK(hipMemcpy(&v, w, 4, hipMemcpyDeviceToHost));
        if (v) {
            // a wait that gave up may have let a counter be reset before its
            // last arrivals: every launch has ended, so zero the slot's
            // fused-step counters along with the count
            total += v;
            int32_t* step = c->sync + (size_t)i * kSyncWords + kStepSyncAttn;
            HIPCHK(hipMemset(step, 0, (size_t)(kSyncWords - kStepSyncAttn) * 4));
        }
    }
    if (timeouts) *timeouts = total;
    return LP_OK;
}

int lp_profile_enable(lp_ctx* c, int enable) {
    if (int r = check_ctx(c)) return r;
    c->prof = enable != 0;
    return LP_OK;
}

int lp_profile_reset(lp_ctx* c) {
    if (int r = check_ctx(c)) return r;
    HIPCHK(hipDeviceSynchronize());
    std::lock_guard<std::mutex> g(c->prof_mu);
    prof_drain(c);
    for (int f = 0; f < kNumFns; ++f) {
        c->prof_ms[f] = 0.0;
        c->prof_n[f] = 0;
    }
    return LP_OK;
}

int lp_profile_read_sync(lp_ctx* c, const char* kernel, double* total_ms, int64_t* launches) {
    if (int r = check_ctx(c)) return r;
    if (!kernel) return fail(LP_E_INVALID, "null kernel name");
    HIPCHK(hipDeviceSynchronize());
    std::lock_guard<std::mutex> g(c->prof_mu);
    prof_drain(c);
    for (int f = 0; f < kNumFns; ++f) {
        if (strcmp(kSpecs[f].name, kernel) == 0) {
            if (total_ms) *total_ms = c->prof_ms[f];
            if (launches) *launches = c->prof_n[f];
            return LP_OK;
        }
    }
    return fail(LP_E_INVALID, std::string("unknown kernel ") + kernel);
}

float lp_route_expf(float x) { return lp::expf_glibc(x); }

int lp_route_expf_device(lp_ctx* c, uint32_t first, uint32_t stride, uint64_t n, uint64_t out,
                         lp_stream s) {
    if (int r = check_ctx(c)) return r;
    if (!out || n == 0) return fail(LP_E_INVALID, "lp_route_expf_device: bad arguments");
    ExpfSweepArgs a{out, n, first, stride};
    return launch(c, kExpfWave, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, a);
}

void lp_route_expf_sweep(uint32_t first, uint32_t stride, uint64_t n, float* out) {
    for (uint64_t i = 0; i < n; ++i) {
        const uint32_t b = first + (uint32_t)(i * stride);
        float f;
        memcpy(&f, &b, 4);
        out[i] = lp::expf_glibc(f);
    }
}

}  // extern "C"
