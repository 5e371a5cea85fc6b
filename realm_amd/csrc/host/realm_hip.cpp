// Host side of the MI355X quantized compute path: the C ABI of
// include/realm_hip.h on top of the HIP runtime.  The gfx950 code object is
// embedded in this library at build time and loaded with hipModuleLoadData;
// every kernel is launched with hipModuleLaunchKernel.
//
// Mirrors, for this path, the reference's GpuBackendTrait
// (crates/realm-compute-gpu/src/gpu_backend_trait.rs:17-143) and its
// candle_matmul host functions (crates/realm-runtime/src/memory64_host.rs:
// 853-1087), plus what the reference lacks: device-resident weights and a
// batched multi-adapter LoRA.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "kernel_args.h"
#include "noalloc.h"
#include "realm_hip.h"

#define REALM_STR2(x) #x
#define REALM_STR(x) REALM_STR2(x)

// The code objects (REALM_HSACO_COUNT of them: the non-GEMV kernels, the
// GEMV variants of each weight format and token count, and the LDS-tiled
// GEMM), embedded at link time.
#define REALM_EMBED(I, FILE)                                                                   \
    __asm__(".pushsection .rodata.realm_hsaco" #I ",\"a\",@progbits\n"                        \
            ".balign 4096\n"                                                                  \
            ".globl realm_hsaco" #I "\n"                                                      \
            ".hidden realm_hsaco" #I "\n"                                                     \
            "realm_hsaco" #I ":\n"                                                            \
            ".incbin \"" REALM_STR(FILE) "\"\n"                                                \
            ".byte 0\n"                                                                       \
            ".popsection\n");                                                                 \
    extern "C" const unsigned char realm_hsaco##I[];
REALM_EMBED(0, REALM_HSACO_FILE0)
REALM_EMBED(1, REALM_HSACO_FILE1)
REALM_EMBED(2, REALM_HSACO_FILE2)
REALM_EMBED(3, REALM_HSACO_FILE3)
REALM_EMBED(4, REALM_HSACO_FILE4)
REALM_EMBED(5, REALM_HSACO_FILE5)
REALM_EMBED(6, REALM_HSACO_FILE6)
REALM_EMBED(7, REALM_HSACO_FILE7)
REALM_EMBED(8, REALM_HSACO_FILE8)
REALM_EMBED(9, REALM_HSACO_FILE9)
REALM_EMBED(10, REALM_HSACO_FILE10)
REALM_EMBED(11, REALM_HSACO_FILE11)
REALM_EMBED(12, REALM_HSACO_FILE12)
REALM_EMBED(13, REALM_HSACO_FILE13)
REALM_EMBED(14, REALM_HSACO_FILE14)
REALM_EMBED(15, REALM_HSACO_FILE15)
REALM_EMBED(16, REALM_HSACO_FILE16)
REALM_EMBED(17, REALM_HSACO_FILE17)
static_assert(REALM_HSACO_COUNT == 18, "the build embeds eighteen code objects");
static const unsigned char *const realm_hsacos[REALM_HSACO_COUNT] = {
    realm_hsaco0, realm_hsaco1, realm_hsaco2,  realm_hsaco3,  realm_hsaco4,
    realm_hsaco5, realm_hsaco6, realm_hsaco7,  realm_hsaco8,  realm_hsaco9,
    realm_hsaco10, realm_hsaco11, realm_hsaco12, realm_hsaco13, realm_hsaco14,
    realm_hsaco15, realm_hsaco16, realm_hsaco17};

#define REALM_API extern "C" __attribute__((visibility("default")))

// Sets the calling thread's last-error message and returns code (for the
// library's other translation units; not exported).
int realm_set_error(int code, const std::string &msg);

using realm::GemmArgs;
using realm::LoraEntry;
using realm::LoraChunk;

namespace {

// ------------------------------------------------------------------ errors

thread_local std::string t_last_error;

int fail(int code, const std::string &msg)
{
    t_last_error = msg;
    return code;
}

int hip_code(hipError_t e)
{
    return e == hipErrorOutOfMemory ? REALM_OUT_OF_MEMORY : REALM_GENERIC_FAILURE;
}

#define HIP_TRY(expr)                                                                     \
    do {                                                                                  \
        hipError_t e_ = (expr);                                                           \
        if (e_ != hipSuccess)                                                             \
            return fail(hip_code(e_), std::string(#expr) + ": " + hipGetErrorString(e_)); \
    } while (0)

#define CHECK(expr)            \
    do {                       \
        int rc_ = (expr);      \
        if (rc_ != REALM_OK)   \
            return rc_;        \
    } while (0)

constexpr int GGML_Q8_0 = REALM_GGML_Q8_0, GGML_Q4_K = REALM_GGML_Q4_K,
              GGML_Q6_K = REALM_GGML_Q6_K;

// The reference's 32-element formats Q4_0, Q4_1, Q5_0, Q5_1, Q8_1
// (quant.rs:10-70): dequantized on the device, products through the dense
// f32 GEMM (as CandleGpuBackend's fused_dequant_matmul_q40 etc.).
bool is_block32(int t) { return t == 2 || t == 3 || t == 6 || t == 7 || t == 9; }
// The reference's own 256-element Q2_K, Q3_K, Q5_K, Q8_K layouts
// (quant.rs:71-95, 200-222; #[repr(C)] sizes 116, 196, 178, 292 bytes, not
// ggml's): the same treatment as the 32-element formats.
bool is_kq(int t) { return t == 10 || t == 11 || t == 13 || t == 15; }
// formats kept dequantized in f32 on the device
bool is_dq(int t) { return is_block32(t) || is_kq(t); }
size_t dq_bytes(int t)
{
    return t == 2 ? 18 : t == 3 ? 20 : t == 6 ? 22 : t == 7 ? 24 : t == 9 ? 36
         : t == 10 ? 116 : t == 11 ? 196 : t == 13 ? 178 : t == 15 ? 292 : 0;
}
size_t block_bytes(int t)
{
    return t == GGML_Q4_K ? 144 : t == GGML_Q6_K ? 210 : is_dq(t) ? dq_bytes(t) : 34;
}
size_t block_elems(int t) { return (t == GGML_Q4_K || t == GGML_Q6_K || is_kq(t)) ? 256 : 32; }
const char *dq_name(int t)
{
    switch (t) {
    case 2: return "Q4_0";
    case 3: return "Q4_1";
    case 6: return "Q5_0";
    case 7: return "Q5_1";
    case 9: return "Q8_1";
    case 10: return "Q2_K";
    case 11: return "Q3_K";
    case 13: return "Q5_K";
    default: return "Q8_K";
    }
}
size_t align256(size_t v) { return (v + 255) & ~size_t(255); }
size_t round_up(size_t v, size_t m) { return (v + m - 1) / m * m; }
// kernel-name stem of a resident format ("q8m": the 32-element formats as
// int8 q', f16 scale, f16 delta)
const char *fmt_name(int t)
{
    return t == GGML_Q4_K ? "q4k" : t == GGML_Q6_K ? "q6k" : t == GGML_Q8_0 ? "q80" : "q8m";
}

// ------------------------------------------------------------------ device

struct Device {
    bool ready = false;
    int id = 0;
    int cu_count = 256;
    size_t max_lds = 65536;
    // this device's copy of the no-allocation entry point's scratch array
    // (noalloc.hip), resolved once at init with the device current
    void *noalloc_scratch = nullptr;
    hipModule_t modules[REALM_HSACO_COUNT] = {};
    std::unordered_map<std::string, hipFunction_t> fns;
};

std::mutex g_mu; // device init, function cache, registries, workspaces
Device g_dev;
std::atomic<int> g_nan_fb{0};

int init_locked(int device)
{
    if (g_dev.ready) {
        if (device != g_dev.id)
            return fail(REALM_INVALID_ARGUMENT, "realm_hip already initialised on device " +
                                                    std::to_string(g_dev.id));
        return REALM_OK;
    }
    int count = 0;
    HIP_TRY(hipGetDeviceCount(&count));
    if (device < 0 || device >= count)
        return fail(REALM_INVALID_ARGUMENT, "device " + std::to_string(device) +
                                                " out of range (" + std::to_string(count) + ")");
    HIP_TRY(hipSetDevice(device));
    hipDeviceProp_t prop;
    HIP_TRY(hipGetDeviceProperties(&prop, device));
    if (std::string(prop.gcnArchName).find("gfx950") == std::string::npos)
        return fail(REALM_BACKEND_UNSUPPORTED,
                    std::string("code object is built for gfx950, device is ") + prop.gcnArchName);
    g_dev.cu_count = prop.multiProcessorCount;
    g_dev.max_lds = prop.sharedMemPerBlock;
    for (int i = 0; i < REALM_HSACO_COUNT; ++i)
        HIP_TRY(hipModuleLoadData(&g_dev.modules[i], realm_hsacos[i]));
    if (int e = realm_noalloc_scratch_address(&g_dev.noalloc_scratch))
        return fail(REALM_GENERIC_FAILURE,
                    std::string("hipGetSymbolAddress of the no-allocation scratch: ") +
                        hipGetErrorString((hipError_t)e));
    g_dev.id = device;
    g_dev.ready = true;
    return REALM_OK;
}

int ensure_init()
{
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_dev.ready) {
        HIP_TRY(hipSetDevice(g_dev.id));
        return REALM_OK;
    }
    return init_locked(0);
}

int get_fn(const std::string &name, hipFunction_t *out)
{
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_dev.fns.find(name);
    if (it != g_dev.fns.end()) {
        *out = it->second;
        return REALM_OK;
    }
    hipFunction_t f = nullptr;
    for (int i = 0; i < REALM_HSACO_COUNT && !f; ++i)
        if (hipModuleGetFunction(&f, g_dev.modules[i], name.c_str()) != hipSuccess)
            f = nullptr;
    (void)hipGetLastError(); // lookups in the other code objects set it
    if (!f)
        return fail(REALM_GENERIC_FAILURE, "kernel " + name + " not found in the code objects");
    g_dev.fns[name] = f;
    *out = f;
    return REALM_OK;
}

thread_local std::string t_last_kernel;

int launch(const std::string &name, dim3 grid, dim3 block, size_t lds, hipStream_t s,
           void **args)
{
    if (grid.x == 0 || grid.y == 0 || grid.z == 0)
        return REALM_OK;
    hipFunction_t f;
    CHECK(get_fn(name, &f));
    t_last_kernel = name;
    HIP_TRY(hipModuleLaunchKernel(f, grid.x, grid.y, grid.z, block.x, block.y, block.z,
                                  (unsigned)lds, s, args, nullptr));
    return REALM_OK;
}

// ------------------------------------------------------------ streams etc.

thread_local hipStream_t t_stream = nullptr;

int thread_stream(hipStream_t *s)
{
    if (!t_stream)
        HIP_TRY(hipStreamCreateWithFlags(&t_stream, hipStreamNonBlocking));
    *s = t_stream;
    return REALM_OK;
}

// A second stream per thread, and a fork/join event pair, for work that can
// run beside the main stream's (the LoRA shrink beside the base product).
// Under graph capture the fork's event pulls the side stream into the graph.
thread_local hipStream_t t_side = nullptr;
thread_local hipEvent_t t_fork = nullptr, t_join = nullptr;

int side_stream(hipStream_t *side, hipEvent_t *fork, hipEvent_t *join)
{
    if (!t_side) {
        HIP_TRY(hipStreamCreateWithFlags(&t_side, hipStreamNonBlocking));
        HIP_TRY(hipEventCreateWithFlags(&t_fork, hipEventDisableTiming));
        HIP_TRY(hipEventCreateWithFlags(&t_join, hipEventDisableTiming));
    }
    *side = t_side;
    *fork = t_fork;
    *join = t_join;
    return REALM_OK;
}

int pick_stream(void *user, hipStream_t *s)
{
    if (user) {
        *s = (hipStream_t)user;
        return REALM_OK;
    }
    return thread_stream(s);
}

// Per-stream scratch buffers (grow-only).  Work on one stream is ordered, so
// reusing a stream's buffers for its next call is safe.
//
// A HIP graph captured on a stream holds the addresses of the buffers its
// calls used.  So while such a graph is alive (captured through
// realm_hip_graph_begin/end and not yet released), or while the stream is
// capturing, a buffer that has to grow is not freed: it goes on the
// stream's retired list, freed when the stream's last graph is released.
// Buffers replaced while the stream was capturing outside
// realm_hip_graph_begin are never freed (the library cannot tell when such
// a graph ends).
enum Slot { WS_RAW, WS_WEIGHT, WS_X, WS_Y, WS_XH, WS_XL, WS_XM, WS_TS, WS_U, WS_IDS, WS_PART,
            WS_LAYER, WS_ATT, WS_NF, WS_N };

struct Workspace {
    void *buf[WS_N] = {};
    size_t cap[WS_N] = {};
    int graphs = 0;              // live graphs captured on this stream (and open captures)
    std::vector<void *> retired; // replaced buffers a live graph may still use
};
std::unordered_map<hipStream_t, std::unique_ptr<Workspace>> g_ws;

// During a call of the no-allocation entry point, every scratch request of
// the calling thread is cut from the device's fixed scratch array (in
// order, 256-byte aligned) instead of the stream's workspace; a request
// that does not fit fails instead of allocating.
struct FixedScratch {
    uint8_t *base;
    size_t cap, used = 0;
    size_t room() const { return used >= cap ? 0 : cap - align256(used); }
};
thread_local FixedScratch *t_fixed = nullptr;

// The stream's workspace (created on first use); g_mu must be held.
Workspace *ws_of_locked(hipStream_t s)
{
    auto &p = g_ws[s];
    if (!p)
        p.reset(new Workspace);
    return p.get();
}

int ws_get(hipStream_t s, Slot slot, size_t bytes, void **out)
{
    if (FixedScratch *f = t_fixed) {
        const size_t off = align256(f->used);
        if (off > f->cap || bytes > f->cap - off)
            return fail(REALM_INVALID_ARGUMENT,
                        "the product needs more scratch than the no-allocation entry point's " +
                            std::to_string(f->cap >> 20) + " MiB");
        *out = f->base + off;
        f->used = off + bytes;
        return REALM_OK;
    }
    Workspace *w;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        w = ws_of_locked(s);
    }
    bytes = std::max<size_t>(bytes, 256);
    if (w->cap[slot] < bytes) {
        if (w->buf[slot]) {
            hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
            HIP_TRY(hipStreamIsCapturing(s, &cs));
            int graphs;
            {
                std::lock_guard<std::mutex> lk(g_mu);
                graphs = w->graphs;
                if (graphs > 0)
                    w->retired.push_back(w->buf[slot]);
            }
            if (graphs == 0 && cs == hipStreamCaptureStatusNone) {
                HIP_TRY(hipStreamSynchronize(s));
                HIP_TRY(hipFree(w->buf[slot]));
            } // else: retired (or, under a capture the library does not track, kept)
            w->buf[slot] = nullptr;
            w->cap[slot] = 0;
        }
        size_t cap = align256(bytes + bytes / 4);
        HIP_TRY(hipMalloc(&w->buf[slot], cap));
        w->cap[slot] = cap;
    }
    *out = w->buf[slot];
    return REALM_OK;
}

// ----------------------------------------------------------------- weights

struct Weight {
    int type = 0;
    size_t n = 0, k = 0, kx = 0; // kx: padded K of the device layout
    size_t bytes = 0;
    void *dev = nullptr;          // owned allocation (null for a per-call weight)
    const void *w0 = nullptr, *w1 = nullptr, *w2 = nullptr;
    bool wide = false;            // Q6_K with some |sub-scale| > 63
};

std::unordered_map<uint64_t, Weight> g_weights;
uint64_t g_next_handle = 1;

// Byte offsets of the streams of the device layout (see kernels/common.h).
// Device layout of an [n, k] matrix (offsets of its streams in one
// allocation).  Every stream has 4 zeroed rows of padding past row n-1: a
// GEMV pass covers up to 4 rows and reads them without per-row clamping.
size_t layout(int type, size_t n, size_t k, size_t off[3], size_t *kx)
{
    size_t B = k / 256;
    size_t np = n + 4;
    if (type == GGML_Q4_K) {
        off[0] = 0;
        off[1] = align256(np * B * 16);
        off[2] = 0;
        *kx = k;
        return off[1] + np * (k / 2);
    }
    if (type == GGML_Q6_K) {
        off[0] = 0;
        off[1] = align256(np * B * 2);
        off[2] = off[1] + align256(np * B * 16);
        *kx = k;
        return off[2] + np * B * 192;
    }
    // Q8_0, and the 32-element formats as q8m (the Q8_0 streams plus a delta
    // stream shaped like the scales)
    size_t kp = round_up(k, 64);
    off[0] = 0;
    off[1] = align256(np * (kp / 32) * 2);
    *kx = kp;
    if (type == GGML_Q8_0) {
        off[2] = 0;
        return off[1] + np * kp;
    }
    off[2] = align256(off[1] + np * kp);
    return off[2] + np * (kp / 32) * 2;
}

bool q6k_wide(const uint8_t *blocks, size_t nblocks)
{
    for (size_t b = 0; b < nblocks; ++b) {
        const int8_t *sc = reinterpret_cast<const int8_t *>(blocks + b * 210 + 192);
        for (int i = 0; i < 16; ++i)
            if (sc[i] > 63 || sc[i] < -63)
                return true;
    }
    return false;
}

// Upload reference-layout blocks and repack them into `dst` (device layout).
int upload_repack(int type, const void *blocks, size_t n, size_t k, void *dst, Weight *w,
                  hipStream_t s)
{
    size_t nblocks = n * (k / block_elems(type));
    size_t raw_bytes = nblocks * block_bytes(type);
    size_t off[3], kx;
    size_t total = layout(type, n, k, off, &kx);
    w->type = type;
    w->n = n;
    w->k = k;
    w->kx = kx;
    w->bytes = total;
    uint8_t *base = (uint8_t *)dst;
    w->w0 = base + off[0];
    w->w1 = base + off[1];
    w->w2 = type == GGML_Q6_K || is_block32(type) ? base + off[2] : nullptr;
    w->wide = type == GGML_Q6_K && q6k_wide((const uint8_t *)blocks, nblocks);
    // zeroes the row padding (and the Q8_0 K padding) of every stream
    HIP_TRY(hipMemsetAsync(dst, 0, total, s));
    if (nblocks == 0)
        return REALM_OK;
    void *raw;
    CHECK(ws_get(s, WS_RAW, raw_bytes, &raw));
    HIP_TRY(hipMemcpyAsync(raw, blocks, raw_bytes, hipMemcpyHostToDevice, s));
    long long nb = (long long)nblocks;
    if (type == GGML_Q4_K) {
        void *hdr = (void *)w->w0, *qs = (void *)w->w1;
        int bpr = (int)(k / 256);
        void *args[] = {&raw, &hdr, &qs, &nb, &bpr};
        CHECK(launch("realm_repack_q4k", dim3((unsigned)((nblocks * 9 + 255) / 256)), dim3(256),
                     0, s, args));
    } else if (type == GGML_Q6_K) {
        void *dq = (void *)w->w0, *scq = (void *)w->w1, *qq = (void *)w->w2;
        int bpr = (int)(k / 256);
        void *args[] = {&raw, &dq, &scq, &qq, &nb, &bpr};
        CHECK(launch("realm_repack_q6k", dim3((unsigned)((nblocks * 64 + 255) / 256)),
                     dim3(256), 0, s, args));
    } else if (type == GGML_Q8_0) {
        void *dq = (void *)w->w0, *qq = (void *)w->w1;
        int kbr = (int)(k / 32), kp = (int)kx;
        void *args[] = {&raw, &dq, &qq, &nb, &kbr, &kp};
        CHECK(launch("realm_repack_q80", dim3((unsigned)((nblocks * 32 + 255) / 256)),
                     dim3(256), 0, s, args));
    } else { // the 32-element formats: q8m
        void *dq = (void *)w->w0, *qq = (void *)w->w1, *mq = (void *)w->w2;
        int kbr = (int)(k / 32), kp = (int)kx, it = type;
        void *args[] = {&raw, &dq, &qq, &mq, &nb, &kbr, &kp, &it};
        CHECK(launch("realm_repack_q32", dim3((unsigned)((nblocks * 32 + 255) / 256)),
                     dim3(256), 0, s, args));
    }
    return REALM_OK;
}

// ------------------------------------------------------------------ LoRA

struct Adapter {
    int dtype = 0;
    void *a = nullptr, *b = nullptr;
    size_t rank = 0, in = 0, out = 0;
    float alpha = 0.f;
    int uses = 0; // number of sets holding it
};
struct AdapterSet {
    void *table = nullptr;  // device: count LoraEntry, then the chunk list
    void *chunks = nullptr; // device: nchunks LoraChunk (fused shrink), inside table's allocation
    size_t count = 0, in = 0, out = 0, nchunks = 0;
    int rmax = 0;
    std::vector<uint64_t> members;
};
std::unordered_map<uint64_t, Adapter> g_adapters;
std::unordered_map<uint64_t, AdapterSet> g_sets;

struct LoraCall {
    const AdapterSet *set;
    const int32_t *d_ids;
};

// --------------------------------------------------------------- dispatch

// The decoder layer's step before a one-token product, fused into the
// GEMV's x staging (gemv.hip "_n" and "_s" kernels): mode 1, RMSNorm of
// x + a (a may be null) times w, x + a written to sum by workgroup 0 (sum
// may be null); mode 2, SwiGLU of gate = x and up = a.
struct GemvPre {
    int mode = 0;
    const float *a = nullptr;
    const float *w = nullptr;
    float *sum = nullptr;
    float eps = 0.f;
};

// M = 1..4 tokens, f32 activations: the integer-dot GEMV over 1..4
// matrices of one format that share x (rows concatenated); 2 tokens run the
// 2-token kernels, 3 and 4 the 4-token ones (every weight load serves all of
// them).  Returns BACKEND_UNSUPPORTED when the row is too long for the
// kernel's register budget or the quantized x of all tokens does not fit in
// LDS (the caller then uses the MFMA path), and, with a fused pre-step
// (one token of Q4_K, Q6_K or Q8_0, SwiGLU on one matrix), before any
// launch when the fused kernels cannot take the call.
int run_gemv(const Weight *const *ws, int count, const float *d_x, int M, float *const *d_y,
             hipStream_t s, const GemvPre *pre = nullptr)
{
    const Weight &w = *ws[0];
    int U = (int)(w.kx / 64);
    int lpr = U <= 16 ? 16 : (U <= 32 ? 32 : 64);
    int upl = (U + lpr - 1) / lpr;
    const int rpp = 64 / lpr;
    const int nt = M <= 1 ? 1 : (M == 2 ? 2 : 4);
    const int pmode = pre ? pre->mode : 0;
    // per token: 8 x records + up to 2 meta float4 per unit; then one flag
    // word per token (its x needs the exact path)
    size_t lds = (size_t)U * 16 * 10 * nt + 16;
    if (M < 1 || M > 4 || upl > 8 || lds + (pmode ? 64 : 0) > g_dev.max_lds || count < 1 ||
        count > REALM_GEMV_MAX_MATS)
        return REALM_BACKEND_UNSUPPORTED;
    if (pmode) {
        bool ok = M == 1 && (pmode == 1 || count == 1);
        for (int i = 0; i < count; ++i)
            ok = ok && (ws[i]->type == GGML_Q4_K || ws[i]->type == GGML_Q6_K ||
                        ws[i]->type == GGML_Q8_0) &&
                 ws[i]->type == w.type && ws[i]->n % rpp == 0;
        if (!ok)
            return REALM_BACKEND_UNSUPPORTED;
    }
    // A grouped launch needs every matrix to start on a pass boundary;
    // otherwise the matrices go one launch each.
    for (int i = 0; count > 1 && i < count; ++i)
        if (ws[i]->n % rpp) {
            for (int j = 0; j < count; ++j)
                CHECK(run_gemv(ws + j, 1, d_x, M, d_y + j, s));
            return REALM_OK;
        }
    realm::GemvArgs a;
    std::memset(&a, 0, sizeof a);
    int rows = 0;
    for (int i = 0; i < count; ++i) {
        a.w0[i] = ws[i]->w0;
        a.w1[i] = ws[i]->w1;
        a.w2[i] = ws[i]->w2;
        a.y[i] = d_y[i];
        a.row_start[i] = rows;
        rows += (int)ws[i]->n;
    }
    for (int i = count; i <= REALM_GEMV_MAX_MATS; ++i)
        a.row_start[i] = rows;
    a.nmat = count;
    a.x = d_x;
    a.K = (int)w.k;
    a.KX = (int)w.kx;
    a.nan_fb = g_nan_fb.load();
    a.m = M;
    if (pmode) {
        a.pre_a = pre->a;
        a.pre_w = pre->w;
        a.pre_sum = pre->sum;
        a.pre_eps = pre->eps;
    }
    // At most one workgroup per CU (each stages x in its LDS); each wave
    // keeps a ring of D passes in flight, D the smallest variant that holds
    // all of the wave's passes (so the whole weight stream is requested
    // before the first pass is computed).  The workgroup size follows the
    // variant's register budget (GEMV_TH in gemv.hip).
    static const int d_u1[] = {1, 2, 3, 4, 6, 8, 12}, d_u2[] = {1, 2, 3, 4},
                     d_u3[] = {1, 2, 3, 4, 6}, d_u45[] = {1, 2}, d_big[] = {1};
    const int *ds = upl == 1 ? d_u1 : upl == 2 ? d_u2 : upl == 3 ? d_u3 : upl <= 5 ? d_u45 : d_big;
    int nd = upl == 1 ? 7 : upl == 2 ? 4 : upl == 3 ? 5 : upl <= 5 ? 2 : 1;
    if (nt > 1) // the multi-token kernels: depths 1-4, 1-2 and 1 (gemv.hip)
        nd = upl == 1 ? 4 : upl <= 3 ? 2 : 1;
    auto threads_of = [&](int d) { // GEMV_TH and GEMV_THN in gemv.hip
        if (nt == 1)
            return upl == 1 ? (d <= 4 ? 1024 : 512)
                            : (upl <= 3 ? (d == 1 ? 1024 : (upl == 2 || d == 2 ? 512 : 256)) : 256);
        if (upl == 1)
            return nt == 2 || d <= 3 ? 512 : 256;
        return upl == 2 ? (d == 1 && nt == 2 ? 1024 : 512) : (upl == 3 && d == 1 ? 512 : 256);
    };
    const long cu = g_dev.cu_count;
    const long npass = ((long)rows + rpp - 1) / rpp;
    // Measured policy: with one unit per lane, all of a wave's passes in
    // flight when there are at most 3, else two (the next pass loads while
    // the current one computes); with 2-3 units per lane two passes once
    // the halved workgroup (register budget) leaves each wave two of them.
    // Deeper rings cost more registers than they gain.
    int d = 1;
    if (upl == 1 && nt > 1) {
        // multi-token (8 waves per workgroup): all of a wave's passes in
        // flight up to 3 (measured at 7B shapes: Wo best at 2, Q/K/V and
        // gate/up at 3)
        const long t8 = (npass + cu * 8 - 1) / (cu * 8);
        d = (int)std::min<long>(std::max<long>(t8, 1), 3);
    } else if (upl == 1) {
        // one pass in flight while a wave has at most 3 (7B Q/K/V 7.76 us
        // against 8.05 us at depth 3), two beyond (gate/up: 11.46 us at
        // depth 2, 11.83 at 1, 11.93 at 3)
        const long t1 = (npass + cu * 16 - 1) / (cu * 16); // passes per wave
        d = t1 <= 3 ? 1 : 2;
    } else if ((upl == 2 || upl == 3) && npass >= 2 * cu * 8 && nt == 1) {
        d = 2; // (multi-token: one pass in flight measured faster)
    }
    if (w.type == GGML_Q8_0 && d > 8) // its 12-deep ring does not fit the registers
        d = 8;
    if (is_block32(w.type) && d > 3) // q8m (one more dword per unit) spills from depth 4
        d = 3;
    d = std::min(d, ds[nd - 1]);
    if (const char *env = getenv("REALM_GEMV_D")) { // tuning override
        int v = atoi(env);
        for (int i = 0; i < nd; ++i)
            if (ds[i] == v && !(is_block32(w.type) && v > 3))
                d = v;
    }
    if (pmode) // the fused kernels' ring depths (gemv.hip DEF_GEMV_PRE)
        d = std::min(d, upl == 1 ? 3 : upl <= 3 ? 2 : 1);
    const int threads = threads_of(d);
    if (pmode == 1) { // the norm needs every round of x in registers (GEMV_XR)
        const int xr = std::min((512 * upl + threads - 1) / threads, 8);
        if ((8 * U + threads - 1) / threads > xr)
            return REALM_BACKEND_UNSUPPORTED;
    }
    const int wpb = threads / 64;
    long wgs = std::min<long>(cu, (npass + wpb - 1) / wpb);
    if (const char *env = getenv("REALM_GEMV_WGS")) { // tuning override
        long v = atol(env);
        if (v >= 1 && v <= 16 * cu)
            wgs = v;
    }
    // the fused norm kernels take the grouped form (any count), SwiGLU the
    // single one
    const bool m4 = pmode == 1 || (pmode == 0 && count > 1);
    std::string name = std::string("realm_gemv_") + fmt_name(w.type) + "_l" +
                       std::to_string(lpr) + "_u" + std::to_string(upl) + "_d" +
                       std::to_string(d) + "_m" + (m4 ? "4" : "1") +
                       (nt == 1 ? "" : "_t" + std::to_string(nt)) +
                       (pmode == 1 ? "_n" : pmode == 2 ? "_s" : "");
    void *args[] = {&a};
    return launch(name, dim3((unsigned)std::max<long>(wgs, 1)), dim3(threads), lds, s, args);
}

// MFMA path for any M: activation prep (once per input, shared by a group
// of weights), optional LoRA shrink, then the MFMA kernel.
struct GemmTile {
    std::string name;
    unsigned rows_per_wg, toks_per_wg, threads;
    bool tiled = false; // LDS-tiled kernel (gemm_tiled.hip): 1-D grid over tiles
    int ord = 0;        // activation slot order the kernel reads
    int ks = 1;         // tiled: K splits (parts summed by realm_gemm_tiled_reduce)
};

// LDS-tiled kernel "t<WR><WT><TN><TM><mode><NS>": WR x WT waves, each TN
// 32-row tiles x TM 32-slot token tiles; mode p = packed f32 (16 tokens per
// tile), s = f32 with separate lo MFMAs, b = bf16; NS pipeline stages.
// Returns false for a malformed name or a mode that does not match the input.
bool tiled_tile(const std::string &name, bool bf16, int ks, GemmTile *t)
{
    if (name.size() != 7 || name[0] != 't' || ks < 1 || ks > 64 || name[6] < '2' ||
        name[6] > '4')
        return false;
    for (int i = 1; i < 5; ++i)
        if (name[i] < '1' || name[i] > '8')
            return false;
    const unsigned wr = name[1] - '0', wt = name[2] - '0', tn = name[3] - '0', tm = name[4] - '0';
    const char mode = name[5];
    if ((mode == 'b') != bf16 || (mode != 'b' && mode != 'p' && mode != 's'))
        return false;
    *t = GemmTile{name, wr * tn * 32, wt * tm * (mode == 'p' ? 16u : 32u), wr * wt * 64, true, 1,
                  ks};
    return true;
}

// Kernel choice for a batched product with M tokens against w:
//  * M <= 8 (f32) or M <= 32 (bf16): gemm.hip's small-batch tiles (16 rows x
//    8..32 tokens, K split over the workgroup's waves);
//  * otherwise, Q4_K / Q6_K / Q8_0 (K a multiple of 256): the LDS-tiled
//    kernel on 32x32x16 MFMAs (gemm_tiled.hip) -- packed f32 (16 or 32
//    tokens per workgroup) or bf16 (64 tokens) -- with the K range split so
//    that a launch has at least 256 workgroups;
//  * Q8_0 with K not a multiple of 256: gemm.hip's decode (16 rows x 16..64
//    tokens) or prefill (128 rows x 64 tokens) tiles.
// The tiled kernel's formats; its per-lane weight offsets are 32-bit.
bool tiled_ok(const Weight &w)
{
    return (w.type == GGML_Q4_K || w.type == GGML_Q6_K || w.type == GGML_Q8_0) && w.kx % 256 == 0 &&
           w.bytes < ((size_t)1 << 32);
}

GemmTile gemm_tile(const Weight &w, size_t M, bool bf16)
{
    if (const char *env = getenv("REALM_GEMM_TILE")) { // tuning override (Q4_K, Q6_K)
        const char *ks = getenv("REALM_GEMM_KS");
        GemmTile t;
        if (tiled_ok(w) && tiled_tile(env, bf16, ks ? atoi(ks) : 1, &t))
            return t;
    }
    size_t M16 = round_up(M, 16);
    if (!bf16 && M <= 8)
        return {"s1", 16, 8, 1024};
    if (bf16 && M <= 32)
        return M <= 16 ? GemmTile{"s1", 16, 16, 1024} : GemmTile{"s2", 16, 32, 512};
    if (tiled_ok(w)) {
        GemmTile t;
        // f32 Q6_K past 448 tokens: the lo part as a second MFMA (`s`)
        // beat the packed slots by 8-11% at 511 and 1024 tokens (W_down and
        // 11008 x 4096); it lost at 256 and below, and for Q4_K everywhere
        const char *name = bf16 ? "t4112b2"
                           : M <= 16 ? "t4111p2"
                           : (w.type == GGML_Q6_K && M > 448) ? "t4112s2" : "t4112p2";
        tiled_tile(name, bf16, 1, &t);
        const size_t tiles = ((w.n + t.rows_per_wg - 1) / t.rows_per_wg) *
                             ((M + t.toks_per_wg - 1) / t.toks_per_wg);
        const int nblk = (int)(w.kx / 256);
        int ks = 1;
        while ((size_t)ks * tiles < 256 && ks < 16 && 2 * ks <= nblk)
            ks *= 2;
        t.ks = ks;
        return t;
    }
    if (!bf16 && M <= 32)
        return M <= 16 ? GemmTile{"s2", 16, 16, 512} : GemmTile{"s4", 16, 32, 256};
    if (M16 >= 128)
        return {"p4", 128, 64, 256};
    if (M16 <= 16)
        return {"d1", 16, 16, 256};
    if (M16 <= 32 && !bf16)
        return {"d2", 16, 32, 256};
    return {"d4", 16, 64, 256};
}

struct XPrep {
    void *xh = nullptr, *xl = nullptr, *xm = nullptr, *ts = nullptr;
    size_t Mp = 0;
    size_t rows = 0;         // token rows xprep writes (Mp, plus a zero row for the tiled kernels)
    const void *x = nullptr; // the caller's activations (read again on the exact path)
    bool bf16 = false;
};

int fmt_code(int type) { return type == GGML_Q4_K ? 0 : type == GGML_Q6_K ? 1 : 2; }

// xprep limit: the kernel holds 4 rounds of 1024 x 8 positions per thread
constexpr size_t XPREP_MAX_KX = 32768;

// The prepared-activation buffers of a batched product (no launch).
int prep_x_alloc(const Weight &w, const void *d_x, bool bf16, size_t M, const GemmTile &tile,
                 hipStream_t s, XPrep *p)
{
    if (w.kx > XPREP_MAX_KX)
        return fail(REALM_INVALID_ARGUMENT,
                    "K " + std::to_string(w.k) + " exceeds the batched path's limit of " +
                        std::to_string(XPREP_MAX_KX));
    // every token a workgroup reads must exist in the prepared activations;
    // the tiled kernels also read one all-zero token past them
    p->Mp = round_up(M, tile.toks_per_wg);
    const size_t rows = p->Mp + (tile.tiled ? 1 : 0);
    p->rows = rows;
    size_t B = w.k / 256;
    CHECK(ws_get(s, WS_XH, rows * w.kx * 2, &p->xh));
    if (!bf16)
        CHECK(ws_get(s, WS_XL, rows * w.kx * 2, &p->xl));
    else
        p->xl = nullptr;
    if (w.type == GGML_Q4_K)
        CHECK(ws_get(s, WS_XM, rows * B * 64, &p->xm));
    CHECK(ws_get(s, WS_TS, rows * 4, &p->ts));
    p->x = d_x;
    p->bf16 = bf16;
    return REALM_OK;
}

// The xprep launch; with L, `nshrink` workgroups past its rows run the fused
// LoRA shrink (realm_xprep_lora_*).
int prep_x_launch(const Weight &w, const XPrep &p, size_t M, const GemmTile &tile, hipStream_t s,
                  const realm::LoraGroupArgs *L = nullptr, int nshrink = 0)
{
    const void *d_x = p.x;
    void *xh = p.xh, *xl = p.xl, *xm = p.xm, *ts = p.ts;
    int ibf = p.bf16 ? 1 : 0, iM = (int)M, iK = (int)w.k, iKX = (int)w.kx, irows = (int)p.rows;
    const std::string ord = tile.ord ? "_o1" : "";
    if (L) {
        realm::LoraGroupArgs g = *L;
        void *args[] = {(void *)&d_x, &ibf, &xh, &xl, &xm, &ts, &iM, &iK, &iKX, &irows, &g};
        return launch(std::string("realm_xprep_lora_") + fmt_name(w.type) + ord,
                      dim3((unsigned)(p.rows + (size_t)nshrink)), dim3(1024), 0, s, args);
    }
    void *args[] = {(void *)&d_x, &ibf, &xh, &xl, &xm, &ts, &iM, &iK, &iKX};
    // threads per token: 256 for K <= 8192, 512 for K <= 16384, else 1024
    // (four rounds of 8 positions per thread; none idle at 4096, and all of
    // a thread's loads in one round trip)
    const int th = w.kx <= 8192 ? 256 : w.kx <= 16384 ? 512 : 1024;
    return launch(std::string("realm_xprep_") + fmt_name(w.type) + ord +
                      (th < 1024 ? "_t" + std::to_string(th) : std::string()),
                  dim3((unsigned)p.rows), dim3(th), 0, s, args);
}

int prep_x(const Weight &w, const void *d_x, bool bf16, size_t M, const GemmTile &tile,
           hipStream_t s, XPrep *p)
{
    CHECK(prep_x_alloc(w, d_x, bf16, M, tile, s, p));
    return prep_x_launch(w, *p, M, tile, s);
}

// One launch of the LDS-tiled kernel over 1..4 matrices of one format and K
// that share the prepared activations (Q/K/V, gate/up), each padded to whole
// row tiles.  With a K split, realm_gemm_tiled_reduce then sums each tile's
// parts in split order (deterministic) into the matrices' outputs.
int tiled_launch(const Weight *const *w, float *const *d_y, int count, const XPrep &p, bool bf16,
                 size_t M, const GemmTile &tile, hipStream_t s,
                 const realm::LoraGroupArgs *L = nullptr)
{
    if (count < 1 || count > REALM_GEMM_MAX_SEGS)
        return fail(REALM_INVALID_ARGUMENT, "a tiled launch takes 1..4 matrices");
    const Weight &w0 = *w[0];
    if (w0.kx % 256)
        return fail(REALM_INVALID_ARGUMENT, "tiled GEMM needs K padded to a multiple of 256");
    // Q6_K with some sub-scale beyond +-63 needs the wide decode; it is exact
    // for every Q6_K matrix, so a group with one such matrix uses it for all
    bool wide = false;
    for (int i = 0; i < count; ++i)
        wide = wide || (w[i]->type == GGML_Q6_K && w[i]->wide);
    const std::string name =
        "realm_gemm_" + std::string(wide ? "q6kw" : fmt_name(w0.type)) + "_" + tile.name;
    GemmArgs g;
    std::memset(&g, 0, sizeof g);
    g.w0 = w0.w0;
    g.w1 = w0.w1;
    g.w2 = w0.w2;
    g.y = d_y[0];
    g.N = (int)w0.n;
    g.xh = p.xh;
    g.xl = p.xl;
    g.xm = p.xm;
    g.tscale = (const float *)p.ts;
    g.x = p.x;
    g.xbf16 = p.bf16 ? 1 : 0;
    g.fmt = fmt_code(w0.type);
    g.K = (int)w0.k;
    g.KX = (int)w0.kx;
    g.M = (int)M;
    g.nan_fb = g_nan_fb.load();
    g.nseg = count;
    size_t rt = 0;
    for (int i = 0; i < REALM_GEMM_MAX_SEGS; ++i) {
        g.seg_tile[i] = i < count ? (int)rt : INT32_MAX;
        if (i >= count)
            continue;
        g.seg_n[i] = (int)w[i]->n;
        g.seg_w0[i] = w[i]->w0;
        g.seg_w1[i] = w[i]->w1;
        g.seg_w2[i] = w[i]->w2;
        g.seg_y[i] = d_y[i];
        rt += (w[i]->n + tile.rows_per_wg - 1) / tile.rows_per_wg;
    }
    g.seg_tile[REALM_GEMM_MAX_SEGS] = INT32_MAX;
    const size_t TT = (p.Mp + tile.toks_per_wg - 1) / tile.toks_per_wg;
    if (rt * TT * 8 > (size_t)INT32_MAX)
        return fail(REALM_INVALID_ARGUMENT, "batched product too large for one launch");
    g.rtiles = (int)rt;
    const int nblk = (int)(w0.kx / 256);
    g.ksplit = tile.ks < nblk ? tile.ks : nblk;
    // in the fixed scratch region, fewer K splits when the parts would not fit
    while (t_fixed && g.ksplit > 1 &&
           rt * TT * g.ksplit * tile.rows_per_wg * tile.toks_per_wg * sizeof(float) >
               t_fixed->room())
        g.ksplit /= 2;
    // parts for a K split, and for the LoRA-fused reduce even without one
    if (g.ksplit > 1 || L) {
        void *part = nullptr;
        CHECK(ws_get(s, WS_PART,
                     rt * TT * g.ksplit * tile.rows_per_wg * tile.toks_per_wg * sizeof(float),
                     &part));
        g.part = (float *)part;
    }
    // XCDs along the token tiles: enough that each XCD's share of the
    // activations (f16, hi and lo for f32 input) stays within 2 MB of L2
    const size_t xbytes = p.Mp * w0.kx * (bf16 ? 2 : 4);
    int xt = 1;
    while (xt < 8 && (size_t)xt < TT && xbytes / xt > ((size_t)2 << 20))
        xt *= 2;
    if (const char *env = getenv("REALM_GEMM_XT")) { // tuning override
        const int e = atoi(env);
        xt = e == 1 || e == 2 || e == 4 || e == 8 ? e : xt;
    }
    g.xt = xt;
    const size_t xr = 8 / xt, rk = rt * (size_t)g.ksplit;
    const dim3 grid((unsigned)(8 * ((rk + xr - 1) / xr) * ((TT + xt - 1) / xt)));
    void *args[] = {&g};
    CHECK(launch(name, grid, dim3(tile.threads), 0, s, args));
    if (g.part) {
        int grows = (int)tile.rows_per_wg, gtok = (int)tile.toks_per_wg;
        const dim3 rgrid((unsigned)(rt * TT), (unsigned)((grows * gtok + 255) / 256));
        if (L) {
            realm::LoraGroupArgs lg = *L;
            void *rargs[] = {&g, &grows, &gtok, &lg};
            CHECK(launch("realm_gemm_tiled_reduce_lora", rgrid, dim3(256), 0, s, rargs));
        } else {
            void *rargs[] = {&g, &grows, &gtok};
            CHECK(launch("realm_gemm_tiled_reduce", rgrid, dim3(256), 0, s, rargs));
        }
    }
    return REALM_OK;
}

// Whether the LoRA shrink runs on the per-thread side stream beside the base
// product (REALM_LORA_SIDE=1, for tuning) or on the caller's stream before it
// (default: on MI355X the cross-queue fork and join of a graph cost more, 5-10
// us each, than the overlap saves).
bool lora_side()
{
    const char *e = getenv("REALM_LORA_SIDE");
    return e && e[0] == '1';
}

// LoRA shrink output: one part per 512 positions of K (summed by the
// expand), [part][token][rmax rounded to 8] f32 per matrix
struct LoraU {
    int nparts, pstride;
    size_t bytes() const { return (size_t)nparts * pstride * 4; }
};
LoraU lora_u(const Weight &w, const AdapterSet &set, const XPrep &p)
{
    return {(int)((w.kx + 511) / 512), (int)(p.Mp * round_up(set.rmax, 8))};
}

// Kernel arguments of a LoRA shrink or expand launch over `count`
// projections that share the prepared input and the token ids; u[i] is
// projection i's slice of the shrink output, y[i] its output.
realm::LoraGroupArgs lora_group_args(const Weight *const *w, const LoraCall *lc, int count,
                                     const XPrep &p, size_t M, void *const *u, float *const *y)
{
    realm::LoraGroupArgs g;
    std::memset(&g, 0, sizeof g);
    g.xh = p.xh;
    g.xl = p.xl;
    g.tscale = (const float *)p.ts;
    g.x = p.x;
    g.xbf16 = p.bf16 ? 1 : 0;
    g.ids = lc[0].d_ids;
    g.M = (int)M;
    g.K = (int)w[0]->k;
    g.KX = (int)w[0]->kx;
    g.nparts = lora_u(*w[0], *lc[0].set, p).nparts;
    int slots = 0;
    for (int i = 0; i < count; ++i) {
        const AdapterSet &set = *lc[i].set;
        g.a_start[i] = slots;
        slots += (int)set.count;
        g.table[i] = (const LoraEntry *)set.table;
        g.u[i] = (float *)u[i];
        g.y[i] = y ? y[i] : nullptr;
        g.N[i] = (int)w[i]->n;
        g.rmax[i] = (int)round_up(set.rmax, 8);
        g.pstride[i] = lora_u(*w[i], set, p).pstride;
    }
    g.a_start[count] = slots;
    for (int i = count + 1; i <= REALM_GEMM_MAX_SEGS; ++i)
        g.a_start[i] = INT32_MAX;
    return g;
}

// u = A_a x for every token's adapter a, from the prepared activations, for
// `count` projections in one launch (optionally on the side stream, joined
// again before the expand).
int lora_shrink_launch(const Weight *const *w, const LoraCall *lc, int count, const XPrep &p,
                       bool bf16, size_t M, const GemmTile &tile, void *const *u, hipStream_t s)
{
    realm::LoraGroupArgs g = lora_group_args(w, lc, count, p, M, u, nullptr);
    int rmax = 0;
    for (int i = 0; i < count; ++i)
        rmax = std::max(rmax, lc[i].set->rmax);
    const unsigned slots = (unsigned)g.a_start[count];
    if (slots == 0)
        return REALM_OK;
    void *args[] = {&g};
    const std::string name = std::string("realm_lora_shrink_") + fmt_name(w[0]->type) +
                             (bf16 ? "_bf16" : "_f32") + (tile.ord ? "_o1" : "");
    const bool use_side = lora_side();
    hipStream_t side = s;
    hipEvent_t fork = nullptr, join = nullptr;
    if (use_side) {
        CHECK(side_stream(&side, &fork, &join));
        HIP_TRY(hipEventRecord(fork, s));
        HIP_TRY(hipStreamWaitEvent(side, fork, 0));
    }
    CHECK(launch(name, dim3(slots, (unsigned)((rmax + 15) / 16), (unsigned)g.nparts), dim3(256),
                 0, side, args));
    if (use_side)
        HIP_TRY(hipEventRecord(join, side));
    return REALM_OK;
}

// y += scale_a B_a u per token for `count` projections in one launch, one
// workgroup per (adapter slot, 64 rt rows, 16 tokens); y already holds the
// base product.
int lora_expand_launch(const Weight *const *w, const LoraCall *lc, int count, const XPrep &p,
                       size_t M, void *const *u, float *const *d_y, hipStream_t s)
{
    if (lora_side()) {
        hipStream_t side;
        hipEvent_t fork, join;
        CHECK(side_stream(&side, &fork, &join));
        HIP_TRY(hipStreamWaitEvent(s, join, 0));
    }
    realm::LoraGroupArgs g = lora_group_args(w, lc, count, p, M, u, d_y);
    size_t nmax = 0;
    for (int i = 0; i < count; ++i)
        nmax = std::max(nmax, w[i]->n);
    const unsigned slots = (unsigned)g.a_start[count];
    if (slots == 0 || nmax == 0)
        return REALM_OK;
    // 64-row tiles per workgroup: 8, or 4 (twice the workgroups) when the
    // adapter slots x row groups of 512 leave fewer than two per CU
    // (measured: config-4 q/k/v/o 4.8% LoRA overhead at 4 against 10% at 8;
    // 2 was slower than either for config 3)
    int rt = (long)slots * (long)((nmax + 511) / 512) < 2L * g_dev.cu_count ? 4 : 8;
    if (const char *env = getenv("REALM_LORA_EXPAND_RT")) { // tuning override
        const int v = atoi(env);
        if (v == 2 || v == 4 || v == 8)
            rt = v;
    }
    void *args[] = {&g};
    const std::string name = rt == 8 ? "realm_lora_expand" : "realm_lora_expand_rt" + std::to_string(rt);
    return launch(name,
                  dim3(slots, (unsigned)((nmax + 64 * rt - 1) / (64 * rt)), (unsigned)((M + 15) / 16)),
                  dim3(256), 0, s, args);
}

// Small-batch multi-LoRA with the shrink folded into the xprep launch and
// the expand into the K-split reduce (gemm.hip lora_shrink_fused,
// gemm_tiled.hip realm_gemm_tiled_reduce_lora): the three launches of a
// base call.  Taken for f32 activations (16-byte aligned) of at most
// LORA_FUSED_MAX_M tokens on the tiled kernels, ranks up to LORA_FUSED_RMAX;
// otherwise (and with REALM_LORA_FUSED=0, for comparison) the separate
// shrink and expand launches.
constexpr size_t LORA_FUSED_MAX_WGS = 65536;

bool lora_fused_ok(const GemmTile &tile, size_t M, bool bf16, const Weight &w0, const void *d_x,
                   const LoraCall *lc, int count)
{
    if (const char *env = getenv("REALM_LORA_FUSED"))
        if (env[0] == '0')
            return false;
    // the fused reduce: a workgroup's 256 elements span at most 3 tokens
    if (!tile.tiled || bf16 || M > LORA_FUSED_MAX_M || tile.rows_per_wg < 128 ||
        ((uintptr_t)d_x & 15) != 0)
        return false;
    const size_t np = (w0.k + LORA_FUSED_KP - 1) / LORA_FUSED_KP;
    size_t wgs = 0;
    for (int i = 0; i < count; ++i) {
        if (lc[i].set->rmax > LORA_FUSED_RMAX)
            return false;
        wgs += lc[i].set->nchunks * np;
    }
    return wgs <= LORA_FUSED_MAX_WGS;
}

int lora_fused_run(const Weight *const *w, const LoraCall *lc, int count, const void *d_x,
                   size_t M, const GemmTile &tile, float *const *d_y, hipStream_t s)
{
    XPrep p;
    CHECK(prep_x_alloc(*w[0], d_x, false, M, tile, s, &p));
    const int np = (int)((w[0]->k + LORA_FUSED_KP - 1) / LORA_FUSED_KP);
    size_t uoff[REALM_GEMM_MAX_SEGS], ubytes = 0;
    for (int i = 0; i < count; ++i) {
        uoff[i] = ubytes;
        ubytes += align256((size_t)np * p.Mp * round_up(lc[i].set->rmax, 8) * sizeof(float));
    }
    void *u = nullptr;
    CHECK(ws_get(s, WS_U, ubytes, &u));
    void *us[REALM_GEMM_MAX_SEGS];
    for (int i = 0; i < count; ++i)
        us[i] = (uint8_t *)u + uoff[i];
    realm::LoraGroupArgs L = lora_group_args(w, lc, count, p, M, us, d_y);
    L.nparts = np;
    int wgs = 0;
    for (int i = 0; i < count; ++i) {
        const AdapterSet &set = *lc[i].set;
        L.pstride[i] = (int)(p.Mp * round_up(set.rmax, 8));
        L.chunks[i] = (const realm::LoraChunk *)set.chunks;
        L.wg_start[i] = wgs;
        wgs += (int)set.nchunks * np;
    }
    for (int i = count; i <= REALM_GEMM_MAX_SEGS; ++i)
        L.wg_start[i] = i == count ? wgs : INT32_MAX;
    CHECK(prep_x_launch(*w[0], p, M, tile, s, &L, wgs));
    return tiled_launch(w, d_y, count, p, false, M, tile, s, &L);
}

int gemm_launch(const Weight &w, const XPrep &p, bool bf16, size_t M, const GemmTile &tile,
                float *d_y, hipStream_t s, const LoraCall *lora)
{
    void *u = nullptr;
    if (lora) {
        CHECK(ws_get(s, WS_U, lora_u(w, *lora->set, p).bytes(), &u));
        const Weight *wp = &w;
        CHECK(lora_shrink_launch(&wp, lora, 1, p, bf16, M, tile, &u, s));
    }
    if (tile.tiled) {
        const Weight *wp = &w;
        CHECK(tiled_launch(&wp, &d_y, 1, p, bf16, M, tile, s));
    } else {
        std::string fmt = fmt_name(w.type);
        if (w.type == GGML_Q6_K && w.wide)
            fmt = "q6kw";
        const std::string name = "realm_gemm_" + fmt + "_" + tile.name + (bf16 ? "_bf16" : "_f32");
        GemmArgs g;
        std::memset(&g, 0, sizeof g);
        g.w0 = w.w0;
        g.w1 = w.w1;
        g.w2 = w.w2;
        g.xh = p.xh;
        g.xl = p.xl;
        g.xm = p.xm;
        g.tscale = (const float *)p.ts;
        g.x = p.x;
        g.xbf16 = p.bf16 ? 1 : 0;
        g.fmt = fmt_code(w.type);
        g.y = d_y;
        g.N = (int)w.n;
        g.K = (int)w.k;
        g.KX = (int)w.kx;
        g.M = (int)M;
        g.nan_fb = g_nan_fb.load();
        g.ksplit = 1;
        void *args[] = {&g};
        const dim3 grid((unsigned)((w.n + tile.rows_per_wg - 1) / tile.rows_per_wg),
                        (unsigned)((p.Mp + tile.toks_per_wg - 1) / tile.toks_per_wg));
        CHECK(launch(name, grid, dim3(tile.threads), 0, s, args));
    }
    if (lora) {
        const Weight *wp = &w;
        CHECK(lora_expand_launch(&wp, lora, 1, p, M, &u, &d_y, s));
    }
    return REALM_OK;
}

int run_gemm(const Weight &w, const void *d_x, bool bf16, size_t M, float *d_y, hipStream_t s,
             const LoraCall *lora)
{
    if (M == 0 || w.n == 0)
        return REALM_OK;
    const GemmTile tile = gemm_tile(w, M, bf16);
    if (lora && lora_fused_ok(tile, M, bf16, w, d_x, lora, 1)) {
        const Weight *wp = &w;
        return lora_fused_run(&wp, lora, 1, d_x, M, tile, &d_y, s);
    }
    XPrep p;
    CHECK(prep_x(w, d_x, bf16, M, tile, s, &p));
    return gemm_launch(w, p, bf16, M, tile, d_y, s, lora);
}

int dense_launch(const float *da, const float *db, float *dc, size_t m, size_t k, size_t n,
                 int bt, hipStream_t s);

// The 32-element formats (q8m layout): the int8-dot GEMV for up to 4
// tokens, 4 tokens per launch up to Q8M_GEMV_MAX_M, and beyond that the
// matrix dequantized into the stream's workspace (bit-exact,
// realm_dequant_q8m) for the dense f32 GEMM.  Measured on 4096 x 4096: one
// token 5.6 us (the dense product over f32 weights took 88 us), 4 tokens
// 8.1 us, 16 tokens 30 us (98 us dense), 64 tokens 124-132 us dequantized +
// dense, about what 16 four-token launches take.
constexpr size_t Q8M_GEMV_MAX_M = 48;

int run_q8m(const Weight &w, const float *d_x, size_t M, float *d_y, hipStream_t s)
{
    if (M <= Q8M_GEMV_MAX_M) {
        int rc = REALM_OK;
        for (size_t t0 = 0; t0 < M && rc == REALM_OK; t0 += 4) {
            const Weight *ws[1] = {&w};
            float *ys[1] = {d_y + t0 * w.n};
            rc = run_gemv(ws, 1, d_x + t0 * w.k, (int)std::min<size_t>(4, M - t0), ys, s);
        }
        if (rc != REALM_BACKEND_UNSUPPORTED) // (rows too long for the GEMV: dense)
            return rc;
    }
    void *wf = nullptr;
    CHECK(ws_get(s, WS_WEIGHT, w.n * w.k * sizeof(float), &wf));
    long long ln = (long long)w.n;
    int ik = (int)w.k, ikp = (int)w.kx, it = w.type;
    const void *dq = w.w0, *qq = w.w1, *mq = w.w2;
    void *args[] = {(void *)&dq, (void *)&qq, (void *)&mq, &wf, &ln, &ik, &ikp, &it};
    CHECK(launch("realm_dequant_q8m", dim3((unsigned)((w.n * w.k + 255) / 256)), dim3(256), 0,
                 s, args));
    return dense_launch(d_x, (const float *)wf, d_y, M, w.k, w.n, 1, s);
}

int run_matmul(const Weight &w, const void *d_x, bool bf16, size_t M, float *d_y,
               hipStream_t s, const LoraCall *lora)
{
    if (is_block32(w.type)) {
        if (bf16 || lora)
            return fail(REALM_BACKEND_UNSUPPORTED,
                        "bf16 input and LoRA take Q4_K, Q6_K or Q8_0 weights");
        if (M == 0 || w.n == 0)
            return REALM_OK;
        return run_q8m(w, (const float *)d_x, M, d_y, s);
    }
    if (is_kq(w.type)) { // resident as dequantized f32 [n][k]: y = x W^T
        if (bf16 || lora)
            return fail(REALM_BACKEND_UNSUPPORTED,
                        "bf16 input and LoRA take Q4_K, Q6_K or Q8_0 weights");
        if (M == 0 || w.n == 0)
            return REALM_OK;
        return dense_launch((const float *)d_x, (const float *)w.w0, d_y, M, w.k, w.n, 1, s);
    }
    if (M <= 4 && !bf16 && !lora) {
        const Weight *ws[1] = {&w};
        float *ys[1] = {d_y};
        int rc = run_gemv(ws, 1, (const float *)d_x, (int)M, ys, s);
        if (rc != REALM_BACKEND_UNSUPPORTED)
            return rc;
    }
    return run_gemm(w, d_x, bf16, M, d_y, s, lora);
}

int get_weight(uint64_t h, Weight *out)
{
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_weights.find(h);
    if (it == g_weights.end())
        return fail(REALM_INVALID_ARGUMENT, "unknown weight handle " + std::to_string(h));
    *out = it->second;
    return REALM_OK;
}

// Validation of GpuBackendTrait::fused_dequant_matmul_* (candle_backend.rs:
// 448-464 and 1115-1131; lib.rs:339-345).
int validate_fused(int type, size_t n_blocks, size_t input_len, size_t batch, size_t n,
                   size_t k)
{
    size_t qk = block_elems(type);
    if (k % qk)
        return fail(REALM_INVALID_ARGUMENT, "K dimension " + std::to_string(k) +
                                                " must be multiple of " + std::to_string(qk));
    size_t expected = n * (k / qk);
    if (n_blocks != expected)
        return fail(REALM_INVALID_ARGUMENT, "Expected " + std::to_string(expected) + " " +
                                                (type == GGML_Q4_K   ? "Q4_K"
                                                 : type == GGML_Q6_K ? "Q6_K"
                                                                     : "Q8_0") +
                                                " blocks, got " + std::to_string(n_blocks));
    if (input_len != batch * k)
        return fail(REALM_INVALID_ARGUMENT, "Input size mismatch: expected " +
                                                std::to_string(batch * k) + ", got " +
                                                std::to_string(input_len));
    if (k > (size_t)INT32_MAX || n > (size_t)INT32_MAX || batch > (size_t)INT32_MAX)
        return fail(REALM_INVALID_ARGUMENT, "dimension exceeds 2^31-1");
    return REALM_OK;
}

int dense_launch(const float *da, const float *db, float *dc, size_t m, size_t k, size_t n,
                 int bt, hipStream_t s);

// Dequantize nb blocks of a kept-dequantized format (raw reference bytes on
// the device) into f32 y on stream s.
int dq_launch(int type, const void *raw, float *y, size_t nb, hipStream_t s)
{
    long long lnb = (long long)nb;
    int it = type;
    void *args[] = {(void *)&raw, &y, &lnb, &it};
    const size_t per = block_elems(type);
    return launch(is_kq(type) ? "realm_dequant_kq" : "realm_dequant_q32",
                  dim3((unsigned)((nb * per + 255) / 256)), dim3(256), 0, s, args);
}

// Q4_0 / Q4_1 / Q5_0 / Q5_1 / Q8_1 (candle_backend.rs:837-1103) and the
// reference's Q5_K / Q8_K / Q2_K / Q3_K (candle_backend.rs:507-571,
// 639-836): validated as the reference does, dequantized on the device into
// f32 W [n][k], then y = x W^T on the f32 MFMA GEMM.
int fused_block32(int type, const void *blocks, size_t n_blocks, const float *input,
                  size_t input_len, size_t batch, size_t n, size_t k, float *out)
{
    const size_t qk = block_elems(type);
    if (k % qk)
        return fail(REALM_INVALID_ARGUMENT, "K dimension " + std::to_string(k) +
                                                " must be multiple of " + std::to_string(qk));
    if (n_blocks != n * (k / qk))
        return fail(REALM_INVALID_ARGUMENT, "Expected " + std::to_string(n * (k / qk)) + " " +
                                                dq_name(type) + " blocks, got " +
                                                std::to_string(n_blocks));
    if (input_len != batch * k) {
        // the 32-element formats check the input length (InvalidShape); for
        // the K formats the tensor creation fails (Error::Runtime)
        if (is_kq(type))
            return fail(REALM_GENERIC_FAILURE, "Failed to create input tensor: shape mismatch");
        return fail(REALM_INVALID_ARGUMENT, "Input length " + std::to_string(input_len) +
                                                " does not match batch_size * k = " +
                                                std::to_string(batch * k));
    }
    if (!out || (n_blocks && !blocks) || (input_len && !input))
        return fail(REALM_INVALID_ARGUMENT, "null pointer argument");
    if (n > (size_t)INT32_MAX || k > (size_t)INT32_MAX || batch > (size_t)INT32_MAX)
        return fail(REALM_INVALID_ARGUMENT, "dimension exceeds 2^31-1");
    CHECK(ensure_init());
    if (batch == 0 || n == 0)
        return REALM_OK;
    if (k == 0) {
        std::memset(out, 0, batch * n * sizeof(float));
        return REALM_OK;
    }
    hipStream_t s;
    CHECK(thread_stream(&s));
    void *raw, *w, *dx, *dy;
    const size_t bb = dq_bytes(type);
    CHECK(ws_get(s, WS_RAW, n_blocks * bb, &raw));
    CHECK(ws_get(s, WS_WEIGHT, n * k * 4, &w));
    CHECK(ws_get(s, WS_X, batch * k * 4, &dx));
    CHECK(ws_get(s, WS_Y, batch * n * 4, &dy));
    HIP_TRY(hipMemcpyAsync(raw, blocks, n_blocks * bb, hipMemcpyHostToDevice, s));
    HIP_TRY(hipMemcpyAsync(dx, input, batch * k * 4, hipMemcpyHostToDevice, s));
    CHECK(dq_launch(type, raw, (float *)w, n_blocks, s));
    CHECK(dense_launch((const float *)dx, (const float *)w, (float *)dy, batch, k, n, 1, s));
    HIP_TRY(hipMemcpyAsync(out, dy, batch * n * 4, hipMemcpyDeviceToHost, s));
    HIP_TRY(hipStreamSynchronize(s));
    return REALM_OK;
}

int fused_host(int type, const void *blocks, size_t n_blocks, const float *input,
               size_t input_len, size_t batch, size_t n, size_t k, float *out)
{
    if (is_dq(type))
        return fused_block32(type, blocks, n_blocks, input, input_len, batch, n, k, out);
    if (type != GGML_Q4_K && type != GGML_Q6_K && type != GGML_Q8_0)
        return fail(REALM_BACKEND_UNSUPPORTED,
                    "ggml type " + std::to_string(type) + " is not supported by the HIP backend");
    CHECK(validate_fused(type, n_blocks, input_len, batch, n, k));
    CHECK(ensure_init());
    if (batch == 0 || n == 0)
        return REALM_OK;
    if (k == 0) {
        std::memset(out, 0, batch * n * sizeof(float));
        return REALM_OK;
    }
    hipStream_t s;
    CHECK(thread_stream(&s));
    size_t off[3], kx;
    size_t total = layout(type, n, k, off, &kx);
    void *wbuf, *dx, *dy;
    CHECK(ws_get(s, WS_WEIGHT, total, &wbuf));
    Weight w;
    CHECK(upload_repack(type, blocks, n, k, wbuf, &w, s));
    CHECK(ws_get(s, WS_X, batch * k * 4, &dx));
    CHECK(ws_get(s, WS_Y, batch * n * 4, &dy));
    HIP_TRY(hipMemcpyAsync(dx, input, batch * k * 4, hipMemcpyHostToDevice, s));
    CHECK(run_matmul(w, dx, false, batch, (float *)dy, s, nullptr));
    HIP_TRY(hipMemcpyAsync(out, dy, batch * n * 4, hipMemcpyDeviceToHost, s));
    HIP_TRY(hipStreamSynchronize(s));
    return REALM_OK;
}

// Dense f32 C = A @ B (or A @ B^T, bt = 1) on device pointers; m, n, k >= 1
// and below 2^31.  One workgroup per TMR x 128 tile of C: TMR = 32 or 64 for
// up to 32 or 64 rows (skinny products), 128 otherwise.
int dense_launch(const float *da, const float *db, float *dc, size_t m, size_t k, size_t n,
                 int bt, hipStream_t s)
{
    const size_t tmr = m <= 32 ? 32 : m <= 64 ? 64 : 128;
    const char *kname = m <= 32 ? "realm_dense_f32_m32" : m <= 64 ? "realm_dense_f32_m64"
                                                                   : "realm_dense_f32";
    // K splits (parts summed in split order) until the launch has 256
    // workgroups, keeping at least 256 positions of K per split; skinny
    // tiles until 1024 workgroups and 128 positions (a skinny product streams
    // B once, and a workgroup holds one 16-position slice of it in flight:
    // 32 x 4096 x 4096 B^T took 58 us at 8 splits, 41 us at 32)
    const size_t tiles = ((n + 127) / 128) * ((m + tmr - 1) / tmr);
    const size_t want = tmr < 128 ? 1024 : 256, kmin = tmr < 128 ? 128 : 256;
    int ks = 1;
    while (tiles * ks < want && k / (2 * (size_t)ks) >= kmin && ks < 32)
        ks *= 2;
    if (const char *env = getenv("REALM_DENSE_KS")) // tuning override
        ks = std::max(1, std::min(64, atoi(env)));
    ks = (int)std::min<size_t>((size_t)ks, k); // every split owns at least one k
    while (t_fixed && ks > 1 && (size_t)ks * m * n * sizeof(float) > t_fixed->room())
        ks /= 2; // fixed scratch region: fewer K splits when the parts would not fit
    void *part = nullptr;
    if (ks > 1)
        CHECK(ws_get(s, WS_PART, (size_t)ks * m * n * sizeof(float), &part));
    int M = (int)m, N = (int)n, K = (int)k;
    void *args[] = {(void *)&da, (void *)&db, (void *)&dc, &M, &N, &K, &bt, &ks, &part};
    CHECK(launch(kname,
                 dim3((unsigned)((n + 127) / 128), (unsigned)((m + tmr - 1) / tmr), (unsigned)ks),
                 dim3(256), 0, s, args));
    if (ks > 1) {
        long long total = (long long)(m * n);
        void *rargs[] = {&part, (void *)&dc, &total, &ks};
        CHECK(launch("realm_dense_reduce", dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                     rargs));
    }
    return REALM_OK;
}

// out[0 .. n) = v on stream s.
int fill_launch(float *out, size_t n, float v, hipStream_t s)
{
    if (n == 0)
        return REALM_OK;
    long long ln = (long long)n;
    const unsigned wgs = (unsigned)std::min<size_t>((n + 255) / 256, (size_t)g_dev.cu_count * 8);
    void *args[] = {&out, &ln, &v};
    return launch("realm_fill_f32", dim3(wgs), dim3(256), 0, s, args);
}

// Dense f32 C = A @ B (or A @ B^T) with host pointers.
int dense_host(const float *a, const float *b, float *c, size_t m, size_t k, size_t n, int bt)
{
    CHECK(ensure_init());
    if (m == 0 || n == 0)
        return REALM_OK;
    if (k == 0) {
        std::memset(c, 0, m * n * sizeof(float));
        return REALM_OK;
    }
    if (m > (size_t)INT32_MAX || n > (size_t)INT32_MAX || k > (size_t)INT32_MAX)
        return fail(REALM_INVALID_ARGUMENT, "dimension exceeds 2^31-1");
    hipStream_t s;
    CHECK(thread_stream(&s));
    void *da, *db, *dc;
    CHECK(ws_get(s, WS_X, m * k * 4, &da));
    CHECK(ws_get(s, WS_WEIGHT, k * n * 4, &db));
    CHECK(ws_get(s, WS_Y, m * n * 4, &dc));
    HIP_TRY(hipMemcpyAsync(da, a, m * k * 4, hipMemcpyHostToDevice, s));
    HIP_TRY(hipMemcpyAsync(db, b, k * n * 4, hipMemcpyHostToDevice, s));
    CHECK(dense_launch((const float *)da, (const float *)db, (float *)dc, m, k, n, bt, s));
    HIP_TRY(hipMemcpyAsync(c, dc, m * n * 4, hipMemcpyDeviceToHost, s));
    HIP_TRY(hipStreamSynchronize(s));
    return REALM_OK;
}

int32_t candle_matmul_impl(uint8_t *mem, size_t mem_len, uint32_t a_ptr, uint32_t b_ptr,
                           uint32_t r_ptr, uint32_t m, uint32_t k, uint32_t n, int bt)
{
    size_t a_bytes = (size_t)m * k * 4, b_bytes = (size_t)k * n * 4, r_bytes = (size_t)m * n * 4;
    if (!mem || (size_t)a_ptr + a_bytes > mem_len) {
        fail(REALM_INVALID_ARGUMENT, "Failed to read matrix A: out of bounds");
        return -3;
    }
    if ((size_t)b_ptr + b_bytes > mem_len) {
        fail(REALM_INVALID_ARGUMENT, "Failed to read matrix B: out of bounds");
        return -4;
    }
    // linear memory offsets need not be 4-byte aligned: copy out first
    std::vector<float> A((size_t)m * k), B((size_t)k * n), C((size_t)m * n);
    if (a_bytes)
        std::memcpy(A.data(), mem + a_ptr, a_bytes);
    if (b_bytes)
        std::memcpy(B.data(), mem + b_ptr, b_bytes);
    if (dense_host(A.data(), B.data(), C.data(), m, k, n, bt) != REALM_OK)
        return -5;
    if ((size_t)r_ptr + r_bytes > mem_len) {
        fail(REALM_INVALID_ARGUMENT, "Failed to write result: out of bounds");
        return -6;
    }
    if (r_bytes)
        std::memcpy(mem + r_ptr, C.data(), r_bytes);
    return (int32_t)((size_t)m * n);
}

} // namespace

// ======================================================================= ABI

REALM_API int realm_hip_init(int device)
{
    std::lock_guard<std::mutex> lk(g_mu);
    return init_locked(device);
}

REALM_API const char *realm_hip_last_error(void) { return t_last_error.c_str(); }

REALM_API const char *realm_hip_last_kernel(void) { return t_last_kernel.c_str(); }

REALM_API const char *realm_hip_backend_name(void) { return "HIP (gfx950)"; }

REALM_API int realm_hip_set_nan_fallback(int enable)
{
    g_nan_fb.store(enable ? 1 : 0);
    return REALM_OK;
}

REALM_API int realm_hip_matmul(const float *a, size_t a_len, const float *b, size_t b_len,
                               uint32_t m, uint32_t k, uint32_t n, float *out)
{
    // CandleGpuBackend::matmul fails in tensor creation on a size mismatch
    // (candle_backend.rs:419-425), an Error::Runtime.
    if (a_len != (size_t)m * k || b_len != (size_t)k * n)
        return fail(REALM_GENERIC_FAILURE, "Candle GPU tensor creation failed: shape mismatch");
    return dense_host(a, b, out, m, k, n, 0);
}

REALM_API int realm_hip_matmul_dev(const float *d_a, const float *d_b, float *d_c, uint32_t m,
                                   uint32_t k, uint32_t n, int b_transposed, void *stream)
{
    if ((m && k && !d_a) || (k && n && !d_b) || (m && n && !d_c))
        return fail(REALM_INVALID_ARGUMENT, "null pointer argument");
    CHECK(ensure_init());
    hipStream_t s;
    CHECK(pick_stream(stream, &s));
    if (m == 0 || n == 0)
        return REALM_OK;
    if (m > (uint32_t)INT32_MAX || n > (uint32_t)INT32_MAX || k > (uint32_t)INT32_MAX)
        return fail(REALM_INVALID_ARGUMENT, "dimension exceeds 2^31-1");
    if (k == 0) // C = 0 by a fill kernel: no memset node goes into a captured graph
        return fill_launch(d_c, (size_t)m * n, 0.f, s);
    return dense_launch(d_a, d_b, d_c, m, k, n, b_transposed ? 1 : 0, s);
}

// ------------------------------------------------ element-wise layer ops

namespace {
bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }
} // namespace

REALM_API int realm_hip_rms_norm_dev(const float *d_x, const float *d_residual,
                                     const float *d_weight, float eps, size_t rows, size_t hidden,
                                     float *d_sum, float *d_out, void *stream)
{
    if (rows == 0 || hidden == 0)
        return REALM_OK;
    if (!d_x || !d_weight || !d_out || (d_sum && !d_residual))
        return fail(REALM_INVALID_ARGUMENT, "rms_norm: null pointer argument");
    if (hidden % 4 || hidden > (size_t)INT32_MAX || rows > (size_t)INT32_MAX)
        return fail(REALM_INVALID_ARGUMENT, "rms_norm: hidden must be a multiple of 4 below 2^31");
    if (!aligned16(d_x) || !aligned16(d_weight) || !aligned16(d_out) ||
        (d_residual && !aligned16(d_residual)) || (d_sum && !aligned16(d_sum)))
        return fail(REALM_INVALID_ARGUMENT, "rms_norm: pointers must be 16-byte aligned");
    if (d_sum && (d_sum == d_x || d_sum == d_residual))
        return fail(REALM_INVALID_ARGUMENT, "rms_norm: the sum may not overwrite an input");
    CHECK(ensure_init());
    hipStream_t s;
    CHECK(pick_stream(stream, &s));
    int ih = (int)hidden;
    void *args[] = {(void *)&d_x, (void *)&d_residual, (void *)&d_weight, &eps, &ih, &d_sum,
                    &d_out};
    return launch("realm_rms_norm", dim3((unsigned)rows), dim3(256), 0, s, args);
}

REALM_API int realm_hip_swiglu_dev(const float *d_gate, const float *d_up, size_t n, float *d_out,
                                   void *stream)
{
    if (n == 0)
        return REALM_OK;
    if (!d_gate || !d_up || !d_out)
        return fail(REALM_INVALID_ARGUMENT, "swiglu: null pointer argument");
    if (n % 4 || !aligned16(d_gate) || !aligned16(d_up) || !aligned16(d_out))
        return fail(REALM_INVALID_ARGUMENT,
                    "swiglu: n must be a multiple of 4 and pointers 16-byte aligned");
    CHECK(ensure_init());
    hipStream_t s;
    CHECK(pick_stream(stream, &s));
    size_t n4 = n / 4;
    const unsigned wgs = (unsigned)std::min<size_t>((n4 + 255) / 256, (size_t)g_dev.cu_count * 8);
    void *args[] = {(void *)&d_gate, (void *)&d_up, &n4, &d_out};
    return launch("realm_swiglu", dim3(wgs), dim3(256), 0, s, args);
}

REALM_API int realm_hip_rope_dev(float *d_x, size_t seq_len, size_t num_heads, size_t head_dim,
                                size_t start_pos, float theta, void *stream)
{
    if (seq_len == 0 || num_heads == 0)
        return REALM_OK;
    if (!d_x || head_dim == 0 || head_dim % 2 || ((uintptr_t)d_x & 7))
        return fail(REALM_INVALID_ARGUMENT, "rope: head_dim must be even, x 8-byte aligned");
    const size_t pairs = seq_len * num_heads * (head_dim / 2);
    if (start_pos + seq_len > (size_t)INT32_MAX || pairs / 256 >= (size_t)UINT32_MAX ||
        head_dim > (size_t)INT32_MAX || num_heads > (size_t)INT32_MAX)
        return fail(REALM_INVALID_ARGUMENT, "rope: sizes exceed 2^31-1");
    CHECK(ensure_init());
    hipStream_t s;
    CHECK(pick_stream(stream, &s));
    int is = (int)seq_len, ih = (int)num_heads, id = (int)head_dim, ip = (int)start_pos;
    void *args[] = {&d_x, &is, &ih, &id, &ip, &theta};
    return launch("realm_rope", dim3((unsigned)((pairs + 255) / 256)), dim3(256), 0, s, args);
}

namespace {
// Key splits of a decode attention: small grids split the keys of each
// (token, head) over up to 16 workgroups of at least 64 keys; any cache
// length takes at least as many splits as keep a chunk's scores in LDS.
size_t att_splits(size_t seq_len, size_t kv_len, size_t num_heads, size_t head_dim)
{
    size_t splits = 1;
    if (seq_len * num_heads < 2 * (size_t)g_dev.cu_count && kv_len >= 256)
        splits = std::min<size_t>({16, (2 * (size_t)g_dev.cu_count + seq_len * num_heads - 1) /
                                           (seq_len * num_heads),
                                   (kv_len + 63) / 64});
    if (const char *env = getenv("REALM_ATT_SPLITS")) { // tuning / test override
        const long v = atol(env);
        if (v >= 1 && v <= 64)
            splits = (size_t)v;
    }
    const size_t att_threads = 1024; // ATT_TH in layer_ops.hip
    const size_t max_chunk = g_dev.max_lds / sizeof(float) - head_dim - 256 - 16;
    if ((head_dim + kv_len + att_threads) * sizeof(float) + 64 > g_dev.max_lds)
        splits = std::max(splits, (kv_len + max_chunk - 1) / max_chunk);
    return splits;
}

// The split attention of a one-token decode step with RoPE fused in
// (realm_attention_split_rope): q and this step's key row k_new arrive
// unrotated; the kernel rotates them by the (cos, sin) table of the step's
// position (realm_rope_table) and writes the rotated row into the cache at
// `position`.  The caller checked the arguments and that att_splits() > 1.
int attention_rope_run(const float *d_q, float *d_k_cache, const float *d_v_cache,
                       const float *k_new, size_t kv_len, size_t position, size_t num_heads,
                       size_t num_kv_heads, size_t head_dim, const void *rope_cs, float *d_out,
                       hipStream_t s)
{
    const size_t splits = att_splits(1, kv_len, num_heads, head_dim);
    const size_t chunk = (kv_len + splits - 1) / splits;
    const size_t lds = (head_dim + chunk + 256) * sizeof(float);
    if (splits < 2 || lds + 64 > g_dev.max_lds)
        return fail(REALM_BACKEND_UNSUPPORTED, "attention: no split form for fused RoPE");
    void *part = nullptr;
    CHECK(ws_get(s, WS_ATT, num_heads * splits * (head_dim + 2) * sizeof(float), &part));
    int ikv = (int)kv_len, ipos = (int)position, ih = (int)num_heads, ikh = (int)num_kv_heads,
        id = (int)head_dim, isp = (int)splits, ich = (int)chunk;
    float scale = 1.0f / std::sqrt((float)head_dim);
    void *args[] = {(void *)&d_q, (void *)&d_k_cache, (void *)&d_v_cache, &ikv, &ipos, &ih,
                    &ikh, &id, &scale, &isp, &ich, &part, (void *)&k_new, (void *)&rope_cs};
    CHECK(launch("realm_attention_split_rope", dim3((unsigned)(num_heads * splits)), dim3(256),
                 lds, s, args));
    void *cargs[] = {&part, &isp, &id, &d_out};
    return launch("realm_attention_combine", dim3((unsigned)num_heads), dim3(256), 0, s, cargs);
}
} // namespace

REALM_API int realm_hip_attention_dev(const float *d_q, const float *d_k_cache,
                                      const float *d_v_cache, size_t seq_len, size_t kv_len,
                                      size_t position, size_t num_heads, size_t num_kv_heads,
                                      size_t head_dim, float *d_out, void *stream)
{
    if (seq_len == 0 || num_heads == 0)
        return REALM_OK;
    if (!d_q || !d_out || (kv_len && (!d_k_cache || !d_v_cache)))
        return fail(REALM_INVALID_ARGUMENT, "attention: null pointer argument");
    if (head_dim < 4 || head_dim > 256 || 256 % head_dim || num_kv_heads == 0 ||
        num_heads % num_kv_heads)
        return fail(REALM_INVALID_ARGUMENT,
                    "attention: head_dim must divide 256 (4..256) and kv heads divide heads");
    if (!aligned16(d_k_cache) || !aligned16(d_v_cache))
        return fail(REALM_INVALID_ARGUMENT, "attention: caches must be 16-byte aligned");
    if (seq_len * num_heads > (size_t)UINT32_MAX || position + seq_len > (size_t)INT32_MAX ||
        kv_len > (size_t)INT32_MAX || num_heads > (size_t)INT32_MAX)
        return fail(REALM_INVALID_ARGUMENT, "attention: sizes exceed 2^31-1");
    CHECK(ensure_init());
    // Chunks of many query tokens (prefill): the tiled kernel stages each
    // block of 32 keys once for 32 queries and takes any cache length; its
    // keys split over workgroups when the query tiles alone leave the chip
    // idle (partials combined by realm_attention_combine).
    // REALM_ATT_TILED=1 / 0 forces it on / off (a forced split count,
    // REALM_ATT_SPLITS, turns it off); REALM_ATT_TSPLITS forces its splits.
    bool tiled = seq_len >= 4 && !getenv("REALM_ATT_SPLITS");
    if (const char *env = getenv("REALM_ATT_TILED"))
        tiled = env[0] == '1';
    if (tiled && head_dim % 32 == 0 && num_heads <= 65535 && seq_len <= ((size_t)1 << 26) &&
        aligned16(d_q) && aligned16(d_out)) {
        hipStream_t s;
        CHECK(pick_stream(stream, &s));
        const size_t tiles = (seq_len + 31) / 32;
        const size_t kvis = std::min(kv_len, position + seq_len); // keys the last token sees
        size_t splits = 1;
        if (tiles * num_heads < 2 * (size_t)g_dev.cu_count)
            splits = std::min<size_t>({32, (2 * (size_t)g_dev.cu_count + tiles * num_heads - 1) /
                                               (tiles * num_heads),
                                       (kvis + 63) / 64});
        if (const char *env = getenv("REALM_ATT_TSPLITS")) {
            const long v = atol(env);
            if (v >= 1 && v <= 64)
                splits = (size_t)v;
        }
        splits = std::max<size_t>(splits, 1);
        // chunks of whole 32-key blocks; the split count that covers kvis
        size_t chunk = ((std::max<size_t>(kvis, 1) + splits - 1) / splits + 31) / 32 * 32;
        splits = std::max<size_t>((kvis + chunk - 1) / chunk, 1);
        void *part = nullptr;
        if (splits > 1)
            CHECK(ws_get(s, WS_ATT, seq_len * num_heads * splits * (head_dim + 2) * sizeof(float),
                         &part));
        int is = (int)seq_len, ikv = (int)kv_len, ipos = (int)position, ih = (int)num_heads,
            ikh = (int)num_kv_heads, isp = (int)splits, ich = (int)chunk, id = (int)head_dim;
        float scale = 1.0f / std::sqrt((float)head_dim);
        void *args[] = {(void *)&d_q, (void *)&d_k_cache, (void *)&d_v_cache, &is, &ikv, &ipos,
                        &ih, &ikh, &scale, &isp, &ich, &d_out, &part};
        const std::string kname = "realm_attention_tiled_h" + std::to_string(head_dim);
        CHECK(launch(kname.c_str(), dim3((unsigned)tiles, (unsigned)num_heads, (unsigned)splits),
                     dim3(256), 0, s, args));
        if (splits == 1)
            return REALM_OK;
        void *cargs[] = {&part, &isp, &id, &d_out};
        return launch("realm_attention_combine", dim3((unsigned)(seq_len * num_heads)),
                      dim3(256), 0, s, cargs);
    }
    // Small grids (decode) and long caches: the keys split over workgroups,
    // then the partials combined (att_splits)
    const size_t att_threads = 1024; // ATT_TH in layer_ops.hip
    const size_t splits = att_splits(seq_len, kv_len, num_heads, head_dim);
    if (splits > 1) {
        const size_t chunk = (kv_len + splits - 1) / splits;
        const size_t lds = (head_dim + chunk + 256) * sizeof(float);
        if (lds + 64 > g_dev.max_lds)
            return fail(REALM_BACKEND_UNSUPPORTED,
                        "attention: " + std::to_string(chunk) + " keys per split exceed the LDS");
        if (seq_len * num_heads * splits > (size_t)UINT32_MAX)
            return fail(REALM_INVALID_ARGUMENT, "attention: too many (token, head, split) groups");
        hipStream_t s;
        CHECK(pick_stream(stream, &s));
        void *part = nullptr;
        CHECK(ws_get(s, WS_ATT, seq_len * num_heads * splits * (head_dim + 2) * sizeof(float),
                     &part));
        int ikv = (int)kv_len, ipos = (int)position, ih = (int)num_heads,
            ikh = (int)num_kv_heads, id = (int)head_dim, isp = (int)splits, ich = (int)chunk;
        float scale = 1.0f / std::sqrt((float)head_dim);
        void *args[] = {(void *)&d_q, (void *)&d_k_cache, (void *)&d_v_cache, &ikv, &ipos, &ih,
                        &ikh, &id, &scale, &isp, &ich, &part};
        CHECK(launch("realm_attention_split", dim3((unsigned)(seq_len * num_heads * splits)),
                     dim3(256), lds, s, args));
        void *cargs[] = {&part, &isp, &id, &d_out};
        return launch("realm_attention_combine", dim3((unsigned)(seq_len * num_heads)),
                      dim3(256), 0, s, cargs);
    }
    hipStream_t s;
    CHECK(pick_stream(stream, &s));
    const size_t lds = (head_dim + kv_len + att_threads) * sizeof(float);
    if (lds + 64 > g_dev.max_lds)
        return fail(REALM_BACKEND_UNSUPPORTED,
                    "attention: " + std::to_string(kv_len) + " cached keys exceed the LDS");
    int ikv = (int)kv_len, ipos = (int)position, ih = (int)num_heads, ikh = (int)num_kv_heads,
        id = (int)head_dim;
    float scale = 1.0f / std::sqrt((float)head_dim);
    void *args[] = {(void *)&d_q, (void *)&d_k_cache, (void *)&d_v_cache, &ikv, &ipos, &ih, &ikh,
                    &id, &scale, &d_out};
    return launch("realm_attention", dim3((unsigned)(seq_len * num_heads)),
                  dim3((unsigned)att_threads), lds, s, args);
}

REALM_API int realm_hip_kv_append_dev(const float *d_k, const float *d_v, size_t seq_len,
                                      size_t kv_dim, size_t cur_len, size_t max_len,
                                      float *d_k_cache, float *d_v_cache, void *stream)
{
    if (cur_len + seq_len > max_len)
        return fail(REALM_MODEL_PARSE_ERROR, "KV cache overflow: " + std::to_string(cur_len) +
                                                 " + " + std::to_string(seq_len) + " > " +
                                                 std::to_string(max_len));
    if (seq_len == 0 || kv_dim == 0)
        return REALM_OK;
    if (!d_k || !d_v || !d_k_cache || !d_v_cache)
        return fail(REALM_INVALID_ARGUMENT, "kv_append: null pointer argument");
    CHECK(ensure_init());
    hipStream_t s;
    CHECK(pick_stream(stream, &s));
    const size_t off = cur_len * kv_dim, bytes = seq_len * kv_dim * sizeof(float);
    HIP_TRY(hipMemcpyAsync(d_k_cache + off, d_k, bytes, hipMemcpyDeviceToDevice, s));
    HIP_TRY(hipMemcpyAsync(d_v_cache + off, d_v, bytes, hipMemcpyDeviceToDevice, s));
    return REALM_OK;
}

REALM_API int realm_hip_add_dev(const float *d_a, const float *d_b, size_t n, float *d_out,
                               void *stream)
{
    if (n == 0)
        return REALM_OK;
    if (!d_a || !d_b || !d_out)
        return fail(REALM_INVALID_ARGUMENT, "add: null pointer argument");
    if (n % 4 || !aligned16(d_a) || !aligned16(d_b) || !aligned16(d_out))
        return fail(REALM_INVALID_ARGUMENT,
                    "add: n must be a multiple of 4 and pointers 16-byte aligned");
    CHECK(ensure_init());
    hipStream_t s;
    CHECK(pick_stream(stream, &s));
    size_t n4 = n / 4;
    const unsigned wgs = (unsigned)std::min<size_t>((n4 + 255) / 256, (size_t)g_dev.cu_count * 8);
    void *args[] = {(void *)&d_a, (void *)&d_b, &n4, &d_out};
    return launch("realm_add", dim3(wgs), dim3(256), 0, s, args);
}

namespace {

// Checks one layer's shape, cache room and weights; type[] gets the seven
// weights' formats (Wq, Wk, Wv, Wo, W_gate, W_up, W_down).
int check_layer(const realm_layer *L, size_t seq_len, size_t position, size_t max_seq_len,
                int type[7])
{
    if (!L->attn_norm || !L->ffn_norm)
        return fail(REALM_INVALID_ARGUMENT, "forward_layer: null norm weights");
    const size_t H = L->hidden, heads = L->num_heads, kvh = L->num_kv_heads, hd = L->head_dim,
                 I = L->intermediate, kv_dim = kvh * hd;
    if (H == 0 || heads * hd != H || kvh == 0 || heads % kvh || I == 0 || I % 4 || H % 4 ||
        hd % 4 || 256 % hd || seq_len * (heads + kvh) * (hd / 2) / 256 >= (size_t)UINT32_MAX)
        return fail(REALM_INVALID_ARGUMENT,
                    "forward_layer: hidden must be heads x head_dim, kv heads divide heads, "
                    "hidden and intermediate multiples of 4");
    if (position + seq_len > max_seq_len)
        return fail(REALM_MODEL_PARSE_ERROR, "KV cache overflow: " + std::to_string(position) +
                                                 " + " + std::to_string(seq_len) + " > " +
                                                 std::to_string(max_seq_len));
    const uint64_t h[7] = {L->wq, L->wk, L->wv, L->wo, L->w_gate, L->w_up, L->w_down};
    const uint64_t lora[7] = {L->lora_q,  L->lora_k,    L->lora_v,   L->lora_o,
                              L->lora_gate, L->lora_up, L->lora_down};
    bool any_lora = false;
    for (int i = 0; i < 7; ++i)
        any_lora = any_lora || lora[i] != 0;
    if (any_lora && !L->d_adapter_ids)
        return fail(REALM_INVALID_ARGUMENT,
                    "forward_layer: adapter sets given without device adapter ids");
    if (any_lora && seq_len > 1024)
        return fail(REALM_INVALID_ARGUMENT,
                    "forward_layer: calls with adapters take at most 1024 tokens");
    const size_t n[7] = {H, kv_dim, kv_dim, H, I, I, H}, k[7] = {H, H, H, H, H, H, I};
    for (int i = 0; i < 7; ++i) {
        Weight w;
        CHECK(get_weight(h[i], &w));
        type[i] = w.type;
        if (w.n != n[i] || w.k != k[i])
            return fail(REALM_INVALID_ARGUMENT,
                        "forward_layer: weight " + std::to_string(h[i]) + " is " +
                            std::to_string(w.n) + " x " + std::to_string(w.k) + ", the layer needs " +
                            std::to_string(n[i]) + " x " + std::to_string(k[i]));
    }
    return REALM_OK;
}

// The steps of one layer up to (not including) the final residual add.  The
// layer's input is x, or x + x_res when x_res is set (the previous layer's
// output left as its two addends: the add is fused into this layer's first
// norm, the sum going to h_in).  Leaves h2 = input + attention output and
// down = the FFN output, whose sum is the layer's output.  h2 and down may be
// the buffers x and x_res came in (both are consumed by the first norm).
int layer_steps(const realm_layer *L, const int type[7], const float *x, const float *x_res,
                size_t seq_len, size_t position, float *kc, float *vc, float *ws, float *h_in,
                float *h2, float *down, const void *rope_cs, hipStream_t s)
{
    const size_t H = L->hidden, heads = L->num_heads, kvh = L->num_kv_heads, hd = L->head_dim,
                 I = L->intermediate, kv_dim = kvh * hd;
    const size_t sh = align256(seq_len * H * 4) / 4, si = align256(seq_len * I * 4) / 4;
    float *normed = ws, *q = ws + sh, *att = ws + 2 * sh, *o = ws + 3 * sh, *gate = ws + 4 * sh,
          *up = ws + 4 * sh + si;
    float *k_rows = kc + position * kv_dim, *v_rows = vc + position * kv_dim;
    const float *h = x_res ? h_in : x;
    // One-token calls fuse each RMSNorm into the x staging of the grouped
    // GEMV after it (Q/K/V, gate/up) and SwiGLU into W_down's, for
    // projections without adapters whose matrices share a Q4_K, Q6_K or Q8_0
    // format (REALM_LAYER_FUSE=0 keeps the separate launches).  run_gemv
    // refuses before launching anything when its fused kernels cannot take
    // the call; then the separate launches run.
    const char *fenv = getenv("REALM_LAYER_FUSE");
    const bool fuse = seq_len == 1 && !(fenv && fenv[0] == '0') && aligned16(L->attn_norm) &&
                      aligned16(L->ffn_norm);
    auto fused = [&](const uint64_t *hs, const uint64_t *sets, int n, const float *in,
                     float *const *out, const GemvPre &pre, bool *done) {
        *done = false;
        if (!fuse || !aligned16(in) || (pre.a && !aligned16(pre.a)) ||
            (pre.sum && !aligned16(pre.sum)))
            return (int)REALM_OK;
        Weight w[REALM_GEMV_MAX_MATS];
        const Weight *wp[REALM_GEMV_MAX_MATS];
        for (int i = 0; i < n; ++i) {
            if (sets[i])
                return (int)REALM_OK;
            CHECK(get_weight(hs[i], &w[i]));
            wp[i] = &w[i];
        }
        const int rc = run_gemv(wp, n, in, 1, out, s, &pre);
        if (rc == REALM_BACKEND_UNSUPPORTED)
            return (int)REALM_OK;
        *done = rc == REALM_OK;
        return rc;
    };
    // matrices of one format share a grouped product (GGUF quant mixes
    // often keep V or up in Q6_K: then separate products); with adapter sets
    // on every member, one grouped multi-LoRA product, on some of them, one
    // product per projection
    const int32_t *ids = L->d_adapter_ids;
    auto one = [&](uint64_t hw, uint64_t set, const float *in, float *out) {
        return set ? realm_hip_multi_lora_matmul_dev(hw, set, in, seq_len, ids, out, s)
                   : realm_hip_weights_matmul_dev(hw, in, seq_len, out, s);
    };
    auto products = [&](const uint64_t *hs, const uint64_t *sets, const int *ts,
                        float *const *out, int n) {
        bool same = true, any = false, all = true;
        for (int i = 0; i < n; ++i) {
            same = same && ts[i] == ts[0];
            any = any || sets[i] != 0;
            all = all && sets[i] != 0;
        }
        if (same && !any)
            return realm_hip_weights_matmul_group_dev(hs, n, normed, seq_len, out, s);
        if (same && all)
            return realm_hip_multi_lora_matmul_group_dev(hs, sets, n, normed, seq_len, ids, out, s);
        for (int i = 0; i < n; ++i)
            if (int rc = one(hs[i], sets[i], normed, out[i]))
                return rc;
        return (int)REALM_OK;
    };
    const uint64_t qkv[3] = {L->wq, L->wk, L->wv};
    const uint64_t qkv_sets[3] = {L->lora_q, L->lora_k, L->lora_v};
    float *const qkv_out[3] = {q, k_rows, v_rows};
    // With the fused norm, `normed` is free: the new key row goes there
    // unrotated and the split attention applies RoPE itself (and writes the
    // rotated row into the cache), when the step runs the split form
    const bool rope_fuse = fuse && rope_cs && att_splits(1, position + 1, heads, hd) > 1;
    float *const qkv_fout[3] = {q, rope_fuse ? normed : k_rows, v_rows};
    bool done = false;
    GemvPre norm1;
    norm1.mode = 1;
    norm1.a = x_res;
    norm1.w = L->attn_norm;
    norm1.sum = x_res ? h_in : nullptr;
    norm1.eps = L->rms_norm_eps;
    CHECK(fused(qkv, qkv_sets, 3, x, qkv_fout, norm1, &done));
    if (done && rope_fuse) {
        CHECK(attention_rope_run(q, kc, vc, normed, position + 1, position, heads, kvh, hd,
                                 rope_cs, att, s));
    } else {
        if (!done) {
            CHECK(realm_hip_rms_norm_dev(x, x_res, L->attn_norm, L->rms_norm_eps, seq_len, H,
                                         x_res ? h_in : nullptr, normed, s));
            CHECK(products(qkv, qkv_sets, type, qkv_out, 3));
        }
        { // RoPE of Q and of this call's K rows in one launch (rotations
          // from the call's table of these positions when there is one)
            int iq = (int)heads, ik = (int)kvh, is = (int)seq_len, id = (int)hd,
                ip = (int)position;
            float theta = L->rope_theta;
            const size_t pairs = seq_len * (heads + kvh) * (hd / 2);
            if (rope_cs) {
                void *args[] = {&q, &iq, &k_rows, &ik, &is, &id, (void *)&rope_cs};
                CHECK(launch("realm_rope_qk_tab", dim3((unsigned)((pairs + 255) / 256)),
                             dim3(256), 0, s, args));
            } else {
                void *args[] = {&q, &iq, &k_rows, &ik, &is, &id, &ip, &theta};
                CHECK(launch("realm_rope_qk", dim3((unsigned)((pairs + 255) / 256)), dim3(256),
                             0, s, args));
            }
        }
        CHECK(realm_hip_attention_dev(q, kc, vc, seq_len, position + seq_len, position, heads,
                                      kvh, hd, att, s));
    }
    CHECK(one(L->wo, L->lora_o, att, o));
    const uint64_t gu[2] = {L->w_gate, L->w_up};
    const uint64_t gu_sets[2] = {L->lora_gate, L->lora_up};
    float *const gu_out[2] = {gate, up};
    GemvPre norm2;
    norm2.mode = 1;
    norm2.a = o;
    norm2.w = L->ffn_norm;
    norm2.sum = h2;
    norm2.eps = L->rms_norm_eps;
    CHECK(fused(gu, gu_sets, 2, h, gu_out, norm2, &done));
    if (!done) {
        CHECK(realm_hip_rms_norm_dev(h, o, L->ffn_norm, L->rms_norm_eps, seq_len, H, h2, normed,
                                     s));
        CHECK(products(gu, gu_sets, type + 4, gu_out, 2));
    }
    const uint64_t dn[1] = {L->w_down}, dn_sets[1] = {L->lora_down};
    float *const dn_out[1] = {down};
    GemvPre act;
    act.mode = 2;
    act.a = up;
    CHECK(fused(dn, dn_sets, 1, gate, dn_out, act, &done));
    if (done)
        return REALM_OK;
    CHECK(realm_hip_swiglu_dev(gate, up, seq_len * I, gate, s));
    return one(L->w_down, L->lora_down, gate, down);
}

} // namespace

// n_layers decoder layers of realm_forward_layer (memory64_host.rs:
// 2059-2458) on the device, every step on `stream`: per layer RMSNorm, Q/K/V
// in one grouped product with K and V written straight into the cache rows
// of this call's tokens, RoPE on Q and on those K rows, attention over the
// cache, Wo, the residual add fused with the FFN norm, gate/up in one grouped
// product, SwiGLU, W_down; between layers the residual add is fused into the
// next layer's first norm, and only the last layer's output is summed.
REALM_API int realm_hip_forward_layers_dev(const realm_layer *layers, size_t n_layers,
                                           const float *d_hidden, size_t seq_len,
                                           size_t position, float *const *d_k_caches,
                                           float *const *d_v_caches, size_t max_seq_len,
                                           float *d_out, void *stream)
{
    if (!layers || !d_hidden || !d_out || (n_layers && (!d_k_caches || !d_v_caches)))
        return fail(REALM_INVALID_ARGUMENT, "forward_layers: null pointer argument");
    if (seq_len == 0 || n_layers == 0)
        return REALM_OK;
    std::vector<int> types(7 * n_layers);
    size_t wsize = 0;
    for (size_t l = 0; l < n_layers; ++l) {
        if (!d_k_caches[l] || !d_v_caches[l])
            return fail(REALM_INVALID_ARGUMENT, "forward_layers: null KV cache");
        if (layers[l].hidden != layers[0].hidden)
            return fail(REALM_INVALID_ARGUMENT, "forward_layers: layers of different widths");
        CHECK(check_layer(&layers[l], seq_len, position, max_seq_len, &types[7 * l]));
        wsize = std::max(wsize, 4 * align256(seq_len * layers[l].hidden * 4) +
                                    2 * align256(seq_len * layers[l].intermediate * 4));
    }
    CHECK(ensure_init());
    hipStream_t s;
    CHECK(pick_stream(stream, &s));
    // per-layer intermediates, then the chained h_in, h2 and down [seq][H],
    // then the one-token step's rotation table
    const size_t sh = align256(seq_len * layers[0].hidden * 4);
    const size_t hd0 = layers[0].head_dim;
    void *ws = nullptr;
    CHECK(ws_get(s, WS_LAYER, wsize + 3 * sh + align256(seq_len * hd0 * 4), &ws));
    uint8_t *base = static_cast<uint8_t *>(ws);
    float *h_in = (float *)(base + wsize), *h2 = (float *)(base + wsize + sh),
          *down = (float *)(base + wsize + 2 * sh);
    // One token: the (cos, sin) of its position's rotary angles, once for
    // every layer that shares layer 0's head_dim and theta (the fused
    // decode attention reads them instead of evaluating them per layer)
    void *rope_tab = nullptr;
    const char *fenv = getenv("REALM_LAYER_FUSE");
    if (seq_len == 1 && !(fenv && fenv[0] == '0') &&
        att_splits(1, position + 1, layers[0].num_heads, hd0) > 1) {
        rope_tab = base + wsize + 3 * sh;
        int ihd = (int)hd0, ipos = (int)position;
        float th = layers[0].rope_theta;
        void *args[] = {&rope_tab, &ihd, &ipos, &th};
        CHECK(launch("realm_rope_table", dim3((unsigned)((hd0 / 2 + 255) / 256)), dim3(256), 0, s,
                     args));
    } else if (seq_len > 1) {
        // a chunk of tokens: the rotations of its positions, once for every
        // layer that shares layer 0's head_dim and theta (realm_rope_qk_tab
        // reads them instead of evaluating powf and sincos per pair)
        rope_tab = base + wsize + 3 * sh;
        int ihd = (int)hd0, ipos = (int)position, iseq = (int)seq_len;
        float th = layers[0].rope_theta;
        void *args[] = {&rope_tab, &ihd, &ipos, &iseq, &th};
        CHECK(launch("realm_rope_table_seq",
                     dim3((unsigned)((seq_len * (hd0 / 2) + 255) / 256)), dim3(256), 0, s, args));
    }
    for (size_t l = 0; l < n_layers; ++l) {
        const bool same = layers[l].head_dim == hd0 && layers[l].rope_theta == layers[0].rope_theta;
        CHECK(layer_steps(&layers[l], &types[7 * l], l ? h2 : d_hidden, l ? down : nullptr,
                          seq_len, position, d_k_caches[l], d_v_caches[l], (float *)base, h_in,
                          h2, down, same ? rope_tab : nullptr, s));
    }
    return realm_hip_add_dev(h2, down, seq_len * layers[0].hidden, d_out, s);
}

REALM_API int realm_hip_forward_layer_dev(const realm_layer *L, const float *d_hidden,
                                          size_t seq_len, size_t position, float *d_k_cache,
                                          float *d_v_cache, size_t max_seq_len, float *d_out,
                                          void *stream)
{
    if (!L || !d_k_cache || !d_v_cache)
        return fail(REALM_INVALID_ARGUMENT, "forward_layer: null pointer argument");
    return realm_hip_forward_layers_dev(L, 1, d_hidden, seq_len, position, &d_k_cache,
                                        &d_v_cache, max_seq_len, d_out, stream);
}

REALM_API int realm_hip_fused_dequant_matmul_q40(const void *blocks, size_t n_blocks,
                                                 const float *input, size_t input_len,
                                                 size_t batch_size, size_t n, size_t k,
                                                 float *out)
{
    return fused_host(2, blocks, n_blocks, input, input_len, batch_size, n, k, out);
}

REALM_API int realm_hip_fused_dequant_matmul_q41(const void *blocks, size_t n_blocks,
                                                 const float *input, size_t input_len,
                                                 size_t batch_size, size_t n, size_t k,
                                                 float *out)
{
    return fused_host(3, blocks, n_blocks, input, input_len, batch_size, n, k, out);
}

REALM_API int realm_hip_fused_dequant_matmul_q50(const void *blocks, size_t n_blocks,
                                                 const float *input, size_t input_len,
                                                 size_t batch_size, size_t n, size_t k,
                                                 float *out)
{
    return fused_host(6, blocks, n_blocks, input, input_len, batch_size, n, k, out);
}

REALM_API int realm_hip_fused_dequant_matmul_q51(const void *blocks, size_t n_blocks,
                                                 const float *input, size_t input_len,
                                                 size_t batch_size, size_t n, size_t k,
                                                 float *out)
{
    return fused_host(7, blocks, n_blocks, input, input_len, batch_size, n, k, out);
}

REALM_API int realm_hip_fused_dequant_matmul_q81(const void *blocks, size_t n_blocks,
                                                 const float *input, size_t input_len,
                                                 size_t batch_size, size_t n, size_t k,
                                                 float *out)
{
    return fused_host(9, blocks, n_blocks, input, input_len, batch_size, n, k, out);
}

REALM_API int realm_hip_fused_dequant_matmul_q5k(const void *blocks, size_t n_blocks,
                                                 const float *input, size_t input_len,
                                                 size_t batch_size, size_t n, size_t k,
                                                 float *out)
{
    return fused_host(13, blocks, n_blocks, input, input_len, batch_size, n, k, out);
}

REALM_API int realm_hip_fused_dequant_matmul_q8k(const void *blocks, size_t n_blocks,
                                                 const float *input, size_t input_len,
                                                 size_t batch_size, size_t n, size_t k,
                                                 float *out)
{
    return fused_host(15, blocks, n_blocks, input, input_len, batch_size, n, k, out);
}

REALM_API int realm_hip_fused_dequant_matmul_q2k(const void *blocks, size_t n_blocks,
                                                 const float *input, size_t input_len,
                                                 size_t batch_size, size_t n, size_t k,
                                                 float *out)
{
    return fused_host(10, blocks, n_blocks, input, input_len, batch_size, n, k, out);
}

REALM_API int realm_hip_fused_dequant_matmul_q3k(const void *blocks, size_t n_blocks,
                                                 const float *input, size_t input_len,
                                                 size_t batch_size, size_t n, size_t k,
                                                 float *out)
{
    return fused_host(11, blocks, n_blocks, input, input_len, batch_size, n, k, out);
}

REALM_API int realm_hip_fused_dequant_matmul_q4k(const void *blocks, size_t n_blocks,
                                                 const float *input, size_t input_len,
                                                 size_t batch_size, size_t n, size_t k,
                                                 float *out)
{
    return fused_host(GGML_Q4_K, blocks, n_blocks, input, input_len, batch_size, n, k, out);
}

REALM_API int realm_hip_fused_dequant_matmul_q6k(const void *blocks, size_t n_blocks,
                                                 const float *input, size_t input_len,
                                                 size_t batch_size, size_t n, size_t k,
                                                 float *out)
{
    return fused_host(GGML_Q6_K, blocks, n_blocks, input, input_len, batch_size, n, k, out);
}

REALM_API int realm_hip_fused_dequant_matmul_q80(const void *blocks, size_t n_blocks,
                                                 const float *input, size_t input_len,
                                                 size_t batch_size, size_t n, size_t k,
                                                 float *out)
{
    return fused_host(GGML_Q8_0, blocks, n_blocks, input, input_len, batch_size, n, k, out);
}

REALM_API int realm_hip_fused_dequant_matmul(int ggml_type, const void *blocks, size_t n_blocks,
                                             const float *input, size_t input_len,
                                             size_t batch_size, size_t n, size_t k, float *out)
{
    return fused_host(ggml_type, blocks, n_blocks, input, input_len, batch_size, n, k, out);
}

REALM_API int32_t realm_hip_candle_matmul(uint8_t *mem, size_t mem_len, uint32_t a_ptr,
                                          uint32_t b_ptr, uint32_t result_ptr, uint32_t m,
                                          uint32_t k, uint32_t n)
{
    return candle_matmul_impl(mem, mem_len, a_ptr, b_ptr, result_ptr, m, k, n, 0);
}

REALM_API int32_t realm_hip_candle_matmul_transposed(uint8_t *mem, size_t mem_len,
                                                     uint32_t a_ptr, uint32_t b_ptr,
                                                     uint32_t result_ptr, uint32_t m,
                                                     uint32_t k, uint32_t n)
{
    return candle_matmul_impl(mem, mem_len, a_ptr, b_ptr, result_ptr, m, k, n, 1);
}

REALM_API int realm_hip_dequantize(int type, const void *data, size_t nbytes,
                                   size_t element_count, float *out)
{
    if (type != GGML_Q4_K && type != GGML_Q6_K && type != GGML_Q8_0 && !is_dq(type))
        return fail(REALM_BACKEND_UNSUPPORTED,
                    "ggml type " + std::to_string(type) + " is not supported by the HIP backend");
    size_t bb = block_bytes(type), qk = block_elems(type);
    size_t nb = nbytes / bb;
    if (type == GGML_Q4_K) {
        if (nbytes % bb)
            return fail(REALM_MODEL_PARSE_ERROR, "Q4_K data size " + std::to_string(nbytes) +
                                                     " is not a multiple of block size 144");
        if (element_count != nb * qk)
            return fail(REALM_INVALID_ARGUMENT, "Element count mismatch: expected " +
                                                    std::to_string(nb * qk) + ", got " +
                                                    std::to_string(element_count));
    } else if (nb * qk > element_count) {
        return fail(REALM_INVALID_ARGUMENT, "element_count " + std::to_string(element_count) +
                                                " is smaller than the " + std::to_string(nb) +
                                                " blocks' output");
    }
    CHECK(ensure_init());
    if (element_count > nb * qk)
        std::memset(out + nb * qk, 0, (element_count - nb * qk) * sizeof(float));
    if (nb == 0)
        return REALM_OK;
    hipStream_t s;
    CHECK(thread_stream(&s));
    void *raw, *dy;
    CHECK(ws_get(s, WS_RAW, nb * bb, &raw));
    CHECK(ws_get(s, WS_Y, nb * qk * 4, &dy));
    HIP_TRY(hipMemcpyAsync(raw, data, nb * bb, hipMemcpyHostToDevice, s));
    long long lnb = (long long)nb;
    if (is_dq(type)) {
        CHECK(dq_launch(type, raw, (float *)dy, nb, s));
    } else {
        void *args[] = {&raw, &dy, &lnb};
        size_t threads = nb * (type == GGML_Q4_K ? 128 : type == GGML_Q6_K ? 64 : 32);
        CHECK(launch(std::string("realm_dequant_") + fmt_name(type),
                     dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, args));
    }
    HIP_TRY(hipMemcpyAsync(out, dy, nb * qk * 4, hipMemcpyDeviceToHost, s));
    HIP_TRY(hipStreamSynchronize(s));
    return REALM_OK;
}

REALM_API int realm_hip_weights_register(int type, const void *blocks, size_t nbytes, size_t n,
                                         size_t k, uint64_t *handle)
{
    if (!handle)
        return fail(REALM_INVALID_ARGUMENT, "handle is null");
    if (type != GGML_Q4_K && type != GGML_Q6_K && type != GGML_Q8_0 && !is_dq(type))
        return fail(REALM_BACKEND_UNSUPPORTED,
                    "ggml type " + std::to_string(type) + " is not supported by the HIP backend");
    size_t qk = block_elems(type);
    if (k == 0 || n == 0 || k % qk)
        return fail(REALM_INVALID_ARGUMENT, "K dimension " + std::to_string(k) +
                                                " must be a positive multiple of " +
                                                std::to_string(qk));
    if (nbytes != n * (k / qk) * block_bytes(type))
        return fail(REALM_INVALID_ARGUMENT, "nbytes " + std::to_string(nbytes) +
                                                " does not match n*k/" + std::to_string(qk) +
                                                " blocks");
    if (k > (size_t)INT32_MAX || n > (size_t)INT32_MAX)
        return fail(REALM_INVALID_ARGUMENT, "dimension exceeds 2^31-1");
    CHECK(ensure_init());
    hipStream_t s;
    CHECK(thread_stream(&s));
    if (is_kq(type)) {
        // the reference's own Q2_K / Q3_K / Q5_K / Q8_K stay resident
        // dequantized (f32 [n][k], 4 bytes per weight), their products on the
        // f32 GEMM (the 32-element formats are repacked as q8m below)
        void *dev = nullptr, *raw = nullptr;
        CHECK(ws_get(s, WS_RAW, nbytes, &raw));
        HIP_TRY(hipMalloc(&dev, n * k * 4));
        int rc = hipMemcpyAsync(raw, blocks, nbytes, hipMemcpyHostToDevice, s) == hipSuccess
                     ? dq_launch(type, raw, (float *)dev, n * (k / qk), s)
                     : fail(REALM_GENERIC_FAILURE, "upload failed");
        if (rc == REALM_OK && hipStreamSynchronize(s) != hipSuccess)
            rc = fail(REALM_GENERIC_FAILURE, "dequantization failed");
        if (rc != REALM_OK) {
            (void)hipFree(dev);
            return rc;
        }
        Weight w;
        w.type = type;
        w.n = n;
        w.k = w.kx = k;
        w.bytes = n * k * 4;
        w.dev = dev;
        w.w0 = dev;
        std::lock_guard<std::mutex> lk(g_mu);
        uint64_t h = g_next_handle++;
        g_weights[h] = w;
        *handle = h;
        return REALM_OK;
    }
    size_t off[3], kx;
    size_t total = layout(type, n, k, off, &kx);
    void *dev;
    HIP_TRY(hipMalloc(&dev, total));
    Weight w;
    int rc = upload_repack(type, blocks, n, k, dev, &w, s);
    if (rc == REALM_OK && hipStreamSynchronize(s) != hipSuccess)
        rc = fail(REALM_GENERIC_FAILURE, "repack failed");
    if (rc != REALM_OK) {
        (void)hipFree(dev);
        return rc;
    }
    w.dev = dev;
    std::lock_guard<std::mutex> lk(g_mu);
    uint64_t h = g_next_handle++;
    g_weights[h] = w;
    *handle = h;
    return REALM_OK;
}

REALM_API int realm_hip_weights_release(uint64_t handle)
{
    void *dev = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        auto it = g_weights.find(handle);
        if (it == g_weights.end())
            return fail(REALM_INVALID_ARGUMENT, "unknown weight handle " + std::to_string(handle));
        dev = it->second.dev;
        g_weights.erase(it);
    }
    HIP_TRY(hipDeviceSynchronize());
    HIP_TRY(hipFree(dev));
    return REALM_OK;
}

REALM_API int realm_hip_weights_info(uint64_t handle, int *type, size_t *n, size_t *k,
                                     size_t *device_bytes)
{
    Weight w;
    CHECK(get_weight(handle, &w));
    if (type)
        *type = w.type;
    if (n)
        *n = w.n;
    if (k)
        *k = w.k;
    if (device_bytes)
        *device_bytes = w.bytes;
    return REALM_OK;
}

REALM_API int realm_hip_weights_matmul(uint64_t handle, const float *input, size_t batch,
                                       float *out)
{
    Weight w;
    CHECK(get_weight(handle, &w));
    CHECK(ensure_init());
    if (batch == 0)
        return REALM_OK;
    if (batch > (size_t)INT32_MAX)
        return fail(REALM_INVALID_ARGUMENT, "batch exceeds 2^31-1");
    hipStream_t s;
    CHECK(thread_stream(&s));
    void *dx, *dy;
    CHECK(ws_get(s, WS_X, batch * w.k * 4, &dx));
    CHECK(ws_get(s, WS_Y, batch * w.n * 4, &dy));
    HIP_TRY(hipMemcpyAsync(dx, input, batch * w.k * 4, hipMemcpyHostToDevice, s));
    CHECK(run_matmul(w, dx, false, batch, (float *)dy, s, nullptr));
    HIP_TRY(hipMemcpyAsync(out, dy, batch * w.n * 4, hipMemcpyDeviceToHost, s));
    HIP_TRY(hipStreamSynchronize(s));
    return REALM_OK;
}

REALM_API int realm_hip_weights_matmul_dev(uint64_t handle, const float *d_input, size_t batch,
                                           float *d_out, void *stream)
{
    Weight w;
    CHECK(get_weight(handle, &w));
    CHECK(ensure_init());
    if (batch > (size_t)INT32_MAX)
        return fail(REALM_INVALID_ARGUMENT, "batch exceeds 2^31-1");
    hipStream_t s;
    CHECK(pick_stream(stream, &s));
    return run_matmul(w, d_input, false, batch, d_out, s, nullptr);
}

// realm_hip_weights_matmul_dev with every scratch buffer cut from the
// device's fixed scratch array: no hipMalloc, hipFree or other allocating
// call.  The library must already be initialised on the device and the
// stream given; calls that overlap on one GPU share the array and race.
REALM_API int realm_hip_weights_matmul_noalloc_dev(uint64_t handle, const float *d_input,
                                                   size_t batch, float *d_out, void *stream)
{
    if (!stream)
        return fail(REALM_INVALID_ARGUMENT, "noalloc: needs an explicit stream");
    {
        std::lock_guard<std::mutex> lk(g_mu);
        if (!g_dev.ready || !g_dev.noalloc_scratch)
            return fail(REALM_INVALID_ARGUMENT,
                        "noalloc: call realm_hip_init first (this entry point allocates nothing)");
    }
    Weight w;
    CHECK(get_weight(handle, &w));
    if (batch > (size_t)INT32_MAX)
        return fail(REALM_INVALID_ARGUMENT, "batch exceeds 2^31-1");
    if (batch && (!d_input || !d_out))
        return fail(REALM_INVALID_ARGUMENT, "noalloc: null pointer argument");
    HIP_TRY(hipSetDevice(g_dev.id));
    FixedScratch fixed{(uint8_t *)g_dev.noalloc_scratch, REALM_NOALLOC_SCRATCH_BYTES};
    t_fixed = &fixed;
    const int rc = run_matmul(w, d_input, false, batch, d_out, (hipStream_t)stream, nullptr);
    t_fixed = nullptr;
    return rc;
}

REALM_API int realm_hip_weights_matmul_group_dev(const uint64_t *handles, size_t count,
                                                 const float *d_input, size_t batch,
                                                 float *const *d_outs, void *stream)
{
    if (!handles || !d_outs || count == 0 || count > REALM_GEMV_MAX_MATS)
        return fail(REALM_INVALID_ARGUMENT, "group needs 1..4 weight handles");
    Weight w[REALM_GEMV_MAX_MATS];
    const Weight *wp[REALM_GEMV_MAX_MATS];
    for (size_t i = 0; i < count; ++i) {
        CHECK(get_weight(handles[i], &w[i]));
        if (w[i].type != w[0].type || w[i].k != w[0].k)
            return fail(REALM_INVALID_ARGUMENT, "grouped weights must share format and K");
        wp[i] = &w[i];
    }
    CHECK(ensure_init());
    if (batch > (size_t)INT32_MAX)
        return fail(REALM_INVALID_ARGUMENT, "batch exceeds 2^31-1");
    hipStream_t s;
    CHECK(pick_stream(stream, &s));
    // dequantized f32 weights, and q8m batches past the GEMV's 4 tokens: one
    // product each (q8m groups of 1-4 tokens take the grouped GEMV below)
    if (is_kq(w[0].type) || (is_block32(w[0].type) && batch > 4)) {
        for (size_t i = 0; i < count; ++i)
            CHECK(run_matmul(w[i], d_input, false, batch, d_outs[i], s, nullptr));
        return REALM_OK;
    }
    if (batch >= 1 && batch <= 4) {
        int rc = run_gemv(wp, (int)count, d_input, (int)batch, d_outs, s);
        if (rc != REALM_BACKEND_UNSUPPORTED)
            return rc;
    }
    if (is_block32(w[0].type)) { // q8m rows too long for the GEMV: dense, one each
        for (size_t i = 0; i < count; ++i)
            CHECK(run_matmul(w[i], d_input, false, batch, d_outs[i], s, nullptr));
        return REALM_OK;
    }
    // batched: one activation prep for the whole group (the matrices share
    // format and K, so the prepared layout is the same), then one MFMA launch
    // per matrix
    if (batch == 0)
        return REALM_OK;
    // the tile and K split are chosen for the group's rows together
    Weight all = w[0];
    all.n = 0;
    for (size_t i = 0; i < count; ++i) {
        all.n += w[i].n;
        all.bytes = std::max(all.bytes, w[i].bytes); // each matrix within the tiled limit
    }
    if (all.n == 0)
        return REALM_OK;
    const GemmTile tile = gemm_tile(all, batch, false);
    XPrep p;
    CHECK(prep_x(w[0], d_input, false, batch, tile, s, &p));
    if (tile.tiled) { // one launch for the whole group
        const Weight *live[REALM_GEMV_MAX_MATS];
        float *ys[REALM_GEMV_MAX_MATS];
        int nlive = 0;
        for (size_t i = 0; i < count; ++i)
            if (w[i].n) {
                live[nlive] = &w[i];
                ys[nlive++] = d_outs[i];
            }
        return tiled_launch(live, ys, nlive, p, false, batch, tile, s);
    }
    for (size_t i = 0; i < count; ++i)
        if (w[i].n)
            CHECK(gemm_launch(w[i], p, false, batch, tile, d_outs[i], s, nullptr));
    return REALM_OK;
}

REALM_API int realm_hip_weights_matmul_bf16_dev(uint64_t handle, const uint16_t *d_input,
                                                size_t batch, float *d_out, void *stream)
{
    Weight w;
    CHECK(get_weight(handle, &w));
    CHECK(ensure_init());
    if (batch > (size_t)INT32_MAX)
        return fail(REALM_INVALID_ARGUMENT, "batch exceeds 2^31-1");
    hipStream_t s;
    CHECK(pick_stream(stream, &s));
    return run_gemm(w, d_input, true, batch, d_out, s, nullptr);
}

REALM_API int realm_hip_lora_register(int dtype, const void *lora_a, const void *lora_b,
                                      size_t rank, float alpha, size_t in_dim, size_t out_dim,
                                      uint64_t *handle)
{
    if (!handle || !lora_a || !lora_b)
        return fail(REALM_INVALID_ARGUMENT, "null pointer argument");
    if (dtype != REALM_DTYPE_F32 && dtype != REALM_DTYPE_F16)
        return fail(REALM_INVALID_ARGUMENT, "dtype must be REALM_DTYPE_F32 or REALM_DTYPE_F16");
    if (rank == 0 || rank > 256)
        return fail(REALM_INVALID_ARGUMENT, "rank must be 1..256");
    if (in_dim == 0 || out_dim == 0 || in_dim > (size_t)INT32_MAX || out_dim > (size_t)INT32_MAX)
        return fail(REALM_INVALID_ARGUMENT, "bad adapter dimensions");
    CHECK(ensure_init());
    size_t es = dtype == REALM_DTYPE_F16 ? 2 : 4;
    size_t abytes = rank * in_dim * es, bbytes = out_dim * rank * es;
    Adapter ad;
    ad.dtype = dtype;
    ad.rank = rank;
    ad.alpha = alpha;
    ad.in = in_dim;
    ad.out = out_dim;
    HIP_TRY(hipMalloc(&ad.a, abytes));
    if (hipMalloc(&ad.b, bbytes) != hipSuccess) {
        (void)hipFree(ad.a);
        return fail(REALM_OUT_OF_MEMORY, "hipMalloc of LoRA B failed");
    }
    if (hipMemcpy(ad.a, lora_a, abytes, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(ad.b, lora_b, bbytes, hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipFree(ad.a);
        (void)hipFree(ad.b);
        return fail(REALM_GENERIC_FAILURE, "upload of LoRA factors failed");
    }
    std::lock_guard<std::mutex> lk(g_mu);
    uint64_t h = g_next_handle++;
    g_adapters[h] = ad;
    *handle = h;
    return REALM_OK;
}

REALM_API int realm_hip_lora_release(uint64_t handle)
{
    Adapter ad;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        auto it = g_adapters.find(handle);
        if (it == g_adapters.end())
            return fail(REALM_INVALID_ARGUMENT, "unknown adapter handle " + std::to_string(handle));
        if (it->second.uses > 0)
            return fail(REALM_INVALID_ARGUMENT, "adapter is still part of an adapter set");
        ad = it->second;
        g_adapters.erase(it);
    }
    HIP_TRY(hipDeviceSynchronize());
    HIP_TRY(hipFree(ad.a));
    HIP_TRY(hipFree(ad.b));
    return REALM_OK;
}

REALM_API int realm_hip_lora_set_create(const uint64_t *lora_handles, size_t count,
                                        uint64_t *set_handle)
{
    if (!set_handle || (!lora_handles && count))
        return fail(REALM_INVALID_ARGUMENT, "null pointer argument");
    if (count == 0 || count > 65535)
        return fail(REALM_INVALID_ARGUMENT, "adapter set needs 1..65535 adapters");
    CHECK(ensure_init());
    std::vector<LoraEntry> table(count);
    AdapterSet set;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        for (size_t i = 0; i < count; ++i) {
            auto it = g_adapters.find(lora_handles[i]);
            if (it == g_adapters.end())
                return fail(REALM_INVALID_ARGUMENT,
                            "unknown adapter handle " + std::to_string(lora_handles[i]));
            const Adapter &ad = it->second;
            if (i == 0) {
                set.in = ad.in;
                set.out = ad.out;
            } else if (ad.in != set.in || ad.out != set.out) {
                return fail(REALM_INVALID_ARGUMENT, "adapters of a set must share in/out dims");
            }
            table[i].a = ad.a;
            table[i].b = ad.b;
            table[i].rank = (int32_t)ad.rank;
            table[i].dtype = ad.dtype;
            table[i].scale = ad.alpha / (float)ad.rank; // lora.rs:49-52
            table[i].pad = 0;
            set.rmax = std::max(set.rmax, (int)ad.rank);
        }
        for (size_t i = 0; i < count; ++i)
            g_adapters[lora_handles[i]].uses++;
    }
    set.count = count;
    set.members.assign(lora_handles, lora_handles + count);
    // the 16-row chunks of every adapter's A, for the fused shrink
    std::vector<LoraChunk> chunks;
    for (size_t i = 0; i < count; ++i)
        for (int rc = 0; rc * 16 < table[i].rank; ++rc) {
            LoraChunk c;
            std::memset(&c, 0, sizeof c);
            c.e = table[i];
            c.a = (int32_t)i;
            c.rc = rc;
            chunks.push_back(c);
        }
    set.nchunks = chunks.size();
    const size_t tbytes = align256(count * sizeof(LoraEntry));
    int rc = REALM_OK;
    if (hipMalloc(&set.table, tbytes + chunks.size() * sizeof(LoraChunk)) != hipSuccess) {
        set.table = nullptr;
        rc = fail(REALM_OUT_OF_MEMORY, "hipMalloc of adapter table failed");
    } else {
        set.chunks = (uint8_t *)set.table + tbytes;
        if (hipMemcpy(set.table, table.data(), count * sizeof(LoraEntry),
                      hipMemcpyHostToDevice) != hipSuccess ||
            hipMemcpy(set.chunks, chunks.data(), chunks.size() * sizeof(LoraChunk),
                      hipMemcpyHostToDevice) != hipSuccess)
            rc = fail(REALM_GENERIC_FAILURE, "upload of adapter table failed");
    }
    std::lock_guard<std::mutex> lk(g_mu);
    if (rc != REALM_OK) {
        if (set.table)
            (void)hipFree(set.table);
        for (size_t i = 0; i < count; ++i)
            g_adapters[lora_handles[i]].uses--;
        return rc;
    }
    uint64_t h = g_next_handle++;
    g_sets[h] = set;
    *set_handle = h;
    return REALM_OK;
}

REALM_API int realm_hip_lora_set_release(uint64_t set_handle)
{
    void *table;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        auto it = g_sets.find(set_handle);
        if (it == g_sets.end())
            return fail(REALM_INVALID_ARGUMENT, "unknown adapter set " + std::to_string(set_handle));
        for (uint64_t m : it->second.members) {
            auto a = g_adapters.find(m);
            if (a != g_adapters.end())
                a->second.uses--;
        }
        table = it->second.table;
        g_sets.erase(it);
    }
    HIP_TRY(hipDeviceSynchronize());
    HIP_TRY(hipFree(table));
    return REALM_OK;
}

namespace {
int lora_lookup(uint64_t wh, uint64_t sh, size_t batch, Weight *w, AdapterSet *set)
{
    CHECK(get_weight(wh, w));
    if (is_dq(w->type))
        return fail(REALM_BACKEND_UNSUPPORTED, "multi-LoRA takes Q4_K, Q6_K or Q8_0 base weights");
    {
        std::lock_guard<std::mutex> lk(g_mu);
        auto it = g_sets.find(sh);
        if (it == g_sets.end())
            return fail(REALM_INVALID_ARGUMENT, "unknown adapter set " + std::to_string(sh));
        *set = it->second;
    }
    if (set->in != w->k || set->out != w->n)
        return fail(REALM_INVALID_ARGUMENT, "adapter set dims do not match the weight");
    if (batch > 1024)
        return fail(REALM_INVALID_ARGUMENT, "multi-LoRA batch is limited to 1024 tokens");
    return REALM_OK;
}
} // namespace

REALM_API int realm_hip_multi_lora_matmul_dev(uint64_t weight_handle, uint64_t set_handle,
                                              const float *d_input, size_t batch,
                                              const int32_t *d_adapter_ids, float *d_out,
                                              void *stream)
{
    Weight w;
    AdapterSet set;
    CHECK(lora_lookup(weight_handle, set_handle, batch, &w, &set));
    CHECK(ensure_init());
    hipStream_t s;
    CHECK(pick_stream(stream, &s));
    LoraCall lc{&set, d_adapter_ids};
    return run_gemm(w, d_input, false, batch, d_out, s, &lc);
}

REALM_API int realm_hip_multi_lora_matmul_group_dev(const uint64_t *weight_handles,
                                                    const uint64_t *set_handles, size_t count,
                                                    const float *d_input, size_t batch,
                                                    const int32_t *d_adapter_ids,
                                                    float *const *d_outs, void *stream)
{
    if (!weight_handles || !set_handles || !d_outs || count == 0 ||
        count > REALM_GEMM_MAX_SEGS)
        return fail(REALM_INVALID_ARGUMENT, "group needs 1..4 weight and adapter-set handles");
    Weight w[REALM_GEMM_MAX_SEGS];
    AdapterSet set[REALM_GEMM_MAX_SEGS];
    for (size_t i = 0; i < count; ++i) {
        CHECK(lora_lookup(weight_handles[i], set_handles[i], batch, &w[i], &set[i]));
        if (w[i].type != w[0].type || w[i].k != w[0].k)
            return fail(REALM_INVALID_ARGUMENT, "grouped weights must share format and K");
    }
    CHECK(ensure_init());
    hipStream_t s;
    CHECK(pick_stream(stream, &s));
    if (batch == 0)
        return REALM_OK;
    Weight all = w[0];
    all.n = 0;
    for (size_t i = 0; i < count; ++i) {
        all.n += w[i].n;
        all.bytes = std::max(all.bytes, w[i].bytes);
    }
    const GemmTile tile = gemm_tile(all, batch, false);
    LoraCall lc[REALM_GEMM_MAX_SEGS];
    for (size_t i = 0; i < count; ++i)
        lc[i] = LoraCall{&set[i], d_adapter_ids};
    if (lora_fused_ok(tile, batch, false, w[0], d_input, lc, (int)count)) {
        const Weight *wp[REALM_GEMM_MAX_SEGS];
        for (size_t i = 0; i < count; ++i)
            wp[i] = &w[i];
        return lora_fused_run(wp, lc, (int)count, d_input, batch, tile, d_outs, s);
    }
    XPrep p;
    CHECK(prep_x(w[0], d_input, false, batch, tile, s, &p));
    if (!tile.tiled) { // per matrix: shrink, base product, expand
        for (size_t i = 0; i < count; ++i)
            CHECK(gemm_launch(w[i], p, false, batch, tile, d_outs[i], s, &lc[i]));
        return REALM_OK;
    }
    // one shrink launch for every projection (each into its own slice of
    // the u workspace), one launch of the base products, one expand launch
    size_t uoff[REALM_GEMM_MAX_SEGS], ubytes = 0;
    for (size_t i = 0; i < count; ++i) {
        uoff[i] = ubytes;
        ubytes += align256(lora_u(w[i], set[i], p).bytes());
    }
    void *u = nullptr;
    CHECK(ws_get(s, WS_U, ubytes, &u));
    void *us[REALM_GEMM_MAX_SEGS];
    const Weight *wp[REALM_GEMM_MAX_SEGS];
    for (size_t i = 0; i < count; ++i) {
        us[i] = (uint8_t *)u + uoff[i];
        wp[i] = &w[i];
    }
    CHECK(lora_shrink_launch(wp, lc, (int)count, p, false, batch, tile, us, s));
    CHECK(tiled_launch(wp, d_outs, (int)count, p, false, batch, tile, s));
    CHECK(lora_expand_launch(wp, lc, (int)count, p, batch, us, d_outs, s));
    return REALM_OK;
}

REALM_API int realm_hip_multi_lora_matmul(uint64_t weight_handle, uint64_t set_handle,
                                          const float *input, size_t batch,
                                          const int32_t *adapter_ids, float *out)
{
    Weight w;
    AdapterSet set;
    CHECK(lora_lookup(weight_handle, set_handle, batch, &w, &set));
    CHECK(ensure_init());
    if (batch == 0)
        return REALM_OK;
    hipStream_t s;
    CHECK(thread_stream(&s));
    void *dx, *dy, *di;
    CHECK(ws_get(s, WS_X, batch * w.k * 4, &dx));
    CHECK(ws_get(s, WS_Y, batch * w.n * 4, &dy));
    CHECK(ws_get(s, WS_IDS, batch * 4, &di));
    HIP_TRY(hipMemcpyAsync(dx, input, batch * w.k * 4, hipMemcpyHostToDevice, s));
    HIP_TRY(hipMemcpyAsync(di, adapter_ids, batch * 4, hipMemcpyHostToDevice, s));
    LoraCall lc{&set, (const int32_t *)di};
    CHECK(run_gemm(w, dx, false, batch, (float *)dy, s, &lc));
    HIP_TRY(hipMemcpyAsync(out, dy, batch * w.n * 4, hipMemcpyDeviceToHost, s));
    HIP_TRY(hipStreamSynchronize(s));
    return REALM_OK;
}

// ------------------------------------------------------------ HIP graphs

namespace {
// A live graph and the stream it was captured on (whose workspace buffers
// it may use: see ws_get).
struct GraphRec {
    hipGraphExec_t exec;
    hipStream_t stream;
};
std::unordered_map<uint64_t, GraphRec> g_graphs;

// One graph of stream s fewer (a release, or a capture that failed): when
// none is left, the buffers retired meanwhile are freed.
int graph_unpin(hipStream_t s)
{
    std::vector<void *> drop;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        Workspace *w = ws_of_locked(s);
        if (w->graphs > 0 && --w->graphs == 0)
            drop.swap(w->retired);
    }
    if (!drop.empty())
        HIP_TRY(hipDeviceSynchronize());
    for (void *p : drop)
        HIP_TRY(hipFree(p));
    return REALM_OK;
}
} // namespace

REALM_API int realm_hip_graph_begin(void *stream)
{
    if (!stream)
        return fail(REALM_INVALID_ARGUMENT, "graph capture needs an explicit stream");
    CHECK(ensure_init());
    HIP_TRY(hipStreamBeginCapture((hipStream_t)stream, hipStreamCaptureModeThreadLocal));
    std::lock_guard<std::mutex> lk(g_mu);
    ws_of_locked((hipStream_t)stream)->graphs++;
    return REALM_OK;
}

REALM_API int realm_hip_graph_end(void *stream, uint64_t *graph_handle)
{
    if (!stream || !graph_handle)
        return fail(REALM_INVALID_ARGUMENT, "null argument");
    const hipStream_t s = (hipStream_t)stream;
    hipGraph_t graph;
    hipError_t e = hipStreamEndCapture(s, &graph);
    if (e != hipSuccess) {
        (void)graph_unpin(s);
        return fail(hip_code(e), std::string("hipStreamEndCapture: ") + hipGetErrorString(e));
    }
    hipGraphExec_t exec;
    e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (e != hipSuccess) {
        (void)graph_unpin(s);
        return fail(hip_code(e), std::string("hipGraphInstantiate: ") + hipGetErrorString(e));
    }
    std::lock_guard<std::mutex> lk(g_mu);
    uint64_t h = g_next_handle++;
    g_graphs[h] = GraphRec{exec, s};
    *graph_handle = h;
    return REALM_OK;
}

REALM_API int realm_hip_graph_launch(uint64_t graph_handle, void *stream)
{
    hipGraphExec_t exec;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        auto it = g_graphs.find(graph_handle);
        if (it == g_graphs.end())
            return fail(REALM_INVALID_ARGUMENT, "unknown graph " + std::to_string(graph_handle));
        exec = it->second.exec;
    }
    hipStream_t s;
    CHECK(pick_stream(stream, &s));
    HIP_TRY(hipGraphLaunch(exec, s));
    return REALM_OK;
}

REALM_API int realm_hip_graph_release(uint64_t graph_handle)
{
    GraphRec rec;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        auto it = g_graphs.find(graph_handle);
        if (it == g_graphs.end())
            return fail(REALM_INVALID_ARGUMENT, "unknown graph " + std::to_string(graph_handle));
        rec = it->second;
        g_graphs.erase(it);
    }
    HIP_TRY(hipDeviceSynchronize());
    HIP_TRY(hipGraphExecDestroy(rec.exec));
    return graph_unpin(rec.stream);
}

REALM_API int realm_hip_workspace_info(void *stream, size_t *bytes, size_t *retired,
                                       int *graphs)
{
    CHECK(ensure_init());
    hipStream_t s;
    CHECK(pick_stream(stream, &s));
    std::lock_guard<std::mutex> lk(g_mu);
    const Workspace *w = ws_of_locked(s);
    size_t total = 0;
    for (int i = 0; i < WS_N; ++i)
        total += w->cap[i];
    if (bytes)
        *bytes = total;
    if (retired)
        *retired = w->retired.size();
    if (graphs)
        *graphs = w->graphs;
    return REALM_OK;
}

// ------------------------------------------------------------- checksum

REALM_API int realm_hip_checksum_dev(const void *d_buf, size_t nbytes, uint32_t *d_partials,
                                     size_t n_partials, void *stream)
{
    if (n_partials == 0 || n_partials > 4096 || !d_partials || (nbytes && !d_buf))
        return fail(REALM_INVALID_ARGUMENT, "checksum: 1..4096 partials and non-null pointers");
    if (nbytes > ((size_t)1 << 62))
        return fail(REALM_INVALID_ARGUMENT, "checksum: buffer too large");
    CHECK(ensure_init());
    hipStream_t s;
    CHECK(pick_stream(stream, &s));
    long long n = (long long)nbytes;
    void *args[] = {(void *)&d_buf, &n, &d_partials};
    return launch("realm_checksum", dim3((unsigned)n_partials), dim3(1024), 0, s, args);
}

REALM_API int realm_hip_checksum(const void *d_buf, size_t nbytes, uint32_t *checksum)
{
    if (!checksum)
        return fail(REALM_INVALID_ARGUMENT, "checksum: null output");
    CHECK(ensure_init());
    hipStream_t s;
    CHECK(thread_stream(&s));
    const size_t np = (size_t)g_dev.cu_count;
    void *part;
    CHECK(ws_get(s, WS_IDS, np * 4, &part));
    CHECK(realm_hip_checksum_dev(d_buf, nbytes, (uint32_t *)part, np, s));
    std::vector<uint32_t> h(np);
    HIP_TRY(hipMemcpyAsync(h.data(), part, np * 4, hipMemcpyDeviceToHost, s));
    HIP_TRY(hipStreamSynchronize(s));
    uint32_t r = 0;
    for (uint32_t v : h)
        r ^= v;
    *checksum = r;
    return REALM_OK;
}

// ------------------------------------------------------------- plumbing

REALM_API int realm_hip_malloc(void **d_ptr, size_t nbytes)
{
    CHECK(ensure_init());
    HIP_TRY(hipMalloc(d_ptr, std::max<size_t>(nbytes, 1)));
    return REALM_OK;
}

REALM_API int realm_hip_free(void *d_ptr)
{
    CHECK(ensure_init());
    HIP_TRY(hipFree(d_ptr));
    return REALM_OK;
}

REALM_API int realm_hip_memcpy_htod(void *d_dst, const void *h_src, size_t nbytes)
{
    CHECK(ensure_init());
    HIP_TRY(hipMemcpy(d_dst, h_src, nbytes, hipMemcpyHostToDevice));
    return REALM_OK;
}

REALM_API int realm_hip_memcpy_dtoh(void *h_dst, const void *d_src, size_t nbytes)
{
    CHECK(ensure_init());
    HIP_TRY(hipMemcpy(h_dst, d_src, nbytes, hipMemcpyDeviceToHost));
    return REALM_OK;
}

REALM_API int realm_hip_memcpy_dtod(void *d_dst, const void *d_src, size_t nbytes)
{
    CHECK(ensure_init());
    HIP_TRY(hipMemcpy(d_dst, d_src, nbytes, hipMemcpyDeviceToDevice));
    return REALM_OK;
}

REALM_API int realm_hip_stream(void **stream)
{
    CHECK(ensure_init());
    hipStream_t s;
    CHECK(thread_stream(&s));
    *stream = s;
    return REALM_OK;
}

REALM_API int realm_hip_stream_synchronize(void *stream)
{
    CHECK(ensure_init());
    hipStream_t s;
    CHECK(pick_stream(stream, &s));
    HIP_TRY(hipStreamSynchronize(s));
    return REALM_OK;
}

REALM_API int realm_hip_device_synchronize(void)
{
    CHECK(ensure_init());
    HIP_TRY(hipDeviceSynchronize());
    return REALM_OK;
}

REALM_API int realm_hip_event_create(void **event)
{
    CHECK(ensure_init());
    hipEvent_t e;
    HIP_TRY(hipEventCreate(&e));
    *event = e;
    return REALM_OK;
}

REALM_API int realm_hip_event_destroy(void *event)
{
    HIP_TRY(hipEventDestroy((hipEvent_t)event));
    return REALM_OK;
}

REALM_API int realm_hip_event_record(void *event, void *stream)
{
    hipStream_t s;
    CHECK(pick_stream(stream, &s));
    HIP_TRY(hipEventRecord((hipEvent_t)event, s));
    return REALM_OK;
}

REALM_API int realm_hip_event_elapsed_ms(void *start, void *stop, float *ms)
{
    HIP_TRY(hipEventSynchronize((hipEvent_t)stop));
    HIP_TRY(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop));
    return REALM_OK;
}

int realm_set_error(int code, const std::string &msg) { return fail(code, msg); }

int realm_device_free_bytes(size_t *bytes)
{
    CHECK(ensure_init());
    size_t total = 0;
    HIP_TRY(hipMemGetInfo(bytes, &total));
    return REALM_OK;
}
