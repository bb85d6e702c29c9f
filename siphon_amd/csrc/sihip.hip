// libsiphon_hip.so: C-ABI implementation (declarations in include/sihip.h).
//
// Owns device copies of the weights in the planar layout of formats.h and
// launches the gfx950 kernels of matvec.h. Every entry point validates its
// arguments on the host before any launch, so a kernel never sees a shape
// its grid and LDS sizing do not cover.
#include <hip/hip_runtime.h>

#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <cmath>
#include <mutex>
#include <utility>
#include <vector>

#include "../../include/sihip.h"
#include "attn.h"
#include "formats.h"
#include "gemm.h"
#include "f32w.h"
#include "gemm2.h"
#include "gemm2s.h"
#include "gemmks.h"
#include "gemmkf.h"
#include "gemm6.h"
#include "gemmh.h"
#include "gemmq.h"
#include "matvec.h"
#include "quant.h"

using namespace sihip;

// Tuning knobs, read once from the environment at sihip_init (variable
// SIHIP_<NAME>) and changed afterwards only through sihip_set_option; a
// negative value means "the built-in rule".
struct Options {
    int64_t wg_per_cu = -1;    // matvec workgroups per CU when rows exceed waves (rule: 2)
    int64_t wave_target = -1;  // row tiles a matvec layout aims for (rule: 800)
    int64_t split_elems = -1;  // column-slice length in elements, 0: none (rule: kSliceElems)
    int64_t tile_cols = -1;    // matvec tile width at upload (rule: choose_G)
    int64_t gemm_min_m = -1;   // smallest M on the matrix cores (rule: 5)
    int64_t gemm_mt = -1;      // GEMM m-tile rows / 32 (rule: by M)
    int64_t gemm_sbk = -1;     // GEMM K-slice length in super-blocks, 0: none (rule: by tiles)
    int64_t gemm2_min_m = -1;  // smallest M on the 16x16 Q4_K GEMM (rule: kGemm2MinM)
    int64_t gemm2_waves = -1;  // waves per SIMD of the 16x16 GEMMs, 1 or 2 (rule: 2)
    int64_t gemm6_min_m = -1;  // smallest M on the Q6_K GEMM (rule: kGemm6MinM)
    int64_t gemmh_min_m = -1;  // smallest M on the F16 GEMM (rule: kGemmhMinM)
    int64_t gemmq_min_m = -1;  // smallest M on the Q4_0/Q5_0/Q8_0 GEMM (rule: kGemmqMinM)
    int64_t gemmq_xmode = -1;  // Q8_0-pair GEMM record mode 0 or 1 (gemmq_kernel XM; rule: 1 where it fits)
    int64_t gemmq_fuse = -1;   // Q8_0-pair GEMM quantizing X itself (XM 2) at 16-row m blocks, 0: off (rule: on)
    int64_t gemmh_fuse = -1;   // F16 GEMM converting X itself (XF) at 16-row m blocks, 0: off (rule: on)
    int64_t attn_fuse = -1;    // decode attention in two launches up to 1024 positions (softmax in the value launch), 0: three
    int64_t gemm2s_max_m = -1; // largest M on the small-M Q4_K GEMM, 0: none (rule: 16)
    int64_t gemmks_max_m = -1; // largest M on the small-M K-quant GEMM, 0: none (rule: 16)
    int64_t gemmks_q4k = -1;   // Q4_K small M on gemmks.h (1) or gemm2s.h (0) (rule: 0)
    int64_t gemms_waves = -1;  // waves per workgroup of the small-M GEMMs, 4 or 8 (rule: by rows)
    int64_t gemmkf_max_m = -1; // largest M on the fused small-M K-quant launch, 0: none (rule: 8)
    int64_t gemmkf_sbk = -1;   // its K-slice length in super-blocks, 0: fewest slices (rule: by tiles)
    int64_t gemm_group = -1;   // Q4_K matrices over one X in one 16x16 GEMM launch, 0: off (rule: on)
    int64_t q80_scalar = -1;   // Q8_0 activations by the scalar quantizer (reference
                               // kernels.c:542-558, its SI_SCALAR mode), 1: on (rule: off)
};

struct OptionName {
    const char *name;
    int64_t Options::*field;
};

static const OptionName kOptionNames[] = {
    {"WG_PER_CU", &Options::wg_per_cu},   {"WAVE_TARGET", &Options::wave_target},
    {"SPLIT_ELEMS", &Options::split_elems}, {"TILE_COLS", &Options::tile_cols},
    {"GEMM_MIN_M", &Options::gemm_min_m}, {"GEMM_MT", &Options::gemm_mt},
    {"GEMM_SBK", &Options::gemm_sbk},     {"GEMM2_MIN_M", &Options::gemm2_min_m},
    {"GEMM2_WAVES", &Options::gemm2_waves}, {"GEMM6_MIN_M", &Options::gemm6_min_m},
    {"GEMMH_MIN_M", &Options::gemmh_min_m}, {"GEMMQ_MIN_M", &Options::gemmq_min_m},
    {"GEMMQ_XMODE", &Options::gemmq_xmode}, {"Q80_SCALAR", &Options::q80_scalar},
    {"GEMMQ_FUSE", &Options::gemmq_fuse}, {"GEMMH_FUSE", &Options::gemmh_fuse},
    {"ATTN_FUSE", &Options::attn_fuse},
    {"GEMM2S_MAX_M", &Options::gemm2s_max_m}, {"GEMMKS_MAX_M", &Options::gemmks_max_m},
    {"GEMMKS_Q4K", &Options::gemmks_q4k},
    {"GEMMS_WAVES", &Options::gemms_waves},
    {"GEMMKF_MAX_M", &Options::gemmkf_max_m}, {"GEMMKF_SBK", &Options::gemmkf_sbk},
    {"GEMM_GROUP", &Options::gemm_group},
};

// Order of launches that share mutable device state across streams: a
// context's GEMM and attention workspaces, a column-sliced weight's partial
// sums and arrival counters. While all of them come on one stream nothing
// is added. The first launch on a second stream waits for the device to
// drain (hipDeviceSynchronize; no stream handle of an earlier call is
// touched, since the caller may have destroyed it); from then on the state
// carries an event recorded after each of its launches, and a launch on
// another stream than the last one waits for that event. Launches made
// during a graph capture are neither recorded nor made to wait: a captured
// sequence is ordered by its graph, and its replays must not overlap eager
// use of the same state on another stream.
struct StreamOrder {
    hipStream_t last = nullptr;
    bool used = false;
    bool multi = false;
    hipEvent_t ev = nullptr;
};

struct sihip_ctx {
    int device;
    int n_cu;
    size_t lds_limit;
    hipStream_t stream;  // for host-pointer entry points
    char err[512];
    Options opt;
    void *d_in = nullptr;
    size_t d_in_cap = 0;
    void *d_out = nullptr;
    size_t d_out_cap = 0;
    void *d_aux = nullptr;
    size_t d_aux_cap = 0;
    void *d_ws = nullptr;  // prefill GEMM: quantized activation planes
    size_t d_ws_cap = 0;
    void *d_gpart = nullptr;  // prefill GEMM K slices: partial sums
    size_t d_gpart_cap = 0;
    uint32_t *d_gcnt = nullptr;  // prefill GEMM K slices: arrival counters (zero between calls)
    void *d_attn = nullptr;  // decode attention: scores and f16 probabilities
    size_t d_attn_cap = 0;
    // workspaces replaced by larger ones: a graph captured earlier may still
    // hold their addresses, so they stay allocated until sihip_shutdown
    std::vector<void *> retired;
    // this device's copy of the static scratch of sihip_gemm_dev_noalloc
    uint8_t *scratch = nullptr;
    StreamOrder order;  // of the launches using the workspaces above
};

// Arrival counters of K-sliced GEMM tiles, allocated (and zeroed) at
// sihip_init; launches with more tiles than this are not sliced.
constexpr int64_t kGemmCounters = 65536;

struct sihip_weight {
    Layout L;
    uint8_t *dev;
    uint8_t *gemm = nullptr;  // GEMM-ordered copy, built on the first prefill call
    int64_t gemm_bytes = 0;
    // Q4_K and Q6_K: the copy of the 16x16 matrix-core GEMM of the type
    // (gemm2.h, gemm6.h); Q4_K: its exponent E (the min operand holds
    // -dmin * mn * 2^E)
    uint8_t *gemm2 = nullptr;
    int64_t gemm2_bytes = 0;
    // K-quants: the near-GGUF-size copy of the small-M GEMM (gemmks.h),
    // built on the first call with 3 <= M <= 16 or by
    // sihip_weight_prepare_gemm
    uint8_t *gsmall = nullptr;
    int64_t gsmall_bytes = 0;
    int gexp = 0;
    // column slices of the matvec (split == 1: whole rows per workgroup);
    // part and cnt live in the same allocation as the planes
    uint32_t split = 1, spr = 0;
    float *part = nullptr;
    uint32_t *cnt = nullptr;
    int64_t split_bytes = 0;
    mutable StreamOrder order;  // of the launches using part and cnt (split > 1)
};

static char g_init_err[512];

static int set_err(sihip_ctx *ctx, int code, const char *fmt, ...) {
    char *dst = ctx ? ctx->err : g_init_err;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(dst, 512, fmt, ap);
    va_end(ap);
    return code;
}

#define HIP_OK(ctx, call)                                                              \
    do {                                                                               \
        hipError_t e_ = (call);                                                        \
        if (e_ != hipSuccess)                                                          \
            return set_err((ctx), SIHIP_EDEVICE, "%s: %s", #call, hipGetErrorString(e_)); \
    } while (0)

// True if work on st is being captured into a graph (allocations and
// synchronous calls are not allowed then).
static bool capturing(hipStream_t st) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess) return false;
    return cs != hipStreamCaptureStatusNone;
}

// Before a launch on stream st that uses the state ordered by o.
static int order_before(sihip_ctx *ctx, StreamOrder &o, hipStream_t st) {
    if (!o.used || o.last == st || capturing(st)) return SIHIP_OK;
    if (!o.multi) {
        HIP_OK(ctx, hipDeviceSynchronize());
        HIP_OK(ctx, hipEventCreateWithFlags(&o.ev, hipEventDisableTiming));
        o.multi = true;
        return SIHIP_OK;
    }
    HIP_OK(ctx, hipStreamWaitEvent(st, o.ev, 0));
    return SIHIP_OK;
}

// After that launch was enqueued.
static int order_after(sihip_ctx *ctx, StreamOrder &o, hipStream_t st) {
    if (capturing(st)) return SIHIP_OK;
    o.used = true;
    o.last = st;
    if (o.multi) HIP_OK(ctx, hipEventRecord(o.ev, st));
    return SIHIP_OK;
}

static void order_free(StreamOrder &o) {
    if (o.ev) (void)hipEventDestroy(o.ev);
    o = StreamOrder();
}

// A context workspace of at least `bytes`. Growing it allocates a new
// buffer and retires the old one (kept until sihip_shutdown, since a graph
// captured before may reference it); under graph capture growing is an
// error, as allocation is not allowed there.
static int ensure(sihip_ctx *ctx, void **buf, size_t *cap, size_t bytes, hipStream_t st = nullptr) {
    if (*cap >= bytes) return SIHIP_OK;
    if (st && capturing(st))
        return set_err(ctx, SIHIP_EINVAL,
                       "workspace of %zu bytes needed during graph capture (it holds %zu): run "
                       "the call once outside capture first, or use sihip_gemm_dev_noalloc",
                       bytes, *cap);
    void *nb = nullptr;
    if (hipMalloc(&nb, bytes) != hipSuccess)
        return set_err(ctx, SIHIP_ENOMEM, "device allocation of %zu bytes failed", bytes);
    if (*buf) ctx->retired.push_back(*buf);
    *buf = nb;
    *cap = bytes;
    return SIHIP_OK;
}

// ---- the scratch of sihip_gemm_dev_noalloc ------------------------------------
//
// Device memory of fixed size that the allocation-free GEMM entry point
// uses in place of the context's workspaces: the quantized activation
// planes and K-slice partial sums from offset 0, and kGemmCounters arrival
// counters in the last kNoAllocCntBytes (zero at module load; each sliced
// launch leaves them zero again). Each device holds its own copy for the
// life of the process. In host code `scratch` only names the symbol: its
// device address comes from hipGetSymbolAddress at sihip_init (ctx->scratch).
constexpr size_t kNoAllocCntBytes = (size_t)kGemmCounters * 4;
constexpr size_t kNoAllocBytes = ((size_t)16 << 20) + kNoAllocCntBytes;  // 16 MiB + counters
static __device__ __align__(256) uint8_t scratch[kNoAllocBytes];
// devices whose scratch counters sihip_init clears (one flag each)
constexpr int kMaxDevices = 64;

extern "C" int sihip_abi_version(void) { return SIHIP_ABI_VERSION; }

static void read_env_options(Options &o) {
    char name[64];
    for (const OptionName &n : kOptionNames) {
        snprintf(name, sizeof name, "SIHIP_%s", n.name);
        if (const char *e = getenv(name)) o.*(n.field) = atoll(e);
    }
}

extern "C" int sihip_init(int device, sihip_ctx **out) {
    if (!out) return set_err(nullptr, SIHIP_EINVAL, "sihip_init: out is NULL");
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0)
        return set_err(nullptr, SIHIP_EDEVICE, "sihip_init: no HIP device");
    if (device < 0 || device >= n)
        return set_err(nullptr, SIHIP_EINVAL, "sihip_init: device %d of %d", device, n);
    if (hipSetDevice(device) != hipSuccess)
        return set_err(nullptr, SIHIP_EDEVICE, "sihip_init: hipSetDevice(%d) failed", device);
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess)
        return set_err(nullptr, SIHIP_EDEVICE, "sihip_init: hipGetDeviceProperties failed");
    void *sp = nullptr;
    const hipError_t se = hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch));
    if (se != hipSuccess || !sp)
        return set_err(nullptr, SIHIP_EDEVICE, "sihip_init: scratch symbol address: %s",
                       hipGetErrorString(se));
    void *cnt = nullptr;
    if (hipMalloc(&cnt, kGemmCounters * 4) != hipSuccess)
        return set_err(nullptr, SIHIP_ENOMEM, "sihip_init: GEMM slice counters");
    if (hipMemset(cnt, 0, kGemmCounters * 4) != hipSuccess) {
        (void)hipFree(cnt);
        return set_err(nullptr, SIHIP_EDEVICE, "sihip_init: GEMM slice counters: memset failed");
    }
    // The scratch counters start at zero (each sliced launch leaves them
    // so). The scratch is one per device and shared by every context, so
    // they are cleared once per device and process, by its first context:
    // clearing them again when a later context is created could reset them
    // under a sliced launch of another context still running on another
    // stream.
    {
        static std::mutex mu;
        static bool cleared[kMaxDevices];
        std::lock_guard<std::mutex> lock(mu);
        if (device >= kMaxDevices) {
            (void)hipFree(cnt);
            return set_err(nullptr, SIHIP_EINVAL, "sihip_init: device %d past %d", device,
                           kMaxDevices);
        }
        if (!cleared[device]) {
            if (hipMemset((uint8_t *)sp + (kNoAllocBytes - kNoAllocCntBytes), 0, kNoAllocCntBytes) !=
                    hipSuccess ||
                hipDeviceSynchronize() != hipSuccess) {
                (void)hipFree(cnt);
                return set_err(nullptr, SIHIP_EDEVICE, "sihip_init: scratch counters: memset failed");
            }
            cleared[device] = true;
        }
    }
    sihip_ctx *c = new sihip_ctx();
    c->device = device;
    c->n_cu = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
    c->lds_limit = prop.sharedMemPerBlock;
    c->err[0] = 0;
    c->d_gcnt = (uint32_t *)cnt;
    c->scratch = (uint8_t *)sp;
    read_env_options(c->opt);
    if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
        (void)hipFree(cnt);
        delete c;
        return set_err(nullptr, SIHIP_EDEVICE, "sihip_init: stream creation failed");
    }
    *out = c;
    return SIHIP_OK;
}

extern "C" void sihip_shutdown(sihip_ctx *ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    (void)hipDeviceSynchronize();
    for (void *p : {ctx->d_in, ctx->d_out, ctx->d_aux, ctx->d_ws, ctx->d_gpart,
                    (void *)ctx->d_gcnt, ctx->d_attn})
        if (p) (void)hipFree(p);
    for (void *p : ctx->retired) (void)hipFree(p);
    order_free(ctx->order);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
}

extern "C" int sihip_set_option(sihip_ctx *ctx, const char *name, int64_t value) {
    if (!ctx || !name) return set_err(ctx, SIHIP_EINVAL, "set_option: NULL argument");
    for (const OptionName &n : kOptionNames)
        if (!strcmp(name, n.name)) {
            ctx->opt.*(n.field) = value < 0 ? -1 : value;
            return SIHIP_OK;
        }
    return set_err(ctx, SIHIP_EINVAL, "set_option: unknown option %s", name);
}

extern "C" const char *sihip_last_error(const sihip_ctx *ctx) {
    return ctx ? ctx->err : g_init_err;
}

// ---- weights ------------------------------------------------------------------

// Workgroup cap per CU for matvec launches with more row tiles than waves:
// two, the number resident at once for the heavier kernels, so the whole
// grid is one generation of long-lived workgroups (each walks several
// tiles) instead of several generations that each repeat the prologue
// (measured 2-4% faster than 4 or 8 on heads and 27648-row matrices).
// SIHIP_WG_PER_CU overrides.
static int wgs_per_cu(const Options &o) { return o.wg_per_cu > 0 ? (int)o.wg_per_cu : 2; }

static int64_t wave_target(const Options &o) { return o.wave_target > 0 ? o.wave_target : 800; }

// Activation elements per column slice (slice_rounds in formats.h); the
// SPLIT_ELEMS option overrides kSliceElems (0: no slices).
static int64_t split_elems(const Options &o) { return o.split_elems >= 0 ? o.split_elems : kSliceElems; }

// Columns (super-blocks for K-quants, 32-element units otherwise) per wave
// tile: the smallest power of two that keeps at least 80% of the lanes busy
// and gives at least wave_target() row tiles (about one per resident wave
// of a decode launch, so no second wave of workgroups trails behind), while
// each lane keeps as many rounds (and as few shuffle steps) as possible.
// A matrix that this leaves with fewer than 256 row tiles (few rows and
// long rows, e.g. a 1024-row kv projection) takes wider tiles at down to 50%
// busy lanes: padding slots cost lanes but no memory traffic (they re-read a
// real column), and more waves in flight matter more there.
//
// Rows of at least two slice lengths are cut into column slices; their tiles
// are narrow, 4 super-blocks (K-quants) or 8 blocks wide, so that a wave
// keeps several rounds per slice (measured on rows of 14336 and 27648: 4-29%
// faster than the widest tiles without slices), and wider only while the
// launch would have fewer than 256 workgroups.
static int choose_G(const Options &o, uint32_t type, int64_t n_out, int64_t n_in) {
    const int64_t ncols = is_kquant(type) ? n_in / 256 : n_in / 32;
    if (o.tile_cols > 0) {
        const int G = (int)o.tile_cols;
        if (G >= 1 && G <= 64 && !(G & (G - 1))) return G;
    }
    const int64_t elems = split_elems(o);
    if (sliced_rows(n_in, elems)) {
        int G = is_kquant(type) ? 4 : 8;
        for (; G < 64; G *= 2) {
            Layout L;
            if (!make_layout(type, n_out, n_in, G, &L)) break;
            const int64_t spr = slice_rounds(L, elems);
            const int64_t wgs = (L.ntiles + kWaves - 1) / kWaves * ((L.S + spr - 1) / spr);
            if (wgs >= 256) break;
        }
        return G;
    }
    const int64_t target = wave_target(o);
    // Two lanes per row at least (one lane per row lost 4-8% on 151936-row
    // heads of 4 and 28 columns) and 16 rounds per lane at most (a lane that
    // walks 80 units of a 27648 x 5120 Q5_0 or F16 row lost 3-32% to tiles
    // 16 wide); a row of one column keeps one lane.
    const int min_g = ncols >= 2 ? 2 : 1;
    // Unit columns (Q4_0, Q5_0, Q8_0, F16): where the narrowest tile with at
    // most 6 rounds per lane (80% of the lanes busy) gives 512-4096 row
    // tiles, it is taken. The tile-count rule below leaves 2 or 3 rounds
    // there, or 10: Q8_0 4864 x 896 4.77 us at 16 wide against 4.14 at 8,
    // Q5_0 5120 x 5120 9.47 at 16 against 8.01 at 32, Q5_0 and F16
    // 1024 x 5120 5.45 and 6.32 at 64 against 5.28 and 5.83 at 32. Fewer
    // tiles (896 x 896, 128 x 896: 4.0 and 3.8 us at 8 wide, 3.5 at 32) or
    // more (27648-row and 151936-row matrices) keep the tile-count rule.
    if (!is_kquant(type)) {
        for (int G = min_g; G <= 64; G *= 2) {
            const int64_t S = (ncols + G - 1) / G;
            if (S > 6 || ncols * 100 < S * G * 80) continue;
            const int64_t tiles = (n_out + 64 / G - 1) / (64 / G);
            if (tiles >= 512 && tiles <= 4096) return G;
            break;
        }
    }
    auto pick = [&](int pct, int64_t max_rounds) {
        int best = 0;
        int64_t best_tiles = 0;
        for (int G = min_g; G <= 64; G *= 2) {
            const int64_t S = (ncols + G - 1) / G;
            if (ncols * 100 < S * G * pct) continue;  // too few lanes busy
            if (S > max_rounds) continue;
            const int64_t tiles = (n_out + 64 / G - 1) / (64 / G);
            if (tiles > best_tiles) { best = G; best_tiles = tiles; }
            if (tiles >= target) break;
        }
        return std::make_pair(best, best_tiles);
    };
    auto choose = [&](int64_t max_rounds) {
        auto [G, tiles] = pick(80, max_rounds);
        if (tiles < 256) G = pick(50, max_rounds).first;
        return G;
    };
    const int G = choose(16);
    return G > 0 ? G : std::max(choose(INT64_MAX), 1);
}

// Exponent E of the Q4_K 16x16 GEMM's min operand (gemm2.h): the largest
// E <= 14 with max |dmin| * 63 * 2^E <= 2^15 over the tensor's blocks, so
// the hi halves stay far inside the f16 range. dmin is the f16 at bytes
// 2..3 of each 144-byte block (reference quant.h:71-78).
static int q4k_min_exponent(const uint8_t *blocks, uint64_t nblocks) {
    float mx = 0.0f;
    for (uint64_t i = 0; i < nblocks; i++) {
        const uint8_t *b = blocks + i * 144;
        const float v = fabsf(half_to_float((uint32_t)b[2] | ((uint32_t)b[3] << 8)));
        if (v > mx) mx = v;  // NaN never enters
    }
    int e = 14;
    while (e > -24 && (double)mx * 63.0 * std::ldexp(1.0, e) > 32768.0) e--;
    return e;
}

// F32 weights: the rows as they are (f32w.h). Layout fields other than
// type and shape stay zero; no plane, slice or GEMM copy exists.
static int upload_f32(sihip_ctx *ctx, uint64_t n_out, uint64_t n_in, const void *host,
                      uint64_t bytes, sihip_weight **out) {
    if (n_out == 0 || n_in == 0)
        return set_err(ctx, SIHIP_EINVAL, "weight_upload: empty F32 tensor");
    if (n_in > (1ull << 30) || n_out > (1ull << 31))
        return set_err(ctx, SIHIP_ERANGE, "weight_upload: shape too large");
    if (bytes != n_out * n_in * 4)
        return set_err(ctx, SIHIP_EINVAL, "weight_upload: %llu bytes given, %llu expected",
                       (unsigned long long)bytes, (unsigned long long)(n_out * n_in * 4));
    HIP_OK(ctx, hipSetDevice(ctx->device));
    uint8_t *dev = nullptr;
    if (hipMalloc((void **)&dev, (size_t)bytes) != hipSuccess)
        return set_err(ctx, SIHIP_ENOMEM, "weight_upload: %llu device bytes", (unsigned long long)bytes);
    hipError_t e = hipMemcpyAsync(dev, host, (size_t)bytes, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        (void)hipFree(dev);
        return set_err(ctx, SIHIP_EDEVICE, "weight_upload: %s", hipGetErrorString(e));
    }
    sihip_weight *w = new sihip_weight();
    memset(&w->L, 0, sizeof w->L);
    w->L.type = T_F32;
    w->L.n_out = (int64_t)n_out;
    w->L.n_in = (int64_t)n_in;
    w->L.total_bytes = (int64_t)bytes;
    w->dev = dev;
    *out = w;
    return SIHIP_OK;
}

extern "C" int sihip_weight_upload(sihip_ctx *ctx, uint32_t type, uint64_t n_out,
                                   uint64_t n_in, const void *host_blocks, uint64_t bytes,
                                   sihip_weight **out) {
    if (!ctx || !out || !host_blocks) return set_err(ctx, SIHIP_EINVAL, "weight_upload: NULL argument");
    if (type == T_F32) return upload_f32(ctx, n_out, n_in, host_blocks, bytes, out);
    uint32_t be, bb;
    if (!geometry(type, &be, &bb) || type == T_Q8_K)
        return set_err(ctx, SIHIP_ENOTSUP, "weight_upload: unsupported ggml type %u", type);
    if (n_out == 0 || n_in == 0 || n_in % be != 0 || n_in % 32 != 0)
        return set_err(ctx, SIHIP_EINVAL,
                       "weight_upload: n_in %llu is not a multiple of the block size %u",
                       (unsigned long long)n_in, be);
    if (n_in > (1ull << 24) || n_out > (1ull << 31))
        return set_err(ctx, SIHIP_ERANGE, "weight_upload: shape too large");
    const uint64_t row_bytes = n_in / be * bb;
    if (bytes != row_bytes * n_out)
        return set_err(ctx, SIHIP_EINVAL, "weight_upload: %llu bytes given, %llu expected",
                       (unsigned long long)bytes, (unsigned long long)(row_bytes * n_out));
    HIP_OK(ctx, hipSetDevice(ctx->device));
    const int64_t nunits = (int64_t)n_in / 32;
    Layout L;
    if (!make_layout(type, (int64_t)n_out, (int64_t)n_in, choose_G(ctx->opt, type, n_out, n_in), &L))
        return set_err(ctx, SIHIP_EINVAL, "weight_upload: no layout for this shape");
    const uint32_t spr = (uint32_t)slice_rounds(L, split_elems(ctx->opt));
    const uint32_t split = (uint32_t)((L.S + spr - 1) / spr);
    // slices: partial sums for up to kMaxCols columns, then one counter per
    // group of kWaves row tiles
    const int64_t part_bytes = split > 1 ? (int64_t)split * kMaxCols * L.ntiles * L.R * 4 : 0;
    const int64_t cnt_bytes = split > 1 ? ((L.ntiles + kWaves - 1) / kWaves) * 4 : 0;
    const int64_t alloc = L.total_bytes + part_bytes + cnt_bytes;
    uint8_t *dev = nullptr;
    if (hipMalloc((void **)&dev, (size_t)alloc) != hipSuccess)
        return set_err(ctx, SIHIP_ENOMEM, "weight_upload: %lld device bytes", (long long)alloc);
    uint8_t *raw = nullptr;
    if (hipMalloc((void **)&raw, (size_t)bytes) != hipSuccess) {
        (void)hipFree(dev);
        return set_err(ctx, SIHIP_ENOMEM, "weight_upload: %llu staging bytes",
                       (unsigned long long)bytes);
    }
    int rc = SIHIP_OK;
    const int64_t recs = (type == T_F16) ? nunits : (int64_t)(n_in / be);
    const int64_t rec_bytes = (type == T_F16) ? 64 : bb;
    const int64_t total = (int64_t)n_out * recs;
    hipError_t e = hipMemsetAsync(dev, 0, (size_t)alloc, ctx->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(raw, host_blocks, (size_t)bytes, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) {
        hipLaunchKernelGGL(repack_kernel, dim3((unsigned)((total + kThreads - 1) / kThreads)),
                           dim3(kThreads), 0, ctx->stream, L, raw, dev, (int64_t)row_bytes, recs,
                           rec_bytes);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    (void)hipFree(raw);
    if (e != hipSuccess) {
        (void)hipFree(dev);
        return set_err(ctx, SIHIP_EDEVICE, "weight_upload: %s", hipGetErrorString(e));
    }
    sihip_weight *w = new sihip_weight();
    w->L = L;
    w->dev = dev;
    w->split = split;
    w->spr = spr;
    if (type == T_Q4_K) w->gexp = q4k_min_exponent((const uint8_t *)host_blocks, bytes / bb);
    if (split > 1) {
        w->part = reinterpret_cast<float *>(dev + L.total_bytes);
        w->cnt = reinterpret_cast<uint32_t *>(dev + L.total_bytes + part_bytes);
        w->split_bytes = part_bytes + cnt_bytes;
    }
    *out = w;
    return rc;
}

extern "C" int sihip_weight_free(sihip_ctx *ctx, sihip_weight *w) {
    if (!w) return SIHIP_OK;
    if (ctx) HIP_OK(ctx, hipSetDevice(ctx->device));
    (void)hipFree(w->dev);
    if (w->gemm) (void)hipFree(w->gemm);
    if (w->gemm2) (void)hipFree(w->gemm2);
    if (w->gsmall) (void)hipFree(w->gsmall);
    order_free(w->order);
    delete w;
    return SIHIP_OK;
}

extern "C" uint64_t sihip_weight_device_bytes(const sihip_weight *w) {
    return w ? (uint64_t)(w->L.total_bytes + w->split_bytes + w->gemm_bytes + w->gemm2_bytes + w->gsmall_bytes) : 0;
}

extern "C" int sihip_weight_tile_cols(const sihip_weight *w) { return w ? w->L.G : 0; }

extern "C" int sihip_weight_slice_rounds(const sihip_weight *w) { return w ? (int)w->spr : 0; }

// ---- launches -----------------------------------------------------------------

// Q8_K passes of the activation loaded before the weights (16 blocks of
// 256 each): all four for long unsliced rows of a single column where the
// kernel has register room (the instances with Q6_K run at 2 waves per
// SIMD with registers to spare); two for the other K-quants' single-matrix
// launches of rows up to 8192 (16 more VGPRs: Q2_K 148 -> 164 and Q3_K 137
// -> 153 keep three waves per SIMD, Q4_K and Q5_K two), so a 5120-element
// row's last 4 blocks do not wait for a second round trip after the first
// pass is quantized; else the first. Launches with sliced matrices take one
// pass (a slice of about 4096 elements is one).
template <uint32_t F0, uint32_t F1>
static int prologue_passes(const MVArgs &A) {
    if (pair_of(F0) != T_Q8_K || A.nc != 1 || A.n_in <= 4096) return 1;
    if (F0 == T_Q6_K || F1 == T_Q6_K) return 4;
    return A.nseg == 1 && A.n_in <= 8192 ? 2 : 1;
}

static bool any_sliced(const MVArgs &A) {
    for (int i = 0; i < A.nseg; i++)
        if (A.seg[i].split > 1) return true;
    return false;
}

template <uint32_t F0, uint32_t F1, int NC, bool MULTI>
static hipError_t launch_nc(const MVArgs &A, dim3 grid, size_t lds, hipStream_t st) {
    if (any_sliced(A)) {
        hipLaunchKernelGGL((matvec_kernel<F0, F1, NC, 1, true, MULTI>), grid, dim3(kThreads), lds,
                           st, A);
        return hipGetLastError();
    }
    if constexpr (NC == 1 && (F0 == T_Q6_K || F1 == T_Q6_K)) {
        if (prologue_passes<F0, F1>(A) == 4) {
            hipLaunchKernelGGL((matvec_kernel<F0, F1, NC, 4, false, MULTI>), grid, dim3(kThreads),
                               lds, st, A);
            return hipGetLastError();
        }
    } else if constexpr (NC == 1 && !MULTI && F0 == F1 && pair_of(F0) == T_Q8_K) {
        if (prologue_passes<F0, F1>(A) == 2) {
            hipLaunchKernelGGL((matvec_kernel<F0, F1, NC, 2, false, MULTI>), grid, dim3(kThreads),
                               lds, st, A);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL((matvec_kernel<F0, F1, NC, 1, false, MULTI>), grid, dim3(kThreads), lds, st,
                       A);
    return hipGetLastError();
}

// Launches of several matrices are single-column (gemv_multi); a launch of
// one matrix takes 1, 2, 4 or 8 columns (at most 4 for the K-quants).
template <uint32_t F0, uint32_t F1>
static hipError_t launch_fmt(const MVArgs &A, dim3 grid, size_t lds, hipStream_t st) {
    if (A.nseg > 1)
        return A.nc == 1 ? launch_nc<F0, F1, 1, true>(A, grid, lds, st) : hipErrorInvalidValue;
    if constexpr (F0 != F1) {
        return hipErrorInvalidValue;
    } else {
        switch (A.nc) {
            case 1: return launch_nc<F0, F0, 1, false>(A, grid, lds, st);
            case 2: return launch_nc<F0, F0, 2, false>(A, grid, lds, st);
            case 4: return launch_nc<F0, F0, 4, false>(A, grid, lds, st);
            case 8:
                if constexpr (!is_kquant(F0)) return launch_nc<F0, F0, 8, false>(A, grid, lds, st);
                return hipErrorInvalidValue;
            default: return hipErrorInvalidValue;
        }
    }
}

// Format pairs one launch can mix (the K-quant mixes of Q4_K_M / Q5_K_M
// models); f0 < f1.
static bool mix_supported(uint32_t f0, uint32_t f1) {
    return f0 == f1 || (f0 == T_Q4_K && f1 == T_Q6_K) || (f0 == T_Q5_K && f1 == T_Q6_K);
}

static hipError_t launch_any(const MVArgs &A, uint32_t f0, uint32_t f1, dim3 grid, size_t lds,
                             hipStream_t st) {
    if (f0 == T_Q4_K && f1 == T_Q6_K) return launch_fmt<T_Q4_K, T_Q6_K>(A, grid, lds, st);
    if (f0 == T_Q5_K && f1 == T_Q6_K) return launch_fmt<T_Q5_K, T_Q6_K>(A, grid, lds, st);
    if (f0 != f1) return hipErrorInvalidValue;
    switch (f0) {
        case T_F16:  return launch_fmt<T_F16, T_F16>(A, grid, lds, st);
        case T_Q4_0: return launch_fmt<T_Q4_0, T_Q4_0>(A, grid, lds, st);
        case T_Q5_0: return launch_fmt<T_Q5_0, T_Q5_0>(A, grid, lds, st);
        case T_Q8_0: return launch_fmt<T_Q8_0, T_Q8_0>(A, grid, lds, st);
        case T_Q2_K: return launch_fmt<T_Q2_K, T_Q2_K>(A, grid, lds, st);
        case T_Q3_K: return launch_fmt<T_Q3_K, T_Q3_K>(A, grid, lds, st);
        case T_Q4_K: return launch_fmt<T_Q4_K, T_Q4_K>(A, grid, lds, st);
        case T_Q5_K: return launch_fmt<T_Q5_K, T_Q5_K>(A, grid, lds, st);
        case T_Q6_K: return launch_fmt<T_Q6_K, T_Q6_K>(A, grid, lds, st);
        default: return hipErrorInvalidValue;
    }
}

static int64_t col_bytes_aligned(uint32_t pair, int64_t n_in) {
    return (lds_col_bytes(pair, n_in) + 15) & ~(int64_t)15;
}

// LDS bytes past the activation columns of a launch with a sliced matrix
// (the arrival flag of split_reduce).
constexpr int64_t kSliceLds = 16;

// Largest supported column count (1, 2, 4 or 8) whose LDS fits.
static int max_cols(const sihip_ctx *ctx, uint32_t pair, int64_t n_in) {
    const int64_t cb = col_bytes_aligned(pair, n_in);
    for (int nc = kMaxCols; nc >= 1; nc >>= 1)
        if ((size_t)(cb * nc + kSliceLds) <= ctx->lds_limit) return nc;
    return 0;
}

// One launch computes `count` matrices against the same activation
// columns [0, M) of x (f32, ldx) or xq (pair format, ldxq); matrix i writes
// rows [0, n_out[i]) of y[i] (column stride ldy[i]). The caller checks that
// the matrices share n_in and that mix_supported() holds for their formats.
// M is split into launches of 8/4/2/1 columns.
// F32 weights (f32w.h): launches of up to kF32Cols columns of x (f32;
// the pair format of F32 is f32 itself).
static int run_f32(sihip_ctx *ctx, const sihip_weight *w, int64_t n_out, float *y, int64_t ldy,
                   const float *x, int64_t ldx, int64_t M, hipStream_t st) {
    const dim3 grid((unsigned)((n_out + kF32Threads / 64 - 1) / (kF32Threads / 64)));
    const float *W = (const float *)w->dev;
    for (int64_t m = 0; m < M;) {
        const int64_t nc = M - m >= kF32Cols ? kF32Cols : M - m;
        switch (nc) {
            case 4: hipLaunchKernelGGL(f32_matvec_kernel<4>, grid, dim3(kF32Threads), 0, st, W, w->L.n_in, n_out, x + m * ldx, ldx, y + m * ldy, ldy); break;
            case 3: hipLaunchKernelGGL(f32_matvec_kernel<3>, grid, dim3(kF32Threads), 0, st, W, w->L.n_in, n_out, x + m * ldx, ldx, y + m * ldy, ldy); break;
            case 2: hipLaunchKernelGGL(f32_matvec_kernel<2>, grid, dim3(kF32Threads), 0, st, W, w->L.n_in, n_out, x + m * ldx, ldx, y + m * ldy, ldy); break;
            default: hipLaunchKernelGGL(f32_matvec_kernel<1>, grid, dim3(kF32Threads), 0, st, W, w->L.n_in, n_out, x + m * ldx, ldx, y + m * ldy, ldy); break;
        }
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return set_err(ctx, SIHIP_EDEVICE, "f32 matvec launch: %s", hipGetErrorString(e));
        m += nc;
    }
    return SIHIP_OK;
}

static int run_matvec_multi(sihip_ctx *ctx, int count, const sihip_weight *const *w,
                            const int64_t *n_out, float *const *y, const int64_t *ldy,
                            const float *x, int64_t ldx, const uint8_t *xq, int64_t ldxq,
                            int64_t M, hipStream_t st) {
    if (w[0]->L.type == T_F32) {  // callers pass F32 weights one at a time
        const float *xf = x ? x : (const float *)xq;
        return run_f32(ctx, w[0], n_out[0], y[0], ldy[0], xf, x ? ldx : ldxq / 4, M, st);
    }
    const int64_t n_in = w[0]->L.n_in;
    const uint32_t pair = pair_of(w[0]->L.type);
    uint32_t f0 = w[0]->L.type, f1 = w[0]->L.type;
    for (int i = 1; i < count; i++) {
        const uint32_t t = w[i]->L.type;
        if (t < f0) f0 = t;
        if (t > f1) f1 = t;
    }
    // LDS per activation column: a whole row, or for a sliced matrix one
    // slice (its workgroups stage only their slice)
    int64_t n_lds = 0;
    for (int i = 0; i < count; i++) {
        const Layout &L = w[i]->L;
        const int64_t need = w[i]->split > 1
                                 ? (int64_t)w[i]->spr * L.G * (is_kquant(L.type) ? 256 : 32)
                                 : n_in;
        n_lds = need > n_lds ? need : n_lds;
    }
    int ncmax = max_cols(ctx, pair, n_lds);
    if (ncmax == 0)
        return set_err(ctx, SIHIP_ERANGE, "activation row of %lld does not fit in LDS",
                       (long long)n_in);
    if (is_kquant(f1) && ncmax > 4) ncmax = 4;  // 8 K-quant columns exceed the VGPR file
    if (count > 1) {
        if (M != 1) return set_err(ctx, SIHIP_EINVAL, "a launch of several matrices takes one column");
        ncmax = 1;
    }
    const int64_t cb = col_bytes_aligned(pair, n_lds);
    // workgroups: one row tile per wave when the chip has room; otherwise
    // each matrix gets a share of the cap proportional to its bytes
    const int64_t wg_cap = (int64_t)ctx->n_cu * wgs_per_cu(ctx->opt);
    // (a sliced matrix always takes one workgroup per tile group and slice)
    int64_t want[kMaxSegs], nwg[kMaxSegs], want_sum = 0, bytes_sum = 0;
    for (int i = 0; i < count; i++) {
        const int64_t ntiles = (n_out[i] + w[i]->L.R - 1) / w[i]->L.R;
        want[i] = (ntiles + kWaves - 1) / kWaves;
        if (w[i]->split > 1) want[i] *= w[i]->split;
        want_sum += want[i];
        bytes_sum += w[i]->L.total_bytes;
    }
    for (int i = 0; i < count; i++) {
        nwg[i] = want[i];
        if (want_sum > wg_cap && w[i]->split == 1) {
            const int64_t share = (int64_t)((double)wg_cap * (double)w[i]->L.total_bytes /
                                            (double)bytes_sum);
            nwg[i] = share < 1 ? 1 : (share < want[i] ? share : want[i]);
        }
    }
    // A launch of several matrices that would need between one and two
    // workgroups per CU halves the workgroups of its largest whole-row
    // matrix (each wave then walks two of its tiles) where that brings it to
    // one per CU: otherwise half the CUs run two workgroups and the rest one.
    // Llama-3-8B q/k/v (256 + 64 + 64 workgroups): 6.34 -> 5.52 us.
    // (Only where the halved matrix still cuts into ranges as wide as the
    // narrowest matrix, below, so the grid keeps no surplus workgroups.)
    if (count > 1 && want_sum > ctx->n_cu && want_sum <= wg_cap) {
        int big = -1;
        for (int i = 0; i < count; i++)
            if (w[i]->split == 1 && (big < 0 || nwg[i] > nwg[big])) big = i;
        if (big >= 0 && nwg[big] % 2 == 0 && want_sum - nwg[big] / 2 <= ctx->n_cu) {
            const int64_t half = nwg[big] / 2;
            int64_t narrow_other = 0;
            for (int i = 0; i < count; i++)
                if (i != big && (narrow_other == 0 || nwg[i] < narrow_other)) narrow_other = nwg[i];
            const int64_t ntiles = (n_out[big] + w[big]->L.R - 1) / w[big]->L.R;
            if (narrow_other > 0 && half >= narrow_other && half % narrow_other == 0 &&
                ntiles % (half * kWaves) == 0)
                nwg[big] = half;
        }
    }
    for (int i = 0; i < count; i++) {
        if (w[i]->split > 1) {
            const int rc = order_before(ctx, w[i]->order, st);
            if (rc) return rc;
        }
    }
    // A launch of several matrices gets a grid of (its widest segment's
    // workgroups) x (segments), and a segment narrower than the widest
    // leaves the surplus to exit at once. Those exits still hold workgroup
    // slots while their arguments load, and with two resident per CU the
    // q/k/v launch (768 workgroups, 384 of them surplus) kept its Q6_K wv
    // workgroups waiting for slots. A whole-row matrix whose workgroup count
    // is a multiple of the narrowest matrix's is therefore cut into ranges
    // of consecutive row tiles of that many workgroups (a range is the same
    // matrix from a later tile: plane bases, y and rows offset), so every
    // segment is equally wide: q/k/v runs as 4 x 64 workgroups, wq in two
    // ranges whose waves walk two tiles each.
    int parts[kMaxSegs];
    int nsegs = 0;
    int64_t narrow = 0;
    for (int i = 0; i < count; i++)
        if (narrow == 0 || nwg[i] < narrow) narrow = nwg[i];
    for (int i = 0; i < count; i++) {
        const int64_t ntiles = (n_out[i] + w[i]->L.R - 1) / w[i]->L.R;
        parts[i] = 1;
        if (count > 1 && w[i]->split == 1 && nwg[i] > narrow && nwg[i] % narrow == 0 &&
            ntiles % (nwg[i] * kWaves) == 0)
            parts[i] = (int)(nwg[i] / narrow);
        nsegs += parts[i];
    }
    if (nsegs > kMaxLaunchSegs)
        for (int i = 0; i < count; i++) parts[i] = 1;
    int64_t m = 0;
    while (m < M) {
        int nc = ncmax;
        while (nc > 1 && m + nc > M) nc >>= 1;
        MVArgs A;
        memset(&A, 0, sizeof(A));
        uint32_t wg = 0;
        int ns = 0;
        for (int i = 0; i < count; i++) {
            const Layout &L = w[i]->L;
            const int64_t ntiles = (n_out[i] + L.R - 1) / L.R;
            const int64_t per = ntiles / parts[i];  // row tiles of a range (parts[i] divides)
            for (int k = 0; k < parts[i]; k++) {
                const int64_t t0 = k * per;
                const int64_t rows = k + 1 < parts[i] ? per * L.R : n_out[i] - t0 * L.R;
                MVSeg &sg = A.seg[ns++];
                // the records of tile t0 start at record (t0 * S) * 64 of a
                // column-level plane, 8 times that of a unit-level one
                for (int p = 0; p < 4; p++) {
                    const int64_t per_col = is_kquant(L.type) && !L.plane_blk[p] ? 8 : 1;
                    sg.plane[p] = w[i]->dev + L.plane_off[p] +
                                  t0 * L.S * 64 * per_col * L.plane_bytes[p];
                }
                sg.y = y[i] + m * ldy[i] + t0 * L.R;
                sg.ldy = ldy[i];
                sg.part = w[i]->part;
                sg.cnt = w[i]->cnt;
                sg.split = w[i]->split;
                sg.spr = w[i]->spr;
                sg.type = L.type;
                sg.n_out = (uint32_t)rows;
                sg.ntiles = (uint32_t)((rows + L.R - 1) / L.R);
                sg.nwg = (uint32_t)(nwg[i] / parts[i]);
                sg.G = (uint32_t)L.G;
                sg.logG = (uint32_t)L.logG;
                sg.R = (uint32_t)L.R;
                sg.S = (uint32_t)L.S;
                sg.ncols = (uint32_t)L.ncols;
                wg = sg.nwg > wg ? sg.nwg : wg;
            }
        }
        A.nseg = ns;
        A.n_in = n_in;
        A.q80s = ctx->opt.q80_scalar > 0;
        A.x = x ? x + m * ldx : nullptr;
        A.xq = xq ? xq + m * ldxq : nullptr;
        A.ldx = ldx;
        A.ldxq = ldxq;
        A.nc = nc;
        A.col_bytes = cb;
        const hipError_t e =
            launch_any(A, f0, f1, dim3(wg, (unsigned)ns),
                       (size_t)(cb * nc + (any_sliced(A) ? kSliceLds : 0)), st);
        if (e != hipSuccess)
            return set_err(ctx, SIHIP_EDEVICE, "matvec launch: %s", hipGetErrorString(e));
        m += nc;
    }
    for (int i = 0; i < count; i++) {
        if (w[i]->split > 1) {
            const int rc = order_after(ctx, w[i]->order, st);
            if (rc) return rc;
        }
    }
    return SIHIP_OK;
}

static int run_matvec(sihip_ctx *ctx, const sihip_weight *w, const float *x, int64_t ldx,
                      const uint8_t *xq, int64_t ldxq, int64_t M, float *y, int64_t ldy,
                      int64_t n_out, hipStream_t st) {
    return run_matvec_multi(ctx, 1, &w, &n_out, &y, &ldy, x, ldx, xq, ldxq, M, st);
}

static bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

// ---- prefill GEMM on MFMA -----------------------------------------------------

// Smallest M that takes the MFMA GEMM (below it the matvec kernel, which
// streams the weights once per 1-4 columns, is cheaper: Q4_K 14336 x 4096
// at M = 4 takes 17.5 us there against 22 us on the matrix cores, at M = 8
// 33.7 against 22). Q5_K, Q2_K and Q3_K use the same threshold: at M = 8
// (config 4's 32B-class shapes) their matrix-core calls take 2.0-3.9x less
// time than the matvec kernel's. With the small-M kernels (gemm2s.h,
// gemmks.h) the threshold is 3: Llama-3-8B shapes per call at M = 3, matvec
// against small-M kernel: q/k/v 28.6 / 22.1 us, gate/up 35.5 / 27.8,
// ffn_down (Q6_K) 27.6 / 18.8; at M = 4 27.7 / 22.4, 31.9 / 28.2, 21.4 /
// 18.9; at M = 2 the matvec kernel wins (17.1 / 21.8, 19.8 / 27.7, 15.7 /
// 18.7). The GEMM_MIN_M option overrides it (tests force both paths).
static int64_t gemm_min_m(const Options &o) { return o.gemm_min_m > 0 ? o.gemm_min_m : 3; }

static bool is_q80_pair(uint32_t t) { return t == T_Q4_0 || t == T_Q5_0 || t == T_Q8_0; }

static bool gemm_mfma_supported(const Layout &L) {
    const uint32_t t = L.type;
    if (t == T_F16 || is_q80_pair(t)) return L.n_in % 128 == 0;  // steps of 128 elements
    return t == T_Q4_K || t == T_Q5_K || t == T_Q2_K || t == T_Q3_K || t == T_Q6_K;
}

// Types whose 32x32 GEMM copy exists (gemm.h): the K-quants but Q6_K.
static bool gemm32_supported(const Layout &L) {
    return gemm_mfma_supported(L) && (L.type == T_Q4_K || L.type == T_Q5_K || L.type == T_Q2_K ||
                                      L.type == T_Q3_K);
}

// Types with a 16x16 GEMM copy (w->gemm2): Q4_K (gemm2.h), Q6_K (gemm6.h),
// F16 (gemmh.h), Q4_0 / Q5_0 / Q8_0 (gemmq.h).
static bool gemm16_supported(const Layout &L) {
    return gemm_mfma_supported(L) && (L.type == T_Q4_K || L.type == T_Q6_K || L.type == T_F16 ||
                                      is_q80_pair(L.type));
}

// The weight's copy in the GEMM's order (gemm_layout_kernel), built from
// its matvec copy on stream st.
static int build_gemm_copy(sihip_ctx *ctx, sihip_weight *w, hipStream_t st) {
    if (capturing(st))
        return set_err(ctx, SIHIP_EINVAL,
                       "the weight's GEMM copy would be built during graph capture: call "
                       "sihip_weight_prepare_gemm before capturing");
    const Layout &L = w->L;
    const int64_t nb = L.n_in / 256;
    const int64_t nblk32 = (L.n_out + kGemmBN - 1) / kGemmBN * (kGemmBN / 32);
    const int64_t bytes = gemm_layout_bytes(nblk32, nb, L.type);
    uint8_t *g = nullptr;
    hipError_t e = hipMalloc(&g, (size_t)bytes);
    if (e != hipSuccess)
        return set_err(ctx, SIHIP_ENOMEM, "gemm weight copy (%lld bytes): %s", (long long)bytes,
                       hipGetErrorString(e));
    const int64_t threads = nblk32 * nb * (gemm_chunk_bytes(L.type) / 16);
    hipLaunchKernelGGL(gemm_layout_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                       st, L, (const uint8_t *)w->dev, g, nblk32);
    e = hipGetLastError();
    if (e != hipSuccess) {
        (void)hipFree(g);
        return set_err(ctx, SIHIP_EDEVICE, "gemm layout: %s", hipGetErrorString(e));
    }
    w->gemm = g;
    w->gemm_bytes = bytes;
    return SIHIP_OK;
}

// Q4_K, Q6_K and F16: the weight's copy in the order of the type's 16x16
// GEMM (gemm2.h, gemm6.h, gemmh.h).
static int build_gemm2_copy(sihip_ctx *ctx, sihip_weight *w, hipStream_t st) {
    if (capturing(st))
        return set_err(ctx, SIHIP_EINVAL,
                       "the weight's GEMM copy would be built during graph capture: call "
                       "sihip_weight_prepare_gemm before capturing");
    const Layout &L = w->L;
    const int64_t nblk32 = (L.n_out + kG2BN - 1) / kG2BN * (kG2BN / 32);
    int64_t bytes, threads;
    const int64_t nk = L.n_in / 128;
    if (L.type == T_Q8_0) {
        bytes = gemmq_layout_bytes<T_Q8_0>(nblk32, nk);
        threads = nblk32 * nk * (gq_chunk<T_Q8_0>() / 16);
    } else if (L.type == T_Q4_0) {
        bytes = gemmq_layout_bytes<T_Q4_0>(nblk32, nk);
        threads = nblk32 * nk * (gq_chunk<T_Q4_0>() / 16);
    } else if (L.type == T_Q5_0) {
        bytes = gemmq_layout_bytes<T_Q5_0>(nblk32, nk);
        threads = nblk32 * nk * (gq_chunk<T_Q5_0>() / 16);
    } else if (L.type == T_F16) {
        bytes = gemmh_layout_bytes(nblk32, L.n_in / 128);
        threads = nblk32 * (L.n_in / 128) * (kGHChunk / 16);
    } else if (L.type == T_Q6_K) {
        bytes = gemm6_layout_bytes(nblk32, L.n_in / 256);
        threads = nblk32 * (L.n_in / 256) * (kG6Chunk / 16);
    } else {
        bytes = gemm2_layout_bytes(nblk32, L.n_in / 256);
        threads = nblk32 * (L.n_in / 256) * (kG2ChunkQ4K / 16);
    }
    uint8_t *g = nullptr;
    hipError_t e = hipMalloc(&g, (size_t)bytes);
    if (e != hipSuccess)
        return set_err(ctx, SIHIP_ENOMEM, "gemm weight copy (%lld bytes): %s", (long long)bytes,
                       hipGetErrorString(e));
    const dim3 grid((unsigned)((threads + 255) / 256));
    if (L.type == T_Q8_0)
        hipLaunchKernelGGL(gemmq_layout<T_Q8_0>, grid, dim3(256), 0, st, L, (const uint8_t *)w->dev,
                           g, nblk32);
    else if (L.type == T_Q4_0)
        hipLaunchKernelGGL(gemmq_layout<T_Q4_0>, grid, dim3(256), 0, st, L, (const uint8_t *)w->dev,
                           g, nblk32);
    else if (L.type == T_Q5_0)
        hipLaunchKernelGGL(gemmq_layout<T_Q5_0>, grid, dim3(256), 0, st, L, (const uint8_t *)w->dev,
                           g, nblk32);
    else if (L.type == T_F16)
        hipLaunchKernelGGL(gemmh_layout_f16, grid, dim3(256), 0, st, L, (const uint8_t *)w->dev, g,
                           nblk32);
    else if (L.type == T_Q6_K)
        hipLaunchKernelGGL(gemm6_layout_q6k, grid, dim3(256), 0, st, L, (const uint8_t *)w->dev, g,
                           nblk32);
    else
        hipLaunchKernelGGL(gemm2_layout_q4k, grid, dim3(256), 0, st, L, (const uint8_t *)w->dev, g,
                           nblk32, std::ldexp(1.0f, w->gexp));
    e = hipGetLastError();
    if (e != hipSuccess) {
        (void)hipFree(g);
        return set_err(ctx, SIHIP_EDEVICE, "gemm layout: %s", hipGetErrorString(e));
    }
    w->gemm2 = g;
    w->gemm2_bytes = bytes;
    return SIHIP_OK;
}

static int64_t gemmks_max_m(const Options &o, uint32_t type);
// Largest M on the fused small-M K-quant launch (gemmkf.h, at most
// kKFMaxM); option GEMMKF_MAX_M, 0 turns it off.
static int64_t gemmkf_max_m(const Options &o) {
    return o.gemmkf_max_m >= 0 ? (o.gemmkf_max_m < kKFMaxM ? o.gemmkf_max_m : kKFMaxM) : kKFMaxM;
}

// The near-GGUF-size K-quant copy of the small-M GEMM (gemmks.h).
static int build_gemmks_copy(sihip_ctx *ctx, sihip_weight *w, hipStream_t st) {
    if (capturing(st))
        return set_err(ctx, SIHIP_EINVAL,
                       "the weight's GEMM copy would be built during graph capture: call "
                       "sihip_weight_prepare_gemm before capturing");
    const Layout &L = w->L;
    const int64_t nblk32 = (L.n_out + 31) / 32, nb = L.n_in / 256;
    const int64_t bytes = nblk32 * nb * gemmks_chunk(L.type);
    const int64_t threads = nblk32 * nb * (gemmks_chunk(L.type) / 16);
    uint8_t *g = nullptr;
    hipError_t e = hipMalloc(&g, (size_t)bytes);
    if (e != hipSuccess)
        return set_err(ctx, SIHIP_ENOMEM, "gemm weight copy (%lld bytes): %s", (long long)bytes,
                       hipGetErrorString(e));
    const dim3 grid((unsigned)((threads + 255) / 256));
    const uint8_t *src = (const uint8_t *)w->dev;
    switch (L.type) {
        case T_Q2_K: hipLaunchKernelGGL(gemmks_layout<T_Q2_K>, grid, dim3(256), 0, st, L, src, g, nblk32); break;
        case T_Q3_K: hipLaunchKernelGGL(gemmks_layout<T_Q3_K>, grid, dim3(256), 0, st, L, src, g, nblk32); break;
        case T_Q4_K: hipLaunchKernelGGL(gemmks_layout<T_Q4_K>, grid, dim3(256), 0, st, L, src, g, nblk32); break;
        case T_Q5_K: hipLaunchKernelGGL(gemmks_layout<T_Q5_K>, grid, dim3(256), 0, st, L, src, g, nblk32); break;
        default: hipLaunchKernelGGL(gemmks_layout<T_Q6_K>, grid, dim3(256), 0, st, L, src, g, nblk32); break;
    }
    e = hipGetLastError();
    if (e != hipSuccess) {
        (void)hipFree(g);
        return set_err(ctx, SIHIP_EDEVICE, "gemm layout: %s", hipGetErrorString(e));
    }
    w->gsmall = g;
    w->gsmall_bytes = bytes;
    return SIHIP_OK;
}

extern "C" int sihip_weight_prepare_gemm(sihip_ctx *ctx, sihip_weight *w) {
    if (!ctx || !w) return set_err(ctx, SIHIP_EINVAL, "weight_prepare_gemm: NULL argument");
    if (!gemm_mfma_supported(w->L)) return SIHIP_OK;
    HIP_OK(ctx, hipSetDevice(ctx->device));
    if (gemm32_supported(w->L) && !w->gemm) {
        const int rc = build_gemm_copy(ctx, w, ctx->stream);
        if (rc) return rc;
    }
    if (gemm16_supported(w->L) && !w->gemm2) {
        const int rc = build_gemm2_copy(ctx, w, ctx->stream);
        if (rc) return rc;
    }
    if (is_kquant(w->L.type) && !w->gsmall &&
        (gemmkf_max_m(ctx->opt) > 0 ||
         (gemmks_max_m(ctx->opt, w->L.type) > 0 &&
          !(w->L.type == T_Q4_K && ctx->opt.gemmks_q4k != 1)))) {
        const int rc = build_gemmks_copy(ctx, w, ctx->stream);
        if (rc) return rc;
    }
    HIP_OK(ctx, hipStreamSynchronize(ctx->stream));
    return SIHIP_OK;
}

// Smallest M that takes the 16x16 Q4_K GEMM (gemm2.h); option GEMM2_MIN_M.
// It needs two of its 128-row workgroups per CU to hide latency: at the
// 14336 x 4096 shape it is faster from M = 512 (83 against 95 us per call;
// M = 2048: 323 against 357 us) and slower at M = 256 (67 against 50 us).
constexpr int64_t kGemm2MinM = 384;
static int64_t gemm2_min_m(const Options &o) { return o.gemm2_min_m > 0 ? o.gemm2_min_m : kGemm2MinM; }
// Largest M that takes the small-M Q4_K GEMM (gemm2s.h; at most its 16-row
// m tile); option GEMM2S_MAX_M, 0 turns it off.
static int64_t gemm2s_max_m(const Options &o) {
    return o.gemm2s_max_m >= 0 ? (o.gemm2s_max_m < 16 ? o.gemm2s_max_m : 16) : 16;
}
// Largest M that takes the small-M K-quant GEMM (gemmks.h; at most 16);
// option GEMMKS_MAX_M (all K-quants), 0 turns it off. The rule is by
// format: past 8 rows the kernel takes 3 or 4 activation groups per MFMA
// and its registers spill, so the matrix-core GEMMs above take over.
// Config-4 shapes (27648 x 5120, 5120 x 27648, 5120 x 5120), us per call:
//   M = 12: Q2_K 33.8 / 65.5 / 20.4 here, 24.2 / 28.3 / 14.5 there;
//           Q5_K 111 / 155 / 32.4 here, 33.7 / 36.1 / 16.2 there;
//           Q3_K 25.2 / 32.0 / 12.6 here, 30.7 / 34.6 / 15.9 there;
//           Q6_K 37.2 / 43.3 / 14.1 here, 52.0 / 58.8 / 15.7 there;
//   M = 16: Q3_K 106 / 110 / 28.1 here, Q6_K 160 / 191 / 43.7 here.
static int64_t gemmks_max_m(const Options &o, uint32_t type) {
    if (o.gemmks_max_m >= 0) return o.gemmks_max_m < 16 ? o.gemmks_max_m : 16;
    return type == T_Q3_K || type == T_Q6_K ? 12 : 8;
}

// Smallest M that takes a Q6_K GEMM (the small-M kernel of gemmks.h up to
// M = 12, gemm6.h above); option GEMM6_MIN_M. As for the other K-quants
// (gemm_min_m) 3: the small-M kernel streams the GGUF bytes once, so it
// wins from M = 3 (ffn_down 4096 x 14336: 18.8 against 27.6 us on the
// matvec kernel), which stays faster at M = 2.
constexpr int64_t kGemm6MinM = 3;
static int64_t gemm6_min_m(const Options &o) { return o.gemm6_min_m > 0 ? o.gemm6_min_m : kGemm6MinM; }

// Smallest M that takes the F16 GEMM (gemmh.h); option GEMMH_MIN_M. Its copy
// holds the same bytes as the weights and streams them once for up to 128
// rows per m block, where the matvec kernel's time grows with the columns
// (config 4 at M = 8: ffn_up 27648 x 5120 61 us against 103, ffn_down 67
// against 153, attn 20 against 66); at M = 1 and 2 the matvec kernel is as
// fast or faster (kv 1024 x 5120 at M = 2: 10.2 us against 15.8).
constexpr int64_t kGemmhMinM = 3;
static int64_t gemmh_min_m(const Options &o) { return o.gemmh_min_m > 0 ? o.gemmh_min_m : kGemmhMinM; }

// Smallest M that takes the Q4_0 / Q5_0 / Q8_0 GEMM (gemmq.h); option
// GEMMQ_MIN_M. At M = 3 (the matvec kernel: a launch of two columns and
// one of one) the GEMM is the faster on every config shape (config 0 Q4_0
// 7.9 against 10.2 us, config 1 Q8_0 8.2 against 9.6, config 4 Q5_0 attn
// 12.5 against 19.5, kv 9.5 against 13.1, ffn_up 29.9 against 43.9); at
// M = 2 the matvec kernel is (6.1 / 5.5 / 11.6 / 7.9 / 26.6 against 8.0 /
// 8.3 / 12.4 / 9.5 / 29.8).
constexpr int64_t kGemmqMinM = 3;
static int64_t gemmq_min_m(const Options &o) { return o.gemmq_min_m > 0 ? o.gemmq_min_m : kGemmqMinM; }

// Shape of one matrix-core GEMM call: tile height, padded rows, workspace
// sizes and K slices.
struct GemmPlan {
    bool v2;           // a 16x16 kernel (Q4_K: gemm2.h, Q6_K: gemm6.h); mt counts 16-row m tiles
    bool small = false;  // M <= 16: gemmks_kernel (gemmks.h), or for Q4_K gemm2s_q4k_kernel
    bool q4s = false;    // Q4_K small M on gemm2s.h (the 16x16 GEMM's copy)
    int mt;            // 32-row MFMA tiles per wave along m
    int64_t Mp;        // M rounded up to the workgroup's rows
    int64_t ws_bytes;  // quantized activation planes
    int S, SBK;        // K slices (S == 1: none) and K steps per slice
    int64_t steps;     // K steps of a tile: super-blocks, or 128-element
                       // steps for the F16 and Q8_0-pair kernels
    int64_t part_bytes;
    bool fuseq = false;  // a GEMM that quantizes or converts X itself (gemmq_kernel XM 2,
                         // gemmh_f16_kernel XF)
};

// K slices of the 16x16 GEMMs: when the output tiles would fill at most
// half of `want` workgroups (by default two per CU, the slots of the
// kernels built for two waves per SIMD), the K steps of a tile
// (super-blocks, or 128-element steps) are split over S workgroups, as many
// as keep within `want` (a workgroup past the slots waits for a whole
// round: Q5_0 27648 x 5120 at M = 8 on two slots takes 25 us in 432
// workgroups against 31 us in 648), at least min_sbk steps each (a slice's
// fixed cost, its partial sums and the last workgroup's sum, outweighs a
// few steps); the GEMM_SBK option overrides (0: none). Above half of
// `want`, the partial sums' extra traffic costs more than the idle slots.
static void plan_slices(const sihip_ctx *ctx, GemmPlan &p, int64_t tiles, int64_t nb, int64_t NB,
                        int64_t min_sbk = 2, int64_t want = 0) {
    if (want <= 0) want = 2 * ctx->n_cu;
    int64_t sbk = 0;
    if (2 * tiles <= want) {
        int64_t S = want / tiles;
        if (S > nb / min_sbk) S = nb / min_sbk;
        if (S > 1) sbk = (nb + S - 1) / S;
    }
    if (ctx->opt.gemm_sbk >= 0) sbk = ctx->opt.gemm_sbk;
    p.S = 1;
    p.SBK = (int)nb;
    p.steps = nb;
    p.part_bytes = 0;
    if (sbk > 0 && sbk < nb && tiles <= kGemmCounters) {
        p.S = (int)((nb + sbk - 1) / sbk);
        p.SBK = (int)sbk;
        p.part_bytes = (int64_t)p.S * p.Mp * NB * kG2BN * (int64_t)sizeof(float);
    }
}

// force_mt > 0 sets the m tiles per wave where the kernel has that
// instance (as the GEMM_MT option does; sihip_gemm_multi_dev uses it to
// give weights that share X one activation record layout).
static GemmPlan plan_gemm(const sihip_ctx *ctx, const Layout &L, int64_t M, int force_mt = 0) {
    const int64_t opt_mt = force_mt > 0 ? force_mt : ctx->opt.gemm_mt;
    GemmPlan p;
    const int64_t K = L.n_in, nb = K / 256;
    const int64_t NB = (L.n_out + kGemmBN - 1) / kGemmBN;
    if (L.type == T_F16 || is_q80_pair(L.type)) {
        // m blocks of 16 to 128 rows by M (Q4_0/Q5_0/Q8_0: to 64), shorter
        // while the output tiles reach fewer than a quarter of the CUs (the
        // GEMM_MT option, 1, 2, 4 or 8, overrides); K slices over steps of
        // 128 elements
        const int64_t nk = K / 128;
        p.v2 = true;
        p.mt = M <= 16 ? 1 : M <= 32 ? 2 : M <= 64 ? 4 : 8;
        if (L.type != T_F16 && p.mt > 4) p.mt = 4;
        while (p.mt > 1 && (M + 16 * p.mt - 1) / (16 * p.mt) * NB < ctx->n_cu / 4) p.mt /= 2;
        if (opt_mt == 1 || opt_mt == 2 || opt_mt == 4 || (opt_mt == 8 && L.type == T_F16))
            p.mt = (int)opt_mt;
        const int64_t BM = 16 * p.mt;
        p.Mp = (M + BM - 1) / BM * BM;
        p.ws_bytes = p.Mp / BM * nk *
                     (L.type == T_F16 ? gh_rec_bytes((int)BM) : gq_rec_bytes((int)BM));
        // The Q8_0-pair kernel holds three workgroups per CU from 32-row m
        // blocks (at M = 8, 16-row blocks, two per CU are faster than three:
        // 25.3 against 28.8 us for 27648 x 5120; at M = 512, 5120 x 27648 in
        // 640 workgroups 313 us against 503 in 320). The F16 kernel streams
        // 8 KB per wave and step with no epilogue: up to 64-row blocks it is
        // fastest at about three workgroups per four CUs (M = 8: 27648 x
        // 5120 unsliced, 216 workgroups, 47.6 us against 53.6 in 432;
        // 5120 x 27648 in 160, 52.8 against 56.5 in 480; kv 1024 x 5120 in
        // 64, 8.6 against 12.6 in 160), 128-row blocks at two per CU.
        // Q8_0 pairs in 16-row m blocks take slices of 3 steps or more, which
        // on the shapes below makes them 4 steps (512 elements) long; rows of
        // 896 (7 steps) get two. At M = 8, slices of 4 steps against the
        // earlier 5-step floor: config 0 Q4_0 5632 x 2048 9.2 -> 8.5 us,
        // 2048 x 2048 9.0 -> 8.2, 256 x 2048 8.7 -> 7.6, Q8_0 4864 x 896
        // (unsliced before) 8.75 -> 8.14, 896 x 896 8.4 -> 7.8, 896 x 4864
        // 10.7 -> 10.4, Q5_0 5120 x 5120 and 1024 x 5120 unchanged (13.6,
        // 10.8); 2- and 3-step slices were slower on all but 896 x 896.
        if (L.type == T_F16)
            plan_slices(ctx, p, (p.Mp / BM) * NB, nk, NB, p.mt <= 4 ? 5 : 2,
                        p.mt <= 4 ? 3 * ctx->n_cu / 4 : 0);
        else
            plan_slices(ctx, p, (p.Mp / BM) * NB, nk, NB, p.mt == 1 ? 3 : 5,
                        (p.mt == 1 ? 2 : 3) * ctx->n_cu);
        // 16-row m blocks whose K slice holds at most two Q8_0 blocks of X
        // per thread: the launch quantizes X itself (gemmq_kernel XM 2), no
        // quantization launch before it. At M = 8: config 0 Q4_0 5632 x
        // 2048 (slices of 6 steps) 13.1 -> 9.2 us, config 4 Q5_0 5120 x 5120
        // and 1024 x 5120 (5 steps) 16.6 -> 13.7 and 13.4 -> 10.8; with 18-20
        // steps (2.3-2.5 blocks per thread, 27648 x 5120 and 5120 x 27648)
        // no faster than the separate launch (32.2 against 32.3, 35.7
        // against 35.1)
        p.fuseq = L.type != T_F16 && p.mt == 1 && gq_lds_bytes(16, p.SBK) <= kGQSliceLds &&
                  std::min<int64_t>(M, 16) * 4 * p.SBK <= 2 * kG2Threads &&
                  ctx->opt.gemmq_xmode != 0 && ctx->opt.gemmq_fuse != 0;
        // F16 in 16-row m blocks converts X as it stages each step's record
        // (a 4 KB record: one 32-byte f32 read per thread and step), with no
        // conversion launch before it
        if (L.type == T_F16) p.fuseq = p.mt == 1 && ctx->opt.gemmh_fuse != 0;
        return p;
    }
    // (Q4_K: gemm2s.h below, unless the GEMMKS_Q4K option is 1; on the
    // Llama-3-8B shapes at M = 8 it took 10.0 / 7.9 / 15.8 us per call for
    // 4096 / 1024 / 14336 x 4096 against 10.9 / 9.9 / 16.0 here)
    if (is_kquant(L.type) && M <= gemmks_max_m(ctx->opt, L.type) &&
        !(L.type == T_Q4_K && ctx->opt.gemmks_q4k != 1)) {
        // one 16-row record block, a workgroup per 32 weight rows whose
        // waves split the super-blocks, the near-GGUF-size copy (gemmks.h)
        p.v2 = true;
        p.small = true;
        p.mt = 1;
        p.Mp = 16;
        p.ws_bytes = nb * g2_rec_bytes(16);
        p.S = 1;
        p.SBK = (int)nb;
        p.steps = nb;
        p.part_bytes = 0;
        return p;
    }
    if (L.type == T_Q6_K) {
        // m blocks of 16, 32 or 64 rows (the GEMM_MT option, 1, 2 or 4,
        // overrides); K slices as plan_slices decides
        // (shorter m blocks while the output tiles would not reach a quarter
        // of the CUs: ffn_down 4096 x 14336 at M = 64 takes 41 us in 32-row
        // blocks against 48 us in 16-row ones, and 1024 x 4096 at M = 512
        // the same 24 us in 64- or 32-row blocks)
        p.v2 = true;
        p.mt = M <= 16 ? 1 : M <= 32 ? 2 : 4;
        while (p.mt > 1 && (M + 16 * p.mt - 1) / (16 * p.mt) * NB < ctx->n_cu / 4) p.mt /= 2;
        if (opt_mt == 1 || opt_mt == 2 || opt_mt == 4) p.mt = (int)opt_mt;
        const int64_t BM = 16 * p.mt;
        p.Mp = (M + BM - 1) / BM * BM;
        p.ws_bytes = p.Mp / BM * nb * g2_rec_bytes((int)BM);
        // K slices: with 16- and 32-row blocks (no operand decode, 2-byte
        // digits streamed) about one workgroup per CU is fastest (M = 8:
        // ffn_down 4096 x 14336 in 224 workgroups 25.6 us against 29.5 in
        // 448; 27648 x 5120 unsliced 48.4 against 54.8), with 64-row blocks
        // two (ffn_down at M = 512: 83.8 us in 512 against 107 in 256), at
        // least 4 super-blocks per slice (wv 1024 x 4096 at M = 512: 20.3 us
        // in 4 slices of 4 against 22.8 in 8 of 2)
        plan_slices(ctx, p, (p.Mp / BM) * NB, nb, NB, 4, p.mt <= 2 ? ctx->n_cu : 0);
        return p;
    }
    if (L.type == T_Q4_K && M <= gemm2s_max_m(ctx->opt)) {
        // one 16-row record block, a workgroup per 32 weight rows whose
        // waves split the super-blocks (gemm2s.h): no K slices
        p.v2 = true;
        p.small = true;
        p.q4s = true;
        p.mt = 1;
        p.Mp = 16;
        p.ws_bytes = nb * g2_rec_bytes(16);
        p.S = 1;
        p.SBK = (int)nb;
        p.steps = nb;
        p.part_bytes = 0;
        return p;
    }
    if (L.type == T_Q4_K && M >= gemm2_min_m(ctx->opt)) {
        // 128-row m blocks, shorter ones (64, 32 rows) while the output
        // tiles would not reach one per CU, then K slices (plan_slices); the
        // GEMM_MT option (2, 4 or 8) overrides. At M = 512: 4096 x 4096 in
        // 64-row blocks 35.0 us (128-row: 55.4), 1024 x 4096 in 32-row
        // blocks 21.2 us (128-row: 46.5).
        p.v2 = true;
        p.mt = 8;
        while (p.mt > 2 && (M + 16 * p.mt - 1) / (16 * p.mt) * NB < ctx->n_cu) p.mt /= 2;
        if (opt_mt == 2 || opt_mt == 4 || opt_mt == 8) p.mt = (int)opt_mt;
        const int64_t BM = 16 * p.mt;
        p.Mp = (M + BM - 1) / BM * BM;
        p.ws_bytes = p.Mp / BM * nb * g2_rec_bytes((int)BM);
        plan_slices(ctx, p, (p.Mp / BM) * NB, nb, NB);
        return p;
    }
    p.v2 = false;
    // small M: 32-row m tiles (twice the workgroups) with four super-blocks
    // of weights in flight per wave; the GEMM_MT option (1 or 2) overrides
    p.mt = M <= 128 ? 1 : 2;
    if (opt_mt > 0) p.mt = opt_mt == 1 ? 1 : 2;
    // Q5_K's fifth-bit words and bias term do not fit two 32-row tiles or
    // four super-blocks in flight in 256 VGPRs: 32-row tiles, two in flight
    if (L.type == T_Q5_K) p.mt = 1;
    const int64_t BM = 32 * p.mt;
    p.Mp = (M + BM - 1) / BM * BM;
    p.ws_bytes = gemm_x_bytes(p.Mp, K);
    // K slices when the output tiles alone would leave CUs idle (M <= 32
    // at the benchmark shapes: 112 tiles on 256 CUs), at least 4
    // super-blocks per slice, as many as keep within two workgroups per CU
    // (plan_slices; M = 8 ffn_down 5120 x 27648 in 480 workgroups: Q4_K
    // 30.7 us, Q5_K 32.3, Q2_K 25.5, against 39.0 / 43.3 / 30.8 in 280 and
    // 39.1 / 42.1 / 32.3 in 560). The partial sums cost a write and a read
    // of S x M x N floats, which outweighs the extra parallelism once the
    // tiles fill the chip (measured M = 64: 26.2 us unsliced, 32.3 us in 4
    // slices).
    plan_slices(ctx, p, (p.Mp / BM) * NB, nb, NB, 4);
    return p;
}

// Device buffers of one GEMM call: the activation planes, and for K slices
// the partial sums and the arrival counters (zero between calls). quant:
// the launch first writes the activation planes from X; false when an
// earlier launch on the stream wrote the same planes (several weights
// sharing one X and one record layout, sihip_gemm_multi_dev).
// xmode: the Q8_0-pair GEMM's record mode (gemmq_kernel XM; -1: its rule;
// the plan's fuseq takes mode 2).
struct GemmBufs {
    uint8_t *ws;
    float *part;
    uint32_t *cnt;
    bool quant = true;
    int xmode = -1;
    int q80s = 0;  // the scalar Q8_0 quantizer (Q80_SCALAR option)
};

// Y_i[m, :] = W_i x[m, :] for m < M on the matrix cores, for `count` Q4_K
// weights over one X in one grid (their n blocks one after another), with
// the workspaces in B (sized by plan_gemm for their n blocks together); the
// weights' GEMM copies must exist.
template <int MT, int W>
static hipError_t launch_gemm2_multi(int count, const sihip_weight *const *w, const GemmPlan &p,
                                     const GemmBufs &B, const float *X, int64_t ldx, int64_t M,
                                     float *const *Y, const int64_t *ldy, hipStream_t st) {
    uint8_t *ws = B.ws;
    constexpr int BM = 16 * MT;
    if (count < 1 || count > kG2MaxSegs) return hipErrorInvalidValue;
    const int64_t nb = w[0]->L.n_in / 256;
    const int64_t blocks = p.Mp * nb;
    if (B.quant)
        hipLaunchKernelGGL(gemm2_quantize_x<BM>, dim3((unsigned)gemm2_quantize_grid(blocks)),
                           dim3(kG2Threads), 0, st, X, ldx, M, p.Mp, nb, ws);
    G2Args A{};
    A.x = ws;
    A.M = M;
    A.Mp = p.Mp;
    A.nb = (int)nb;
    A.MB = (int)(p.Mp / BM);
    int NB = 0;
    for (int i = 0; i < count; i++) {
        G2Seg &g = A.seg[i];
        g.w = w[i]->gemm2;
        g.y = Y[i];
        g.ldy = ldy[i];
        g.n_out = w[i]->L.n_out;
        g.yscale = std::ldexp(1.0f, -w[i]->gexp);
        g.nb0 = NB;
        NB += (int)((w[i]->L.n_out + kG2BN - 1) / kG2BN);
    }
    A.nseg = count;
    A.NB = NB;
    A.S = p.S;
    A.SBK = p.SBK;
    A.part = p.S > 1 ? B.part : nullptr;
    A.cnt = p.S > 1 ? B.cnt : nullptr;
    const dim3 grid((unsigned)((int64_t)8 * ((A.NB + 7) / 8) * A.MB * A.S));
    hipLaunchKernelGGL((gemm2_q4k_kernel<MT, W>), grid, dim3(kG2Threads), 0, st, A);
    return hipGetLastError();
}

template <int MT, int W>
static hipError_t launch_gemm2(const sihip_weight *w, const GemmPlan &p, const GemmBufs &B,
                               const float *X, int64_t ldx, int64_t M, float *Y, int64_t ldy,
                               hipStream_t st) {
    return launch_gemm2_multi<MT, W>(1, &w, p, B, X, ldx, M, &Y, &ldy, st);
}

template <uint32_t FMT, int MT>
static hipError_t launch_gemmq(const sihip_weight *w, const GemmPlan &p, const GemmBufs &B,
                               const float *X, int64_t ldx, int64_t M, float *Y, int64_t ldy,
                               hipStream_t st) {
    constexpr int BM = 16 * MT;
    const Layout &L = w->L;
    const int64_t nk = L.n_in / 128;
    const int64_t threads = p.Mp * L.n_in / 32;
    constexpr int bias = FMT == T_Q4_0 ? 8 : FMT == T_Q5_0 ? 16 : 0;
    // record mode: with up to 32-row m blocks and a K slice whose records
    // fit kGQSliceLds, the slice's records go to LDS up front (mode 1: 2-7%
    // faster than the ring at M = 8-16, e.g. kv 1024 x 5120 13.1 against
    // 14.1 us per call). The GEMMQ_XMODE option 0 forces the ring.
    const int64_t lds = gq_lds_bytes(BM, p.SBK);
    int xm = MT <= 2 && lds <= kGQSliceLds ? 1 : 0;
    if (B.xmode == 0) xm = 0;
    const bool fused = MT == 1 && p.fuseq;
    if (B.quant && !fused)
        hipLaunchKernelGGL((gemmq_quantize_x<BM, bias>), dim3((unsigned)((threads + 255) / 256)),
                           dim3(256), 0, st, X, ldx, M, p.Mp, L.n_in, B.ws, B.q80s);
    GQArgs A{};
    A.q80s = B.q80s;
    A.w = w->gemm2;
    A.x = B.ws;
    A.y = Y;
    A.ldy = ldy;
    A.n_out = L.n_out;
    A.M = M;
    A.Mp = p.Mp;
    A.nk = (int)nk;
    A.MB = (int)(p.Mp / BM);
    A.NB = (int)((L.n_out + kG2BN - 1) / kG2BN);
    A.S = p.S;
    A.SBK = p.SBK;
    A.part = p.S > 1 ? B.part : nullptr;
    A.cnt = p.S > 1 ? B.cnt : nullptr;
    const int64_t cons = (int64_t)8 * ((A.NB + 7) / 8) * A.MB * A.S;
    if constexpr (MT == 1) {
        if (fused) {
            A.xf = X;
            A.ldx = ldx;
            hipLaunchKernelGGL((gemmq_kernel<FMT, MT, 2>), dim3((unsigned)cons), dim3(kG2Threads),
                               (unsigned)lds, st, A);
            return hipGetLastError();
        }
    }
    if constexpr (MT <= 2) {
        if (xm == 1) {
            hipLaunchKernelGGL((gemmq_kernel<FMT, MT, 1>), dim3((unsigned)cons), dim3(kG2Threads),
                               (unsigned)lds, st, A);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL((gemmq_kernel<FMT, MT, 0>), dim3((unsigned)cons), dim3(kG2Threads), 0, st, A);
    return hipGetLastError();
}

template <uint32_t FMT>
static hipError_t launch_gemmq_mt(const sihip_weight *w, const GemmPlan &p, const GemmBufs &B,
                                  const float *X, int64_t ldx, int64_t M, float *Y, int64_t ldy,
                                  hipStream_t st) {
    switch (p.mt) {
        case 1: return launch_gemmq<FMT, 1>(w, p, B, X, ldx, M, Y, ldy, st);
        case 2: return launch_gemmq<FMT, 2>(w, p, B, X, ldx, M, Y, ldy, st);
        default: return launch_gemmq<FMT, 4>(w, p, B, X, ldx, M, Y, ldy, st);
    }
}

template <int MT>
static hipError_t launch_gemmh(const sihip_weight *w, const GemmPlan &p, const GemmBufs &B,
                               const float *X, int64_t ldx, int64_t M, float *Y, int64_t ldy,
                               hipStream_t st) {
    constexpr int BM = 16 * MT;
    const Layout &L = w->L;
    const int64_t nk = L.n_in / 128;
    const int64_t threads = p.Mp * L.n_in / 8;
    const bool fused = MT == 1 && p.fuseq;
    if (B.quant && !fused)
        hipLaunchKernelGGL(gemmh_convert_x<BM>, dim3((unsigned)((threads + 255) / 256)), dim3(256),
                           0, st, X, ldx, M, p.Mp, L.n_in, B.ws);
    GHArgs A;
    A.w = w->gemm2;
    A.x = B.ws;
    A.y = Y;
    A.ldy = ldy;
    A.n_out = L.n_out;
    A.M = M;
    A.Mp = p.Mp;
    A.nk = (int)nk;
    A.MB = (int)(p.Mp / BM);
    A.NB = (int)((L.n_out + kG2BN - 1) / kG2BN);
    A.S = p.S;
    A.SBK = p.SBK;
    A.part = p.S > 1 ? B.part : nullptr;
    A.cnt = p.S > 1 ? B.cnt : nullptr;
    A.xf = fused ? X : nullptr;
    A.ldx = ldx;
    const dim3 grid((unsigned)((int64_t)8 * ((A.NB + 7) / 8) * A.MB * A.S));
    if (fused)
        hipLaunchKernelGGL((gemmh_f16_kernel<MT, true>), grid, dim3(kG2Threads), 0, st, A);
    else
        hipLaunchKernelGGL((gemmh_f16_kernel<MT, false>), grid, dim3(kG2Threads), 0, st, A);
    return hipGetLastError();
}

template <int MT>
static hipError_t launch_gemm6(const sihip_weight *w, const GemmPlan &p, const GemmBufs &B,
                               const float *X, int64_t ldx, int64_t M, float *Y, int64_t ldy,
                               hipStream_t st) {
    constexpr int BM = 16 * MT;
    const Layout &L = w->L;
    const int64_t nb = L.n_in / 256;
    const int64_t blocks = p.Mp * nb;
    if (B.quant)
        hipLaunchKernelGGL(gemm2_quantize_x<BM>, dim3((unsigned)gemm2_quantize_grid(blocks)),
                           dim3(kG2Threads), 0, st, X, ldx, M, p.Mp, nb, B.ws);
    G6Args A;
    A.w = w->gemm2;
    A.x = B.ws;
    A.y = Y;
    A.ldy = ldy;
    A.n_out = L.n_out;
    A.M = M;
    A.Mp = p.Mp;
    A.nb = (int)nb;
    A.MB = (int)(p.Mp / BM);
    A.NB = (int)((L.n_out + kG2BN - 1) / kG2BN);
    A.S = p.S;
    A.SBK = p.SBK;
    A.part = p.S > 1 ? B.part : nullptr;
    A.cnt = p.S > 1 ? B.cnt : nullptr;
    const dim3 grid((unsigned)((int64_t)8 * ((A.NB + 7) / 8) * A.MB * A.S));
    hipLaunchKernelGGL((gemm6_q6k_kernel<MT>), grid, dim3(kG2Threads), 0, st, A);
    return hipGetLastError();
}

template <uint32_t FMT, int NH>
static void launch_gemmks_nh(int kw, dim3 grid, hipStream_t st, const GKSArgs &A) {
    constexpr int SW = gemmks_sw<FMT, NH>();
    if (kw == 2)
        hipLaunchKernelGGL((gemmks_kernel<FMT, NH, 2, SW>), grid, dim3(128), 0, st, A);
    else if (kw == 4)
        hipLaunchKernelGGL((gemmks_kernel<FMT, NH, 4, SW>), grid, dim3(256), 0, st, A);
    else
        hipLaunchKernelGGL((gemmks_kernel<FMT, NH, 8, SW>), grid, dim3(512), 0, st, A);
}

// The small-M K-quant GEMM for M <= 4 nh activation rows.
template <uint32_t FMT>
static void launch_gemmks(int nh, int kw, dim3 grid, hipStream_t st, const GKSArgs &A) {
    switch (nh) {
        case 1: launch_gemmks_nh<FMT, 1>(kw, grid, st, A); break;
        case 2: launch_gemmks_nh<FMT, 2>(kw, grid, st, A); break;
        case 3: launch_gemmks_nh<FMT, 3>(kw, grid, st, A); break;
        default: launch_gemmks_nh<FMT, 4>(kw, grid, st, A); break;
    }
}

// Waves per workgroup of the small-M GEMMs (gemm2s.h, gemmks.h), which
// split a 32-row block's super-blocks: the most of 8, 4, 2 that keep the
// launch's waves within 10 per CU (about 2.5 per SIMD: two resident at the
// VGPRs these kernels use, so the workgroups run in little more than one
// round). M = 8, per call: Q2_K 27648 x 5120 (864 blocks) 23.6 us in 2
// waves, 25.4 in 4, 32.2 in 8; 5120 x 27648 (160 blocks) 28.5 in 8, 32.7
// in 4, 56.9 in 2; Q4_K 14336 x 4096 (448 blocks) 15.9 in 4 against 17.4
// in 8. Except for Q2_K (the smallest blocks), eight waves also need at
// least 8 super-blocks each: rows of 4096 and 5120 (16 and 20 per row) run
// faster in 4 (M = 8, per call: Llama-3-8B q/k/v 24.6 to 22.6 us, wo 10.1
// to 9.6; Q3_K 5120 x 5120 12.4 to 11.7, Q5_K 14.1 to 13.2; ffn_down, 56
// per row, 20.5 to 20.2), while Q2_K 5120 x 5120 is faster in 8 (11.8
// against 12.9). The Q4_K kernel of gemm2s.h has 4 and 8. The GEMMS_WAVES
// option (2, 4 or 8) overrides.
static int small_gemm_waves(const sihip_ctx *ctx, const Layout &L) {
    if (ctx->opt.gemms_waves == 2 || ctx->opt.gemms_waves == 4 || ctx->opt.gemms_waves == 8)
        return (int)ctx->opt.gemms_waves;
    const int64_t blocks = (L.n_out + 31) / 32, room = 10 * (int64_t)ctx->n_cu;
    if (blocks * 8 <= room && (L.type == T_Q2_K || L.n_in / 256 >= 64)) return 8;
    return blocks * 4 <= room ? 4 : 2;
}

static int launch_gemm_mfma(sihip_ctx *ctx, const sihip_weight *w, const GemmPlan &p,
                            const GemmBufs &B, const float *X, int64_t ldx, int64_t M, float *Y,
                            int64_t ldy, hipStream_t st) {
    const Layout &L = w->L;
    if (p.v2 && is_q80_pair(L.type)) {
        GemmBufs BQ = B;
        BQ.xmode = (int)ctx->opt.gemmq_xmode;
        BQ.q80s = ctx->opt.q80_scalar > 0;
        const hipError_t e =
            L.type == T_Q8_0   ? launch_gemmq_mt<T_Q8_0>(w, p, BQ, X, ldx, M, Y, ldy, st)
            : L.type == T_Q4_0 ? launch_gemmq_mt<T_Q4_0>(w, p, BQ, X, ldx, M, Y, ldy, st)
                               : launch_gemmq_mt<T_Q5_0>(w, p, BQ, X, ldx, M, Y, ldy, st);
        if (e != hipSuccess) return set_err(ctx, SIHIP_EDEVICE, "gemm launch: %s", hipGetErrorString(e));
        return SIHIP_OK;
    }
    if (p.v2 && L.type == T_F16) {
        hipError_t e;
        switch (p.mt) {
            case 1: e = launch_gemmh<1>(w, p, B, X, ldx, M, Y, ldy, st); break;
            case 2: e = launch_gemmh<2>(w, p, B, X, ldx, M, Y, ldy, st); break;
            case 4: e = launch_gemmh<4>(w, p, B, X, ldx, M, Y, ldy, st); break;
            default: e = launch_gemmh<8>(w, p, B, X, ldx, M, Y, ldy, st); break;
        }
        if (e != hipSuccess) return set_err(ctx, SIHIP_EDEVICE, "gemm launch: %s", hipGetErrorString(e));
        return SIHIP_OK;
    }
    if (p.v2 && p.small && !p.q4s) {
        const int64_t nb = L.n_in / 256;
        if (B.quant)
            hipLaunchKernelGGL(gemm2_quantize_x<16>, dim3((unsigned)gemm2_quantize_grid(16 * nb)),
                               dim3(kG2Threads), 0, st, X, ldx, M, (int64_t)16, nb, B.ws);
        GKSArgs A;
        A.w = w->gsmall;
        A.x = B.ws;
        A.y = Y;
        A.ldy = ldy;
        A.n_out = L.n_out;
        A.M = M;
        A.nb = (int)nb;
        const dim3 grid((unsigned)((L.n_out + 31) / 32));
        const int kw = small_gemm_waves(ctx, L);
        const int nh = (int)((M + 3) / 4);
        switch (L.type) {
            case T_Q2_K: launch_gemmks<T_Q2_K>(nh, kw, grid, st, A); break;
            case T_Q3_K: launch_gemmks<T_Q3_K>(nh, kw, grid, st, A); break;
            case T_Q4_K: launch_gemmks<T_Q4_K>(nh, kw, grid, st, A); break;
            case T_Q5_K: launch_gemmks<T_Q5_K>(nh, kw, grid, st, A); break;
            default: launch_gemmks<T_Q6_K>(nh, kw, grid, st, A); break;
        }
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return set_err(ctx, SIHIP_EDEVICE, "gemm launch: %s", hipGetErrorString(e));
        return SIHIP_OK;
    }
    if (p.v2 && L.type == T_Q6_K) {
        hipError_t e;
        switch (p.mt) {
            case 1: e = launch_gemm6<1>(w, p, B, X, ldx, M, Y, ldy, st); break;
            case 2: e = launch_gemm6<2>(w, p, B, X, ldx, M, Y, ldy, st); break;
            default: e = launch_gemm6<4>(w, p, B, X, ldx, M, Y, ldy, st); break;
        }
        if (e != hipSuccess) return set_err(ctx, SIHIP_EDEVICE, "gemm launch: %s", hipGetErrorString(e));
        return SIHIP_OK;
    }
    if (p.v2 && p.small) {
        const Layout &L = w->L;
        const int64_t nb = L.n_in / 256;
        if (B.quant)
            hipLaunchKernelGGL(gemm2_quantize_x<16>, dim3((unsigned)gemm2_quantize_grid(16 * nb)),
                               dim3(kG2Threads), 0, st, X, ldx, M, (int64_t)16, nb, B.ws);
        G2SArgs A;
        A.w = w->gemm2;
        A.x = B.ws;
        A.y = Y;
        A.ldy = ldy;
        A.n_out = L.n_out;
        A.M = M;
        A.nb = (int)nb;
        A.yscale = std::ldexp(1.0f, -w->gexp);
        const dim3 grid((unsigned)((L.n_out + 31) / 32));
        if (small_gemm_waves(ctx, L) < 8)
            hipLaunchKernelGGL(gemm2s_q4k_kernel<4>, grid, dim3(256), 0, st, A);
        else
            hipLaunchKernelGGL(gemm2s_q4k_kernel<8>, grid, dim3(512), 0, st, A);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return set_err(ctx, SIHIP_EDEVICE, "gemm launch: %s", hipGetErrorString(e));
        return SIHIP_OK;
    }
    if (p.v2) {
        hipError_t e;
        const bool w1 = ctx->opt.gemm2_waves == 1;
        switch (p.mt) {
            case 2: e = launch_gemm2<2, 2>(w, p, B, X, ldx, M, Y, ldy, st); break;
            case 4: e = w1 ? launch_gemm2<4, 1>(w, p, B, X, ldx, M, Y, ldy, st)
                           : launch_gemm2<4, 2>(w, p, B, X, ldx, M, Y, ldy, st); break;
            default: e = w1 ? launch_gemm2<8, 1>(w, p, B, X, ldx, M, Y, ldy, st)
                            : launch_gemm2<8, 2>(w, p, B, X, ldx, M, Y, ldy, st); break;
        }
        if (e != hipSuccess) return set_err(ctx, SIHIP_EDEVICE, "gemm launch: %s", hipGetErrorString(e));
        return SIHIP_OK;
    }
    const int64_t K = L.n_in, nb = K / 256;
    const int NB = (int)((L.n_out + kGemmBN - 1) / kGemmBN);
    const int64_t BM = 32 * p.mt, Mp = p.Mp;
    GemmX XP;
    XP.q = (int8_t *)B.ws;
    XP.d = (float *)(B.ws + Mp * K);
    XP.bs = (_Float16 *)(B.ws + Mp * K + nb * Mp * 4);
    const int64_t blocks = Mp * nb;
    if (B.quant)
        hipLaunchKernelGGL(gemm_quantize_x, dim3((unsigned)((blocks + 15) / 16)), dim3(kGemmThreads),
                           0, st, X, ldx, M, Mp, nb, XP);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_err(ctx, SIHIP_EDEVICE, "gemm quantize: %s", hipGetErrorString(e));
    GemmArgs A;
    A.w = w->gemm;
    A.n_out = L.n_out;
    A.nb = nb;
    A.M = M;
    A.Mp = Mp;
    A.X = XP;
    A.y = Y;
    A.ldy = ldy;
    A.MB = (int)(Mp / BM);
    A.NB = NB;
    A.S = p.S;
    A.SBK = p.SBK;
    A.part = p.S > 1 ? B.part : nullptr;
    A.cnt = p.S > 1 ? B.cnt : nullptr;
    const dim3 grid((unsigned)((int64_t)8 * ((A.NB + 7) / 8) * A.MB * A.S));
    const int mt = p.mt;
    if (L.type == T_Q5_K) {
        hipLaunchKernelGGL((gemm_kq_kernel<T_Q5_K, 1, 2>), grid, dim3(kGemmThreads), 0, st, A);
    } else if (L.type == T_Q3_K) {
        if (mt == 1)
            hipLaunchKernelGGL((gemm_kq_kernel<T_Q3_K, 1, 4>), grid, dim3(kGemmThreads), 0, st, A);
        else
            hipLaunchKernelGGL((gemm_kq_kernel<T_Q3_K, 2, 2>), grid, dim3(kGemmThreads), 0, st, A);
    } else if (L.type == T_Q2_K) {
        if (mt == 1)
            hipLaunchKernelGGL((gemm_kq_kernel<T_Q2_K, 1, 4>), grid, dim3(kGemmThreads), 0, st, A);
        else
            hipLaunchKernelGGL((gemm_kq_kernel<T_Q2_K, 2, 2>), grid, dim3(kGemmThreads), 0, st, A);
    } else {
        if (mt == 1)
            hipLaunchKernelGGL((gemm_kq_kernel<T_Q4_K, 1, 4>), grid, dim3(kGemmThreads), 0, st, A);
        else
            hipLaunchKernelGGL((gemm_kq_kernel<T_Q4_K, 2, 2>), grid, dim3(kGemmThreads), 0, st, A);
    }
    e = hipGetLastError();
    if (e != hipSuccess) return set_err(ctx, SIHIP_EDEVICE, "gemm launch: %s", hipGetErrorString(e));
    return SIHIP_OK;
}

// The GEMM copy a plan's kernel reads: the small-M Q6_K copy, the 16x16
// kernels' copy or the 32-row K-quant GEMM's copy.
static const uint8_t *plan_copy(const sihip_weight *w, const GemmPlan &p) {
    if (p.small && !(w->L.type == T_Q4_K && p.q4s)) return w->gsmall;
    return p.v2 ? w->gemm2 : w->gemm;
}

static int build_plan_copy(sihip_ctx *ctx, sihip_weight *w, const GemmPlan &p, hipStream_t st) {
    if (plan_copy(w, p)) return SIHIP_OK;
    if (p.small && !(w->L.type == T_Q4_K && p.q4s)) return build_gemmks_copy(ctx, w, st);
    return p.v2 ? build_gemm2_copy(ctx, w, st) : build_gemm_copy(ctx, w, st);
}

// ---- the fused small-M K-quant launch (gemmkf.h) ------------------------------

template <uint32_t F0, uint32_t F1>
static void launch_gemmkf_nh(int nh, dim3 grid, size_t lds, hipStream_t st, const GKFArgs &A) {
    if (nh == 1)
        hipLaunchKernelGGL((gemmkf_kernel<F0, F1, 1>), grid, dim3(kKFThreads), lds, st, A);
    else
        hipLaunchKernelGGL((gemmkf_kernel<F0, F1, 2>), grid, dim3(kKFThreads), lds, st, A);
}

// The instances: one format, or the pairs of the K-quant mixes whose
// matrices share an activation (Q4_K_M and Q5_K_M put Q6_K beside Q4_K or
// Q5_K, Q3_K_M Q5_K beside Q3_K, Q2_K Q3_K beside Q2_K). false: no instance.
static bool launch_gemmkf(uint32_t t0, uint32_t t1, int nh, dim3 grid, size_t lds, hipStream_t st,
                          const GKFArgs &A) {
    if (t0 > t1) std::swap(t0, t1);
    if (t0 == t1) {
        switch (t0) {
            case T_Q2_K: launch_gemmkf_nh<T_Q2_K, T_Q2_K>(nh, grid, lds, st, A); return true;
            case T_Q3_K: launch_gemmkf_nh<T_Q3_K, T_Q3_K>(nh, grid, lds, st, A); return true;
            case T_Q4_K: launch_gemmkf_nh<T_Q4_K, T_Q4_K>(nh, grid, lds, st, A); return true;
            case T_Q5_K: launch_gemmkf_nh<T_Q5_K, T_Q5_K>(nh, grid, lds, st, A); return true;
            case T_Q6_K: launch_gemmkf_nh<T_Q6_K, T_Q6_K>(nh, grid, lds, st, A); return true;
            default: return false;
        }
    }
    static_assert(T_Q2_K < T_Q3_K && T_Q3_K < T_Q4_K && T_Q4_K < T_Q5_K && T_Q5_K < T_Q6_K,
                  "pairs below are listed in type order");
    if (t0 == T_Q4_K && t1 == T_Q6_K) launch_gemmkf_nh<T_Q4_K, T_Q6_K>(nh, grid, lds, st, A);
    else if (t0 == T_Q5_K && t1 == T_Q6_K) launch_gemmkf_nh<T_Q5_K, T_Q6_K>(nh, grid, lds, st, A);
    else if (t0 == T_Q3_K && t1 == T_Q5_K) launch_gemmkf_nh<T_Q3_K, T_Q5_K>(nh, grid, lds, st, A);
    else if (t0 == T_Q2_K && t1 == T_Q3_K) launch_gemmkf_nh<T_Q2_K, T_Q3_K>(nh, grid, lds, st, A);
    else return false;
    return true;
}

// Tiles of one segment: kKFWaves 32-row blocks each.
static int64_t gemmkf_tiles(const Layout &L) {
    return ((L.n_out + 31) / 32 + kKFWaves - 1) / kKFWaves;
}

// Whether weights over one X take the fused launch: K-quants of one row
// length, M on the matrix cores and at most gemmkf_max_m. Q3_K matrices of
// at least 128 tiles (16384 rows) whose rows hold at most 32 super-blocks
// stay on the separate quantization and gemmks.h launches, which need no K
// slices there (config 4 ffn_up 27648 x 5120 at M = 8: 25.6 us against 28.8
// fused); smaller ones and longer rows are faster fused (attn 5120 x 5120
// 11.05 against 11.46, kv 1024 x 5120 9.6 against 10.45, ffn_down
// 5120 x 27648 27.8 against 28.1). Q3_K keeps the four-way masked operand
// there (its scaled 3-bit operand does not fit an int8), whose scale
// arithmetic per result needs many rows in flight.
static bool gemmkf_eligible(const sihip_ctx *ctx, int count, const sihip_weight *const *w,
                            int64_t M) {
    if (count < 1 || M < gemm_min_m(ctx->opt) || M > gemmkf_max_m(ctx->opt)) return false;
    for (int i = 0; i < count; i++) {
        const Layout &L = w[i]->L;
        if (!is_kquant(L.type) || L.n_in != w[0]->L.n_in || L.n_in % 256) return false;
        if (L.type == T_Q3_K && L.n_in / 256 <= 32 && gemmkf_tiles(L) >= 128 &&
            ctx->opt.gemmkf_max_m < 0)
            return false;
    }
    return true;
}

// K slices of a fused launch over `tiles` tiles: as many as keep the grid
// within one workgroup per CU, or within two where one per CU would leave
// slices of more than 16 super-blocks; at least two super-blocks each (a
// slice's fixed cost, its partial sums and the last workgroup's sum,
// outweighs one super-block: Llama-3-8B wo 4096 x 4096 at M = 8 takes 10.4
// us per call in 16 slices of one, 7.7 in 8 of two, 8.1 in 4 of four), and
// at most kKFMaxSBK super-blocks per slice (its LDS image); the GEMMKF_SBK
// option sets the slice length (0: the fewest slices). Measured at M = 8
// with the partial tiles in register order: one workgroup per CU against
// two, q/k/v 10.3 against 10.8 us (4 slices against 8), gate + up 17.6
// against 18.2 (no slices against 2), ffn_down 15.9 against 17.5 (8 slices
// against 14), config 4 attn 5120 x 5120 Q2_K 8.6 against 10.5; the 108
// super-blocks of config 4's 5120 x 27648 ffn_down in 6 slices of 18 took
// 21.6 against 19.8 us in 12 of 9 (Q2_K), hence two per CU past 16.
static void gemmkf_slices(const sihip_ctx *ctx, int64_t tiles, int64_t nb, int &S, int &SBK) {
    const int64_t t = tiles > 0 ? tiles : 1;
    auto slices = [&](int64_t per_cu) {
        int64_t v = per_cu * (int64_t)ctx->n_cu / t;
        if (v < 1) v = 1;
        if (v > (nb + 1) / 2) v = (nb + 1) / 2;
        return v;
    };
    int64_t s = slices(1);
    if ((nb + s - 1) / s > 16) s = slices(2);
    int64_t sbk = (nb + s - 1) / s;
    if (ctx->opt.gemmkf_sbk == 0) sbk = nb;
    else if (ctx->opt.gemmkf_sbk > 0) sbk = ctx->opt.gemmkf_sbk;
    if (sbk > kKFMaxSBK) sbk = kKFMaxSBK;
    if (sbk > nb) sbk = nb;
    SBK = (int)sbk;
    S = (int)((nb + sbk - 1) / sbk);
}

// One fused launch (every weight's gemmks.h copy exists, at most two
// formats with an instance, count <= kKFMaxSegs); the partial sums and
// counters were sized by the caller.
static int launch_gemmkf_group(sihip_ctx *ctx, int count, const sihip_weight *const *w,
                               const float *X, int64_t M, float *const *Y, float *part,
                               uint32_t *cnt, hipStream_t st, bool &done) {
    done = false;
    const int64_t nb = w[0]->L.n_in / 256;
    int64_t tiles = 0;
    for (int i = 0; i < count; i++) tiles += gemmkf_tiles(w[i]->L);
    int S, SBK;
    gemmkf_slices(ctx, tiles, nb, S, SBK);
    GKFArgs A{};
    A.x = X;
    A.ldx = w[0]->L.n_in;
    A.M = M;
    A.nb = (int)nb;
    A.nseg = count;
    uint32_t t0 = w[0]->L.type, t1 = t0;
    int64_t wg = 0, pofs = 0, cofs = 0;
    for (int i = 0; i < count; i++) {
        const Layout &L = w[i]->L;
        if (L.type != t0) {
            if (t1 != t0 && L.type != t1) return SIHIP_OK;  // a third format: not done
            t1 = L.type;
        }
        GKFSeg &g = A.seg[i];
        g.w = w[i]->gsmall;
        g.y = Y[i];
        g.ldy = L.n_out;
        g.n_out = L.n_out;
        g.type = L.type;
        g.nblk = (int)((L.n_out + 31) / 32);
        g.ntile = (int)gemmkf_tiles(L);
        g.S = S;
        g.SBK = SBK;
        g.wg0 = (int)wg;
        g.part = S > 1 ? part + pofs : nullptr;
        g.cnt = S > 1 ? cnt + cofs : nullptr;
        wg += (int64_t)g.ntile * S;
        pofs += (int64_t)S * kKFMp * g.ntile * kKFRows;
        cofs += g.ntile;
    }
    const size_t lds = (size_t)SBK * kKFRec;
    if (!launch_gemmkf(t0, t1, (int)((M + 3) / 4), dim3((unsigned)wg), lds, st, A)) return SIHIP_OK;
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_err(ctx, SIHIP_EDEVICE, "gemm launch: %s", hipGetErrorString(e));
    done = true;
    return SIHIP_OK;
}

// Weights over one X on the fused launch: one launch for all of them where
// their formats have an instance, else one per format (each quantizes X
// itself). Copies are built on first use and the partial sums grown as
// needed (outside graph capture).
static int run_gemmkf(sihip_ctx *ctx, int count, const sihip_weight *const *wc, const float *X,
                      int64_t M, float *const *Y, hipStream_t st) {
    const int64_t nb = wc[0]->L.n_in / 256;
    size_t part = 0;
    int64_t counters = 0;
    for (int i = 0; i < count; i++) {
        sihip_weight *w = const_cast<sihip_weight *>(wc[i]);  // the GEMM copies are caches of w
        if (!w->gsmall) {
            const int rc = build_gemmks_copy(ctx, w, st);
            if (rc) return rc;
        }
    }
    // partial sums: a segment's slices in any launch are at most those of a
    // launch of that segment alone (fewer tiles, more slices)
    for (int i = 0; i < count; i++) {
        const int64_t t = gemmkf_tiles(wc[i]->L);
        int S, SBK;
        gemmkf_slices(ctx, t, nb, S, SBK);
        part += (size_t)S * kKFMp * t * kKFRows * sizeof(float);
        counters += t;
    }
    if (counters > kGemmCounters)
        return set_err(ctx, SIHIP_EINVAL, "gemm: %lld output tiles exceed the %lld counters",
                       (long long)counters, (long long)kGemmCounters);
    int rc = ensure(ctx, &ctx->d_gpart, &ctx->d_gpart_cap, part, st);
    if (rc) return rc;
    rc = order_before(ctx, ctx->order, st);
    if (rc) return rc;
    bool done = false;
    rc = launch_gemmkf_group(ctx, count, wc, X, M, Y, (float *)ctx->d_gpart, ctx->d_gcnt, st, done);
    if (rc) return rc;
    if (!done) {  // one launch per format
        bool used[kKFMaxSegs] = {};
        for (int i = 0; i < count; i++) {
            if (used[i]) continue;
            const sihip_weight *gw[kKFMaxSegs];
            float *gy[kKFMaxSegs];
            int n = 0;
            for (int j = i; j < count; j++)
                if (!used[j] && wc[j]->L.type == wc[i]->L.type) {
                    used[j] = true;
                    gw[n] = wc[j];
                    gy[n] = Y[j];
                    n++;
                }
            rc = launch_gemmkf_group(ctx, n, gw, X, M, gy, (float *)ctx->d_gpart, ctx->d_gcnt, st,
                                     done);
            if (rc) return rc;
            if (!done) return set_err(ctx, SIHIP_EINVAL, "gemm: no fused instance for a format");
        }
    }
    return order_after(ctx, ctx->order, st);
}

// The MFMA GEMM on the context's workspaces (grown as needed, outside
// graph capture) and the weight's GEMM copy (built on first use). The
// activation planes live in the context, so calls on one context must not
// overlap.
static int run_gemm_mfma(sihip_ctx *ctx, const sihip_weight *wc, const float *X, int64_t ldx,
                         int64_t M, float *Y, int64_t ldy, hipStream_t st) {
    if (ldx == wc->L.n_in && ldy == wc->L.n_out && gemmkf_eligible(ctx, 1, &wc, M))
        return run_gemmkf(ctx, 1, &wc, X, M, &Y, st);
    sihip_weight *w = const_cast<sihip_weight *>(wc);  // the GEMM copies are caches of w
    const GemmPlan p = plan_gemm(ctx, w->L, M);
    int rc = build_plan_copy(ctx, w, p, st);
    if (rc) return rc;
    rc = ensure(ctx, &ctx->d_ws, &ctx->d_ws_cap, (size_t)p.ws_bytes, st);
    if (rc) return rc;
    if (p.S > 1) {
        rc = ensure(ctx, &ctx->d_gpart, &ctx->d_gpart_cap, (size_t)p.part_bytes, st);
        if (rc) return rc;
    }
    rc = order_before(ctx, ctx->order, st);
    if (rc) return rc;
    const GemmBufs B{(uint8_t *)ctx->d_ws, (float *)ctx->d_gpart, ctx->d_gcnt};
    rc = launch_gemm_mfma(ctx, w, p, B, X, ldx, M, Y, ldy, st);
    if (rc) return rc;
    return order_after(ctx, ctx->order, st);
}

// The activation records a plan's launch writes, as a key: launches with
// equal keys over the same X write identical planes. Families: the 32-row
// K-quant GEMM (Q8_K planes of Mp rows), the 16x16 Q4_K and Q6_K GEMMs (Q8_K
// records of BM rows), the Q8_0-pair GEMM (Q8_0 records of BM rows with the
// format's bias) and the F16 GEMM (f16 records of BM rows).
struct XKey {
    int fam;
    int64_t bm;
    int bias;
    bool operator==(const XKey &o) const { return fam == o.fam && bm == o.bm && bias == o.bias; }
};
static XKey xkey(const Layout &L, const GemmPlan &p) {
    if (!p.v2) return XKey{0, 32 * p.mt, 0};
    if (L.type == T_F16) return XKey{3, 16 * p.mt, 0};
    if (is_q80_pair(L.type))
        return XKey{2, 16 * p.mt, L.type == T_Q4_0 ? 8 : L.type == T_Q5_0 ? 16 : 0};
    return XKey{1, 16 * p.mt, 0};
}

// The MFMA GEMMs of several weights over one X: the weights of one record
// family get one m-tile count (the largest of their own plans that each
// kernel has), so X is quantized once per distinct record layout and the
// launches after the first of a layout read its planes.
static int run_gemm_multi(sihip_ctx *ctx, int count, const sihip_weight *const *wc,
                          const float *X, int64_t M, float *const *Y, hipStream_t st) {
    if (count <= kKFMaxSegs && gemmkf_eligible(ctx, count, wc, M))
        return run_gemmkf(ctx, count, wc, X, M, Y, st);
    // the Q4_K weights on the 16x16 kernel (M >= gemm2_min_m) share one
    // launch, planned as one matrix of their n blocks together (the
    // GEMM_GROUP option at 0 turns this off)
    bool grp[kMaxSegs] = {};
    int ngrp = 0;
    Layout Lg{};
    if (M >= gemm2_min_m(ctx->opt) && ctx->opt.gemm_group != 0) {
        int64_t nblk = 0;
        for (int i = 0; i < count; i++)
            if (wc[i]->L.type == T_Q4_K && ngrp < kG2MaxSegs) {
                grp[i] = true;
                if (ngrp++ == 0) Lg = wc[i]->L;
                nblk += (wc[i]->L.n_out + kG2BN - 1) / kG2BN;
            }
        Lg.n_out = nblk * kG2BN;
        if (ngrp < 2) {
            for (int i = 0; i < count; i++) grp[i] = false;
            ngrp = 0;
        }
    }
    auto plan_of = [&](int i, int force_mt) {
        return grp[i] ? plan_gemm(ctx, Lg, M, force_mt) : plan_gemm(ctx, wc[i]->L, M, force_mt);
    };
    GemmPlan plan[kMaxSegs];
    XKey key[kMaxSegs];
    for (int i = 0; i < count; i++) {
        plan[i] = plan_of(i, 0);
        key[i] = xkey(wc[i]->L, plan[i]);
    }
    for (int i = 0; i < count; i++) {
        int mt = plan[i].mt;
        for (int j = 0; j < count; j++)
            if (key[j].fam == key[i].fam && plan[j].mt > mt) mt = plan[j].mt;
        if (mt != plan[i].mt) {
            const GemmPlan q = plan_of(i, mt);
            if (q.mt == mt && q.v2 == plan[i].v2) {
                plan[i] = q;
                key[i] = xkey(wc[i]->L, q);
            }
        }
    }
    if (ngrp) {  // the group's plan is the 16x16 kernel's, the same for every member
        int g0 = 0;
        while (!grp[g0]) g0++;
        if (!plan[g0].v2 || plan[g0].small || plan[g0].mt < 2) {
            for (int i = 0; i < count; i++) grp[i] = false;
            ngrp = 0;
            for (int i = 0; i < count; i++) {
                plan[i] = plan_gemm(ctx, wc[i]->L, M);
                key[i] = xkey(wc[i]->L, plan[i]);
            }
        }
    }
    // a launch that quantizes X itself writes no planes: its key is its own,
    // so no later launch of its record layout counts on them
    for (int i = 0; i < count; i++)
        if (plan[i].fuseq) key[i] = XKey{100 + i, 0, 0};
    // one planes buffer per distinct key, 256-byte aligned, one after another
    size_t off[kMaxSegs], total = 0, part = 0;
    bool first[kMaxSegs];
    for (int i = 0; i < count; i++) {
        first[i] = true;
        for (int j = 0; j < i; j++)
            if (key[j] == key[i]) {
                first[i] = false;
                off[i] = off[j];
                break;
            }
        if (first[i]) {
            off[i] = total;
            total += ((size_t)plan[i].ws_bytes + 255) & ~(size_t)255;
        }
        if (plan[i].S > 1 && (size_t)plan[i].part_bytes > part) part = (size_t)plan[i].part_bytes;
    }
    for (int i = 0; i < count; i++) {
        sihip_weight *w = const_cast<sihip_weight *>(wc[i]);  // GEMM copies are caches of w
        const int rc = build_plan_copy(ctx, w, plan[i], st);
        if (rc) return rc;
    }
    int rc = ensure(ctx, &ctx->d_ws, &ctx->d_ws_cap, total, st);
    if (rc) return rc;
    if (part) {
        rc = ensure(ctx, &ctx->d_gpart, &ctx->d_gpart_cap, part, st);
        if (rc) return rc;
    }
    rc = order_before(ctx, ctx->order, st);
    if (rc) return rc;
    bool grp_done = false;
    for (int i = 0; i < count; i++) {
        GemmBufs B{(uint8_t *)ctx->d_ws + off[i], (float *)ctx->d_gpart, ctx->d_gcnt};
        B.quant = first[i];
        if (grp[i]) {
            if (grp_done) continue;
            grp_done = true;
            const sihip_weight *gw[kG2MaxSegs];
            float *gy[kG2MaxSegs];
            int64_t gld[kG2MaxSegs];
            int n = 0;
            for (int j = i; j < count; j++)
                if (grp[j]) {
                    gw[n] = wc[j];
                    gy[n] = Y[j];
                    gld[n] = wc[j]->L.n_out;
                    n++;
                }
            const bool w1 = ctx->opt.gemm2_waves == 1;
            const int64_t ldx = wc[i]->L.n_in;
            hipError_t e;
            switch (plan[i].mt) {
                case 2: e = launch_gemm2_multi<2, 2>(n, gw, plan[i], B, X, ldx, M, gy, gld, st); break;
                case 4: e = w1 ? launch_gemm2_multi<4, 1>(n, gw, plan[i], B, X, ldx, M, gy, gld, st)
                               : launch_gemm2_multi<4, 2>(n, gw, plan[i], B, X, ldx, M, gy, gld, st); break;
                default: e = w1 ? launch_gemm2_multi<8, 1>(n, gw, plan[i], B, X, ldx, M, gy, gld, st)
                                : launch_gemm2_multi<8, 2>(n, gw, plan[i], B, X, ldx, M, gy, gld, st); break;
            }
            if (e != hipSuccess) return set_err(ctx, SIHIP_EDEVICE, "gemm launch: %s", hipGetErrorString(e));
            continue;
        }
        rc = launch_gemm_mfma(ctx, wc[i], plan[i], B, X, wc[i]->L.n_in, M, Y[i], wc[i]->L.n_out, st);
        if (rc) return rc;
    }
    return order_after(ctx, ctx->order, st);
}

// Prefill dispatch: MFMA GEMM where supported and M is large enough,
// otherwise the matvec kernel over column groups.
static bool gemm_on_mfma(const sihip_ctx *ctx, const sihip_weight *w, int64_t M) {
    if (!gemm_mfma_supported(w->L)) return false;
    if (w->L.type == T_Q6_K) return M >= gemm6_min_m(ctx->opt);
    if (w->L.type == T_F16) return M >= gemmh_min_m(ctx->opt);
    if (is_q80_pair(w->L.type)) return M >= gemmq_min_m(ctx->opt);
    return M >= gemm_min_m(ctx->opt);
}

static int run_gemm(sihip_ctx *ctx, const sihip_weight *w, const float *X, int64_t M, float *Y,
                    hipStream_t st) {
    if (gemm_on_mfma(ctx, w, M)) return run_gemm_mfma(ctx, w, X, w->L.n_in, M, Y, w->L.n_out, st);
    return run_matvec(ctx, w, X, w->L.n_in, nullptr, 0, M, Y, w->L.n_out, w->L.n_out, st);
}

// ---- dequantized rows --------------------------------------------------------------

static hipError_t launch_dequant(const Layout &L, const uint8_t *w, int64_t row0, int64_t nrows,
                                 float *out, int64_t ldo, hipStream_t st) {
    if (L.type == T_F32) {
        hipLaunchKernelGGL(f32_rows_kernel, dim3((unsigned)((nrows * L.n_in + kF32Threads - 1) / kF32Threads)),
                           dim3(kF32Threads), 0, st, (const float *)w, L.n_in, row0, nrows, out, ldo);
        return hipGetLastError();
    }
    const dim3 grid((unsigned)((nrows * L.ncols + kThreads - 1) / kThreads)), block(kThreads);
    switch (L.type) {
        case T_F16: hipLaunchKernelGGL(dequant_rows_kernel<T_F16>, grid, block, 0, st, L, w, row0, nrows, out, ldo); break;
        case T_Q4_0: hipLaunchKernelGGL(dequant_rows_kernel<T_Q4_0>, grid, block, 0, st, L, w, row0, nrows, out, ldo); break;
        case T_Q5_0: hipLaunchKernelGGL(dequant_rows_kernel<T_Q5_0>, grid, block, 0, st, L, w, row0, nrows, out, ldo); break;
        case T_Q8_0: hipLaunchKernelGGL(dequant_rows_kernel<T_Q8_0>, grid, block, 0, st, L, w, row0, nrows, out, ldo); break;
        case T_Q2_K: hipLaunchKernelGGL(dequant_rows_kernel<T_Q2_K>, grid, block, 0, st, L, w, row0, nrows, out, ldo); break;
        case T_Q3_K: hipLaunchKernelGGL(dequant_rows_kernel<T_Q3_K>, grid, block, 0, st, L, w, row0, nrows, out, ldo); break;
        case T_Q4_K: hipLaunchKernelGGL(dequant_rows_kernel<T_Q4_K>, grid, block, 0, st, L, w, row0, nrows, out, ldo); break;
        case T_Q5_K: hipLaunchKernelGGL(dequant_rows_kernel<T_Q5_K>, grid, block, 0, st, L, w, row0, nrows, out, ldo); break;
        case T_Q6_K: hipLaunchKernelGGL(dequant_rows_kernel<T_Q6_K>, grid, block, 0, st, L, w, row0, nrows, out, ldo); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ---- calibration -------------------------------------------------------------------

// Streaming read: a grid-stride loop over 16-byte words with the
// nontemporal hint (as the matvec's weight loads), four loads in flight per
// thread, the words folded by xor; the fold is stored only when it hits a
// fixed value, so the reads cannot be dropped and nothing else is written.
__global__ __launch_bounds__(256) void probe_read_kernel(const uint4 *p, int64_t n16,
                                                         uint32_t *sink) {
    typedef unsigned int v4u_t __attribute__((ext_vector_type(4)));
    const v4u_t *q = reinterpret_cast<const v4u_t *>(p);
    const int64_t stride = (int64_t)gridDim.x * 256;
    int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    v4u_t acc = {0, 0, 0, 0};
    for (; i + 3 * stride < n16; i += 4 * stride) {
        const v4u_t a = __builtin_nontemporal_load(q + i);
        const v4u_t b = __builtin_nontemporal_load(q + i + stride);
        const v4u_t c = __builtin_nontemporal_load(q + i + 2 * stride);
        const v4u_t d = __builtin_nontemporal_load(q + i + 3 * stride);
        acc ^= a ^ b ^ c ^ d;
    }
    for (; i < n16; i += stride) acc ^= __builtin_nontemporal_load(q + i);
    const uint32_t f = acc.x ^ acc.y ^ acc.z ^ acc.w;
    if (f == 0x5eed1e55u) sink[blockIdx.x] = f;
}

extern "C" int sihip_probe_read_dev(sihip_ctx *ctx, const void *p, uint64_t bytes, uint32_t *sink,
                                    void *stream) {
    if (!ctx || !p || !sink) return set_err(ctx, SIHIP_EINVAL, "probe_read_dev: NULL argument");
    if (bytes == 0 || bytes % 16 || !aligned16(p))
        return set_err(ctx, SIHIP_EINVAL, "probe_read_dev: p and bytes must be 16-byte aligned");
    HIP_OK(ctx, hipSetDevice(ctx->device));
    const int64_t n16 = (int64_t)(bytes / 16);
    // at least four words per thread, at most 8 workgroups per CU (and the
    // 4096 words of sink)
    int64_t wg = (n16 + 1023) / 1024;
    const int64_t cap = std::min<int64_t>(8 * (int64_t)ctx->n_cu, 4096);
    if (wg > cap) wg = cap;
    hipLaunchKernelGGL(probe_read_kernel, dim3((unsigned)wg), dim3(256), 0, (hipStream_t)stream,
                       (const uint4 *)p, n16, sink);
    HIP_OK(ctx, hipGetLastError());
    return SIHIP_OK;
}

extern "C" int sihip_dequant_rows_dev(sihip_ctx *ctx, const sihip_weight *w, uint64_t row0,
                                      uint64_t nrows, float *out, int64_t ldo, void *stream) {
    if (!ctx || !w || !out) return set_err(ctx, SIHIP_EINVAL, "dequant_rows_dev: NULL argument");
    if (nrows == 0 || row0 >= (uint64_t)w->L.n_out || nrows > (uint64_t)w->L.n_out - row0)
        return set_err(ctx, SIHIP_EINVAL, "dequant_rows_dev: rows %llu..%llu outside 0..%lld",
                       (unsigned long long)row0, (unsigned long long)(row0 + nrows),
                       (long long)w->L.n_out);
    if (ldo < w->L.n_in || ldo % 4 != 0 || !aligned16(out))
        return set_err(ctx, SIHIP_EINVAL,
                       "dequant_rows_dev: out must be 16-byte aligned with a row stride of at "
                       "least n_in, a multiple of 4");
    HIP_OK(ctx, hipSetDevice(ctx->device));
    const hipError_t e =
        launch_dequant(w->L, w->dev, (int64_t)row0, (int64_t)nrows, out, ldo, (hipStream_t)stream);
    if (e != hipSuccess) return set_err(ctx, SIHIP_EDEVICE, "dequant launch: %s", hipGetErrorString(e));
    return SIHIP_OK;
}

extern "C" int sihip_dequant_row(sihip_ctx *ctx, const sihip_weight *w, uint64_t row, float *out) {
    if (!ctx || !w || !out) return set_err(ctx, SIHIP_EINVAL, "dequant_row: NULL argument");
    if (row >= (uint64_t)w->L.n_out)
        return set_err(ctx, SIHIP_EINVAL, "dequant_row: row %llu outside 0..%lld",
                       (unsigned long long)row, (long long)w->L.n_out - 1);
    HIP_OK(ctx, hipSetDevice(ctx->device));
    const size_t ob = (size_t)w->L.n_in * 4;
    const int rc = ensure(ctx, &ctx->d_out, &ctx->d_out_cap, ob);
    if (rc) return rc;
    const hipError_t e = launch_dequant(w->L, w->dev, (int64_t)row, 1, (float *)ctx->d_out,
                                        w->L.n_in, ctx->stream);
    if (e != hipSuccess) return set_err(ctx, SIHIP_EDEVICE, "dequant launch: %s", hipGetErrorString(e));
    HIP_OK(ctx, hipMemcpyAsync(out, ctx->d_out, ob, hipMemcpyDeviceToHost, ctx->stream));
    HIP_OK(ctx, hipStreamSynchronize(ctx->stream));
    return SIHIP_OK;
}

extern "C" int sihip_gemv_dev(sihip_ctx *ctx, const sihip_weight *w, const float *x, float *y,
                              int64_t n_out, void *stream) {
    if (!ctx || !w || !x || !y) return set_err(ctx, SIHIP_EINVAL, "gemv_dev: NULL argument");
    if (n_out <= 0 || n_out > w->L.n_out)
        return set_err(ctx, SIHIP_EINVAL, "gemv_dev: n_out %lld outside 1..%lld",
                       (long long)n_out, (long long)w->L.n_out);
    if (!aligned16(x)) return set_err(ctx, SIHIP_EINVAL, "gemv_dev: x must be 16-byte aligned");
    return run_matvec(ctx, w, x, w->L.n_in, nullptr, 0, 1, y, w->L.n_out, n_out,
                      (hipStream_t)stream);
}

extern "C" int sihip_gemm_dev(sihip_ctx *ctx, const sihip_weight *w, const float *X, int64_t M,
                              float *Y, void *stream) {
    if (!ctx || !w || !X || !Y) return set_err(ctx, SIHIP_EINVAL, "gemm_dev: NULL argument");
    if (M <= 0) return set_err(ctx, SIHIP_EINVAL, "gemm_dev: M must be positive");
    if (!aligned16(X)) return set_err(ctx, SIHIP_EINVAL, "gemm_dev: X must be 16-byte aligned");
    return run_gemm(ctx, w, X, M, Y, (hipStream_t)stream);
}

// sihip_gemm_dev without any allocation: the MFMA path takes its workspaces
// from this device's static scratch (kNoAllocBytes, split as described at
// `scratch`); the matvec path (small M, other formats) uses only the
// weight's own buffers. No hipMalloc, hipFree or allocating library call is
// made, so the call may be captured into a graph.
extern "C" int sihip_gemm_dev_noalloc(sihip_ctx *ctx, const sihip_weight *w, const float *X,
                                      int64_t M, float *Y, void *stream) {
    if (!ctx || !w || !X || !Y) return set_err(ctx, SIHIP_EINVAL, "gemm_dev_noalloc: NULL argument");
    if (M <= 0) return set_err(ctx, SIHIP_EINVAL, "gemm_dev_noalloc: M must be positive");
    if (!aligned16(X)) return set_err(ctx, SIHIP_EINVAL, "gemm_dev_noalloc: X must be 16-byte aligned");
    const hipStream_t st = (hipStream_t)stream;
    if (!gemm_on_mfma(ctx, w, M))
        return run_matvec(ctx, w, X, w->L.n_in, nullptr, 0, M, Y, w->L.n_out, w->L.n_out, st);
    const size_t room = kNoAllocBytes - kNoAllocCntBytes;
    if (gemmkf_eligible(ctx, 1, &w, M)) {
        // the fused small-M launch: its partial sums from offset 0
        if (!w->gsmall)
            return set_err(ctx, SIHIP_EINVAL,
                           "gemm_dev_noalloc: the weight has no GEMM copy; call "
                           "sihip_weight_prepare_gemm first");
        const int64_t t = gemmkf_tiles(w->L);
        int S, SBK;
        gemmkf_slices(ctx, t, w->L.n_in / 256, S, SBK);
        const size_t part = (size_t)S * kKFMp * t * kKFRows * sizeof(float);
        if (part > room)
            return set_err(ctx, SIHIP_ERANGE,
                           "gemm_dev_noalloc: %lld output rows in %d K slices need %zu bytes of "
                           "partial sums; the static scratch holds %zu",
                           (long long)w->L.n_out, S, part, room);
        bool done = false;
        float *Yp = Y;
        const int rc = launch_gemmkf_group(ctx, 1, &w, X, M, &Yp, (float *)ctx->scratch,
                                           (uint32_t *)(ctx->scratch + room), st, done);
        if (rc) return rc;
        return done ? SIHIP_OK : set_err(ctx, SIHIP_EINVAL, "gemm_dev_noalloc: no fused instance");
    }
    GemmPlan p = plan_gemm(ctx, w->L, M);
    if (!plan_copy(w, p))
        return set_err(ctx, SIHIP_EINVAL,
                       "gemm_dev_noalloc: the weight has no GEMM copy; call "
                       "sihip_weight_prepare_gemm first");
    if ((size_t)p.ws_bytes > room)
        return set_err(ctx, SIHIP_ERANGE,
                       "gemm_dev_noalloc: M = %lld x n_in = %lld needs %lld bytes of activation "
                       "planes; the static scratch holds %zu (M * n_in up to about %zu)",
                       (long long)M, (long long)w->L.n_in, (long long)p.ws_bytes, room,
                       room * 256 / 292);
    // K-slice partial sums go after the planes; where they do not fit, the
    // call runs without K slices (same results, fewer workgroups)
    const size_t part_off = ((size_t)p.ws_bytes + 255) & ~(size_t)255;
    if (p.S > 1 && part_off + (size_t)p.part_bytes > room) {
        p.S = 1;
        p.SBK = (int)p.steps;
        p.part_bytes = 0;
    }
    const GemmBufs B{ctx->scratch, (float *)(ctx->scratch + part_off),
                     (uint32_t *)(ctx->scratch + room)};
    return launch_gemm_mfma(ctx, w, p, B, X, w->L.n_in, M, Y, w->L.n_out, st);
}

extern "C" int sihip_attn_decode_dev(sihip_ctx *ctx, const float *q, const uint16_t *k_cache,
                                     const uint16_t *v_cache, int64_t n_head, int64_t n_head_kv,
                                     int64_t head_dim, int64_t n_ctx, int64_t pos, float kq_scale,
                                     float *out, float *scores, uint16_t *probs16, void *stream) {
    if (!ctx || !q || !k_cache || !v_cache || !out)
        return set_err(ctx, SIHIP_EINVAL, "attn_decode_dev: NULL argument");
    if (n_head < 1 || n_head_kv < 1 || n_head % n_head_kv != 0 || n_head > 4096)
        return set_err(ctx, SIHIP_EINVAL,
                       "attn_decode_dev: n_head %lld must be a multiple of n_head_kv %lld (<= 4096)",
                       (long long)n_head, (long long)n_head_kv);
    if (head_dim < 1 || head_dim > kAttnMaxHd)
        return set_err(ctx, SIHIP_EINVAL, "attn_decode_dev: head_dim %lld outside 1..%d",
                       (long long)head_dim, kAttnMaxHd);
    if (n_ctx < 1 || n_ctx > (int64_t)INT32_MAX || pos < 0 || pos >= n_ctx)
        return set_err(ctx, SIHIP_EINVAL, "attn_decode_dev: pos %lld outside 0..n_ctx-1 (n_ctx %lld)",
                       (long long)pos, (long long)n_ctx);
    HIP_OK(ctx, hipSetDevice(ctx->device));
    AttnArgs A;
    A.q = q;
    A.k = k_cache;
    A.v = v_cache;
    A.out = out;
    A.n_ctx = n_ctx;
    A.ld = n_ctx;
    A.n = (int)(pos + 1);
    A.hd = (int)head_dim;
    A.gqa = (int)(n_head / n_head_kv);
    A.n_head = (int)n_head;
    A.kq_scale = kq_scale;
    A.sc = scores;    // NULL: not written
    A.p16 = probs16;  // NULL: not written
    // workspace scores (f32) and probabilities (f16): rows of whole
    // kAttnBlock blocks, so that block loads stay inside the allocation
    A.lw = (A.n + kAttnBlock - 1) / kAttnBlock * kAttnBlock;
    const int rc = ensure(ctx, &ctx->d_attn, &ctx->d_attn_cap, (size_t)(n_head * A.lw * 6),
                          (hipStream_t)stream);
    if (rc) return rc;
    A.sw = (float *)ctx->d_attn;
    A.pw = (uint16_t *)((uint8_t *)ctx->d_attn + n_head * A.lw * 4);
    const int chunks = (A.gqa + kAttnHeads - 1) / kAttnHeads;
    const dim3 gs((unsigned)((A.n + kAttnRows - 1) / kAttnRows), (unsigned)(n_head_kv * chunks));
    const dim3 gv((unsigned)((head_dim + kAttnPvRows - 1) / kAttnPvRows),
                  (unsigned)(n_head_kv * chunks));
    if (gs.y > 65535) return set_err(ctx, SIHIP_EINVAL, "attn_decode_dev: too many KV heads");
    const hipStream_t st = (hipStream_t)stream;
    const int orc = order_before(ctx, ctx->order, st);
    if (orc) return orc;
    // wide loads where rows stay aligned: keys 8 bytes, value rows 16
    const bool kvec = head_dim % 4 == 0 && (uintptr_t)k_cache % 8 == 0;
    const bool vvec = n_ctx % 8 == 0 && (uintptr_t)v_cache % 16 == 0;
    if (kvec)
        hipLaunchKernelGGL(attn_scores_kernel<true>, gs, dim3(kAttnThreads), 0, st, A);
    else
        hipLaunchKernelGGL(attn_scores_kernel<false>, gs, dim3(kAttnThreads), 0, st, A);
    // up to kAttnFuseMax positions the value launch's waves compute their
    // heads' softmax themselves: no softmax launch (8B shape: 11.6 against
    // 15.1 us per layer at position 511)
    const int64_t fmax = ctx->opt.attn_fuse > 0 ? std::min<int64_t>(ctx->opt.attn_fuse * 512, 2048)
                                                : kAttnFuseMax;
    const int ng = ctx->opt.attn_fuse == 0 || A.n > fmax ? 0 : (A.n + 511) / 512;
    if (ng == 0)
        hipLaunchKernelGGL(attn_softmax_kernel, dim3((unsigned)n_head), dim3(kAttnThreads), 0, st, A);
#define SIHIP_PV(V)                                                                                 \
    switch (ng) {                                                                                   \
        case 0: hipLaunchKernelGGL((attn_pv_kernel<V, 0>), gv, dim3(kAttnThreads), 0, st, A); break; \
        case 1: hipLaunchKernelGGL((attn_pv_kernel<V, 1>), gv, dim3(kAttnThreads), 0, st, A); break; \
        case 2: hipLaunchKernelGGL((attn_pv_kernel<V, 2>), gv, dim3(kAttnThreads), 0, st, A); break; \
        default: hipLaunchKernelGGL((attn_pv_kernel<V, 4>), gv, dim3(kAttnThreads), 0, st, A); break; \
    }
    if (vvec) {
        SIHIP_PV(true)
    } else {
        SIHIP_PV(false)
    }
#undef SIHIP_PV
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_err(ctx, SIHIP_EDEVICE, "attention launch: %s", hipGetErrorString(e));
    return order_after(ctx, ctx->order, st);
}

extern "C" int sihip_gemm_multi_dev(sihip_ctx *ctx, int count, const sihip_weight *const *w,
                                    const float *X, int64_t M, float *const *Y, void *stream) {
    if (!ctx || !w || !X || !Y || count < 1 || count > kMaxSegs)
        return set_err(ctx, SIHIP_EINVAL, "gemm_multi_dev: bad arguments");
    if (M <= 0) return set_err(ctx, SIHIP_EINVAL, "gemm_multi_dev: M must be positive");
    if (!aligned16(X)) return set_err(ctx, SIHIP_EINVAL, "gemm_multi_dev: X must be 16-byte aligned");
    for (int i = 0; i < count; i++) {
        if (!w[i] || !Y[i]) return set_err(ctx, SIHIP_EINVAL, "gemm_multi_dev: NULL weight/output");
        if (w[i]->L.n_in != w[0]->L.n_in)
            return set_err(ctx, SIHIP_EINVAL, "gemm_multi_dev: n_in differs between weights");
    }
    const hipStream_t st = (hipStream_t)stream;
    // weights below their matrix-core threshold run on their own; the others
    // share the activation planes
    const sihip_weight *mw[kMaxSegs];
    float *my[kMaxSegs];
    int nm = 0;
    for (int i = 0; i < count; i++) {
        if (gemm_on_mfma(ctx, w[i], M)) {
            mw[nm] = w[i];
            my[nm++] = Y[i];
        } else {
            const int rc = run_matvec(ctx, w[i], X, w[i]->L.n_in, nullptr, 0, M, Y[i],
                                      w[i]->L.n_out, w[i]->L.n_out, st);
            if (rc) return rc;
        }
    }
    return nm ? run_gemm_multi(ctx, nm, mw, X, M, my, st) : SIHIP_OK;
}

extern "C" int sihip_gemv_multi_dev(sihip_ctx *ctx, int count, const sihip_weight *const *w,
                                    const float *x, float *const *y, void *stream) {
    if (!ctx || !w || !x || !y || count < 1 || count > kMaxSegs)
        return set_err(ctx, SIHIP_EINVAL, "gemv_multi_dev: bad arguments");
    if (!aligned16(x)) return set_err(ctx, SIHIP_EINVAL, "gemv_multi_dev: x must be 16-byte aligned");
    for (int i = 0; i < count; i++) {
        if (!w[i] || !y[i]) return set_err(ctx, SIHIP_EINVAL, "gemv_multi_dev: NULL weight/output");
        if (w[i]->L.n_in != w[0]->L.n_in)
            return set_err(ctx, SIHIP_EINVAL, "gemv_multi_dev: n_in differs between weights");
        if (pair_of(w[i]->L.type) != pair_of(w[0]->L.type))
            return set_err(ctx, SIHIP_EINVAL, "gemv_multi_dev: activation formats differ");
    }
    // formats one launch can mix; otherwise one launch per distinct format
    uint32_t f0 = w[0]->L.type, f1 = w[0]->L.type;
    for (int i = 1; i < count; i++) {
        if (w[i]->L.type < f0) f0 = w[i]->L.type;
        if (w[i]->L.type > f1) f1 = w[i]->L.type;
    }
    bool fused = mix_supported(f0, f1) && f0 != T_F32;
    for (int i = 0; i < count && fused; i++)
        fused = w[i]->L.type == f0 || w[i]->L.type == f1;
    int64_t n_out[kMaxSegs], ldy[kMaxSegs];
    for (int i = 0; i < count; i++) n_out[i] = ldy[i] = w[i]->L.n_out;
    if (fused)
        return run_matvec_multi(ctx, count, w, n_out, y, ldy, x, w[0]->L.n_in, nullptr, 0, 1,
                                (hipStream_t)stream);
    for (int i = 0; i < count; i++) {
        const int rc = sihip_gemv_dev(ctx, w[i], x, y[i], w[i]->L.n_out, stream);
        if (rc) return rc;
    }
    return SIHIP_OK;
}

// ---- device memory ---------------------------------------------------------------

extern "C" int sihip_dev_alloc(sihip_ctx *ctx, uint64_t bytes, void **dptr) {
    if (!ctx || !dptr || bytes == 0) return set_err(ctx, SIHIP_EINVAL, "dev_alloc: bad arguments");
    HIP_OK(ctx, hipSetDevice(ctx->device));
    void *p = nullptr;
    const hipError_t e = hipMalloc(&p, (size_t)bytes);
    if (e != hipSuccess)
        return set_err(ctx, SIHIP_ENOMEM, "dev_alloc(%llu): %s", (unsigned long long)bytes,
                       hipGetErrorString(e));
    *dptr = p;
    return SIHIP_OK;
}

extern "C" int sihip_dev_free(sihip_ctx *ctx, void *dptr) {
    if (!ctx) return SIHIP_EINVAL;
    if (!dptr) return SIHIP_OK;
    HIP_OK(ctx, hipSetDevice(ctx->device));
    HIP_OK(ctx, hipFree(dptr));
    return SIHIP_OK;
}

extern "C" int sihip_memcpy_htod(sihip_ctx *ctx, void *dst, const void *src, uint64_t bytes) {
    if (!ctx || !dst || !src) return set_err(ctx, SIHIP_EINVAL, "memcpy_htod: NULL argument");
    HIP_OK(ctx, hipSetDevice(ctx->device));
    HIP_OK(ctx, hipMemcpy(dst, src, (size_t)bytes, hipMemcpyHostToDevice));
    return SIHIP_OK;
}

extern "C" int sihip_memcpy_dtoh(sihip_ctx *ctx, void *dst, const void *src, uint64_t bytes) {
    if (!ctx || !dst || !src) return set_err(ctx, SIHIP_EINVAL, "memcpy_dtoh: NULL argument");
    HIP_OK(ctx, hipSetDevice(ctx->device));
    HIP_OK(ctx, hipMemcpy(dst, src, (size_t)bytes, hipMemcpyDeviceToHost));
    return SIHIP_OK;
}

extern "C" int sihip_synchronize(sihip_ctx *ctx) {
    if (!ctx) return SIHIP_EINVAL;
    HIP_OK(ctx, hipSetDevice(ctx->device));
    HIP_OK(ctx, hipDeviceSynchronize());
    return SIHIP_OK;
}

extern "C" int sihip_gemv(sihip_ctx *ctx, const sihip_weight *w, const float *x, float *y,
                          int64_t n_out) {
    if (!ctx || !w || !x || !y) return set_err(ctx, SIHIP_EINVAL, "gemv: NULL argument");
    if (n_out <= 0 || n_out > w->L.n_out)
        return set_err(ctx, SIHIP_EINVAL, "gemv: n_out %lld outside 1..%lld", (long long)n_out,
                       (long long)w->L.n_out);
    HIP_OK(ctx, hipSetDevice(ctx->device));
    const size_t xb = (size_t)w->L.n_in * 4, yb = (size_t)n_out * 4;
    int rc = ensure(ctx, &ctx->d_in, &ctx->d_in_cap, xb);
    if (rc) return rc;
    rc = ensure(ctx, &ctx->d_out, &ctx->d_out_cap, yb);
    if (rc) return rc;
    HIP_OK(ctx, hipMemcpyAsync(ctx->d_in, x, xb, hipMemcpyHostToDevice, ctx->stream));
    rc = run_matvec(ctx, w, (const float *)ctx->d_in, w->L.n_in, nullptr, 0, 1,
                    (float *)ctx->d_out, n_out, n_out, ctx->stream);
    if (rc) return rc;
    HIP_OK(ctx, hipMemcpyAsync(y, ctx->d_out, yb, hipMemcpyDeviceToHost, ctx->stream));
    HIP_OK(ctx, hipStreamSynchronize(ctx->stream));
    return SIHIP_OK;
}

extern "C" int sihip_gemm(sihip_ctx *ctx, const sihip_weight *w, const float *X, int64_t M,
                          float *Y) {
    if (!ctx || !w || !X || !Y) return set_err(ctx, SIHIP_EINVAL, "gemm: NULL argument");
    if (M <= 0) return set_err(ctx, SIHIP_EINVAL, "gemm: M must be positive");
    HIP_OK(ctx, hipSetDevice(ctx->device));
    const size_t xb = (size_t)M * (size_t)w->L.n_in * 4;
    const size_t yb = (size_t)M * (size_t)w->L.n_out * 4;
    int rc = ensure(ctx, &ctx->d_in, &ctx->d_in_cap, xb);
    if (rc) return rc;
    rc = ensure(ctx, &ctx->d_out, &ctx->d_out_cap, yb);
    if (rc) return rc;
    HIP_OK(ctx, hipMemcpyAsync(ctx->d_in, X, xb, hipMemcpyHostToDevice, ctx->stream));
    rc = run_gemm(ctx, w, (const float *)ctx->d_in, M, (float *)ctx->d_out, ctx->stream);
    if (rc) return rc;
    HIP_OK(ctx, hipMemcpyAsync(Y, ctx->d_out, yb, hipMemcpyDeviceToHost, ctx->stream));
    HIP_OK(ctx, hipStreamSynchronize(ctx->stream));
    return SIHIP_OK;
}

// ---- quantizers and per-row dots (parity-test entry points) ---------------------

extern "C" int sihip_quantize_q8_K(sihip_ctx *ctx, const float *x, void *out, int64_t n) {
    if (!ctx || !x || !out) return set_err(ctx, SIHIP_EINVAL, "quantize_q8_K: NULL argument");
    if (n <= 0 || n % 256) return set_err(ctx, SIHIP_EINVAL, "quantize_q8_K: n %% 256 != 0");
    HIP_OK(ctx, hipSetDevice(ctx->device));
    const int64_t nb = n / 256;
    int rc = ensure(ctx, &ctx->d_in, &ctx->d_in_cap, (size_t)n * 4);
    if (rc) return rc;
    rc = ensure(ctx, &ctx->d_out, &ctx->d_out_cap, (size_t)nb * 292);
    if (rc) return rc;
    HIP_OK(ctx, hipMemcpyAsync(ctx->d_in, x, (size_t)n * 4, hipMemcpyHostToDevice, ctx->stream));
    hipLaunchKernelGGL(quantize_q8K_kernel,
                       dim3((unsigned)((nb + kThreads / 16 - 1) / (kThreads / 16))),
                       dim3(kThreads), 0, ctx->stream, (const float *)ctx->d_in,
                       (uint8_t *)ctx->d_out, nb);
    HIP_OK(ctx, hipGetLastError());
    HIP_OK(ctx, hipMemcpyAsync(out, ctx->d_out, (size_t)nb * 292, hipMemcpyDeviceToHost, ctx->stream));
    HIP_OK(ctx, hipStreamSynchronize(ctx->stream));
    return SIHIP_OK;
}

extern "C" int sihip_quantize_q8_K_rows(sihip_ctx *ctx, const float *X, int64_t M, int64_t n_in,
                                        int bm, void *out) {
    if (!ctx || !X || !out) return set_err(ctx, SIHIP_EINVAL, "quantize_q8_K_rows: NULL argument");
    if (M <= 0 || n_in <= 0 || n_in % 256)
        return set_err(ctx, SIHIP_EINVAL, "quantize_q8_K_rows: M > 0 and n_in %% 256 == 0 needed");
    if (bm != 16 && bm != 32 && bm != 64 && bm != 128)
        return set_err(ctx, SIHIP_EINVAL, "quantize_q8_K_rows: bm must be 16, 32, 64 or 128");
    HIP_OK(ctx, hipSetDevice(ctx->device));
    const int64_t nb = n_in / 256, Mp = (M + bm - 1) / bm * bm;
    const int64_t rec = g2_rec_bytes(bm), rec_total = Mp / bm * nb * rec;
    int rc = ensure(ctx, &ctx->d_in, &ctx->d_in_cap, (size_t)(M * n_in * 4));
    if (rc) return rc;
    rc = ensure(ctx, &ctx->d_out, &ctx->d_out_cap, (size_t)rec_total);
    if (rc) return rc;
    HIP_OK(ctx, hipMemcpyAsync(ctx->d_in, X, (size_t)(M * n_in * 4), hipMemcpyHostToDevice,
                               ctx->stream));
    const dim3 grid((unsigned)gemm2_quantize_grid(Mp * nb)), block(kG2Threads);
    const float *xd = (const float *)ctx->d_in;
    uint8_t *rd = (uint8_t *)ctx->d_out;
    switch (bm) {
        case 16: hipLaunchKernelGGL(gemm2_quantize_x<16>, grid, block, 0, ctx->stream, xd, n_in, M, Mp, nb, rd); break;
        case 32: hipLaunchKernelGGL(gemm2_quantize_x<32>, grid, block, 0, ctx->stream, xd, n_in, M, Mp, nb, rd); break;
        case 64: hipLaunchKernelGGL(gemm2_quantize_x<64>, grid, block, 0, ctx->stream, xd, n_in, M, Mp, nb, rd); break;
        default: hipLaunchKernelGGL(gemm2_quantize_x<128>, grid, block, 0, ctx->stream, xd, n_in, M, Mp, nb, rd); break;
    }
    HIP_OK(ctx, hipGetLastError());
    std::vector<uint8_t> host((size_t)rec_total);
    HIP_OK(ctx, hipMemcpyAsync(host.data(), rd, (size_t)rec_total, hipMemcpyDeviceToHost, ctx->stream));
    HIP_OK(ctx, hipStreamSynchronize(ctx->stream));
    // back to the reference block layout: f32 d, 256 quants, 16 int16 sums
    uint8_t *o = (uint8_t *)out;
    for (int64_t m = 0; m < M; m++)
        for (int64_t c = 0; c < nb; c++) {
            const uint8_t *R = host.data() + ((m / bm) * nb + c) * rec;
            const int mr = (int)(m % bm);
            uint8_t *b = o + (m * nb + c) * 292;
            memcpy(b, R + g2_rec_dx(bm) + 4 * mr, 4);
            for (int e = 0; e < 256; e++)
                b[4 + e] = R[(4 * (mr >> 4) + e / 64) * 1024 + (16 * ((e / 16) & 3) + (mr & 15)) * 16 +
                             e % 16];
            for (int grp = 0; grp < 16; grp++) {
                uint16_t h;
                memcpy(&h, R + g2_rec_bsum(bm) + mr * 32 + 2 * grp, 2);
                const int16_t v = (int16_t)half_to_float(h);
                memcpy(b + 260 + 2 * grp, &v, 2);
            }
        }
    return SIHIP_OK;
}

extern "C" int sihip_quantize_q8_0(sihip_ctx *ctx, const float *x, void *out, int64_t n) {
    if (!ctx || !x || !out) return set_err(ctx, SIHIP_EINVAL, "quantize_q8_0: NULL argument");
    if (n <= 0 || n % 32) return set_err(ctx, SIHIP_EINVAL, "quantize_q8_0: n %% 32 != 0");
    HIP_OK(ctx, hipSetDevice(ctx->device));
    const int64_t nb = n / 32;
    int rc = ensure(ctx, &ctx->d_in, &ctx->d_in_cap, (size_t)n * 4);
    if (rc) return rc;
    rc = ensure(ctx, &ctx->d_out, &ctx->d_out_cap, (size_t)nb * 34);
    if (rc) return rc;
    HIP_OK(ctx, hipMemcpyAsync(ctx->d_in, x, (size_t)n * 4, hipMemcpyHostToDevice, ctx->stream));
    hipLaunchKernelGGL(quantize_q80_kernel, dim3((unsigned)((nb + kThreads - 1) / kThreads)),
                       dim3(kThreads), 0, ctx->stream, (const float *)ctx->d_in,
                       (uint8_t *)ctx->d_out, nb, (int)(ctx->opt.q80_scalar > 0));
    HIP_OK(ctx, hipGetLastError());
    HIP_OK(ctx, hipMemcpyAsync(out, ctx->d_out, (size_t)nb * 34, hipMemcpyDeviceToHost, ctx->stream));
    HIP_OK(ctx, hipStreamSynchronize(ctx->stream));
    return SIHIP_OK;
}

extern "C" int sihip_convert_f16(sihip_ctx *ctx, const float *x, void *out, int64_t n) {
    if (!ctx || !x || !out) return set_err(ctx, SIHIP_EINVAL, "convert_f16: NULL argument");
    if (n <= 0) return set_err(ctx, SIHIP_EINVAL, "convert_f16: n must be positive");
    HIP_OK(ctx, hipSetDevice(ctx->device));
    int rc = ensure(ctx, &ctx->d_in, &ctx->d_in_cap, (size_t)n * 4);
    if (rc) return rc;
    rc = ensure(ctx, &ctx->d_out, &ctx->d_out_cap, (size_t)n * 2);
    if (rc) return rc;
    HIP_OK(ctx, hipMemcpyAsync(ctx->d_in, x, (size_t)n * 4, hipMemcpyHostToDevice, ctx->stream));
    hipLaunchKernelGGL(convert_f16_kernel, dim3((unsigned)((n + kThreads - 1) / kThreads)),
                       dim3(kThreads), 0, ctx->stream, (const float *)ctx->d_in,
                       (uint16_t *)ctx->d_out, n);
    HIP_OK(ctx, hipGetLastError());
    HIP_OK(ctx, hipMemcpyAsync(out, ctx->d_out, (size_t)n * 2, hipMemcpyDeviceToHost, ctx->stream));
    HIP_OK(ctx, hipStreamSynchronize(ctx->stream));
    return SIHIP_OK;
}

extern "C" int sihip_gemv_pair(sihip_ctx *ctx, uint32_t wtype, int64_t n_rows, int64_t n_in,
                               const void *rows, const void *xq, float *y) {
    if (!ctx || !rows || !xq || !y) return set_err(ctx, SIHIP_EINVAL, "gemv_pair: NULL argument");
    uint32_t be, bb;
    if (!geometry(wtype, &be, &bb) || wtype == T_Q8_K)
        return set_err(ctx, SIHIP_ENOTSUP, "gemv_pair: unsupported type %u", wtype);
    if (n_rows <= 0 || n_in <= 0 || (wtype != T_F32 && (n_in % be || n_in % 32)))
        return set_err(ctx, SIHIP_EINVAL, "gemv_pair: bad shape");
    const uint32_t pair = pair_of(wtype);
    uint32_t pe, pb;
    geometry(pair, &pe, &pb);
    const size_t xq_bytes = (size_t)(n_in / pe) * pb;
    sihip_weight *w = nullptr;
    int rc = sihip_weight_upload(ctx, wtype, (uint64_t)n_rows, (uint64_t)n_in, rows,
                                 (uint64_t)(n_in / be * bb) * (uint64_t)n_rows, &w);
    if (rc) return rc;
    rc = ensure(ctx, &ctx->d_aux, &ctx->d_aux_cap, xq_bytes);
    if (!rc) rc = ensure(ctx, &ctx->d_out, &ctx->d_out_cap, (size_t)n_rows * 4);
    if (!rc) {
        hipError_t e = hipMemcpyAsync(ctx->d_aux, xq, xq_bytes, hipMemcpyHostToDevice, ctx->stream);
        if (e != hipSuccess) rc = set_err(ctx, SIHIP_EDEVICE, "gemv_pair: %s", hipGetErrorString(e));
    }
    if (!rc)
        rc = run_matvec(ctx, w, nullptr, 0, (const uint8_t *)ctx->d_aux, (int64_t)xq_bytes, 1,
                        (float *)ctx->d_out, n_rows, n_rows, ctx->stream);
    if (!rc) {
        hipError_t e = hipMemcpyAsync(y, ctx->d_out, (size_t)n_rows * 4, hipMemcpyDeviceToHost,
                                      ctx->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) rc = set_err(ctx, SIHIP_EDEVICE, "gemv_pair: %s", hipGetErrorString(e));
    }
    sihip_weight_free(ctx, w);
    return rc;
}

extern "C" int sihip_vec_dot(sihip_ctx *ctx, uint32_t wtype, int n, float *s, const void *x,
                             const void *y) {
    if (!s) return set_err(ctx, SIHIP_EINVAL, "vec_dot: NULL output");
    return sihip_gemv_pair(ctx, wtype, 1, n, x, y, s);
}
