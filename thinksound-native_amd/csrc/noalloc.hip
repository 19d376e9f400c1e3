// noalloc.hip — the allocation-free GEMM entry point (tsn_gemm_noalloc) for callers that cannot
// allocate device memory: code under hipGraph capture, tight serving loops, harnesses that forbid
// hipMalloc. It runs exactly tsn_gemm's kernels and plans; the one buffer tsn_gemm takes from the
// runtime's grow-on-demand scratch (the f16 hi|lo split of an f32 X, 4*M*K bytes) lives instead in
// a file-scope device array of fixed size, one copy per GPU, held until the process ends. The
// partial sums of a K split go to the runtime's own fixed workspace, allocated when the runtime was
// created, as in tsn_gemm.
//
// In host code the array's name is only a host-side stand-in: its device address on each GPU comes
// from hipGetSymbolAddress, taken once per device with that device current (noalloc_init, called
// from the runtime's init), and only that address is ever passed to a kernel. Every call on one GPU
// shares the array and leaves its contents behind; nothing in it has to start at zero (the split
// kernel writes every element the GEMM reads).
//
// Ordering on the device: every runtime has its own stream, so two runtimes (or two host threads)
// calling one after the other could otherwise run their split and GEMM kernels at the same time on
// one array. Each device keeps one event, created at init: a call waits on it when the previous
// call came from another stream, and records it after its GEMM (hipStreamWaitEvent and
// hipEventRecord allocate nothing). A call made while its stream is being captured into a graph
// cannot order itself against work outside the capture this way; there the caller must order the
// graph's launches against other users of the array (one stream, or its own events).
#include "runtime.h"

#include <mutex>

namespace tsn {

namespace {

constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t)32 << 20;   // hi|lo split of X: M*K <= 8 Mi elements

static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
std::mutex g_mu;
void *g_scratch_dev[MAX_DEVICES] = {};         // device address of `scratch` on each GPU
hipEvent_t g_done[MAX_DEVICES] = {};           // recorded after each (uncaptured) call's GEMM
hipStream_t g_last_stream[MAX_DEVICES] = {};   // the stream that recorded it

} // namespace

size_t noalloc_scratch_bytes() { return NOALLOC_SCRATCH_BYTES; }

int noalloc_init(int device) {
    TSN_REQUIRE(device >= 0 && device < MAX_DEVICES, "noalloc: device index out of range");
    std::lock_guard<std::mutex> lock(g_mu);
    if (g_scratch_dev[device]) return TSN_OK;
    int cur = -1;
    TSN_HIP_CHECK(hipGetDevice(&cur));
    TSN_REQUIRE(cur == device, "noalloc: the device must be current");
    void *p = nullptr;
    TSN_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    TSN_REQUIRE(p != nullptr, "noalloc: no device address for the scratch array");
    hipEvent_t ev = nullptr;
    TSN_HIP_CHECK(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
    g_done[device] = ev;
    g_scratch_dev[device] = p;
    return TSN_OK;
}

int gemm_noalloc(Runtime &rt, int wdt, const void *W, const void *X, int xdt, void *Y, int ydt, const float *bias,
                 const GemmParams &p) {
    TSN_REQUIRE(W && X && Y, "gemm: null operand");
    TSN_REQUIRE(p.M > 0 && p.N > 0 && p.K > 0, "gemm: empty shape");
    const uint32_t ldx = p.ldx ? p.ldx : p.K, ldw = p.ldw ? p.ldw : p.K, ldy = p.ldy ? p.ldy : p.N;
    TSN_REQUIRE(ldx >= p.K && ldw >= p.K && ldy >= p.N, "gemm: leading dimension below the row width");
    if (!(wdt == DT_F16 && xdt == DT_F32 && gemm_hilo_ok(W, ldw, Y, ydt, ldy, bias, p.M, p.N, p.K)))
        return rt.gemm(wdt, W, X, xdt, Y, ydt, bias, p);   // no scratch on these routes: nothing to allocate
    const size_t need = gemm_hilo_bytes(p.M, p.K);
    if (need > NOALLOC_SCRATCH_BYTES) {
        set_error("gemm_noalloc: the f32 X split needs " + std::to_string(need) + " bytes (4*M*K); the static scratch holds " +
                  std::to_string(NOALLOC_SCRATCH_BYTES) + " (M*K <= " + std::to_string(NOALLOC_SCRATCH_BYTES / 4) + ")");
        return TSN_ERR_ARG;
    }
    TSN_TRY(rt.dev.make_current());
    const int d = rt.dev.device();
    bool ready = false;
    {
        std::lock_guard<std::mutex> lock(g_mu);
        ready = g_scratch_dev[d] != nullptr;
    }
    if (!ready) TSN_TRY(noalloc_init(d));
    const hipStream_t st = rt.dev.stream();
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    TSN_HIP_CHECK(hipStreamIsCapturing(st, &cap));
    const bool order = cap == hipStreamCaptureStatusNone;
    // one caller at a time per device from here to the event record, so the wait/record pairs of
    // two host threads cannot interleave
    std::lock_guard<std::mutex> lock(g_mu);
    if (order && g_last_stream[d] && g_last_stream[d] != st) TSN_HIP_CHECK(hipStreamWaitEvent(st, g_done[d], 0));
    TSN_TRY(gemm_hilo((const half_t *)W, ldw, (const float *)X, ldx, Y, ydt, ldy, bias, p.M, p.N, p.K,
                      (half_t *)g_scratch_dev[d], rt.split_ws(), rt.split_ws_bytes(), st));
    if (order) {
        TSN_HIP_CHECK(hipEventRecord(g_done[d], st));
        g_last_stream[d] = st;
    }
    return TSN_OK;
}

} // namespace tsn
