// noalloc.hip — ifx_matmul_qt_noalloc: the prefill GEMM of ifx_matmul_qt for
// callers that cannot allocate device memory (code under HIP graph capture,
// serving loops and harnesses that forbid hipMalloc).
//
// ifx_matmul_qt allocates, per call, the GEMM's activation operand (fp16 hi and
// lo planes, 32-element group sums, row exponents) and a workspace for split-K
// partial tiles.  Here those live in one file-scope device array, `scratch`,
// of kScratchBytes, which each GPU the library runs on holds until the
// process ends.  Its device address is taken once per device with
// hipGetSymbolAddress (the array's name in host code is not a device address)
// and only that address is passed to kernels.  Every call on one GPU shares
// the array: calls that overlap on one GPU (two streams, two threads) race.
// Nothing in it needs to start at zero: the row preparation writes every
// operand element the GEMM reads, and the split-K tiles are written before
// the reduce reads them.
#include <mutex>

#include "ifx_common.h"
#include "kernels.h"

namespace ifx {

int device_init();
hipStream_t library_stream();

namespace {

// Operand planes for m * k <= kMaxElems (two fp16 planes), group sums and row
// exponents for m <= kMaxRows, the rest for split-K partial tiles.
constexpr uint64_t kMaxElems = 1ull << 22;
constexpr uint64_t kMaxRows = 16384;
constexpr uint64_t kPlaneBytes = kMaxElems * 2;                      // 8 MiB each
constexpr uint64_t kGsumBytes = kMaxElems / 8 + kMaxRows * 32;       // m (k/256 + 1) 32 B at most
constexpr uint64_t kRexpBytes = kMaxRows * 4;
constexpr uint64_t kPartBytes = 6ull << 20;
constexpr uint64_t kScratchBytes = 2 * kPlaneBytes + kGsumBytes + kRexpBytes + kPartBytes;  // ~23.1 MiB

__device__ __attribute__((aligned(256))) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices] = {};

// The current device's copy of `scratch`, looked up on the first call there.
int scratch_on_device(uint8_t** out) {
  int dev = 0;
  IFX_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) return set_error(IFX_E_NO_DEVICE, "device %d out of range", dev);
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error(IFX_E_HIP, "hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
    g_ptr[dev] = p;
  }
  *out = (uint8_t*)g_ptr[dev];
  return IFX_OK;
}

uint64_t al256(uint64_t b) { return (b + 255) & ~255ull; }

}  // namespace
}  // namespace ifx

using namespace ifx;

extern "C" {

int ifx_matmul_qt_noalloc(const float* a, uint64_t m, const ifx_tensor* w, float* c, void* stream) {
  IFX_TRY(device_init());
  if (!w || (m && (!a || !c))) return set_error(IFX_E_INVALID_ARG, "null argument");
  hipStream_t st = stream ? (hipStream_t)stream : library_stream();
  const uint64_t k = w->L.cols;
  if (m >= 2 && m <= 0xffffffffull && k <= 0xffffffffull && gemm_type(w->L.type) && gemm_layout_ok(w->L)) {
    uint64_t mk = 0;
    if (m > kMaxRows || !mul_u64(m, k, &mk) || mk > kMaxElems)
      return set_error(IFX_E_INVALID_ARG,
                       "ifx_matmul_qt_noalloc: %llu x %llu activations exceed the fixed scratch (m <= %llu, m*k <= %llu)",
                       (unsigned long long)m, (unsigned long long)k, (unsigned long long)kMaxRows,
                       (unsigned long long)kMaxElems);
    uint8_t* s = nullptr;
    IFX_TRY(scratch_on_device(&s));
    // the same carving as ifx_matmul_qt's allocation, inside the array
    const uint64_t bh = al256(m * k * 2), bg = al256(m * (k / 256 + 1) * 32), br = al256(m * 4);
    const uint64_t used = 2 * bh + bg + br;
    if (used > kScratchBytes) return set_error(IFX_E_INVALID_ARG, "ifx_matmul_qt_noalloc: operand exceeds the scratch");
    const GemmIn in{(const uint16_t*)s, (const uint16_t*)(s + bh), (const uint16_t*)(s + 2 * bh),
                    (const int*)(s + 2 * bh + bg), (uint32_t)m, (uint32_t)k, (float*)(s + used),
                    kScratchBytes - used};
    IFX_HIP(launch_prep_rows(a, (uint32_t)m, (uint32_t)k, (uint32_t)k, nullptr, 0.f, in, st));
    const GemmW gw = gemm_w(w->L);
    IFX_HIP(gemm_store(in, gw, c, (uint32_t)w->L.rows, st));
    return IFX_OK;
  }
  // one row, or a matrix the GEMM does not take: the GEMV row by row, which
  // uses no scratch (as ifx_matmul_qt does)
  for (uint64_t i = 0; i < m; i++) {
    GemvLaunch L;
    L.seg[0] = gemv_seg(w->L);
    L.nseg = 1;
    L.cols = (uint32_t)k;
    L.x = a + i * k;
    IFX_HIP(gemv_store(L, c + i * w->L.rows, st));
  }
  return IFX_OK;
}

}  // extern "C"
