// Long prefill batches the way the reference computes every batch (quant_linear.py:93-113:
// dequantize the packed weight, then F.linear): the weight is dequantized bit-exactly into a dense
// [N, K] matrix of the compute dtype in the caller's workspace (launch_dequant: the reference's
// fp32 (q - z) * s, rounded once to the compute dtype), and hipBLASLt multiplies the activations
// with it, fp32 accumulation, the bias added in its epilogue.
//
// Why two passes here: from about a thousand tokens the product is MFMA-bound, and a dense bf16
// GEMM tile streams its operands through LDS with nothing else in the instruction stream, while
// the fused kernels interleave each tile's dequantization (VALU) and its LDS fragment reads with
// the MFMA work. The extra pass costs the dequantized weight's write and re-read once per call
// (gate_up: 59 MB of codes in, 235 MB out, about 50 us on MI355X), a few percent of a
// 1024-token product's MFMA time and less beyond it. Shorter batches keep the fused kernels,
// which read 4 bits per weight instead of 16.
//
// hipBLASLt state: one handle per device, created on the first dense call on that device, and a
// bounded cache per shape of the matmul descriptors and the heuristic's first candidates
// (kCandidates). Up to 6144 tokens, which candidate runs is measured, not guessed: there the
// heuristic's first choice is up to 18 % slower than the best of its first eight on MI355X, and
// one of its first choices does not run at all. The first call of a size class (M rounded up to
// a power of two or 1.5 times one) on a stream that is not being captured runs every candidate
// on its own inputs, times them with HIP events and waits for them (the one place this library
// blocks the host), then keeps the fastest; later calls of any M in that class run the same
// algorithm when the heuristic offers it for their M. From 8192 tokens the heuristic's first
// choice measured fastest for every Llama-3-8B projection, and measuring there would cost tens
// of milliseconds of GEMMs, so the heuristic's order stands. A candidate that fails to launch is
// dropped and the next one runs; with none left the call reports that the path does not fit
// and the fused kernels run. Both caches are guarded by one mutex, which is also held while a
// call sets its bias pointer and enqueues the matmul. hipblasLtCreate allocates device memory:
// the first dense call on a device must not run under stream capture.
#include <hipblaslt/hipblaslt.h>

#include <string.h>

#include <map>
#include <mutex>
#include <tuple>

#include "qcommon.hpp"
#include "qkernels.hpp"

namespace llmopt {
namespace {

constexpr size_t kBlasWorkspace = size_t(32) << 20;  // hipBLASLt's own workspace (split-K etc.)
constexpr int kMaxDevices = 64;
constexpr size_t kMaxPlans = 256;
constexpr int kCandidates = 8;
constexpr int kTimedRuns = 2;
constexpr int64_t kMeasureMaxTokens = 6144;  // largest size class whose candidates are timed

size_t align256(size_t b) { return (b + 255) / 256 * 256; }

size_t elem_bytes(int act) { return act == kDtF32 ? 4 : 2; }

hipDataType blas_type(int act) {
  return act == kDtF32 ? HIP_R_32F : act == kDtF16 ? HIP_R_16F : HIP_R_16BF;
}

struct PlanKey {
  int device, act;
  int64_t M, N, K, ldx, ldy;
  bool bias;
  bool operator<(const PlanKey& o) const {
    return std::tie(device, act, M, N, K, ldx, ldy, bias) <
           std::tie(o.device, o.act, o.M, o.N, o.K, o.ldx, o.ldy, o.bias);
  }
};

// y^T = W x^T in hipBLASLt's column-major terms: A = W stored as a K x N column-major matrix
// (ld K) taken transposed, B = x as K x M (ld ldx), D = y^T as N x M (ld ldy).
struct Plan {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, d = nullptr;
  hipblasLtMatmulAlgo_t algo[kCandidates] = {};
  bool usable[kCandidates] = {};
  int count = 0;
  int chosen = -1;  // index into algo once measured or matched
};

std::mutex g_mutex;
hipblasLtHandle_t g_handle[kMaxDevices] = {};
hipEvent_t g_events[kMaxDevices][2 * kCandidates] = {};
std::map<PlanKey, Plan> g_plans;
std::map<PlanKey, hipblasLtMatmulAlgo_t> g_measured;  // size class -> fastest algorithm

// The size class whose measurement a batch of M tokens reuses: M rounded up to 2^k or 3 * 2^(k-1).
int64_t size_class(int64_t M) {
  int64_t c = 1;
  while (c < M) {
    if (c >= 2 && c + c / 2 >= M) return c + c / 2;
    c *= 2;
  }
  return c;
}

bool same_algo(const hipblasLtMatmulAlgo_t& x, const hipblasLtMatmulAlgo_t& y) {
  return memcmp(x.data, y.data, sizeof(x.data)) == 0;
}

void destroy(Plan& p) {
  if (p.a) hipblasLtMatrixLayoutDestroy(p.a);
  if (p.b) hipblasLtMatrixLayoutDestroy(p.b);
  if (p.d) hipblasLtMatrixLayoutDestroy(p.d);
  if (p.desc) hipblasLtMatmulDescDestroy(p.desc);
  p = Plan{};
}

// Builds the descriptors and asks the heuristic for up to kCandidates algorithms within
// kBlasWorkspace. A plan with count == 0 means hipBLASLt offers none (the caller then runs the
// fused kernels instead). Called with g_mutex held.
Plan make_plan(hipblasLtHandle_t handle, const PlanKey& k) {
  Plan p;
  const hipDataType t = blas_type(k.act);
  bool good = hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS;
  const hipblasOperation_t op_t = HIPBLAS_OP_T, op_n = HIPBLAS_OP_N;
  good = good && hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &op_t, sizeof(op_t)) ==
                     HIPBLAS_STATUS_SUCCESS;
  good = good && hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &op_n, sizeof(op_n)) ==
                     HIPBLAS_STATUS_SUCCESS;
  if (good && k.bias) {
    const hipblasLtEpilogue_t epi = HIPBLASLT_EPILOGUE_BIAS;
    const int32_t bias_type = int32_t(t);
    good = hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_EPILOGUE, &epi, sizeof(epi)) ==
               HIPBLAS_STATUS_SUCCESS &&
           hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bias_type,
                                           sizeof(bias_type)) == HIPBLAS_STATUS_SUCCESS;
  }
  good = good && hipblasLtMatrixLayoutCreate(&p.a, t, uint64_t(k.K), uint64_t(k.N), k.K) == HIPBLAS_STATUS_SUCCESS;
  good = good && hipblasLtMatrixLayoutCreate(&p.b, t, uint64_t(k.K), uint64_t(k.M), k.ldx) == HIPBLAS_STATUS_SUCCESS;
  good = good && hipblasLtMatrixLayoutCreate(&p.d, t, uint64_t(k.N), uint64_t(k.M), k.ldy) == HIPBLAS_STATUS_SUCCESS;
  hipblasLtMatmulPreference_t pref = nullptr;
  good = good && hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS;
  const uint64_t cap = kBlasWorkspace;
  good = good && hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &cap,
                                                       sizeof(cap)) == HIPBLAS_STATUS_SUCCESS;
  // Room beyond the request in case the library's result record is larger than this header's.
  hipblasLtMatmulHeuristicResult_t results[2 * kCandidates] = {};
  int found = 0;
  good = good && hipblasLtMatmulAlgoGetHeuristic(handle, p.desc, p.a, p.b, p.d, p.d, pref, kCandidates, results,
                                                 &found) == HIPBLAS_STATUS_SUCCESS;
  if (pref) hipblasLtMatmulPreferenceDestroy(pref);
  if (!good) {
    destroy(p);
    return p;
  }
  for (int i = 0; i < found && i < kCandidates; ++i) {
    if (results[i].state != HIPBLAS_STATUS_SUCCESS || results[i].workspaceSize > kBlasWorkspace) continue;
    p.algo[p.count] = results[i].algo;
    p.usable[p.count] = true;
    ++p.count;
  }
  if (p.count == 0) destroy(p);
  return p;
}

// The cached plan for these arguments on the current device, or nullptr (none, or no handle).
// Called with g_mutex held.
Plan* find_plan(const PlanKey& key) {
  if (!g_handle[key.device] && hipblasLtCreate(&g_handle[key.device]) != HIPBLAS_STATUS_SUCCESS) {
    g_handle[key.device] = nullptr;
    return nullptr;
  }
  auto it = g_plans.find(key);
  if (it == g_plans.end()) {
    if (g_plans.size() >= kMaxPlans) {
      for (auto& kv : g_plans) destroy(kv.second);
      g_plans.clear();
    }
    it = g_plans.emplace(key, make_plan(g_handle[key.device], key)).first;
  }
  return it->second.count > 0 ? &it->second : nullptr;
}

struct Operands {
  const void *w, *x;
  void *y, *ws;
};

hipblasStatus_t run(hipblasLtHandle_t h, const Plan& p, int i, const Operands& o, hipStream_t stream) {
  const float alpha = 1.0f, beta = 0.0f;
  return hipblasLtMatmul(h, p.desc, &alpha, o.w, p.a, o.x, p.b, &beta, o.y, p.d, o.y, p.d, &p.algo[i], o.ws,
                         kBlasWorkspace, stream);
}

// Runs each usable candidate once untimed and kTimedRuns times between two events on `stream`,
// waits, and returns the fastest (or -1). Candidates that fail to launch are marked unusable.
int measure(hipblasLtHandle_t h, Plan& p, hipEvent_t* ev, const Operands& o, hipStream_t stream) {
  bool timed[kCandidates] = {};
  for (int i = 0; i < p.count; ++i) {
    if (!p.usable[i]) continue;
    if (run(h, p, i, o, stream) != HIPBLAS_STATUS_SUCCESS) {
      p.usable[i] = false;
      continue;
    }
    if (hipEventRecord(ev[2 * i], stream) != hipSuccess) return -1;
    bool good = true;
    for (int r = 0; r < kTimedRuns && good; ++r) good = run(h, p, i, o, stream) == HIPBLAS_STATUS_SUCCESS;
    if (hipEventRecord(ev[2 * i + 1], stream) != hipSuccess) return -1;
    timed[i] = good;
    if (!good) p.usable[i] = false;
  }
  int best = -1;
  float best_ms = 0.0f;
  for (int i = 0; i < p.count; ++i) {
    if (!timed[i]) continue;
    float ms = 0.0f;
    if (hipEventSynchronize(ev[2 * i + 1]) != hipSuccess ||
        hipEventElapsedTime(&ms, ev[2 * i], ev[2 * i + 1]) != hipSuccess)
      continue;
    if (best < 0 || ms < best_ms) {
      best = i;
      best_ms = ms;
    }
  }
  return best;
}

}  // namespace

int64_t dense_min_tokens(int act) { return act == kDtF32 ? 65 : 1024; }

size_t dense_workspace_bytes(int64_t N, int64_t K, int act) {
  if (N <= 0 || K <= 0) return 0;
  return align256(size_t(N) * size_t(K) * elem_bytes(act)) + kBlasWorkspace;
}

hipError_t launch_linear_dense(const LinearArgs& a, hipStream_t stream, bool* fits) {
  *fits = false;
  if (a.epilogue != kEpiNone || a.out_f32 || a.M < 1 || a.N < 1 || a.K < 1) return hipSuccess;
  if (a.act != kDtBf16 && a.act != kDtF16 && a.act != kDtF32) return hipSuccess;
  const size_t dense = align256(size_t(a.N) * size_t(a.K) * elem_bytes(a.act));
  if (!a.workspace || a.workspace_bytes < dense + kBlasWorkspace ||
      reinterpret_cast<uintptr_t>(a.workspace) % 256 != 0)
    return hipSuccess;
  int device = -1;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return err;
  void* w = a.workspace;
  void* blas_ws = static_cast<uint8_t*>(a.workspace) + dense;

  std::lock_guard<std::mutex> lock(g_mutex);
  if (device < 0 || device >= kMaxDevices) return hipSuccess;
  const PlanKey key{device, a.act, a.M, a.N, a.K, a.ldx, a.ldy, a.bias != nullptr};
  Plan* p = find_plan(key);
  if (!p) return hipSuccess;  // no algorithm for this shape: the fused kernels run instead
  hipblasLtHandle_t h = g_handle[device];
  if (a.bias) {
    const void* bias = a.bias;
    if (hipblasLtMatmulDescSetAttribute(p->desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias, sizeof(bias)) !=
        HIPBLAS_STATUS_SUCCESS)
      return hipSuccess;
  }
  err = launch_dequant(a, w, a.act, stream);
  if (err != hipSuccess) return err;
  *fits = true;
  const Operands o{w, a.x, a.y, blas_ws};

  // Which candidate: the one measured for this size class, else measure now (not under capture).
  PlanKey cls = key;
  cls.M = size_class(a.M);
  if (p->chosen < 0) {
    auto m = g_measured.find(cls);
    if (m != g_measured.end()) {
      for (int i = 0; i < p->count && p->chosen < 0; ++i)
        if (p->usable[i] && same_algo(p->algo[i], m->second)) p->chosen = i;
    }
  }
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &capture) != hipSuccess) capture = hipStreamCaptureStatusActive;
  if (p->chosen < 0 && capture == hipStreamCaptureStatusNone && cls.M <= kMeasureMaxTokens) {
    hipEvent_t* ev = g_events[device];
    bool have = true;
    for (int i = 0; i < 2 * kCandidates && have; ++i)
      have = ev[i] != nullptr || hipEventCreate(&ev[i]) == hipSuccess;
    if (have) {
      p->chosen = measure(h, *p, ev, o, stream);
      if (p->chosen >= 0) {
        if (g_measured.size() >= kMaxPlans) g_measured.clear();
        g_measured[cls] = p->algo[p->chosen];
      }
    }
  }
  // The chosen candidate (or, unmeasured, the heuristic's order); one that fails is dropped.
  for (int attempt = 0; attempt < p->count; ++attempt) {
    int i = p->chosen;
    if (i < 0 || !p->usable[i]) {
      i = -1;
      for (int j = 0; j < p->count && i < 0; ++j)
        if (p->usable[j]) i = j;
      if (i < 0) break;
    }
    if (run(h, *p, i, o, stream) == HIPBLAS_STATUS_SUCCESS) return hipSuccess;
    p->usable[i] = false;
    if (p->chosen == i) p->chosen = -1;
  }
  // No candidate ran: the dense weight in the workspace is dropped and the fused kernels run.
  *fits = false;
  return hipSuccess;
}

}  // namespace llmopt
