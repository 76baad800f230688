// C ABI of libtforge_hip (declared in include/tforge_hip.h): compile = front
// end + instantiation selection, launch = the kernel ABI, and the runner
// (correctness run, timed run, resources, device facts) that replaces the
// reference's tforge-gpu-bench process (runners/gpu/tforge-gpu-bench.cu).
#include <dlfcn.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <memory>
#include <mutex>
#include <new>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#include "frontend.h"
#include "tf_kernels.h"
#include "tforge_hip.h"

namespace {

thread_local std::string g_err;

int fail(int code, const std::string &m) {
  g_err = m;
  return code;
}

// Runs an entry point's body; a C++ exception (an allocation failure, say)
// becomes an error code and message instead of unwinding into the caller.
template <typename F>
int guarded(F &&body) {
  try {
    return body();
  } catch (const std::bad_alloc &) {
    return fail(TF_E_ARG, "out of host memory");
  } catch (const std::exception &e) {
    return fail(TF_E_ARG, std::string("internal error: ") + e.what());
  } catch (...) {
    return fail(TF_E_ARG, "internal error");
  }
}

#define TF_HIP(x)                                                                                  \
  do {                                                                                             \
    hipError_t e_ = (x);                                                                           \
    if (e_ != hipSuccess) return fail(TF_E_HIP, std::string(#x) + " failed: " + hipGetErrorString(e_)); \
  } while (0)

void copy_str(char *dst, size_t cap, const std::string &s) {
  std::snprintf(dst, cap, "%s", s.c_str());
}

// Why a staged configuration has no instantiation (mirrors gen_instances.py).
std::string staged_reason(long bm, long bn, long tm, long tn, long bk, bool promote) {
  const long threads = (bm / tm) * (bn / tn);
  if (threads % 64) return std::to_string(threads) + " threads per block is not a whole number of 64-lane waves";
  if (threads > 1024) return std::to_string(threads) + " threads per block exceeds 1024";
  if (threads * tm * tn > 32768)
    return std::to_string(threads) + " threads x " + std::to_string(tm * tn) +
           " accumulators per lane exceed the register file (512 VGPRs per SIMD lane shared by the block's waves)";
  const long wtm = 8 * tm, wtn = 8 * tn;
  if (wtm % 16 || wtn % 16)
    return "wave tile " + std::to_string(wtm) + "x" + std::to_string(wtn) +
           " (8*TM x 8*TN) is not made of 16x16 or 32x32 MFMA blocks";
  if (bm % wtm || bn % wtn)
    return "block tile " + std::to_string(bm) + "x" + std::to_string(bn) + " is not a multiple of the wave tile " +
           std::to_string(wtm) + "x" + std::to_string(wtn) + " (8*TM x 8*TN)";
  const long mb = (wtm % 32 == 0 && wtn % 32 == 0) ? 32 : 16, kc = 256 / mb;
  if (bk % kc)
    return "tile-k must be a multiple of " + std::to_string(kc) + " for " + std::to_string(mb) + "x" +
           std::to_string(mb) + " MFMA blocks";
  const long lds = promote ? 2 * (bm * (bk + (mb == 32 ? 4 : 8)) + bk * (bn + (mb == 32 ? 8 : 4))) * 4 : 0;
  if (lds > 160 * 1024) return "LDS " + std::to_string(lds) + " B exceeds 160 KiB";
  return "no ahead-of-time instantiation of this configuration in libtforge_hip";
}

// The staged kernel gives each 64-lane wave an (8*TM) x (8*TN) output tile.
// Where that wave tile cannot tile the block -- fewer than 64 threads (the
// reference's 32-thread configurations such as block-tile=32,32
// thread-tile=8,4), or a wave tile taller or wider than the block
// (block-tile=32,64 thread-tile=8,4) -- the kernel runs the wave layout that
// keeps the block tile and tile-k: with fewer than 64 threads one wave owns
// the whole block (thread tile BM/8 x BN/8); otherwise the same number of
// threads and accumulators per lane, with the thread tile's long side
// shortened to fit (TM x TN = 8x4 on a 32-row block becomes 4x8).  ktm, ktn
// receive the thread tile of the instantiation to run; they equal tm, tn
// when the option's own layout fits.
void staged_wave_layout(long bm, long bn, long tm, long tn, long &ktm, long &ktn) {
  ktm = tm;
  ktn = tn;
  if (bm % tm || bn % tn || bm % 8 || bn % 8) return;
  const long threads = (bm / tm) * (bn / tn);
  if (threads < 64) {
    ktm = bm / 8;
    ktn = bn / 8;
  } else if (8 * tm > bm && (tm * tn) % (bm / 8) == 0) {
    ktm = bm / 8;
    ktn = tm * tn / ktm;
  } else if (8 * tn > bn && (tm * tn) % (bn / 8) == 0) {
    ktn = bn / 8;
    ktm = tm * tn / ktn;
  }
  if (8 * ktm > bm || 8 * ktn > bn || bm % ktm || bn % ktn) {
    ktm = tm;
    ktn = tn;
  }
}

struct Launch {
  const tfk::KernelEntry *entry = nullptr;
  dim3 grid, block;
};

long ceil_div(long a, long b) { return (a + b - 1) / b; }

}  // namespace

struct tf_kernel {
  tff::Program prog;
  tff::Options opts;
  tff::Plan plan;
  std::vector<Launch> launches;
  int device = -1;
  std::vector<void *> inter;  // intermediate device buffers, by buffer id
  // Split-K partial sums, shared by the stages (they run in stream order).
  size_t ws_bytes = 0;
  void *ws = nullptr;
  std::vector<double> samples;
  ~tf_kernel() {
    for (void *p : inter)
      if (p) (void)hipFree(p);
    if (ws) (void)hipFree(ws);
  }
};

// ------------------------------------------------------------- helpers ---

namespace {

int select_launches(tf_kernel *k) {
  const tff::Options &o = k->opts;
  for (const tff::Stage &st : k->plan.stages) {
    Launch L;
    const bool gemm = st.kind == tff::STAGE_GEMM;
    const bool staged = gemm && o.tile_k > 0;
    // Shapes that are not tile multiples (allowed by mask-edges) run the
    // masked twin of the configuration.
    const int masked = staged && (st.M % o.bm || st.N % o.bn || st.K % o.tile_k) ? 1 : 0;
    if (masked && !o.promote)
      return fail(TF_E_PLAN, tff::format_error(k->prog.source_name, st.loc,
                                                "tforge-gpu-pipeline: mask-edges needs promote=1 for shapes that are "
                                                "not multiples of the block and K tiles"));
    // Masked kernels index A and B with 32-bit offsets (tiles may run one
    // block past the edges).
    if (masked && ((st.M + 256) * st.K >= (1L << 31) || (st.K + 64) * (st.N + 256) >= (1L << 31)))
      return fail(TF_E_PLAN, tff::format_error(k->prog.source_name, st.loc,
                                                "tforge-gpu-pipeline: mask-edges supports matrices below 2^31 "
                                                "elements; pad this problem instead"));
    // wave-split-k: the wave-split kernel for GEMM stages.
    const bool wavek = o.wave_split_k && gemm;
    if (wavek) {
      std::string why;
      if (!staged) why = "wave-split-k needs tile-k";
      else if (masked) why = "wave-split-k needs M, N and K to be multiples of the block and K tiles (pad the problem)";
      else if (!o.promote || !o.vectorize) why = "wave-split-k needs promote=1 vectorize=1";
      // 32-bit buffer offsets from the tile's origin in A and in B.
      else if ((o.bm * st.K + st.K) * 4 >= (1L << 31) || (st.K * st.N + o.bn) * 4 >= (1L << 31))
        why = "wave-split-k supports (BM+1)*K and K*N below 2^29 elements";
      if (!why.empty()) return fail(TF_E_PLAN, tff::format_error(k->prog.source_name, st.loc, "tforge-gpu-pipeline: " + why));
    }
    // The staged kernel's thread tile: the option's own, or the wave layout
    // that stands in for it when 8*TM x 8*TN waves cannot tile the block.
    long ktm = o.tm, ktn = o.tn;
    if (staged && !wavek) staged_wave_layout(o.bm, o.bn, o.tm, o.tn, ktm, ktn);
    for (const tfk::KernelEntry *e = tfk::registry_begin(); e != tfk::registry_end(); ++e) {
      if (wavek) {
        if (e->family == tfk::FAM_WAVEK && e->bm == o.bm && e->bn == o.bn && e->tm == o.tm && e->tn == o.tn &&
            e->bk == o.tile_k) {
          L.entry = e;
          break;
        }
      } else if (staged) {
        if (e->family == tfk::FAM_STAGED && e->bm == o.bm && e->bn == o.bn && e->tm == ktm && e->tn == ktn &&
            e->bk == o.tile_k && e->promote == (int)o.promote && e->vectorize == (int)o.vectorize &&
            e->masked == masked) {
          L.entry = e;
          break;
        }
      } else {
        const int fam = gemm ? tfk::FAM_DIRECT : tfk::FAM_ELEMENTWISE;
        if (e->family == fam && e->tm == o.tm && e->tn == o.tn) {
          L.entry = e;
          break;
        }
      }
    }
    if (!L.entry && masked) {
      const long threads = (o.bm / ktm) * (o.bn / ktn);
      const long vw = o.vectorize ? 4 : 1;
      const long vecs = (o.bm * o.tile_k / vw + threads - 1) / threads + (o.tile_k * o.bn / vw + threads - 1) / threads;
      if (vecs > 16)
        return fail(TF_E_PLAN, tff::format_error(k->prog.source_name, st.loc,
                                                  "tforge-gpu-pipeline: mask-edges has no instantiation for a "
                                                  "configuration whose threads stage " + std::to_string(vecs) +
                                                      " vectors per slab (at most 16); use more threads or a smaller "
                                                      "tile-k, or pad the problem"));
    }
    if (!L.entry && wavek)
      return fail(TF_E_PLAN, tff::format_error(k->prog.source_name, st.loc,
                                                "tforge-gpu-pipeline: wave-split-k has no instantiation of this "
                                                "configuration; wave-split configurations are listed by "
                                                "tf_registry_entry"));
    if (!L.entry) {
      std::string why = staged ? staged_reason(o.bm, o.bn, ktm, ktn, o.tile_k, o.promote)
                               : "thread-tile " + std::to_string(o.tm) + "," + std::to_string(o.tn) +
                                     " has no instantiation (1, 2, 4 or 8 per dimension)";
      return fail(TF_E_PLAN, tff::format_error(k->prog.source_name, st.loc, "tforge-gpu-pipeline: " + why));
    }
    // The launch geometry is the instantiation's: (BN / TN, BM / TM) threads
    // as in the reference (lib/Pipelines/Pipelines.cpp:139), with the
    // stand-in thread tile where one replaced the option's.
    const long tx = o.bn / ktn, ty = o.bm / ktm;
    if (tx * ty > 1024)
      return fail(TF_E_PLAN, tff::format_error(k->prog.source_name, st.loc,
                                                "tforge-gpu-pipeline: " + std::to_string(tx * ty) +
                                                    " threads per block exceeds 1024"));
    L.block = dim3((unsigned)tx, (unsigned)ty, 1);
    L.grid = dim3((unsigned)std::max(1L, ceil_div(st.N, o.bn)), (unsigned)std::max(1L, ceil_div(st.M, o.bm)), 1);
    // split-k splits the K loop of GEMM stages; the element-op launches of an
    // unfused program run as they are.  Without tile-k it is an error.
    if (o.split_k > 1 && (gemm || o.tile_k == 0)) {
      if (!staged)
        return fail(TF_E_PLAN, tff::format_error(k->prog.source_name, st.loc,
                                                  "tforge-gpu-pipeline: split-k needs tile-k"));
      const long slabs = ceil_div(st.K, o.tile_k);
      if (slabs < o.split_k)
        return fail(TF_E_PLAN, tff::format_error(k->prog.source_name, st.loc,
                                                  "tforge-gpu-pipeline: split-k " + std::to_string(o.split_k) +
                                                      " exceeds the " + std::to_string(slabs) +
                                                      " K slabs of this matmul"));
      L.grid.z = (unsigned)o.split_k;
      // Whole tiles per slice: (grid.y * BM) x (grid.x * BN).
      k->ws_bytes = std::max(k->ws_bytes, (size_t)o.split_k * L.grid.y * o.bm * L.grid.x * o.bn * sizeof(float));
    }
    k->launches.push_back(L);
  }
  return TF_OK;
}

tfk::EpiParams make_epi(const tff::Stage &st, void *const *ptrs) {
  tfk::EpiParams e{};
  e.nops = (int)st.epi.size();
  for (int i = 0; i < e.nops; ++i) {
    e.kind[i] = st.epi[i].kind;
    e.ptr[i] = st.epi[i].buf >= 0 ? static_cast<const float *>(ptrs[st.epi[i].buf]) : nullptr;
    e.ldr[i] = st.N;
  }
  return e;
}

// Enqueues stage s of k.  `ptrs` holds every buffer id's device pointer and
// `ws` the split-K workspace (k->ws_bytes bytes, or null when unused).
int launch_stage(const tf_kernel *k, size_t s, void *const *ptrs, void *ws, hipStream_t stream) {
  const tff::Stage &st = k->plan.stages[s];
  const Launch &L = k->launches[s];
  if (st.M == 0 || st.N == 0) return TF_OK;
  // 128-bit accesses need 16-byte aligned buffers (the reference's ABI
  // guarantees 256-byte alignment: docs/stage8.md:34).
  if (L.entry->family == tfk::FAM_STAGED || L.entry->family == tfk::FAM_WAVEK) {
    std::vector<int> ids = {st.a, st.b, st.out};
    for (const tff::EpiOp &e : st.epi)
      if (e.buf >= 0) ids.push_back(e.buf);
    for (int id : ids)
      if (reinterpret_cast<uintptr_t>(ptrs[id]) % 16 != 0)
        return fail(TF_E_ARG, "buffer " + std::to_string(id) + " is not 16-byte aligned");
  }
  hipError_t err;
  if (st.kind == tff::STAGE_GEMM) {
    tfk::GemmParams p{};
    p.A = static_cast<const float *>(ptrs[st.a]);
    p.B = static_cast<const float *>(ptrs[st.b]);
    p.C = static_cast<float *>(ptrs[st.out]);
    p.M = (int)st.M;
    p.N = (int)st.N;
    p.K = (int)st.K;
    p.lda = st.K;
    p.ldb = st.N;
    p.ldc = st.N;
    p.epi = make_epi(st, ptrs);
    p.swizzle = k->opts.xcd_swizzle ? 1 : 0;
    p.splits = (int)L.grid.z;
    if (p.splits > 1) {
      p.ws = static_cast<float *>(ws);
      p.ws_ld = (long)L.grid.x * L.entry->bn;
      p.ws_slice = p.ws_ld * L.grid.y * L.entry->bm;
    }
    err = L.entry->gemm(p, L.grid, L.block, stream);
    if (err == hipSuccess && p.splits > 1) {
      tfk::ReduceParams r{};
      r.ws = p.ws;
      r.C = p.C;
      r.M = p.M;
      r.N = p.N;
      r.splits = p.splits;
      r.ws_ld = p.ws_ld;
      r.ws_slice = p.ws_slice;
      r.ldc = p.ldc;
      r.epi = p.epi;
      err = tfk::launch_splitk_reduce(r, stream);
    }
  } else {
    tfk::EltParams p{};
    p.X = static_cast<const float *>(ptrs[st.x]);
    p.Y = static_cast<float *>(ptrs[st.out]);
    p.M = (int)st.M;
    p.N = (int)st.N;
    p.ldx = st.N;
    p.ldy = st.N;
    p.epi = make_epi(st, ptrs);
    bool vec = st.N % 4 == 0;
    auto aligned = [](const void *q) { return reinterpret_cast<uintptr_t>(q) % 16 == 0; };
    vec = vec && aligned(p.X) && aligned(p.Y);
    for (int i = 0; i < p.epi.nops; ++i)
      if (p.epi.ptr[i]) vec = vec && aligned(p.epi.ptr[i]);
    p.vec_ok = vec ? 1 : 0;
    err = L.entry->elt(p, L.grid, L.block, stream);
  }
  if (err != hipSuccess)
    return fail(TF_E_HIP, std::string("kernel launch ") + L.entry->name + " failed: " + hipGetErrorString(err));
  return TF_OK;
}

// Full pointer table (arguments, result, intermediates) for a launch.
int pointer_table(tf_kernel *k, void *const *bufs, std::vector<void *> &ptrs) {
  const tff::Plan &pl = k->plan;
  ptrs.assign(pl.buffers.size(), nullptr);
  for (int i = 0; i <= pl.nargs; ++i) ptrs[i] = bufs[i];
  int dev = 0;
  TF_HIP(hipGetDevice(&dev));
  if (k->device != dev) {
    for (void *p : k->inter)
      if (p) (void)hipFree(p);
    k->inter.assign(pl.buffers.size(), nullptr);
    if (k->ws) (void)hipFree(k->ws);
    k->ws = nullptr;
    k->device = dev;
  }
  for (size_t i = pl.nargs + 1; i < pl.buffers.size(); ++i) {
    if (!k->inter[i]) TF_HIP(hipMalloc(&k->inter[i], std::max<int64_t>(1, pl.buffers[i].numel()) * sizeof(float)));
    ptrs[i] = k->inter[i];
  }
  if (k->ws_bytes && !k->ws) TF_HIP(hipMalloc(&k->ws, k->ws_bytes));
  return TF_OK;
}

// ------------------------------------------------------------ runner ---

// amdsmi, loaded lazily: socket power per rep, as the reference samples NVML
// (runners/gpu/tforge-gpu-bench.cu:333-361).  Missing -> -1.  (The clock comes
// from clock_probe: amdsmi's current clock, read once a short rep has ended,
// is already the idle clock.)
struct Smi {
  bool ok = false;
  void *h = nullptr;
  void *proc = nullptr;
  typedef int (*init_t)(uint64_t);
  typedef int (*sockets_t)(uint32_t *, void **);
  typedef int (*procs_t)(void *, uint32_t *, void **);
  struct pwr_t {
    uint64_t socket_power;
    uint32_t current_socket_power, average_socket_power;
    uint64_t gfx_voltage, soc_voltage, mem_voltage;
    uint32_t power_limit;
    uint64_t reserved[18];
  };
  typedef int (*power_t)(void *, pwr_t *);
  power_t get_power = nullptr;

  Smi() {
    if (std::getenv("TF_NO_SMI")) return;
    h = dlopen("libamd_smi.so", RTLD_NOW | RTLD_LOCAL);
    if (!h) h = dlopen("/opt/rocm/lib/libamd_smi.so", RTLD_NOW | RTLD_LOCAL);
    if (!h) return;
    auto init = (init_t)dlsym(h, "amdsmi_init");
    auto sockets = (sockets_t)dlsym(h, "amdsmi_get_socket_handles");
    auto procs = (procs_t)dlsym(h, "amdsmi_get_processor_handles");
    get_power = (power_t)dlsym(h, "amdsmi_get_power_info");
    if (!init || !sockets || !procs || !get_power || init(1u << 1) != 0) return;
    uint32_t ns = 0;
    if (sockets(&ns, nullptr) != 0 || ns == 0) return;
    std::vector<void *> socks(ns);
    if (sockets(&ns, socks.data()) != 0) return;
    for (void *s : socks) {
      uint32_t np = 0;
      if (procs(s, &np, nullptr) != 0 || np == 0) continue;
      std::vector<void *> ps(np);
      if (procs(s, &np, ps.data()) != 0) continue;
      proc = ps[0];
      break;
    }
    ok = proc != nullptr;
  }
  double power_w() {
    pwr_t p{};
    if (!ok || !get_power || get_power(proc, &p) != 0) return -1;
    if (p.current_socket_power != UINT32_MAX && p.current_socket_power) return p.current_socket_power;
    if (p.average_socket_power != UINT32_MAX) return p.average_socket_power;
    return -1;
  }
};

Smi &smi() {
  static Smi s;
  return s;
}

// rocBLAS, loaded lazily: the vendor-library baseline (--mode cublas in the
// reference: runners/gpu/tforge-gpu-bench.cu:303-318).
struct Blas {
  bool ok = false;
  void *h = nullptr, *handle = nullptr;
  typedef int (*create_t)(void **);
  typedef int (*stream_t)(void *, hipStream_t);
  typedef int (*sgemm_t)(void *, int, int, int, int, int, const float *, const float *, int, const float *, int,
                         const float *, float *, int);
  stream_t set_stream = nullptr;
  sgemm_t sgemm = nullptr;
  Blas() {
    h = dlopen("librocblas.so.5", RTLD_NOW | RTLD_LOCAL);
    if (!h) h = dlopen("librocblas.so", RTLD_NOW | RTLD_LOCAL);
    if (!h) return;
    auto create = (create_t)dlsym(h, "rocblas_create_handle");
    set_stream = (stream_t)dlsym(h, "rocblas_set_stream");
    sgemm = (sgemm_t)dlsym(h, "rocblas_sgemm");
    ok = create && set_stream && sgemm && create(&handle) == 0;
  }
};

Blas &blas() {
  static Blas b;
  return b;
}

struct DeviceBuf {
  void *p = nullptr;
  ~DeviceBuf() {
    if (p) (void)hipFree(p);
  }
};

struct Stats {
  double median, min, mean, sd;
};
Stats stats(std::vector<double> v) {
  if (v.empty()) return {-1, -1, -1, -1};
  std::sort(v.begin(), v.end());
  const size_t n = v.size();
  double mean = 0;
  for (double x : v) mean += x;
  mean /= n;
  double var = 0;
  for (double x : v) var += (x - mean) * (x - mean);
  const double med = n % 2 ? v[n / 2] : 0.5 * (v[n / 2 - 1] + v[n / 2]);
  return {med, v.front(), mean, n > 1 ? std::sqrt(var / (n - 1)) : 0.0};
}

// Shader-clock probe: each workgroup (one per XCD: workgroups are dealt to the
// 8 XCDs round-robin) spins for 4 us of the 100 MHz wall clock and records the
// shader-clock cycles (s_memtime) that passed meanwhile.  The spin also ends
// after 2^20 reads, so the kernel exits whatever the counters do.  Each call
// takes the next of kProbeSlots result slots (round robin), so up to that
// many calls may run at once, from any threads and streams, without sharing
// one.
constexpr int kProbeGroups = 8;
constexpr int kProbeSlots = 64;
__device__ unsigned long long g_clock_probe[kProbeSlots][2 * kProbeGroups];
static std::atomic<unsigned> g_probe_next{0};

__global__ void clock_probe_kernel(unsigned long long *out) {
  if (threadIdx.x != 0) return;
  const unsigned long long w0 = wall_clock64(), c0 = clock64();
  unsigned long long w1 = w0;
  for (int i = 0; i < (1 << 20) && w1 - w0 < 400; ++i) w1 = wall_clock64();
  const unsigned long long c1 = clock64();
  out[2 * blockIdx.x] = c1 - c0;
  out[2 * blockIdx.x + 1] = w1 - w0;
}

// Mean, min and max shader clock (MHz) over the XCDs, measured on `stream`
// after the work already queued there.  Synchronises the stream.
int clock_probe(hipStream_t stream, double &mean, double &mn, double &mx) {
  static thread_local int probe_dev = -1;
  static thread_local unsigned long long *probe_ptr = nullptr;
  static thread_local int wall_khz = 0;
  int dev = 0;
  TF_HIP(hipGetDevice(&dev));
  if (dev != probe_dev) {
    TF_HIP(hipGetSymbolAddress(reinterpret_cast<void **>(&probe_ptr), HIP_SYMBOL(g_clock_probe)));
    TF_HIP(hipDeviceGetAttribute(&wall_khz, hipDeviceAttributeWallClockRate, dev));
    probe_dev = dev;
  }
  unsigned long long *slot = probe_ptr + (size_t)(g_probe_next.fetch_add(1) % kProbeSlots) * 2 * kProbeGroups;
  hipLaunchKernelGGL(clock_probe_kernel, dim3(kProbeGroups), dim3(64), 0, stream, slot);
  TF_HIP(hipGetLastError());
  unsigned long long h[2 * kProbeGroups];
  TF_HIP(hipMemcpyAsync(h, slot, sizeof(h), hipMemcpyDeviceToHost, stream));
  TF_HIP(hipStreamSynchronize(stream));
  mean = 0;
  mn = 1e30;
  mx = 0;
  for (int g = 0; g < kProbeGroups; ++g) {
    if (h[2 * g + 1] == 0) return fail(TF_E_HIP, "clock probe: the wall clock did not advance");
    const double mhz = double(h[2 * g]) * wall_khz / (double(h[2 * g + 1]) * 1000.0);
    mean += mhz / kProbeGroups;
    mn = std::min(mn, mhz);
    mx = std::max(mx, mhz);
  }
  return TF_OK;
}

__global__ void fill_u32(uint32_t *p, size_t n, uint32_t v) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = v;
}

// A prepared execution of one program: device buffers at the logical shape,
// padded copies when the compiled shape is larger, and the run() closure that
// the reference's runner times (pad copies + launch(es) + unpad copy).
struct Exec {
  tf_kernel *k = nullptr;
  int mode = TF_MODE_KERNEL;
  hipStream_t stream = nullptr;
  std::vector<DeviceBuf> logical, padded;
  std::vector<void *> ptrs;          // what the kernels see
  std::vector<int64_t> lrows, lcols;  // logical 2-D shape per argN buffer
  std::vector<int64_t> prows, pcols;  // compiled 2-D shape per argN buffer
  bool is_padded = false;
  int64_t M = 0, N = 0, K = 0;        // logical problem of a single-matmul program
  ~Exec() {
    if (stream) (void)hipStreamDestroy(stream);
  }
};

void buffer_2d(const tff::Buffer &b, int64_t &rows, int64_t &cols) {
  cols = b.shape.empty() ? 1 : b.shape.back();
  rows = 1;
  for (size_t i = 0; i + 1 < b.shape.size(); ++i) rows *= b.shape[i];
}

// Host-side 2-D shape of every argN buffer (entry arguments, then the result)
// as tf_run and tf_bench copy it: the compiled shape, or, with logical sizes
// (a single-matmul program compiled at a padded shape), the logical shape of
// the buffer's role in the chain -- A m x k, B k x n, bias 1 x n, residual and
// C m x n.  An argument with no role keeps its compiled shape.  A buffer with
// two roles whose logical shapes differ (A reused as the residual with k != n)
// cannot be padded consistently, and is refused.
int host_shapes(const tf_kernel *k, const long long *logical, std::vector<int64_t> &rows,
                std::vector<int64_t> &cols) {
  const tff::Plan &pl = k->plan;
  const int nb = pl.nargs + 1;
  rows.assign(nb, 0);
  cols.assign(nb, 0);
  for (int i = 0; i < nb; ++i) buffer_2d(pl.buffers[i], rows[i], cols[i]);
  if (!logical) return TF_OK;
  const bool single_gemm = pl.stages.size() == 1 && pl.stages[0].kind == tff::STAGE_GEMM;
  if (!single_gemm) return fail(TF_E_ARG, "logical (unpadded) sizes apply to single-matmul programs only");
  const tff::Stage &st = pl.stages[0];
  const int64_t m = logical[0], n = logical[1], kk = logical[2];
  if (m <= 0 || n <= 0 || kk <= 0 || m > st.M || n > st.N || kk > st.K)
    return fail(TF_E_ARG, "padded sizes must be >= M, N, K");
  std::vector<std::string> role(nb);
  auto assign = [&](int id, int64_t r, int64_t c, const char *what) {
    if (id < 0 || id >= nb) return TF_OK;  // an intermediate
    if (!role[id].empty() && (rows[id] != r || cols[id] != c))
      return fail(TF_E_ARG, "buffer " + std::to_string(id) + " (" + pl.buffers[id].name + ") is both the " +
                                role[id] + " and the " + what +
                                ", whose logical shapes differ; compile the program at its logical shape "
                                "(mask-edges) instead of padding it");
    rows[id] = r;
    cols[id] = c;
    role[id] = what;
    return TF_OK;
  };
  int rc = assign(st.a, m, kk, "matmul lhs");
  if (!rc) rc = assign(st.b, kk, n, "matmul rhs");
  if (!rc) rc = assign(st.out, m, n, "result");
  for (const tff::EpiOp &e : st.epi)
    if (!rc && e.buf >= 0)
      rc = e.kind == tfk::EPI_BIAS ? assign(e.buf, 1, n, "bias") : assign(e.buf, m, n, "add operand");
  return rc;
}

int prepare(tf_kernel *k, int mode, const long long *logical, const float *const *host_in, unsigned seed, Exec &ex) {
  ex.k = k;
  ex.mode = mode;
  const tff::Plan &pl = k->plan;
  const int nb = pl.nargs + 1;
  if (mode != TF_MODE_KERNEL && mode != TF_MODE_BLAS) return fail(TF_E_ARG, "mode must be TF_MODE_KERNEL or TF_MODE_BLAS");
  const bool single_gemm = pl.stages.size() == 1 && pl.stages[0].kind == tff::STAGE_GEMM;
  if (mode == TF_MODE_BLAS && !single_gemm) return fail(TF_E_BLAS, "blas mode needs a program with one matmul chain");
  int rc = host_shapes(k, logical, ex.lrows, ex.lcols);
  if (rc) return rc;
  rc = host_shapes(k, nullptr, ex.prows, ex.pcols);
  if (rc) return rc;
  if (single_gemm) {
    const tff::Stage &st = pl.stages[0];
    ex.M = logical ? logical[0] : st.M;
    ex.N = logical ? logical[1] : st.N;
    ex.K = logical ? logical[2] : st.K;
    ex.is_padded = mode == TF_MODE_KERNEL && (ex.M != st.M || ex.N != st.N || ex.K != st.K);
  }
  TF_HIP(hipSetDevice(0));
  TF_HIP(hipStreamCreate(&ex.stream));
  ex.logical.resize(nb);
  std::mt19937 rng(seed);
  std::uniform_real_distribution<float> dist(-1.0f, 1.0f);
  for (int i = 0; i < nb; ++i) {
    const size_t bytes = std::max<int64_t>(1, ex.lrows[i] * ex.lcols[i]) * sizeof(float);
    TF_HIP(hipMalloc(&ex.logical[i].p, bytes));
    if (i < pl.nargs) {
      if (host_in) {
        TF_HIP(hipMemcpy(ex.logical[i].p, host_in[i], ex.lrows[i] * ex.lcols[i] * sizeof(float), hipMemcpyHostToDevice));
      } else {
        std::vector<float> h(ex.lrows[i] * ex.lcols[i]);
        for (float &x : h) x = dist(rng);
        TF_HIP(hipMemcpy(ex.logical[i].p, h.data(), h.size() * sizeof(float), hipMemcpyHostToDevice));
      }
    }
  }
  std::vector<void *> args(nb);
  if (ex.is_padded) {
    // Zeroed once: the pad regions are never written, so they add exact
    // zeros to every dot product (runners/gpu/tforge-gpu-bench.cu:217-219).
    ex.padded.resize(nb);
    for (int i = 0; i < nb; ++i) {
      const size_t bytes = std::max<int64_t>(1, ex.prows[i] * ex.pcols[i]) * sizeof(float);
      TF_HIP(hipMalloc(&ex.padded[i].p, bytes));
      TF_HIP(hipMemset(ex.padded[i].p, 0, bytes));
      args[i] = ex.padded[i].p;
    }
  } else {
    for (int i = 0; i < nb; ++i) args[i] = ex.logical[i].p;
  }
  if (mode == TF_MODE_KERNEL) {
    int rc = pointer_table(k, args.data(), ex.ptrs);
    if (rc) return rc;
  } else {
    ex.ptrs = args;
    if (!blas().ok) return fail(TF_E_BLAS, "rocBLAS (librocblas.so) could not be loaded or initialised");
  }
  return TF_OK;
}

int run_once(Exec &ex) {
  tf_kernel *k = ex.k;
  const tff::Plan &pl = k->plan;
  const int nb = pl.nargs + 1;
  if (ex.mode == TF_MODE_BLAS) {
    const tff::Stage &st = pl.stages[0];
    const float one = 1.0f, zero = 0.0f;
    Blas &b = blas();
    if (b.set_stream(b.handle, ex.stream) != 0) return fail(TF_E_BLAS, "rocblas_set_stream failed");
    // Row-major C = A B as column-major C^T = B^T A^T; FP32 in, FP32 compute.
    const int M = (int)ex.M, N = (int)ex.N, K = (int)ex.K;
    int rc = b.sgemm(b.handle, 111, 111, N, M, K, &one, static_cast<const float *>(ex.ptrs[st.b]), N,
                     static_cast<const float *>(ex.ptrs[st.a]), K, &zero, static_cast<float *>(ex.ptrs[st.out]), N);
    if (rc != 0) return fail(TF_E_BLAS, "rocblas_sgemm failed with status " + std::to_string(rc));
    if (!st.epi.empty()) {
      // The separate epilogue kernel, in place on C.
      const tfk::KernelEntry *e = nullptr;
      for (const tfk::KernelEntry *x = tfk::registry_begin(); x != tfk::registry_end(); ++x)
        if (x->family == tfk::FAM_ELEMENTWISE && x->tm == 1 && x->tn == 1) e = x;
      tfk::EltParams p{};
      p.X = static_cast<const float *>(ex.ptrs[st.out]);
      p.Y = static_cast<float *>(ex.ptrs[st.out]);
      p.M = M;
      p.N = N;
      p.ldx = p.ldy = N;
      p.epi = make_epi(st, ex.ptrs.data());
      for (int i = 0; i < p.epi.nops; ++i) p.epi.ldr[i] = N;
      hipError_t err = e->elt(p, dim3((N + 15) / 16, (M + 15) / 16, 1), dim3(16, 16, 1), ex.stream);
      if (err != hipSuccess) return fail(TF_E_HIP, std::string("epilogue launch failed: ") + hipGetErrorString(err));
    }
    return TF_OK;
  }
  if (ex.is_padded) {
    for (int i = 0; i < pl.nargs; ++i)
      TF_HIP(hipMemcpy2DAsync(ex.padded[i].p, ex.pcols[i] * 4, ex.logical[i].p, ex.lcols[i] * 4, ex.lcols[i] * 4,
                              ex.lrows[i], hipMemcpyDeviceToDevice, ex.stream));
  }
  for (size_t s = 0; s < pl.stages.size(); ++s) {
    int rc = launch_stage(k, s, ex.ptrs.data(), k->ws, ex.stream);
    if (rc) return rc;
  }
  if (ex.is_padded) {
    const int o = pl.nargs;
    TF_HIP(hipMemcpy2DAsync(ex.logical[o].p, ex.lcols[o] * 4, ex.padded[o].p, ex.pcols[o] * 4, ex.lcols[o] * 4,
                            ex.lrows[o], hipMemcpyDeviceToDevice, ex.stream));
  }
  (void)nb;
  return TF_OK;
}

}  // namespace

// ---------------------------------------------------------------- C ABI ---

extern "C" {

const char *tf_last_error(void) { return g_err.c_str(); }

int tf_device_info(tf_device_info_t *out) {
  if (!out) return fail(TF_E_ARG, "null output");
  hipDeviceProp_t prop;
  TF_HIP(hipGetDeviceProperties(&prop, 0));
  std::memset(out, 0, sizeof(*out));
  copy_str(out->name, sizeof(out->name), prop.name);
  copy_str(out->arch, sizeof(out->arch), prop.gcnArchName);
  out->compute_units = prop.multiProcessorCount;
  out->max_clock_mhz = prop.clockRate / 1000;
  out->lds_bytes_per_cu = (int)prop.maxSharedMemoryPerMultiProcessor;
  out->max_threads_per_cu = prop.maxThreadsPerMultiProcessor;
  out->l2_bytes = prop.l2CacheSize;
  out->global_mem_bytes = (long long)prop.totalGlobalMem;
  TF_HIP(hipDriverGetVersion(&out->driver_version));
  TF_HIP(hipRuntimeGetVersion(&out->runtime_version));
  return TF_OK;
}

static int compile_impl(const char *source_name, const char *program, const char *options, tf_kernel_t **out) {
  if (!program || !out) return fail(TF_E_ARG, "null program or output handle");
  *out = nullptr;
  std::unique_ptr<tf_kernel> k(new tf_kernel());
  std::string err;
  const std::string src = source_name ? source_name : "<input>";
  if (!tff::parse_program(program, src, k->prog, err) || !tff::verify_program(k->prog, err)) {
    return fail(TF_E_PARSE, err);
  }
  if (!tff::parse_options(options ? options : "", k->opts, err)) {
    return fail(TF_E_OPTIONS, err);
  }
  if (!tff::plan_program(k->prog, k->opts, k->plan, err)) {
    return fail(TF_E_PLAN, err);
  }
  int rc = select_launches(k.get());
  if (rc) return rc;
  if (k->opts.print_script || k->opts.print_after_each) {
    for (size_t s = 0; s < k->plan.stages.size(); ++s) {
      const tff::Stage &st = k->plan.stages[s];
      const Launch &L = k->launches[s];
      std::fprintf(stderr, "// tforge-gpu: launch %zu: %s -> %s grid [%u, %u, 1] block [%u, %u, 1] M=%lld N=%lld K=%lld\n",
                   s, st.ops.c_str(), L.entry->name, L.grid.x, L.grid.y, L.block.x, L.block.y, (long long)st.M,
                   (long long)st.N, (long long)st.K);
    }
  }
  *out = k.release();
  return TF_OK;
}

void tf_kernel_free(tf_kernel_t *k) { delete k; }

int tf_kernel_num_launches(const tf_kernel_t *k) { return k ? (int)k->launches.size() : fail(TF_E_ARG, "null kernel"); }

int tf_kernel_launch_info(const tf_kernel_t *k, int launch, tf_launch_info_t *out) {
  if (!k || !out || launch < 0 || launch >= (int)k->launches.size()) return fail(TF_E_ARG, "bad launch index");
  const tff::Stage &st = k->plan.stages[launch];
  const Launch &L = k->launches[launch];
  std::memset(out, 0, sizeof(*out));
  copy_str(out->kernel, sizeof(out->kernel), L.entry->name);
  copy_str(out->ops, sizeof(out->ops), st.ops);
  // Buffer order of this launch in the reference's argN spelling: result first,
  // then operands (the reference's launch lists the out-param first:
  // results/gpu/stage8_ir/full-128x64-t8x4-k16_mbr_2048/launch.json).
  auto argname = [&](int id) {
    return id <= k->plan.nargs ? "arg" + std::to_string(id) : std::string("tmp") + std::to_string(id);
  };
  std::string args = argname(st.out);
  if (st.kind == tff::STAGE_GEMM) args += "," + argname(st.a) + "," + argname(st.b);
  else args += "," + argname(st.x);
  for (const tff::EpiOp &e : st.epi)
    if (e.buf >= 0) args += "," + argname(e.buf);
  copy_str(out->args, sizeof(out->args), args);
  out->family = L.entry->family;
  out->grid[0] = L.grid.x;
  out->grid[1] = L.grid.y;
  out->grid[2] = L.grid.z;
  out->block[0] = L.block.x;
  out->block[1] = L.block.y;
  out->block[2] = L.block.z;
  out->m = st.M;
  out->n = st.N;
  out->k = st.kind == tff::STAGE_GEMM ? st.K : 0;
  out->lds_bytes = L.entry->lds_bytes;
  return TF_OK;
}

int tf_kernel_num_buffers(const tf_kernel_t *k) { return k ? k->plan.nargs + 1 : fail(TF_E_ARG, "null kernel"); }

int tf_kernel_buffer_info(const tf_kernel_t *k, int index, tf_buffer_info_t *out) {
  if (!k || !out || index < 0 || index > k->plan.nargs) return fail(TF_E_ARG, "bad buffer index");
  const tff::Buffer &b = k->plan.buffers[index];
  std::memset(out, 0, sizeof(*out));
  copy_str(out->name, sizeof(out->name), b.name);
  out->role = b.role;
  int64_t r, c;
  buffer_2d(b, r, c);
  out->rows = r;
  out->cols = c;
  return TF_OK;
}

int tf_kernel_info(const tf_kernel_t *k, int launch, tf_kernel_resources_t *out) {
  if (!k || !out || launch < 0 || launch >= (int)k->launches.size()) return fail(TF_E_ARG, "bad launch index");
  const Launch &L = k->launches[launch];
  hipFuncAttributes attr;
  TF_HIP(hipFuncGetAttributes(&attr, L.entry->fn));
  const int threads = (int)(L.block.x * L.block.y * L.block.z);
  int blocks = 0;
  TF_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, L.entry->fn, threads, 0));
  hipDeviceProp_t prop;
  TF_HIP(hipGetDeviceProperties(&prop, 0));
  std::memset(out, 0, sizeof(*out));
  out->regs = attr.numRegs;
  out->local_bytes = (int)attr.localSizeBytes;
  out->static_smem = (int)attr.sharedSizeBytes;
  out->blocks_per_cu = blocks;
  out->threads = threads;
  const int waves = (threads + 63) / 64, max_waves = prop.maxThreadsPerMultiProcessor / 64;
  out->theo_occupancy = max_waves > 0 ? double(blocks * waves) / max_waves : 0.0;
  return TF_OK;
}

int tf_kernel_host_shape(const tf_kernel_t *k, const long long *logical_mnk, int index, long long *rows,
                         long long *cols) {
  if (!k || !rows || !cols || index < 0 || index > k->plan.nargs) return fail(TF_E_ARG, "bad buffer index");
  std::vector<int64_t> r, c;
  int rc = host_shapes(k, logical_mnk, r, c);
  if (rc) return rc;
  *rows = r[index];
  *cols = c[index];
  return TF_OK;
}

// A null pointer for a buffer that a launch reads or writes would fault the
// GPU; it is refused here, before anything is enqueued.
static int check_buffers(const tf_kernel_t *k, void *const *bufs) {
  for (int i = 0; i <= k->plan.nargs; ++i)
    if (!bufs[i] && k->plan.buffers[i].numel() > 0)
      return fail(TF_E_ARG, "buffer " + std::to_string(i) + " (" + k->plan.buffers[i].name + ") is a null pointer");
  return TF_OK;
}

static int launch_impl(tf_kernel_t *k, void *const *device_buffers, void *stream) {
  if (!k || !device_buffers) return fail(TF_E_ARG, "null kernel or buffers");
  int rc0 = check_buffers(k, device_buffers);
  if (rc0) return rc0;
  std::vector<void *> ptrs;
  int rc = pointer_table(k, device_buffers, ptrs);
  if (rc) return rc;
  for (size_t s = 0; s < k->plan.stages.size(); ++s) {
    rc = launch_stage(k, s, ptrs.data(), k->ws, static_cast<hipStream_t>(stream));
    if (rc) return rc;
  }
  return TF_OK;
}

// ------------------------------------------------ allocation-free launch ---
//
// tf_launch_noalloc takes the split-K workspace and the intermediates of
// multi-launch programs from `scratch`, one fixed array per GPU, instead of
// the handle's hipMalloc'd buffers.  The array's host-side name is only a
// stand-in: its device address, which differs per GPU, is fetched once per
// device with hipGetSymbolAddress and kept in g_scratch.
constexpr size_t kScratchBytes = size_t(32) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
struct ScratchSlot {
  std::once_flag once;
  void *ptr = nullptr;
  hipError_t err = hipSuccess;
};
static ScratchSlot g_scratch[kMaxDevices];

// Device address of the current device's scratch array.  `stream` must
// belong to the current device: the kernels run on the stream's device, and
// the address is that of the current device's copy.
static int scratch_base(hipStream_t stream, void **out) {
  int dev = 0;
  TF_HIP(hipGetDevice(&dev));
  if (stream) {
    int sdev = dev;
    TF_HIP(hipStreamGetDevice(stream, &sdev));
    if (sdev != dev)
      return fail(TF_E_ARG, "tf_launch_noalloc: the stream belongs to device " + std::to_string(sdev) +
                                " but device " + std::to_string(dev) + " is current; make the stream's device current");
  }
  if (dev < 0 || dev >= kMaxDevices) return fail(TF_E_ARG, "device " + std::to_string(dev) + " out of range");
  ScratchSlot &slot = g_scratch[dev];
  std::call_once(slot.once, [&] { slot.err = hipGetSymbolAddress(&slot.ptr, HIP_SYMBOL(scratch)); });
  if (slot.err != hipSuccess)
    return fail(TF_E_HIP, std::string("hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(slot.err));
  *out = slot.ptr;
  return TF_OK;
}

static int launch_noalloc_impl(tf_kernel_t *k, void *const *device_buffers, void *stream) {
  if (!k || !device_buffers) return fail(TF_E_ARG, "null kernel or buffers");
  int rc = check_buffers(k, device_buffers);
  if (rc) return rc;
  // Scratch layout: the split-K workspace, then each intermediate, each
  // starting on a 256-byte boundary.  Nothing needs clearing: every split
  // writes its whole slice before the reduction reads it, and every
  // intermediate is written whole by the launch that produces it.
  const tff::Plan &pl = k->plan;
  size_t used = 0;
  auto take = [&](size_t bytes) {
    const size_t at = used;
    used += (bytes + 255) / 256 * 256;
    return at;
  };
  const size_t ws_at = k->ws_bytes ? take(k->ws_bytes) : 0;
  std::vector<size_t> at(pl.buffers.size(), 0);
  for (size_t i = pl.nargs + 1; i < pl.buffers.size(); ++i)
    at[i] = take(std::max<int64_t>(1, pl.buffers[i].numel()) * sizeof(float));
  if (used > kScratchBytes)
    return fail(TF_E_ARG, "this program needs " + std::to_string(used) + " bytes of scratch (split-K workspace and "
                          "intermediates); tf_launch_noalloc has " + std::to_string(kScratchBytes) +
                          " per GPU: use tf_launch, which allocates them");
  void *base = nullptr;
  rc = scratch_base(static_cast<hipStream_t>(stream), &base);
  if (rc) return rc;
  std::vector<void *> ptrs(pl.buffers.size(), nullptr);
  for (int i = 0; i <= pl.nargs; ++i) ptrs[i] = device_buffers[i];
  for (size_t i = pl.nargs + 1; i < pl.buffers.size(); ++i) ptrs[i] = static_cast<unsigned char *>(base) + at[i];
  void *ws = k->ws_bytes ? static_cast<unsigned char *>(base) + ws_at : nullptr;
  for (size_t s = 0; s < pl.stages.size(); ++s) {
    rc = launch_stage(k, s, ptrs.data(), ws, static_cast<hipStream_t>(stream));
    if (rc) return rc;
  }
  return TF_OK;
}

static int run_impl(tf_kernel_t *k, int mode, const long long *logical_mnk, const float *const *host_inputs,
                    float *host_out) {
  if (!k || !host_inputs || !host_out) return fail(TF_E_ARG, "null kernel, inputs or output");
  for (int i = 0; i < k->plan.nargs; ++i)
    if (!host_inputs[i]) return fail(TF_E_ARG, "host input " + std::to_string(i) + " is a null pointer");
  Exec ex;
  int rc = prepare(k, mode, logical_mnk, host_inputs, 0, ex);
  if (rc) return rc;
  const int o = k->plan.nargs;
  // Correctness run: output pre-filled with NaN (0xFF bytes), as the reference
  // runner does (runners/gpu/tforge-gpu-bench.cu:323-331).
  TF_HIP(hipMemset(ex.logical[o].p, 0xFF, ex.lrows[o] * ex.lcols[o] * 4));
  if (ex.is_padded) TF_HIP(hipMemset(ex.padded[o].p, 0xFF, ex.prows[o] * ex.pcols[o] * 4));
  rc = run_once(ex);
  if (rc) return rc;
  TF_HIP(hipStreamSynchronize(ex.stream));
  TF_HIP(hipMemcpy(host_out, ex.logical[o].p, ex.lrows[o] * ex.lcols[o] * 4, hipMemcpyDeviceToHost));
  return TF_OK;
}

static int bench_impl(tf_kernel_t *k, int mode, const long long *logical_mnk, const float *const *host_inputs,
                      unsigned seed, int warmup, int reps, int flush, tf_bench_result_t *out) {
  if (!k || !out || warmup < 0 || reps < 1) return fail(TF_E_ARG, "bad bench arguments");
  for (int i = 0; host_inputs && i < k->plan.nargs; ++i)
    if (!host_inputs[i]) return fail(TF_E_ARG, "host input " + std::to_string(i) + " is a null pointer");
  Exec ex;
  int rc = prepare(k, mode, logical_mnk, host_inputs, seed, ex);
  if (rc) return rc;
  DeviceBuf flushbuf;
  const size_t flush_words = (size_t(512) << 20) / 4;  // 512 MiB > the 256 MB MALL
  if (flush) TF_HIP(hipMalloc(&flushbuf.p, flush_words * 4));
  hipEvent_t e0, e1;
  TF_HIP(hipEventCreate(&e0));
  TF_HIP(hipEventCreate(&e1));
  struct EvGuard {
    hipEvent_t a, b;
    ~EvGuard() {
      (void)hipEventDestroy(a);
      (void)hipEventDestroy(b);
    }
  } guard{e0, e1};
  for (int i = 0; i < warmup; ++i) {
    rc = run_once(ex);
    if (rc) return rc;
  }
  TF_HIP(hipStreamSynchronize(ex.stream));
  std::vector<double> ms(reps), clk, pwr;
  Smi &s = smi();
  for (int i = 0; i < reps; ++i) {
    if (flush) {
      hipLaunchKernelGGL(fill_u32, dim3(4096), dim3(256), 0, ex.stream, static_cast<uint32_t *>(flushbuf.p),
                         flush_words, (uint32_t)(i + 1));
      TF_HIP(hipGetLastError());
    }
    TF_HIP(hipEventRecord(e0, ex.stream));
    rc = run_once(ex);
    if (rc) return rc;
    TF_HIP(hipEventRecord(e1, ex.stream));
    TF_HIP(hipEventSynchronize(e1));
    float t = 0;
    TF_HIP(hipEventElapsedTime(&t, e0, e1));
    ms[i] = t;
    // The shader clock right after the rep, measured on the device (the
    // reference samples NVML per rep); power from amdsmi where it loads.
    double c = 0, cmin = 0, cmax = 0;
    rc = clock_probe(ex.stream, c, cmin, cmax);
    if (rc) return rc;
    clk.push_back(c);
    const double p = s.power_w();
    if (p > 0) pwr.push_back(p);
  }
  TF_HIP(hipGetLastError());
  const Stats st = stats(ms), cs = stats(clk), ps = stats(pwr);
  std::memset(out, 0, sizeof(*out));
  out->median_ms = st.median;
  out->min_ms = st.min;
  out->mean_ms = st.mean;
  out->std_ms = st.sd;
  out->clock_median_mhz = cs.median;
  out->clock_min_mhz = cs.min;
  out->clock_max_mhz = clk.empty() ? -1 : *std::max_element(clk.begin(), clk.end());
  out->power_median_w = ps.median;
  out->warmup = warmup;
  out->reps = reps;
  out->l2_flush = flush ? 1 : 0;
  if (k->plan.stages.size() == 1 && k->plan.stages[0].kind == tff::STAGE_GEMM && mode == TF_MODE_KERNEL) {
    out->padded[0] = k->plan.stages[0].M;
    out->padded[1] = k->plan.stages[0].N;
    out->padded[2] = k->plan.stages[0].K;
  } else {
    out->padded[0] = ex.M;
    out->padded[1] = ex.N;
    out->padded[2] = ex.K;
  }
  k->samples = ms;
  return TF_OK;
}

int tf_clock_probe(void *stream, double *mean_mhz, double *min_mhz, double *max_mhz) {
  if (!mean_mhz) return fail(TF_E_ARG, "null output");
  double mean = 0, mn = 0, mx = 0;
  int rc = clock_probe(static_cast<hipStream_t>(stream), mean, mn, mx);
  if (rc) return rc;
  *mean_mhz = mean;
  if (min_mhz) *min_mhz = mn;
  if (max_mhz) *max_mhz = mx;
  return TF_OK;
}

int tf_bench_samples(const tf_kernel_t *k, double *out_ms, int cap) {
  if (!k || (!out_ms && cap > 0)) return fail(TF_E_ARG, "null kernel or output");
  const int n = std::min<int>(cap, (int)k->samples.size());
  for (int i = 0; i < n; ++i) out_ms[i] = k->samples[i];
  return n;
}

int tf_registry_size(void) { return (int)(tfk::registry_end() - tfk::registry_begin()); }

int tf_registry_entry(int i, int *family, int *cfg7, char *name, int name_cap) {
  if (i < 0 || i >= tf_registry_size()) return fail(TF_E_ARG, "bad registry index");
  const tfk::KernelEntry &e = tfk::registry_begin()[i];
  if (family) *family = e.family;
  if (cfg7) {
    const int v[7] = {e.bm, e.bn, e.tm, e.tn, e.bk, e.promote, e.vectorize};
    std::memcpy(cfg7, v, sizeof(v));
  }
  if (name && name_cap > 0) std::snprintf(name, name_cap, "%s", e.name);
  return TF_OK;
}

// The entry points above that parse user text or allocate host memory run
// behind this guard: no C++ exception crosses the C ABI.
int tf_compile(const char *source_name, const char *program, const char *options, tf_kernel_t **out) {
  return guarded([&] { return compile_impl(source_name, program, options, out); });
}

int tf_launch(tf_kernel_t *k, void *const *device_buffers, void *stream) {
  return guarded([&] { return launch_impl(k, device_buffers, stream); });
}

int tf_launch_noalloc(tf_kernel_t *k, void *const *device_buffers, void *stream) {
  return guarded([&] { return launch_noalloc_impl(k, device_buffers, stream); });
}

int tf_run(tf_kernel_t *k, int mode, const long long *logical_mnk, const float *const *host_inputs, float *host_out) {
  return guarded([&] { return run_impl(k, mode, logical_mnk, host_inputs, host_out); });
}

int tf_bench(tf_kernel_t *k, int mode, const long long *logical_mnk, const float *const *host_inputs, unsigned seed,
             int warmup, int reps, int flush, tf_bench_result_t *out) {
  return guarded([&] { return bench_impl(k, mode, logical_mnk, host_inputs, seed, warmup, reps, flush, out); });
}

}  // extern "C"
