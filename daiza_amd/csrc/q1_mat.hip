// q1_mat.hip — Q1_0 matrices on the device: upload/repack, dequant, and the matrix-level
// C ABI (Q1_0Matrix::{from_gguf, row_into_slice, matvec_into_slice, matvec_add_into_slice,
// matvec_multi_into_slice}, Daiza-engine/src/model/weights.rs:83-972).
#include "runtime.h"
#include "q1_gemm.h"

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <algorithm>
#include <mutex>

struct dz_mat {
  dz::Q1Dev d;
};

namespace dz {

// ------------------------------------------------------------------ errors / device

static thread_local char g_err[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

static int g_device = -1;
static hipStream_t g_stream = nullptr;
static std::mutex g_mu;

// Workspace of dz_q1_0_matvec_dev_noalloc: the split-K partials of one product, for callers that
// cannot allocate.  Each device that runs the library holds its own copy until the process ends.
// In host code `scratch` only names the symbol; its device address (per device) is looked up once
// at set-up and kept in g_scratch_dev, which is what kernels receive.
constexpr size_t kNoAllocScratchFloats = (size_t)4 << 20;  // 16 MiB
static __device__ __align__(256) float scratch[kNoAllocScratchFloats];
constexpr int kMaxDevices = 16;
static float* g_scratch_dev[kMaxDevices] = {};

int ensure_device() {
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_device >= 0) {
    DZ_HIP_CHECK(hipSetDevice(g_device));
    return DZ_OK;
  }
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return set_error(DZ_ERR_DEVICE, "no HIP device visible");
  hipDeviceProp_t prop;
  DZ_HIP_CHECK(hipGetDeviceProperties(&prop, 0));
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return set_error(DZ_ERR_DEVICE, "device 0 is %s; this library is built for gfx950 only", prop.gcnArchName);
  DZ_HIP_CHECK(hipSetDevice(0));
  DZ_HIP_CHECK(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking));
  // the no-alloc workspace of this device (device 0 is current)
  void* sp = nullptr;
  hipError_t e = hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch));
  if (e != hipSuccess || sp == nullptr)
    return set_error(DZ_ERR_DEVICE, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
  g_scratch_dev[0] = static_cast<float*>(sp);
  g_device = 0;
  return DZ_OK;
}

hipStream_t lib_stream() { return g_stream; }

int Scratch::reserve(size_t n) {
  if (n <= bytes) return DZ_OK;
  if (ptr) DZ_HIP_CHECK(hipFree(ptr));
  ptr = nullptr;
  bytes = 0;
  size_t want = n + (n >> 2);
  DZ_HIP_CHECK(hipMalloc(&ptr, want));
  bytes = want;
  return DZ_OK;
}

// ------------------------------------------------------------------ kernels

// AoS blocks -> GEMV layout.  One 64-thread block per (row-block, tile) unit; lane = row in block.
__global__ __launch_bounds__(64) void repack_kernel(const uint8_t* __restrict__ aos, int64_t rows, int64_t cols,
                                                    int64_t ntiles, uint8_t* __restrict__ out) {
  const int64_t unit = blockIdx.x;
  const unsigned L = threadIdx.x;
  const int64_t rb = unit / ntiles;
  const int t = (int)(unit % ntiles);
  const int64_t row = rb * kRowBlock + L;
  const int64_t gpr = cols / kGroup;
  uint8_t* u = out + (size_t)unit * kUnitBytes;
  const bool live = row < rows;
  const uint8_t* rowp = aos + (size_t)(live ? row : 0) * gpr * kBlockBytes;
  for (int c = 0; c < 4; ++c) {
    unsigned w[4] = {0, 0, 0, 0};
    for (int i = 0; i < 16; ++i) {
      const unsigned s = 16u * c + i, p = L ^ s;
      const int64_t g = 4 * t + (p >> 4);
      unsigned byte = 0;
      if (live && g < gpr) byte = rowp[g * kBlockBytes + 2 + (p & 15)];
      w[i >> 2] |= byte << (8 * (i & 3));
    }
    u32x4 v = {w[0], w[1], w[2], w[3]};
    reinterpret_cast<u32x4*>(u)[c * 64 + L] = v;
  }
  unsigned sc[2] = {0, 0};
  for (int j = 0; j < 4; ++j) {
    const int64_t g = 4 * t + ((L >> 4) ^ j);
    unsigned bits = 0;
    if (live && g < gpr) bits = rowp[g * kBlockBytes] | (rowp[g * kBlockBytes + 1] << 8);
    sc[j >> 1] |= bits << (16 * (j & 1));
  }
  u32x2 v2 = {sc[0], sc[1]};
  reinterpret_cast<u32x2*>(u + kUnitSignBytes)[L] = v2;
}

// Daiza-engine/src/tensor/quant.rs:39-74 f16_to_f32, bit for bit.  Note: for a subnormal half the
// reference adds the normalisation shift count to the exponent (127 - 15 + e) where IEEE would
// subtract it, so subnormal scales dequantise larger than IEEE; the GEMV path uses the exact
// hardware conversion, as the reference's _mm256_cvtph_ps does (quant.rs:649-660).
__device__ __forceinline__ float ref_f16_to_f32(unsigned bits) {
  const unsigned sign = (bits >> 15) & 1u, exp = (bits >> 10) & 0x1Fu, mant = bits & 0x3FFu;
  const unsigned s32 = sign << 31;
  unsigned out;
  if (exp == 0) {
    if (mant == 0) {
      out = s32;
    } else {
      unsigned m = mant, e = 1;
      while ((m & 0x400u) == 0) { m <<= 1; ++e; }
      out = s32 | ((112u + e) << 23) | ((m & 0x3FFu) << 13);
    }
  } else if (exp == 0x1F) {
    out = s32 | 0x7F800000u | (mant << 13);
  } else {
    out = s32 | ((exp + 112u) << 23) | (mant << 13);
  }
  return __builtin_bit_cast(float, out);
}

// dequantize_q1_0_row_into (quant.rs:161-194) from the GEMV layout: w = (bit*2 - 1) * scale.
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ data, int64_t cols, int64_t ntiles,
                                                      int64_t r0, int64_t nrows, float* __restrict__ out) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= nrows * cols) return;
  const int64_t row = r0 + i / cols, k = i % cols;
  const int64_t rb = row / kRowBlock;
  const unsigned L = (unsigned)(row % kRowBlock);
  const int t = (int)(k / kTileCols);
  const unsigned p = (unsigned)((k % kTileCols) / 8), j = (unsigned)(k % 8);
  const unsigned s = L ^ p;
  const uint8_t* u = data + ((size_t)rb * ntiles + t) * kUnitBytes;
  const unsigned byte = u[((s >> 4) * 64 + L) * 16 + (s & 15)];
  const unsigned slot = (p >> 4) ^ (L >> 4);
  const uint16_t* scp = reinterpret_cast<const uint16_t*>(u + kUnitSignBytes);
  const float scale = ref_f16_to_f32(scp[L * 4 + slot]);
  const float bit = (float)((byte >> j) & 1u);
  out[i] = (bit * 2.0f - 1.0f) * scale;
}

// y = [y +] sum over tile groups of part[tg][vrow], tile-group order 0..n_tg-1.
struct ReduceArgs {
  ReduceSeg seg[8];
  int nseg;
  const float* part;
  int64_t ld;
  int n_tg;
  int accumulate;
};

__global__ __launch_bounds__(256) void partial_reduce_kernel(const ReduceArgs a) {
  const int64_t v = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  int s = 0;
  while (s + 1 < a.nseg && v >= a.seg[s + 1].vrow_begin) ++s;
  const int64_t r = v - a.seg[s].vrow_begin;
  if (r < 0 || r >= a.seg[s].rows) return;
  const float acc = ordered_sum(a.part + v, a.ld, a.n_tg);
  float* y = a.seg[s].y + r;
  *y = a.accumulate ? *y + acc : acc;
}

hipError_t launch_partial_reduce(const float* part, int64_t ld, int n_tg, const ReduceSeg* segs, int nseg,
                                 int accumulate, hipStream_t s) {
  ReduceArgs a;
  memset(&a, 0, sizeof a);
  for (int i = 0; i < nseg; ++i) a.seg[i] = segs[i];
  a.nseg = nseg;
  a.part = part;
  a.ld = ld;
  a.n_tg = n_tg;
  a.accumulate = accumulate;
  const int64_t n = ld;
  hipLaunchKernelGGL(partial_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, a);
  return hipGetLastError();
}

int plan_gemv(const Q1Dev* const* mats, int n, int tpw, GemvPlan* plan) {
  if (n < 1 || n > 8) return set_error(DZ_ERR_TENSOR, "gemv: %d matrices (1..8 supported)", n);
  GemvGrid g;
  memset(&g, 0, sizeof g);
  const int64_t cols = mats[0]->cols;
  int64_t rb = 0;
  for (int i = 0; i < n; ++i) {
    if (mats[i]->cols != cols) return set_error(DZ_ERR_TENSOR, "gemv: matrices disagree on cols");
    g.seg[i].data = mats[i]->data;
    g.seg[i].rb_begin = rb;
    g.seg[i].nrb = mats[i]->nrb;
    rb += mats[i]->nrb;
  }
  g.nseg = n;
  g.total_rb = rb;
  g.ntiles = (int)mats[0]->ntiles;
  if (tpw <= 0) tpw = 1;
  if (tpw > g.ntiles) tpw = g.ntiles;
  if (tpw > 16) return set_error(DZ_ERR_UNSUPPORTED, "gemv: tiles per workgroup %d > 16", tpw);
  g.tpw = tpw;
  g.n_tg = (g.ntiles + tpw - 1) / tpw;
  g.rbw = kGemvWaves * kGemvM;
  plan->g = g;
  plan->nwg = (unsigned)(((rb + g.rbw - 1) / g.rbw) * g.n_tg);
  plan->shmem = gemv_shmem(tpw);
  plan->ld = rb * kRowBlock;
  return DZ_OK;
}

int upload_q1_host(const uint8_t* aos, int64_t rows, int64_t cols, Q1Dev* d, std::vector<void*>* owner) {
  if (cols % kGroup) return set_error(DZ_ERR_TENSOR, "upload: cols %lld is not a multiple of 128", (long long)cols);
  d->rows = rows;
  d->cols = cols;
  d->nrb = (rows + kRowBlock - 1) / kRowBlock;
  d->ntiles = (cols + kTileCols - 1) / kTileCols;
  const size_t aos_bytes = (size_t)rows * (size_t)(cols / kGroup) * kBlockBytes;
  const size_t dev_bytes = (size_t)d->nrb * d->ntiles * kUnitBytes;
  uint8_t* tmp = nullptr;
  d->data = nullptr;
  hipError_t e = hipMalloc(&d->data, dev_bytes);
  if (e == hipSuccess) e = hipMalloc(&tmp, aos_bytes);
  if (e == hipSuccess) e = hipMemcpyAsync(tmp, aos, aos_bytes, hipMemcpyHostToDevice, lib_stream());
  if (e == hipSuccess) {
    hipLaunchKernelGGL(repack_kernel, dim3((unsigned)(d->nrb * d->ntiles)), dim3(64), 0, lib_stream(), tmp, rows, cols,
                       d->ntiles, d->data);
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipStreamSynchronize(lib_stream());
  if (tmp) (void)hipFree(tmp);
  if (e != hipSuccess) {
    if (d->data) (void)hipFree(d->data);
    d->data = nullptr;
    return set_error(DZ_ERR_DEVICE, "upload: %s", hipGetErrorString(e));
  }
  if (owner) owner->push_back(d->data);
  return DZ_OK;
}

int upload_q1_host(const uint8_t* aos, int64_t rows, int64_t cols, Q1Dev* out, std::vector<void*>& owner) {
  return upload_q1_host(aos, rows, cols, out, &owner);
}

// ------------------------------------------------------------------ N-column products

int packed_x_reserve(Scratch& buf, int n, int64_t K, PackedX* out) {
  const int Np = (n + kGemmTok - 1) / kGemmTok * kGemmTok;
  const int64_t Kp = (K + kTileCols - 1) / kTileCols * kTileCols;
  const size_t part_bytes = (size_t)Np * Kp * 2;
  const int rc = buf.reserve(kGemmParts * part_bytes + (size_t)Np * 4);
  if (rc) return rc;
  char* b = static_cast<char*>(buf.ptr);
  out->xh = reinterpret_cast<uint16_t*>(b);
  out->xm = reinterpret_cast<uint16_t*>(b + part_bytes);
  out->xl = reinterpret_cast<uint16_t*>(b + 2 * part_bytes);
  out->sig = reinterpret_cast<float*>(b + kGemmParts * part_bytes);
  out->Kp = Kp;
  out->Np = Np;
  return DZ_OK;
}

hipError_t launch_x_pack(const float* x, int64_t ldx, int64_t K, int n, const float* w, float eps, const PackedX& p,
                         hipStream_t s) {
  hipLaunchKernelGGL(x_pack_kernel, dim3((unsigned)p.Np), dim3(256), 0, s, x, ldx, K, n, w, eps, p.xh, p.xm, p.xl,
                     p.sig, p.Kp);
  return hipGetLastError();
}

// Workgroups wanted in flight (two per CU): a product with fewer splits its K tiles over
// blockIdx.z and sums the partials in a second pass.
constexpr int kGemmMinWgs = 512;

int gemm_splits(const Q1Dev& W, int n, int* tps) {
  const int nb = n <= 16 ? 1 : kGemmNB;
  const int64_t wgs = ((W.nrb + 3) / 4) * ((n + 16 * nb - 1) / (16 * nb));
  const int nt = (int)W.ntiles;
  int S = 1;
  if (wgs < kGemmMinWgs && nt > 1) S = (int)std::min<int64_t>(nt, (kGemmMinWgs + wgs - 1) / wgs);
  *tps = (nt + S - 1) / S;
  return (nt + *tps - 1) / *tps;
}

// The wide form takes eight row-blocks per workgroup (each wave a whole row-block: half the
// activation reads per weight byte and per matrix instruction) when that costs at most a quarter
// more in whole rounds of workgroups over the CUs (one workgroup per CU either way) than four
// row-blocks do: measured at the prefill shapes, the eight-block form runs 10-16% faster at equal
// round cost and about 4% slower at a third more.
static bool gemm_wide_rb8(const Q1Dev& W, int n, int S) {
  if (S > 1) return false;
  static int cus[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
  if (cus[dev] == 0 && (hipDeviceGetAttribute(&cus[dev], hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
                        cus[dev] <= 0)) {
    cus[dev] = 0;
    return false;
  }
  const int64_t tb = (n + kGemmTok - 1) / kGemmTok, c = cus[dev];
  const int64_t r4 = (((W.nrb + 3) / 4) * tb + c - 1) / c, r8 = (((W.nrb + 7) / 8) * tb + c - 1) / c;
  return 8 * r8 <= 5 * r4;
}

// One product launch: the packed form (p non-null) or the raw form (x f32, row stride ldx).
static hipError_t launch_q1_gemm_any(const Q1Dev& W, const PackedX* p, const float* xr, int64_t ldx, int n, float* y,
                                     int64_t ldy, int accumulate, hipStream_t s, Scratch* split,
                                     GemmDefer* defer = nullptr, const float* norm_w = nullptr, float eps = 0.f) {
  static bool attr = false;
  if (!attr) {
    const void* ks[5] = {reinterpret_cast<const void*>(q1_gemm_kernel<kGemmNB, false>),
                         reinterpret_cast<const void*>(q1_gemm_kernel<kGemmNB, false, false, 8>),
                         reinterpret_cast<const void*>(q1_gemm_kernel<1, false>),
                         reinterpret_cast<const void*>(q1_gemm_kernel<1, true>),
                         reinterpret_cast<const void*>(q1_gemm_kernel<1, true, true>)};
    const size_t sh[5] = {gemm_shmem(kGemmNB), gemm_shmem(kGemmNB), gemm_shmem(1), gemm_shmem(1), gemm_shmem(1, true)};
    for (int i = 0; i < 5; ++i) {
      hipError_t e = hipFuncSetAttribute(ks[i], hipFuncAttributeMaxDynamicSharedMemorySize, (int)sh[i]);
      if (e != hipSuccess) return e;
    }
    attr = true;
  }
  const bool raw = p == nullptr;
  if (!raw && (W.ntiles * kTileCols != p->Kp || n > p->Np)) return hipErrorInvalidValue;
  if (raw && n > 16) return hipErrorInvalidValue;  // the raw form packs one 16-token block per workgroup
  GemmX gx{};
  if (raw) {
    gx.Kp = W.ntiles * kTileCols;
    gx.xf = xr;
    gx.ldx = ldx;
    gx.K = W.cols;
    gx.nw = norm_w;
    gx.eps = eps;
  } else {
    gx.xh = p->xh;
    gx.xm = p->xm;
    gx.xl = p->xl;
    gx.sig = p->sig;
    gx.Kp = p->Kp;
  }
  int tps;
  int S = gemm_splits(W, n, &tps);
  if (S > 1 && !split) S = 1, tps = (int)W.ntiles;
  float* out = y;
  int64_t ld = ldy, zs = 0;
  if (S > 1) {
    zs = (int64_t)n * W.rows;
    // the partials, then (normed raw form) the per-split sums of squares [S][n]
    if (split->reserve(((size_t)S * zs + (norm_w ? (size_t)S * n : 0)) * sizeof(float))) return hipErrorOutOfMemory;
    out = static_cast<float*>(split->ptr);
    ld = W.rows;
    if (raw && norm_w) {
      gx.ssq = out + (size_t)S * zs;
      gx.ssq_ld = n;
    }
  }
  const unsigned gx_ = (unsigned)((W.nrb + 3) / 4);
  const dim3 g1(gx_, 1, (unsigned)S), g2(gx_, (unsigned)((n + kGemmTok - 1) / kGemmTok), (unsigned)S);
  if (n <= 16) {
    if (raw && n <= 8)  // hi and mid of every token in one operand, lo in a second: two matrix instructions per step
      hipLaunchKernelGGL((q1_gemm_kernel<1, true, true>), g1, dim3(64 * gemm_waves(1)), gemm_shmem(1, true), s, W.data, W.rows,
                         W.nrb, (int)W.ntiles, tps, gx, n, out, ld, zs, accumulate);
    else if (raw)
      hipLaunchKernelGGL((q1_gemm_kernel<1, true>), g1, dim3(64 * gemm_waves(1)), gemm_shmem(1), s, W.data, W.rows, W.nrb,
                         (int)W.ntiles, tps, gx, n, out, ld, zs, accumulate);
    else
      hipLaunchKernelGGL((q1_gemm_kernel<1, false>), g1, dim3(64 * gemm_waves(1)), gemm_shmem(1), s, W.data, W.rows, W.nrb,
                         (int)W.ntiles, tps, gx, n, out, ld, zs, accumulate);
  } else if (gemm_wide_rb8(W, n, S)) {
    const dim3 g8((unsigned)((W.nrb + 7) / 8), g2.y, 1);
    hipLaunchKernelGGL((q1_gemm_kernel<kGemmNB, false, false, 8>), g8, dim3(64 * gemm_waves(kGemmNB)), gemm_shmem(kGemmNB), s,
                       W.data, W.rows, W.nrb, (int)W.ntiles, tps, gx, n, out, ld, zs, accumulate);
  } else {
    hipLaunchKernelGGL((q1_gemm_kernel<kGemmNB, false>), g2, dim3(64 * gemm_waves(kGemmNB)), gemm_shmem(kGemmNB), s, W.data, W.rows,
                       W.nrb, (int)W.ntiles, tps, gx, n, out, ld, zs, accumulate);
  }
  hipError_t e = hipGetLastError();
  const float* ssq = S > 1 && raw && norm_w ? gx.ssq : nullptr;
  if (defer) *defer = GemmDefer{out, S, zs, ssq, n, W.cols, eps};
  if (e != hipSuccess || S == 1 || defer) return e;
  hipLaunchKernelGGL(gemm_split_reduce_kernel, dim3((unsigned)((W.rows + 255) / 256), (unsigned)n), dim3(256), 0, s,
                     (const float*)out, S, zs, W.rows, n, y, ldy, accumulate, ssq, n, W.cols, eps);
  return hipGetLastError();
}

hipError_t launch_q1_gemm(const Q1Dev& W, const PackedX& p, int n, float* y, int64_t ldy, int accumulate,
                          hipStream_t s, Scratch* split, GemmDefer* defer) {
  return launch_q1_gemm_any(W, &p, nullptr, 0, n, y, ldy, accumulate, s, split, defer);
}

hipError_t launch_q1_gemm_raw(const Q1Dev& W, const float* x, int64_t ldx, int n, float* y, int64_t ldy,
                              int accumulate, hipStream_t s, Scratch* split, const float* norm_w, float eps,
                              GemmDefer* defer) {
  if ((W.cols & 3) || (ldx & 3)) return hipErrorInvalidValue;  // 16-byte loads of x rows
  return launch_q1_gemm_any(W, nullptr, x, ldx, n, y, ldy, accumulate, s, split, defer, norm_w, eps);
}

// ------------------------------------------------------------------ matrix API state

static Scratch g_x, g_y, g_part, g_pack, g_split;

// ws: the partials' workspace (ws_floats of them), or null for the library's growing buffer.
static int matvec_impl(dz_mat* const* mats, int n, const float* x_dev, float* const* y_dev, int accumulate,
                       hipStream_t s, float* ws = nullptr, size_t ws_floats = 0) {
  int prc = prepare_gemv_kernels();
  if (prc) return prc;
  const Q1Dev* ds[8];
  for (int i = 0; i < n; ++i) ds[i] = &mats[i]->d;
  GemvPlan p;
  int rc = plan_gemv(ds, n, 1, &p);
  if (rc) return rc;
  const size_t need = (size_t)p.g.n_tg * (size_t)p.ld;
  float* part = ws;
  if (ws) {
    if (need > ws_floats)
      return set_error(DZ_ERR_UNSUPPORTED, "matvec_dev_noalloc: %zu partial sums exceed the workspace of %zu", need,
                       ws_floats);
  } else {
    if ((rc = g_part.reserve(need * sizeof(float)))) return rc;
    part = static_cast<float*>(g_part.ptr);
  }
  ReduceSeg segs[8];
  for (int i = 0; i < n; ++i) {
    segs[i].y = y_dev[i];
    segs[i].vrow_begin = p.g.seg[i].rb_begin * kRowBlock;
    segs[i].rows = mats[i]->d.rows;
  }
  PlainSrc src{x_dev, mats[0]->d.cols};
  PartialDst dst{part, p.ld};
  DZ_HIP_CHECK(launch_gemv(p, src, dst, s));
  DZ_HIP_CHECK(launch_partial_reduce(part, p.ld, p.g.n_tg, segs, n, accumulate, s));
  return DZ_OK;
}

// The tagged partials of the one-launch product (gemv_fused_kernel).  The buffer starts zeroed and
// tags grow by one per call; it is cleared again before a tag would wrap.  One buffer serves every
// stream, and a launch needs its whole grid resident, so calls run one after another on the device
// in the order the host made them: while every call has come on one stream, the stream orders them
// and nothing else is enqueued (an event record between launches costs about 1-3 us of device time
// per call); the first call on another stream waits on the host for the device to drain, and from
// then on each launch records g_fused_done and a launch on another stream waits for it.
static Scratch g_tpart;
static unsigned g_tag = 0;
static int g_fused_cap = -1;  // workgroups of gemv_fused_kernel resident at once on the device
static hipEvent_t g_fused_done = nullptr;
static hipStream_t g_fused_last = nullptr;
static bool g_fused_multi = false;  // a second stream has been seen: launches record g_fused_done
static int* g_fused_err = nullptr;  // device word: 1 once a launch's wait gave up (until read)

// Wait bound of the summing threads: DAIZA_GEMV_SPIN=<n> lowers it (0 gives up at once), so that
// tests of the failure path stay on the host's side.
static int fused_spin_limit() {
  if (const char* e = getenv("DAIZA_GEMV_SPIN")) {
    const long v = strtol(e, nullptr, 10);
    if (v >= 0 && v < (1 << 20)) return (int)v;
  }
  return 1 << 20;
}

// DZ_ERR_DEVICE if a launch since the last check gave up on its wait (the word is cleared).
// The caller has synchronised the stream of those launches.
static int fused_check() {
  if (!g_fused_err) return DZ_OK;
  int v = 0;
  DZ_HIP_CHECK(hipMemcpy(&v, g_fused_err, 4, hipMemcpyDeviceToHost));
  if (!v) return DZ_OK;
  DZ_HIP_CHECK(hipMemset(g_fused_err, 0, 4));
  return set_error(DZ_ERR_DEVICE, "matvec: a wait for split-K partials gave up (rows left NaN)");
}

// y = W x in one launch when the whole grid is resident at once (its summing workgroups wait for
// workgroups of lower index); otherwise the split-K kernel and the tile-sum kernel.
static int matvec_fused(dz_mat* const* mats, int n, const float* x_dev, float* const* y_dev, int accumulate,
                        hipStream_t s) {
  constexpr size_t shmem = (size_t)kLutBytes + 64 + kTileCols * 4;
  const void* kfn = (const void*)gemv_fused_kernel<kGemvWaves>;
  if (g_fused_cap < 0) {
    DZ_HIP_CHECK(hipFuncSetAttribute(kfn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)shmem));
    int dev = 0, occ = 0;
    hipDeviceProp_t prop;
    DZ_HIP_CHECK(hipGetDevice(&dev));
    DZ_HIP_CHECK(hipGetDeviceProperties(&prop, dev));
    DZ_HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kfn, kGemvWaves * 64, shmem));
    DZ_HIP_CHECK(hipEventCreateWithFlags(&g_fused_done, hipEventDisableTiming));
    DZ_HIP_CHECK(hipMalloc(&g_fused_err, 4));
    DZ_HIP_CHECK(hipMemset(g_fused_err, 0, 4));
    g_fused_cap = occ * prop.multiProcessorCount;
  }
  const Q1Dev* ds[8];
  for (int i = 0; i < n; ++i) ds[i] = &mats[i]->d;
  GemvPlan p;
  int rc = plan_gemv(ds, n, 1, &p);
  if (rc) return rc;
  if ((int64_t)p.nwg > g_fused_cap) return matvec_impl(mats, n, x_dev, y_dev, accumulate, s);
  std::lock_guard<std::mutex> lk(g_mu);
  const size_t words = (size_t)p.g.n_tg * (size_t)p.ld;
  const size_t pb = g_tpart.bytes;
  if ((rc = g_tpart.reserve(words * 8))) return rc;
  if (g_tpart.bytes != pb || g_tag == 0xFFFFFFFFu) {
    DZ_HIP_CHECK(hipMemsetAsync(g_tpart.ptr, 0, g_tpart.bytes, s));
    g_tag = 0;
  }
  FusedGemvArgs a;
  memset(&a, 0, sizeof a);
  a.g = p.g;
  a.x = x_dev;
  a.K = mats[0]->d.cols;
  a.part = static_cast<unsigned long long*>(g_tpart.ptr);
  a.ld = p.ld;
  a.tag = ++g_tag;
  a.accumulate = accumulate;
  a.spin_limit = fused_spin_limit();
  a.err = g_fused_err;
  for (int i = 0; i < n; ++i) {
    a.seg[i].y = y_dev[i];
    a.seg[i].vrow_begin = p.g.seg[i].rb_begin * kRowBlock;
    a.seg[i].rows = mats[i]->d.rows;
  }
  if (g_fused_last && g_fused_last != s) {
    if (g_fused_multi) {
      DZ_HIP_CHECK(hipStreamWaitEvent(s, g_fused_done, 0));
    } else {
      // the earlier launches' stream may since have been destroyed: no event on it, a device drain
      DZ_HIP_CHECK(hipDeviceSynchronize());
      g_fused_multi = true;
    }
  }
  hipLaunchKernelGGL(gemv_fused_kernel<kGemvWaves>, dim3(p.nwg), dim3(kGemvWaves * 64), shmem, s, a);
  DZ_HIP_CHECK(hipGetLastError());
  if (g_fused_multi) DZ_HIP_CHECK(hipEventRecord(g_fused_done, s));
  g_fused_last = s;
  return DZ_OK;
}

}  // namespace dz

using namespace dz;

extern "C" {

const char* dz_last_error(void) { return g_err; }

int dz_device_init(int device) {
  if (device != 0) return set_error(DZ_ERR_UNSUPPORTED, "only device 0 is supported");
  int rc = ensure_device();
  if (rc) return rc;
  return prepare_gemv_kernels();  // kernel attributes once here, not on a first call of any entry point
}

void dz_config_bonsai27b(dz_config* c, int32_t max_ctx) {
  c->n_layers = 64;
  c->hidden = 5120;
  c->ffn = 17408;
  c->vocab = 248320;
  c->n_head = 24;
  c->n_head_kv = 4;
  c->head_dim = 256;
  c->rope_dim = 64;
  c->rope_base = 1.0e7f;
  c->rms_eps = 1e-6f;
  c->full_attn_interval = 4;
  c->ssm_conv_kernel = 4;
  c->ssm_state = 128;
  c->ssm_k_heads = 16;
  c->ssm_v_heads = 48;
  c->embd_f16 = 1;
  c->max_ctx = max_ctx;
}

int dz_q1_0_upload(const uint8_t* aos, size_t rows, size_t cols, dz_mat** out) {
  if (!aos || !out || rows == 0 || cols == 0) return set_error(DZ_ERR_TENSOR, "upload: empty matrix or null pointer");
  if (cols % kGroup) return set_error(DZ_ERR_TENSOR, "upload: cols %zu is not a multiple of 128", cols);
  int rc = ensure_device();
  if (rc) return rc;
  dz_mat* m = new dz_mat();
  rc = upload_q1_host(aos, (int64_t)rows, (int64_t)cols, &m->d, nullptr);
  if (rc) {
    delete m;
    return rc;
  }
  *out = m;
  return DZ_OK;
}

int dz_q1_0_free(dz_mat* m) {
  if (!m) return DZ_OK;
  if (m->d.data) DZ_HIP_CHECK(hipFree(m->d.data));
  delete m;
  return DZ_OK;
}

int dz_q1_0_shape(const dz_mat* m, size_t* rows, size_t* cols) {
  if (!m) return set_error(DZ_ERR_TENSOR, "shape: null matrix");
  if (rows) *rows = (size_t)m->d.rows;
  if (cols) *cols = (size_t)m->d.cols;
  return DZ_OK;
}

int dz_q1_0_matvec_dev(dz_mat* m, const float* x_dev, float* y_dev, int accumulate, void* stream) {
  if (!m || !x_dev || !y_dev) return set_error(DZ_ERR_TENSOR, "matvec_dev: null pointer");
  int rc = ensure_device();
  if (rc) return rc;
  dz_mat* ms[1] = {m};
  float* ys[1] = {y_dev};
  return matvec_fused(ms, 1, x_dev, ys, accumulate, stream ? (hipStream_t)stream : lib_stream());
}

int dz_q1_0_matvec_dev_status(void* stream) {
  int rc = ensure_device();
  if (rc) return rc;
  const hipStream_t s = stream ? (hipStream_t)stream : lib_stream();
  DZ_HIP_CHECK(hipStreamSynchronize(s));
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_fused_multi)
    DZ_HIP_CHECK(hipEventSynchronize(g_fused_done));
  else if (g_fused_last && g_fused_last != s)
    DZ_HIP_CHECK(hipDeviceSynchronize());
  return fused_check();
}

int dz_q1_0_matvec_dev_noalloc(dz_mat* m, const float* x_dev, float* y_dev, int accumulate, void* stream) {
  if (!m || !x_dev || !y_dev) return set_error(DZ_ERR_TENSOR, "matvec_dev_noalloc: null pointer");
  int dev = -1;
  DZ_HIP_CHECK(hipGetDevice(&dev));
  // set-up (stream, workspace address) happens in dz_device_init, never here: this entry allocates nothing
  if (g_device < 0 || dev < 0 || dev >= kMaxDevices || g_scratch_dev[dev] == nullptr)
    return set_error(DZ_ERR_DEVICE, "matvec_dev_noalloc: call dz_device_init first");
  dz_mat* ms[1] = {m};
  float* ys[1] = {y_dev};
  return matvec_impl(ms, 1, x_dev, ys, accumulate, stream ? (hipStream_t)stream : lib_stream(), g_scratch_dev[dev],
                     kNoAllocScratchFloats);
}

size_t dz_q1_0_noalloc_max_partials(void) { return kNoAllocScratchFloats; }

int dz_q1_0_gemv_partials(dz_mat* m, const float* x_dev, float* part_dev, void* stream) {
  if (!m || !x_dev || !part_dev) return set_error(DZ_ERR_TENSOR, "gemv_partials: null pointer");
  int rc = ensure_device();
  if (rc) return rc;
  if ((rc = prepare_gemv_kernels())) return rc;
  const Q1Dev* ds[1] = {&m->d};
  GemvPlan p;
  if ((rc = plan_gemv(ds, 1, 1, &p))) return rc;
  PlainSrc src{x_dev, m->d.cols};
  PartialDst dst{part_dev, p.ld};
  DZ_HIP_CHECK(launch_gemv(p, src, dst, stream ? (hipStream_t)stream : lib_stream()));
  return DZ_OK;
}

size_t dz_q1_0_partials_ld(const dz_mat* m) { return m ? (size_t)(m->d.nrb * kRowBlock) : 0; }

int dz_q1_0_ntiles(const dz_mat* m) { return m ? (int)m->d.ntiles : 0; }

static int matvec_host(dz_mat* const* mats, int n, const float* x, float* const* ys, int accumulate) {
  if (n < 1 || n > 8) return set_error(DZ_ERR_TENSOR, "matvec: %d matrices (1..8 supported)", n);
  if (!x) return set_error(DZ_ERR_TENSOR, "matvec: null x");
  int rc = ensure_device();
  if (rc) return rc;
  size_t ytot = 0;
  for (int i = 0; i < n; ++i) {
    if (!mats[i] || !ys[i]) return set_error(DZ_ERR_TENSOR, "matvec: null matrix or output");
    if (mats[i]->d.cols != mats[0]->d.cols) return set_error(DZ_ERR_TENSOR, "matvec: matrices disagree on cols");
    ytot += (size_t)mats[i]->d.rows;
  }
  const size_t K = (size_t)mats[0]->d.cols;
  rc = g_x.reserve(K * 4);
  if (rc) return rc;
  rc = g_y.reserve(ytot * 4);
  if (rc) return rc;
  hipStream_t s = lib_stream();
  DZ_HIP_CHECK(hipMemcpyAsync(g_x.ptr, x, K * 4, hipMemcpyHostToDevice, s));
  float* ydev[8];
  size_t off = 0;
  for (int i = 0; i < n; ++i) {
    ydev[i] = static_cast<float*>(g_y.ptr) + off;
    if (accumulate)
      DZ_HIP_CHECK(hipMemcpyAsync(ydev[i], ys[i], (size_t)mats[i]->d.rows * 4, hipMemcpyHostToDevice, s));
    off += (size_t)mats[i]->d.rows;
  }
  rc = matvec_fused(mats, n, static_cast<const float*>(g_x.ptr), ydev, accumulate, s);
  if (rc) return rc;
  for (int i = 0; i < n; ++i)
    DZ_HIP_CHECK(hipMemcpyAsync(ys[i], ydev[i], (size_t)mats[i]->d.rows * 4, hipMemcpyDeviceToHost, s));
  DZ_HIP_CHECK(hipStreamSynchronize(s));
  std::lock_guard<std::mutex> lk(g_mu);
  return fused_check();
}

int dz_q1_0_matvec(dz_mat* m, const float* x, float* y, int accumulate) {
  dz_mat* ms[1] = {m};
  float* ys[1] = {y};
  return matvec_host(ms, 1, x, ys, accumulate);
}

int dz_q1_0_matvec_multi(dz_mat* const* mats, int n, const float* x, float* const* ys) {
  return matvec_host(mats, n, x, ys, 0);
}

int dz_q1_0_matvec_batch(dz_mat* m, const float* x, int n, float* y, int accumulate) {
  if (!m || !x || !y) return set_error(DZ_ERR_TENSOR, "matvec_batch: null pointer");
  if (n < 1) return set_error(DZ_ERR_TENSOR, "matvec_batch: n = %d", n);
  int rc = ensure_device();
  if (rc) return rc;
  const size_t K = (size_t)m->d.cols, R = (size_t)m->d.rows;
  PackedX p;
  if ((rc = packed_x_reserve(g_pack, n, (int64_t)K, &p))) return rc;
  if ((rc = g_x.reserve((size_t)n * K * 4)) || (rc = g_y.reserve((size_t)n * R * 4))) return rc;
  hipStream_t s = lib_stream();
  float* xd = static_cast<float*>(g_x.ptr);
  float* yd = static_cast<float*>(g_y.ptr);
  DZ_HIP_CHECK(hipMemcpyAsync(xd, x, (size_t)n * K * 4, hipMemcpyHostToDevice, s));
  if (accumulate) DZ_HIP_CHECK(hipMemcpyAsync(yd, y, (size_t)n * R * 4, hipMemcpyHostToDevice, s));
  if (n <= 16) {  // few tokens: the product packs its tiles itself (as the batched forward does)
    DZ_HIP_CHECK(launch_q1_gemm_raw(m->d, xd, (int64_t)K, n, yd, (int64_t)R, accumulate, s, &g_split));
  } else {
    DZ_HIP_CHECK(launch_x_pack(xd, (int64_t)K, (int64_t)K, n, nullptr, 0.f, p, s));
    DZ_HIP_CHECK(launch_q1_gemm(m->d, p, n, yd, (int64_t)R, accumulate, s, &g_split));
  }
  DZ_HIP_CHECK(hipMemcpyAsync(y, yd, (size_t)n * R * 4, hipMemcpyDeviceToHost, s));
  DZ_HIP_CHECK(hipStreamSynchronize(s));
  return DZ_OK;
}

int dz_q1_0_dequant_rows(dz_mat* m, size_t r0, size_t n, float* out) {
  if (!m || !out) return set_error(DZ_ERR_TENSOR, "dequant: null pointer");
  if (r0 + n > (size_t)m->d.rows) return set_error(DZ_ERR_TENSOR, "dequant: rows [%zu, %zu) out of range", r0, r0 + n);
  if (n == 0) return DZ_OK;
  int rc = ensure_device();
  if (rc) return rc;
  const size_t total = n * (size_t)m->d.cols;
  rc = g_y.reserve(total * 4);
  if (rc) return rc;
  hipStream_t s = lib_stream();
  hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, m->d.data, m->d.cols,
                     m->d.ntiles, (int64_t)r0, (int64_t)n, static_cast<float*>(g_y.ptr));
  DZ_HIP_CHECK(hipGetLastError());
  DZ_HIP_CHECK(hipMemcpyAsync(out, g_y.ptr, total * 4, hipMemcpyDeviceToHost, s));
  DZ_HIP_CHECK(hipStreamSynchronize(s));
  return DZ_OK;
}

}  // extern "C"
