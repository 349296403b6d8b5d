// runtime.h — host-side helpers shared by the library's translation units.
#pragma once
#include "common.h"
#include "q1_gemv.h"

#include <vector>

namespace dz {

// Makes sure a gfx950 device is current for this thread (first call selects device 0).
int ensure_device();
// Library stream used by the matrix-level entry points.
hipStream_t lib_stream();

// Device scratch buffers owned by the library (grown on demand, reused across calls).
struct Scratch {
  void* ptr = nullptr;
  size_t bytes = 0;
  int reserve(size_t n);
};

// Launch shape of one GEMV: the segment table plus grid size and dynamic LDS bytes.
struct GemvPlan {
  GemvGrid g;
  unsigned nwg = 0;
  size_t shmem = 0;
  int64_t ld = 0;  // rows of the virtual row space padded to 64 (partials leading dimension)
};

// Builds a plan over `mats` (stacked in order), all with the same cols.
// tpw = tiles per workgroup; tpw <= 0 picks the default (1, or all tiles when ntiles == 1).
int plan_gemv(const Q1Dev* const* mats, int n, int tpw, GemvPlan* plan);

// Default launch shape: NWAVES waves per workgroup, M row-blocks per wave.
constexpr int kGemvWaves = 8;
constexpr int kGemvM = 1;
// dynamic LDS: table + 16 reduction floats + up to 16 staged tiles
constexpr size_t kGemvShmemMax = kLutBytes + 64 + 16 * kTileCols * 4;
inline size_t gemv_shmem(int tpw) { return (size_t)kLutBytes + 64 + (size_t)tpw * kTileCols * 4; }

// The kernel's dynamic-LDS limit must have been raised (hipFuncSetAttribute) before the first launch.
template <class Src, class Dst>
hipError_t launch_gemv(const GemvPlan& p, const Src& src, const Dst& dst, hipStream_t s) {
  auto kfn = gemv_lut_kernel<kGemvWaves, kGemvM, Src, Dst>;
  hipLaunchKernelGGL(kfn, dim3(p.nwg), dim3(kGemvWaves * 64), p.shmem, s, p.g, src, dst);
  return hipGetLastError();
}

// Raises the dynamic-LDS limit of every GEMV instantiation the library launches (idempotent).
int prepare_gemv_kernels();

// The model config of a context (model.hip).
const dz_config* ctx_config(const dz_ctx* x);
// DZ_ERR_DEVICE for a context whose last token-kernel launch gave up part-way (every forward and
// save is refused until a reset or a restore), else DZ_OK.
int ctx_usable(const dz_ctx* x);

// Sum of the tile-group partials into each segment's output: y = [y +] sum_tg part[tg][row].
hipError_t launch_partial_reduce(const float* part, int64_t ld, int n_tg, const ReduceSeg* segs, int nseg,
                                 int accumulate, hipStream_t s);

// N-column products on the matrix cores (q1_gemm.h): activations packed once per input, then
// one launch per matrix.
struct PackedX {
  uint16_t* xh = nullptr;
  uint16_t* xm = nullptr;
  uint16_t* xl = nullptr;
  float* sig = nullptr;
  int64_t Kp = 0;  // padded columns
  int Np = 0;      // padded tokens (multiple of kGemmTok)
};
// Carves a PackedX for n tokens of K columns out of `buf` (grown on demand).
int packed_x_reserve(Scratch& buf, int n, int64_t K, PackedX* out);
// x[n][K] (row stride ldx) -> p; RMS-normalised with weight w first when w is non-null.
hipError_t launch_x_pack(const float* x, int64_t ldx, int64_t K, int n, const float* w, float eps, const PackedX& p,
                         hipStream_t s);
// y[n][rows] (row stride ldy) =|+= p · Wᵀ; W.cols must match the packed K.  A product with too
// few workgroups to fill the device splits its K tiles into partials held in `split` (grown on
// demand; NULL keeps it unsplit) and sums them in order.  With `defer` set, a split product leaves
// the sum to the caller: defer receives the partials ([splits][n][W.rows], zstride apart) and
// splits > 1; an unsplit one writes y as usual and reports splits = 1.
struct GemmDefer {
  const float* part = nullptr;
  int splits = 1;
  int64_t zstride = 0;
  // a normed raw product: per-split sums of squares [splits][ssq_ld] (the caller applies 1/rms)
  const float* ssq = nullptr;
  int ssq_ld = 0;
  int64_t K = 0;
  float eps = 0.f;
};
hipError_t launch_q1_gemm(const Q1Dev& W, const PackedX& p, int n, float* y, int64_t ldy, int accumulate,
                          hipStream_t s, Scratch* split, GemmDefer* defer = nullptr);
// The same product for n <= 16 tokens on f32 x[n][W.cols] (row stride ldx, both multiples of 4; a
// larger n is refused with hipErrorInvalidValue: callers pack it first), each K tile packed in
// LDS with its own power-of-two scale per token: no separate packing pass.  With norm_w, the product
// of the RMS-normalised x (weight norm_w, eps): the tiles are packed from x·norm_w and the sums of
// squares gathered on the way; 1/rms is applied to the result (by the deferred consumer when defer
// is given and the product is split).
hipError_t launch_q1_gemm_raw(const Q1Dev& W, const float* x, int64_t ldx, int n, float* y, int64_t ldy,
                              int accumulate, hipStream_t s, Scratch* split, const float* norm_w = nullptr,
                              float eps = 0.f, GemmDefer* defer = nullptr);

}  // namespace dz

struct dz_ctx;
namespace dz {
// dz_verify_forward's checks and forward, enqueued on the context's stream without the final wait.
int ctx_verify_enqueue(dz_ctx* x, const uint32_t* draft, int k);
// The device rows of a context's pending verify forward (see dz_verify_forward), for the sampler.
int ctx_verify_view(dz_ctx* x, const float** row0, const float** rows, hipStream_t* s, Scratch** scratch);
// Sampled decode on the token kernel: ctx_sample_begin feeds `first` and hands out the device feed
// array, the logits buffer, the stream and a scratch buffer (DZ_ERR_UNSUPPORTED, no error set, when
// the context runs the graph path); ctx_sample_launch(i) enqueues forward i of feed[i] at position
// pos + i, logits into the buffer; ctx_sample_end(n) waits, checks every launch and moves the
// position by n.
int ctx_sample_begin(dz_ctx* x, uint32_t first, int n, uint32_t** feed, const float** logits, hipStream_t* s,
                     Scratch** scratch);
int ctx_sample_launch(dz_ctx* x, int i);
int ctx_sample_end(dz_ctx* x, int n);
// Sampled decode of n tokens in one token-kernel launch: forward 0 takes `first`; the draws (top_k k
// <= kPtkSampMax, temperature 1/inv_t, top_p) run inside the kernel; out[i] = the draw after forward
// i, *rng the generator state after the last draw.  DZ_ERR_UNSUPPORTED (no error set) on the graph
// path, for a k beyond kPtkSampMax, or for a plan of more than kPtkFan^2 workgroups.
int ctx_sample_decode(dz_ctx* x, uint32_t first, int n, int k, float inv_t, float top_p, uint64_t* rng,
                      uint32_t* out);
}  // namespace dz
