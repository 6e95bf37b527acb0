// tmnn_hip.hip -- host side of the C-ABI (include/tmnn_hip.h): context,
// trainer state in a hipMalloc arena, step sequencing and kernel launches.
//
// Step sequencing follows DefaultRuntime (src/tiny_metal_nn/runtime/
// default_trainer.cpp:883-1045 and training_step_execution.cpp:887-1324):
//   batch cap -> Morton sort -> fused forward/backward -> loss -> Adam
//   (lazy hash + dense MLP) -> gradients and mask cleared -> step + 1.
// Everything after the input copy runs on the trainer's HIP stream with no
// host round trip; the host waits once, for the loss.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "tmnn_hip.h"
#include "aux_kernels.hpp"
#include "encode_kernel.hpp"
#include "field_kernel.hpp"
#include "grad_kernel.hpp"
#include "layer_kernels.hpp"
#include "rate_kernels.hpp"
#include "mlp_kernel.hpp"
#include "scatter_kernel.hpp"
#include "sort.hpp"
#include "step_kernel.hpp"
#include "wide_kernel.hpp"
#include "wide_train_kernel.hpp"

using namespace tmnn_hip;

// Device scratch of the allocation-free training step
// (tmnn_training_step_device_noalloc): the step's batch-sized buffers --
// sort keys and values, radix histograms, sorted positions and targets, the
// feature tiles and the input-feature gradients -- for batches up to
// TMNN_NOALLOC_SCRATCH_BYTES. Each GPU the library runs on holds its own copy
// until the process ends; host code reaches it only through the device
// address hipGetSymbolAddress returns for the current device (tmnn_context).
// Every kernel of the step writes its region before reading it, so nothing
// in it needs clearing; calls that overlap on one GPU share it and race.
static __device__ __align__(256) unsigned char scratch[TMNN_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr uint32_t kAbiVersion = 3u;
constexpr int kMaxLdsBytes = 160 * 1024;  // gfx950 LDS per CU
constexpr uint32_t kOptimizerBlobVersion = 1u;  // detail/checkpoint_contract.h:14

thread_local std::string g_last_error;

// Per device ordinal: the device address of `scratch` (looked up once per
// device) and the event that serialises the allocation-free steps of every
// context on that device. Each such step waits for the event before its
// first kernel and records it after its last, under g_scratch_mu, so steps
// of trainers on different streams take the scratch one after another
// instead of racing on it.
struct ScratchDevice {
  unsigned char *ptr = nullptr;
  hipEvent_t done = nullptr;
  bool recorded = false;
};
std::mutex g_scratch_mu;
std::vector<ScratchDevice> g_scratch;

int fail(int code, const std::string &msg) {
  g_last_error = msg;
  return code;
}

#define TMNN_HIP_TRY(expr)                                                   \
  do {                                                                       \
    hipError_t e_ = (expr);                                                  \
    if (e_ != hipSuccess)                                                    \
      return fail(TMNN_ERR_GPU, std::string(#expr) + ": " + hipGetErrorString(e_)); \
  } while (0)

// "%.6f" baked constants (mlp_kernel_emitter.cpp:91-92), read back as float.
float baked6(float v) {
  char buf[64];
  std::snprintf(buf, sizeof buf, "%.6f", static_cast<double>(v));
  return std::strtof(buf, nullptr);
}

using FieldKernel = void (*)(FieldArgs);

struct KernelChoice {
  FieldKernel fn = nullptr;
  bool reg_dw = false;  // dW accumulated in registers (compile-time layers)
  bool wide = false;    // hidden width 128: the block-cooperative wide kernel
  bool xmem = false;    // input features from encode_features_kernel
  bool mlp = false;     // mlp_train_kernel (no activation staging in LDS)
  bool wide_train = false;  // wide_train_kernel (fp16 training at width 128)
  bool tile_scatter = false;  // the training kernel runs the hash-grid backward per tile
};

// Hidden width 128: instantiated for the BASELINE 4D shape (16 levels x 2
// features, 4 hidden layers) and a 3D two-layer shape. fp16 training runs
// wide_train_kernel (wide_train_kernel.hpp), the rest wide_kernel.
KernelChoice select_wide_kernel(bool f16, bool train, int D, int F, int NHL) {
#define TMNN_WIDE(d, f, nhl)                                                         \
  if (D == d && F == f && NHL == nhl) {                                              \
    if (train && f16) return {wide_train_kernel<nhl>, false, true, true, false, true}; \
    if (train) return {wide_kernel<d, f, nhl, false, true, true>, false, true, true}; \
    return {f16 ? wide_kernel<d, f, nhl, true, false, true>                          \
                : wide_kernel<d, f, nhl, false, false, true>, false, true, true};    \
  }
  TMNN_WIDE(4, 2, 4)
  TMNN_WIDE(3, 2, 2)
#undef TMNN_WIDE
  return {};
}

// Training kernels read their input features from encode_features_kernel:
// fp16 training of the 64-wide BASELINE shapes runs mlp_train_kernel, their
// fp32 training (compile-time hidden-layer count) keeps dW in registers, the
// rest accumulate it in LDS. Forward kernels encode inline,
// specialised on the BASELINE geometries (compile-time D, F) or on the
// runtime geometry; the hidden-128 forward reads X tiles.
KernelChoice select_kernel(int HP, int INP, bool f16, bool train, int D, int F, int NHL,
                           int family, bool small_table = false, bool split_encode = false) {
  const bool fused = family == TMNN_FAMILY_FULLY_FUSED;
  if (HP == kWideHP)
    return INP == 32 && fused ? select_wide_kernel(f16, train, D, F, NHL) : KernelChoice{};
  // forward passes over tables with level slices above 2 MB: the level-major
  // encode, then the MLP over its X tiles (every family)
#define TMNN_FWD_X(hp, inp)                                                          \
  if (!train && split_encode && HP == hp && INP == inp)                              \
    return {f16 ? field_forward_x_kernel<hp, inp, true> : field_forward_x_kernel<hp, inp, false>, \
            false, false, true};
  TMNN_FWD_X(64, 32)
  TMNN_FWD_X(64, 64)
  TMNN_FWD_X(32, 32)
  TMNN_FWD_X(32, 64)
#undef TMNN_FWD_X
  const int DF = D * 8 + F;
#define TMNN_FWD_SPEC(hp, inp, df)                                                   \
  if (fused && !train && HP == hp && INP == inp && DF == df)                         \
    return {f16 ? field_forward_kernel<hp, inp, true, df>                            \
                : field_forward_kernel<hp, inp, false, df>,                          \
            false};
  TMNN_FWD_SPEC(64, 32, 2 * 8 + 2)  // image fit: 2D, 16x2 features
  TMNN_FWD_SPEC(64, 32, 3 * 8 + 2)  // NeRF density: 3D, 16x2
  TMNN_FWD_SPEC(64, 64, 3 * 8 + 4)  // SDF: 3D, 16x4
#undef TMNN_FWD_SPEC
  // fp16 training of the 64-wide BASELINE shapes: transposes on the matrix
  // cores instead of LDS staging (mlp_kernel.hpp)
  // Tables whose level slices stay cache-sized (the scatter's point-major
  // rule): the 64-wide fp16 kernels run the hash-grid backward of each tile
  // themselves (tile_scatter.hpp)
  if (fused && train && f16 && HP == 64 && INP == 32 && small_table &&
      tile_scatter_shape(D, F)) {
    if (NHL == 2)
      return {D == 2 ? mlp_train_kernel<64, 32, 2, 8, 2, 2> : mlp_train_kernel<64, 32, 2, 8, 3, 2>,
              true, false, true, true, false, true};
    if (NHL == 1)
      return {D == 2 ? mlp_train_kernel<64, 32, 1, 8, 2, 2> : mlp_train_kernel<64, 32, 1, 8, 3, 2>,
              true, false, true, true, false, true};
  }
  if (fused && train && f16 && HP == 64 && INP == 32 && NHL == 2)
    return {mlp_train_kernel<64, 32, 2>, true, false, true, true};
  if (fused && train && f16 && HP == 64 && INP == 32 && NHL == 1)
    return {mlp_train_kernel<64, 32, 1>, true, false, true, true};
  if (fused && train && f16 && HP == 64 && INP == 64 && NHL == 3)
    return {mlp_train_kernel<64, 64, 3>, true, false, true, true};
  if (fused && train) {
    // fp32 training of the 64-wide shapes on cache-sized tables: the field
    // kernel runs each tile's hash-grid backward itself (tile_scatter.hpp)
    if (!f16 && HP == 64 && INP == 32 && small_table && tile_scatter_shape(D, F)) {
      if (NHL == 2)
        return {D == 2 ? field_train_kernel<64, 32, false, 2, 2, 2>
                       : field_train_kernel<64, 32, false, 2, 3, 2>,
                true, false, true, false, false, true};
      if (NHL == 1)
        return {D == 2 ? field_train_kernel<64, 32, false, 1, 2, 2>
                       : field_train_kernel<64, 32, false, 1, 3, 2>,
                true, false, true, false, false, true};
    }
// fp32 training of the BASELINE shapes (fp16 took the kernels above)
#define TMNN_TRAIN_SPEC(hp, inp, nhl)                                              \
  if (!f16 && HP == hp && INP == inp && NHL == nhl)                                \
    return {field_train_kernel<hp, inp, false, nhl>, true, false, true};
    TMNN_TRAIN_SPEC(64, 32, 2)  // image fit: 16x2 features, 64x2 MLP
    TMNN_TRAIN_SPEC(64, 32, 1)  // NeRF density: 16x2, 64x1
    TMNN_TRAIN_SPEC(64, 64, 3)  // SDF: 16x4, 64x3
#undef TMNN_TRAIN_SPEC
  }

#define TMNN_SEL(hp, inp)                                                        \
  if (HP == hp && INP == inp) {                                                  \
    if (train)                                                                   \
      return {f16 ? field_train_kernel<hp, inp, true, 0>                         \
                  : field_train_kernel<hp, inp, false, 0>,                       \
              false, false, true};                                               \
    return {f16 ? field_forward_kernel<hp, inp, true, 0>                         \
                : field_forward_kernel<hp, inp, false, 0>,                       \
            false};                                                              \
  }
  // FULLY_FUSED training needs one of the shape-specialised kernels above;
  // every family's forward may use the generic one
  if (fused && train) return {};
  TMNN_SEL(32, 32)
  TMNN_SEL(32, 64)
  TMNN_SEL(64, 32)
  TMNN_SEL(64, 64)
#undef TMNN_SEL
  return {};
}

struct DevBuf {
  void *ptr = nullptr;
  size_t bytes = 0;
  bool borrowed = false;  // ptr is a region of the device scratch (never freed or grown)
  DevBuf() = default;
  DevBuf(const DevBuf &) = delete;
  DevBuf &operator=(const DevBuf &) = delete;
  ~DevBuf() {
    if (ptr && !borrowed) (void)hipFree(ptr);
  }
  hipError_t ensure(size_t want) {
    if (want <= bytes) return hipSuccess;
    if (borrowed) return hipErrorInvalidValue;  // a scratch region never grows
    if (ptr) {
      (void)hipFree(ptr);
      ptr = nullptr;
      bytes = 0;
    }
    const size_t rounded = (want + 255) / 256 * 256;
    hipError_t e = hipMalloc(&ptr, rounded);
    if (e == hipSuccess) bytes = rounded;
    return e;
  }
  template <class T>
  T *as() const {
    return static_cast<T *>(ptr);
  }
};

struct KernelPlan {
  FieldKernel fn = nullptr;
  bool f16 = false, train = false;
  uint64_t packed_version = ~0ull;  // weights version of the packed LDS image
  void *image = nullptr;            // device copy of the LDS head (weights, biases, res)
  size_t image_bytes = 0;
  int wpb = 0;          // waves per block
  int lds = 0;          // dynamic LDS bytes
  bool dw_global = false;  // dW accumulator outside LDS
  bool reg_dw = false;     // dW accumulator in registers
  bool wide = false;       // block-cooperative hidden-128 kernel (4 waves, 128-point block tiles)
  bool xmem = false;       // features from encode_features_kernel (X tiles in xfeat)
  bool mlp = false;        // mlp_train_kernel
  bool wide_train = false; // wide_train_kernel
  bool tile_scatter = false;  // hash-grid backward fused into the training kernel
  bool layerwise = false;  // layer-wise path (layer_kernels.hpp): one product per layer
  int max_blocks = 0;   // resident blocks on the whole device (layer-wise: batch chunks)
};

}  // namespace

struct tmnn_context {
  int device = 0;
  hipStream_t stream = nullptr;
  int cu_count = 0;
  uint64_t mem_bytes = 0;
  std::string name;
  unsigned char *scratch = nullptr;  // this device's copy of the step scratch (device address)
};

struct tmnn_trainer {
  tmnn_context *ctx = nullptr;
  tmnn_model_desc d{};
  int IN = 0, INP = 0, HP = 0;
  uint32_t hash_count = 0, mlp_count = 0;
  uint32_t hash_entries = 0;  // L * T: one visit flag byte each
  uint32_t mask_words = 0;    // words of the reference's bit-mask layout (debug view)
  float res[kMaxLevels] = {};
  uint32_t step = 0;
  float lr_enc = 0.f, lr_net = 0.f;
  int family = TMNN_FAMILY_FULLY_FUSED;  // of the plan the kernels were chosen from
  tmnn_network_plan plan{};

  DevBuf params, m, v, grad_hash, grad_mlp;
  DevBuf mask[2];  // visit flags, double-buffered: Adam reads one, zeroes the other
  int mask_cur = 0;
  DevBuf partials, loss_partials, loss_out;
  DevBuf in_pos, in_tgt, s_pos, s_tgt, keys0, keys1, vals0, vals1, sort_tmp, out_buf;
  DevBuf dx;  // [batch][IN] input-feature gradients between the two train kernels
  DevBuf xfeat;  // input features of the batch as X tiles (encode_kernel.hpp)
  DevBuf wide_mask, wide_act;  // hidden-128 kernel: per-tile ReLU bits and fp16 activations
  DevBuf lw_act, lw_y, lw_g, lw_d;  // layer-wise path: activations, outputs, d_out, deltas
  // The fused device step sorts its batch on a second stream into one of
  // kSortSets buffer sets, so that a step's sort runs while the previous
  // steps' kernels still execute; the main stream waits for the sort
  // (ev_sorted) and marks the set free again after the step (ev_consumed).
  // Three sets: step N's sort may start once step N - 3 is done, so it has
  // the encode and finish windows of two steps (the MLP kernel leaves no CU
  // room) instead of one.
  static constexpr int kSortSets = 3;
  struct SortSet {
    DevBuf keys0, keys1, vals0, vals1, tmp;
  } step_sort[kSortSets];
  hipStream_t side = nullptr;
  hipEvent_t ev_sorted[kSortSets] = {};
  hipEvent_t ev_consumed[kSortSets] = {};
  hipEvent_t ev_staged = nullptr;  // host-staged batch copied in on the main stream
  bool consumed_recorded[kSortSets] = {};
  int sort_parity = 0;
  DevBuf dbg_a, dbg_b, dbg_c;

  KernelPlan train_plan, fwd_plan, infer_plan;
  KernelPlan grad_plan;          // fp32 backward for evaluate_with_gradient (lazy)
  bool grad_planned = false;
  DevBuf grad_out;               // [n][M][D] Jacobian of evaluate_with_gradient
  uint64_t weights_version = 0;  // bumped whenever the parameters change

  // Step profiling: one set of phase events per profiled step, summed and
  // recycled when the profile is read. prof_every: 0 off, k >= 1 one training
  // step in k (the first, then every k-th); prof_seen counts steps since on.
  static constexpr int kProfEvents = 7;  // sort | encode | fwd/bwd | scatter | reduce | adam |
  // per profiled step also the start / stop events of its main kernels
  // (encode, training kernel, scatter, finish), recorded by the dispatches
  // themselves (launch_step_kernel)
  static constexpr int kProfKernels = 4;
  static constexpr int kProfSet = kProfEvents + 2 * kProfKernels;
  int32_t prof_every = 0;
  uint64_t prof_seen = 0;
  std::vector<std::array<hipEvent_t, kProfSet>> prof_events;
  // per event set: bit k set when boundary k was recorded; a boundary with
  // no work before it (the fused step's scatter and reduce phases) is not
  // recorded and reads as the previous one (a zero-length phase)
  std::vector<uint32_t> prof_recorded;
  size_t prof_used = 0;
  int prof_cur = -1;  // event set of the step being enqueued, or -1
  bool prof_suspended = false;  // allocation-free steps record no events
  tmnn_step_profile prof_acc{};
  // per profiled step, in step order: the phase times (TMNN_PROFILE_*)
  std::vector<std::array<float, TMNN_PROFILE_COLUMNS>> prof_samples;
  // inference calls while profiling is on: one event pair around the
  // forward kernel of one call in prof_every
  uint64_t prof_infer_seen = 0;
  std::vector<std::array<hipEvent_t, 2>> infer_events;
  size_t infer_used = 0;

  // Numerics (NumericsGuard, numerics_guard.cpp:12-36): sampling mode and
  // interval, the anomaly history, and the device rows of the last step whose
  // report was computed (finish_step_kernel<F, true>: one float4 per block;
  // num_loss_row holds the largest |output| and the loss).
  int32_t num_mode = TMNN_NUMERICS_SAMPLED;
  uint32_t num_interval = 128;
  uint32_t num_anomalies = 0, num_last_anomaly = 0;
  bool num_this_step = false;   // the step being enqueued computes its report
  DevBuf num_rows, amax_partials;
  int num_row_count = 0, num_loss_row = 0;
  uint32_t num_step = 0;        // step counter after that step (0: none yet)
  uint32_t num_batch = 0;
  float *dbg_step_out = nullptr;  // tmnn_debug_step_outputs: the training kernel's outputs
  hipEvent_t input_ready = nullptr;  // caller's event the side stream's sort waits for

  ~tmnn_trainer() {
    if (side) {
      (void)hipStreamSynchronize(side);
      (void)hipStreamDestroy(side);
    }
    for (int k = 0; k < kSortSets; ++k)
      for (hipEvent_t e : {ev_sorted[k], ev_consumed[k]})
        if (e) (void)hipEventDestroy(e);
    if (ev_staged) (void)hipEventDestroy(ev_staged);
    for (KernelPlan *p : {&train_plan, &fwd_plan, &infer_plan, &grad_plan})
      if (p->image) (void)hipFree(p->image);
    for (auto &set : prof_events)
      for (hipEvent_t e : set)
        if (e) (void)hipEventDestroy(e);
    for (auto &pair : infer_events)
      for (hipEvent_t e : pair)
        if (e) (void)hipEventDestroy(e);
  }
};

namespace {

bool desc_ok(const tmnn_model_desc *d, std::string &why) {
  auto bad = [&](const char *m) {
    why = m;
    return false;
  };
  if (d->spatial_dims < 2 || d->spatial_dims > 4) return bad("spatial_dims must be 2, 3 or 4");
  if (d->num_levels < 1 || d->num_levels > 32) return bad("num_levels must be in [1, 32]");
  if (d->features_per_level != 1 && d->features_per_level != 2 && d->features_per_level != 4)
    return bad("features_per_level must be 1, 2, or 4");
  if (d->log2_hashmap_size < 10 || d->log2_hashmap_size > 24)
    return bad("log2_hashmap_size must be in [10, 24]");
  if (!(d->base_resolution > 0.f)) return bad("base_resolution must be > 0");
  if (!(d->per_level_scale > 0.f)) return bad("per_level_scale must be > 0");
  if (d->hidden_dim < 1 || d->hidden_dim > 512) return bad("hidden_dim must be in (0, 512]");
  if (d->num_hidden_layers < 1 || d->num_hidden_layers > 8)
    return bad("num_hidden_layers must be in [1, 8]");
  if (d->num_outputs < 1) return bad("num_outputs must be >= 1");
  if (d->loss_kind < TMNN_LOSS_L2 || d->loss_kind > TMNN_LOSS_RELATIVE_L2)
    return bad("invalid loss kind");
  if (d->loss_kind == TMNN_LOSS_HUBER && !(d->huber_delta > 0.f))
    return bad("Huber loss requires huber_delta > 0");
  if (d->loss_kind == TMNN_LOSS_COSINE && d->num_outputs < 2)
    return bad("Cosine loss requires num_outputs >= 2");
  if (d->batch_size < 1) return bad("batch_size must be >= 1");
  if (d->precision != TMNN_PRECISION_FP32 && d->precision != TMNN_PRECISION_FP16)
    return bad("invalid precision");
  if (d->hash_adam_mode != TMNN_HASH_ADAM_LAZY && d->hash_adam_mode != TMNN_HASH_ADAM_DENSE)
    return bad("invalid hash_adam_mode");
  if (d->forced_family < TMNN_FAMILY_AUTO || d->forced_family > TMNN_FAMILY_SAFE_DEBUG)
    return bad("invalid forced_family");
  return true;
}

// Claims the next event set for a profiled step (prof_cur = -1 when off).
int prof_begin_step(tmnn_trainer *tr) {
  tr->prof_cur = -1;
  if (tr->prof_every <= 0 || tr->prof_suspended) return TMNN_OK;
  if (tr->prof_seen++ % static_cast<uint64_t>(tr->prof_every) != 0) return TMNN_OK;
  if (tr->prof_used == tr->prof_events.size()) {
    std::array<hipEvent_t, tmnn_trainer::kProfSet> set{};
    // timing-only events: no system-scope fence (cache writeback and
    // invalidate) at each record; prof_collect synchronizes the stream first
    for (hipEvent_t &e : set)
      TMNN_HIP_TRY(hipEventCreateWithFlags(&e, hipEventDisableSystemFence));
    tr->prof_events.push_back(set);
    tr->prof_recorded.push_back(0u);
  }
  tr->prof_recorded[tr->prof_used] = 0u;
  tr->prof_cur = static_cast<int>(tr->prof_used++);
  return TMNN_OK;
}

// Records phase boundary k of the current profiled step.
int prof_mark(tmnn_trainer *tr, int k) {
  if (tr->prof_cur < 0) return TMNN_OK;
  TMNN_HIP_TRY(hipEventRecord(tr->prof_events[tr->prof_cur][k], tr->ctx->stream));
  tr->prof_recorded[tr->prof_cur] |= 1u << k;
  return TMNN_OK;
}

// The step's main kernels (kernel index k: 0 encode, 1 training kernel, 2
// scatter, 3 finish): on a profiled step launched with start / stop events
// that the dispatch itself records (hipExtLaunchKernel), i.e. the kernel's
// own begin and end as a kernel trace reports them, without the launch
// latency the phase boundaries include; otherwise a plain launch.
template <typename K, typename... Args>
void launch_step_kernel(tmnn_trainer *tr, int k, K kernel, dim3 grid, dim3 block, uint32_t shm,
                        hipStream_t st, Args... args) {
  if (tr->prof_cur >= 0) {
    auto &e = tr->prof_events[tr->prof_cur];
    hipExtLaunchKernelGGL(kernel, grid, block, shm, st, e[tmnn_trainer::kProfEvents + 2 * k],
                          e[tmnn_trainer::kProfEvents + 2 * k + 1], 0u, args...);
    tr->prof_recorded[tr->prof_cur] |= 1u << (tmnn_trainer::kProfEvents + k);
  } else {
    hipLaunchKernelGGL(kernel, grid, block, shm, st, args...);
  }
}
enum : int { kKernEncode = 0, kKernTrain = 1, kKernScatter = 2, kKernFinish = 3 };

// Claims an event pair for a profiled inference call (nullptr when this
// call is not sampled).
int prof_infer_begin(tmnn_trainer *tr, std::array<hipEvent_t, 2> **pair) {
  *pair = nullptr;
  if (tr->prof_every <= 0 || tr->prof_suspended) return TMNN_OK;
  if (tr->prof_infer_seen++ % static_cast<uint64_t>(tr->prof_every) != 0) return TMNN_OK;
  if (tr->infer_used == tr->infer_events.size()) {
    std::array<hipEvent_t, 2> ev{};
    for (hipEvent_t &e : ev) TMNN_HIP_TRY(hipEventCreateWithFlags(&e, hipEventDisableSystemFence));
    tr->infer_events.push_back(ev);
  }
  *pair = &tr->infer_events[tr->infer_used];
  return TMNN_OK;
}

// Folds every recorded step and inference call into prof_acc and recycles
// the event sets.
int prof_collect(tmnn_trainer *tr) {
  if (tr->prof_used == 0 && tr->infer_used == 0) return TMNN_OK;
  TMNN_HIP_TRY(hipStreamSynchronize(tr->ctx->stream));
  for (size_t i = 0; i < tr->infer_used; ++i) {
    float ms = 0.0f;
    TMNN_HIP_TRY(hipEventElapsedTime(&ms, tr->infer_events[i][0], tr->infer_events[i][1]));
    tr->prof_acc.gpu_infer_us += 1e3 * ms;
    tr->prof_acc.infer_calls += 1;
  }
  tr->infer_used = 0;
  for (size_t i = 0; i < tr->prof_used; ++i) {
    const auto &e = tr->prof_events[i];
    // boundary k reads the last recorded boundary at or before k (boundary 0,
    // the step's start, is always recorded)
    int at[tmnn_trainer::kProfEvents];
    for (int k = 0, last = 0; k < tmnn_trainer::kProfEvents; ++k) {
      if (tr->prof_recorded[i] & (1u << k)) last = k;
      at[k] = last;
    }
    float ms[tmnn_trainer::kProfEvents - 1];
    for (int k = 0; k + 1 < tmnn_trainer::kProfEvents; ++k) {
      ms[k] = 0.0f;
      if (at[k] != at[k + 1]) TMNN_HIP_TRY(hipEventElapsedTime(&ms[k], e[at[k]], e[at[k + 1]]));
    }
    float kms[tmnn_trainer::kProfKernels];
    for (int k = 0; k < tmnn_trainer::kProfKernels; ++k) {
      kms[k] = 0.0f;
      if (tr->prof_recorded[i] & (1u << (tmnn_trainer::kProfEvents + k)))
        TMNN_HIP_TRY(hipEventElapsedTime(&kms[k], e[tmnn_trainer::kProfEvents + 2 * k],
                                         e[tmnn_trainer::kProfEvents + 2 * k + 1]));
    }
    {
      std::array<float, TMNN_PROFILE_COLUMNS> smp{};
      for (int k = 0; k + 1 < tmnn_trainer::kProfEvents; ++k) smp[k] = 1e3f * ms[k];
      float total = 0.0f;
      for (int k = 0; k + 1 < tmnn_trainer::kProfEvents; ++k) total += smp[k];
      smp[TMNN_PROFILE_TOTAL] = total;
      for (int k = 0; k < tmnn_trainer::kProfKernels; ++k)
        smp[TMNN_PROFILE_KERNEL_ENCODE + k] = 1e3f * kms[k];
      tr->prof_samples.push_back(smp);
    }
    tr->prof_acc.gpu_encode_kernel_us += 1e3 * kms[0];
    tr->prof_acc.gpu_train_kernel_us += 1e3 * kms[1];
    tr->prof_acc.gpu_scatter_kernel_us += 1e3 * kms[2];
    tr->prof_acc.gpu_finish_kernel_us += 1e3 * kms[3];
    tr->prof_acc.gpu_sort_us += 1e3 * ms[0];
    tr->prof_acc.gpu_encode_us += 1e3 * ms[1];
    tr->prof_acc.gpu_fwd_bwd_us += 1e3 * ms[2];
    tr->prof_acc.gpu_scatter_us += 1e3 * ms[3];
    tr->prof_acc.gpu_reduce_us += 1e3 * ms[4];
    tr->prof_acc.gpu_adam_us += 1e3 * ms[5];
    tr->prof_acc.gpu_total_us += 1e3 * (ms[0] + ms[1] + ms[2] + ms[3] + ms[4] + ms[5]);
    tr->prof_acc.steps += 1;
  }
  tr->prof_used = 0;
  return TMNN_OK;
}

// Padded widths and parameter count of a model (the kernels' view of it).
struct ModelShape {
  int D, F, L, IN, INP, H, HP, NHL, M, mlp_count, log2T;
};

ModelShape shape_of(const tmnn_model_desc &d) {
  ModelShape m{};
  m.D = d.spatial_dims;
  m.F = d.features_per_level;
  m.L = d.num_levels;
  m.log2T = d.log2_hashmap_size;
  m.IN = d.num_levels * d.features_per_level;
  m.INP = m.IN <= 32 ? 32 : (m.IN <= 64 ? 64 : 128);
  m.H = d.hidden_dim;
  m.HP = d.hidden_dim <= 32 ? 32
                            : (d.hidden_dim <= 64 ? 64
                                                  : (d.hidden_dim <= kWideHP ? kWideHP
                                                                             : round_up(d.hidden_dim, 16)));
  m.NHL = d.num_hidden_layers;
  m.M = d.num_outputs;
  m.mlp_count = make_layout(m.INP, m.HP, m.IN, m.H, m.NHL, m.M, 0, false, false, 1).mlp_count();
  return m;
}

// Kernel choice and LDS sizing of one plan (host arithmetic only): the
// family's kernel for the shape, waves per block, LDS bytes against
// lds_limit. Returns false with *why when the family has no kernel or its
// LDS plan does not fit.
// Batch chunks (partial dW rows) of the layer-wise path: at most 256 (one
// weight-gradient block per CU and 64 x 64 output tile at least), and at most
// 64 MiB of partial rows.
int lw_max_chunks(int mlp_count) {
  const int by_mem = static_cast<int>((64u << 20) / (4u * static_cast<unsigned>(std::max(1, mlp_count))));
  return std::max(1, std::min(256, by_mem));
}

bool size_plan_fused(const ModelShape &m, bool f16, bool train, int family, int lds_limit,
                     KernelPlan &out, int *why);

// The family's plan; TILED and SAFE_DEBUG fall back to the layer-wise path
// (layer_kernels.hpp) for shapes no MFMA kernel is instantiated for or whose
// LDS plan does not fit, so every KernelSpec shape has a non-fused plan.
bool size_plan(const ModelShape &m, bool f16, bool train, int family, int lds_limit,
               KernelPlan &out, int *why) {
  if (size_plan_fused(m, f16, train, family, lds_limit, out, why)) return true;
  if (family == TMNN_FAMILY_FULLY_FUSED) return false;
  out = KernelPlan{};
  out.f16 = f16;
  out.train = train;
  out.layerwise = true;
  out.xmem = true;
  out.wpb = 4;
  out.max_blocks = lw_max_chunks(m.mlp_count);
  *why = 0;
  return true;
}

bool size_plan_fused(const ModelShape &m, bool f16, bool train, int family, int lds_limit,
                     KernelPlan &out, int *why) {
  *why = 0;
  if (m.M > 16) {  // the MFMA kernels hold the outputs in one 16-wide tile
    *why = TMNN_PLAN_UNSUPPORTED_OUTPUT_DIMS;
    return false;
  }
  if (m.INP > 64 || m.HP > kWideHP) {
    *why = m.HP > kWideHP ? TMNN_PLAN_HIDDEN_DIM_UNSUPPORTED : TMNN_PLAN_NO_FUSED_INSTANCE;
    return false;
  }
  // level slices up to 8 MB: the scatter runs point-major (level_major());
  // above 2 MB the encode runs level-major (encode_level_major()), and so do
  // the forward passes of F <= 2 tables (C3: 789 -> 510 us at 2^20 points;
  // C4's F = 4 slices measured 571 inline against 578 split, kept inline)
  const size_t slice = static_cast<size_t>(m.F) * 4u << m.log2T;
  const bool small_table = slice <= (8u << 20);
  const bool split_encode = slice > (2u << 20) && m.F <= 2;
  const KernelChoice kc = select_kernel(m.HP, m.INP, f16, train, m.D, m.F, m.NHL, family,
                                        small_table, split_encode);
  out.fn = kc.fn;
  out.reg_dw = kc.reg_dw;
  out.wide = kc.wide;
  out.xmem = kc.xmem;
  out.mlp = kc.mlp;
  out.wide_train = kc.wide_train;
  out.tile_scatter = kc.tile_scatter;
  out.f16 = f16;
  out.train = train;
  *why = 0;
  if (!out.fn) {
    *why = (m.HP == kWideHP && family != TMNN_FAMILY_FULLY_FUSED) ? TMNN_PLAN_HIDDEN_DIM_UNSUPPORTED
                                                                  : TMNN_PLAN_NO_FUSED_INSTANCE;
    return false;
  }
  if (out.mlp) {
    const FieldLayout s = make_layout(m.INP, m.HP, m.IN, m.H, m.NHL, m.M, m.mlp_count, true, true,
                                      mlp_waves(m.INP, m.NHL), false, true);
    out.wpb = mlp_waves(m.INP, m.NHL);
    out.lds = mlp_lds(s, out.wpb).total;
    out.image_bytes = static_cast<size_t>(s.dw_off);
  } else if (out.wide) {
    const FieldLayout fl = make_layout(m.INP, m.HP, m.IN, m.H, m.NHL, m.M, m.mlp_count, f16, train, 1);
    out.wpb = kWideWaves;
    out.lds = out.wide_train ? wide_train_lds(fl).total : make_wide_layout(fl, f16, train).total;
    out.image_bytes = static_cast<size_t>(fl.dw_off);
  } else {
    // Most waves per block whose LDS plan fits; failing that, move the dW
    // accumulator out of LDS (global float atomics into the block's row).
    out.wpb = 0;
    for (int dwg = 0; dwg <= (train && !kc.reg_dw ? 1 : 0) && out.wpb == 0; ++dwg) {
      for (int w = 4; w >= 1; --w) {
        const FieldLayout s = make_layout(m.INP, m.HP, m.IN, m.H, m.NHL, m.M, m.mlp_count, f16,
                                          train, w, dwg != 0, kc.reg_dw);
        if (s.total <= lds_limit) {
          out.lds = s.total;
          out.dw_global = dwg != 0;
          out.wpb = w;
          break;
        }
      }
    }
    if (out.wpb < 1) {
      out.lds = make_layout(m.INP, m.HP, m.IN, m.H, m.NHL, m.M, m.mlp_count, f16, train, 1,
                            train && !kc.reg_dw, kc.reg_dw).total;
    }
    out.image_bytes = static_cast<size_t>(
        make_layout(m.INP, m.HP, m.IN, m.H, m.NHL, m.M, m.mlp_count, f16, train, 1).dw_off);
  }
  if (out.wpb < 1 || out.lds > lds_limit) {
    *why = TMNN_PLAN_THREADGROUP_MEMORY_EXCEEDED;
    return false;
  }
  return true;
}

// FNV-1a over the shape fields the kernels depend on.
uint64_t planner_fingerprint(const tmnn_model_desc &d) {
  uint64_t h = 1469598103934665603ull;
  auto mix = [&](uint64_t v) {
    for (int i = 0; i < 8; ++i) {
      h ^= (v >> (8 * i)) & 0xffu;
      h *= 1099511628211ull;
    }
  };
  mix(static_cast<uint64_t>(d.spatial_dims));
  mix(static_cast<uint64_t>(d.num_levels));
  mix(static_cast<uint64_t>(d.features_per_level));
  mix(static_cast<uint64_t>(d.log2_hashmap_size));
  mix(static_cast<uint64_t>(d.base_resolution * 1000000.0f));
  mix(static_cast<uint64_t>(d.per_level_scale * 1000000.0f));
  mix(static_cast<uint64_t>(d.hidden_dim));
  mix(static_cast<uint64_t>(d.num_hidden_layers));
  mix(static_cast<uint64_t>(d.num_outputs));
  mix(static_cast<uint64_t>(d.precision));
  return h;
}

// plan_with_capabilities (network_planner.cpp:132-300) for this library:
// FULLY_FUSED when its training kernel is instantiated for the shape and its
// LDS plan fits, else TILED (generic kernels), SAFE_DEBUG only when forced;
// the reasons record why a family was not eligible or was overridden.
void plan_network_impl(const tmnn_device_caps &caps, const tmnn_model_desc &d,
                       tmnn_network_plan &p) {
  std::memset(&p, 0, sizeof p);
  p.struct_size = sizeof p;
  p.capabilities = caps;
  p.selected_family = -1;
  p.planner_fingerprint = planner_fingerprint(d);
  auto reason = [&](int r) { p.reasons |= 1u << r; };
  if (!caps.gpu_available) {
    reason(TMNN_PLAN_NO_GPU_CONTEXT);
    return;
  }
  if (d.spatial_dims < 2 || d.spatial_dims > 4 || d.num_levels < 1 || d.num_levels > 32 ||
      d.num_levels * d.features_per_level > 128) {
    reason(TMNN_PLAN_UNSUPPORTED_INPUT_DIMS);
    return;
  }
  if (d.num_outputs < 1) {
    reason(TMNN_PLAN_UNSUPPORTED_OUTPUT_DIMS);
    return;
  }
  if (d.hidden_dim < 1 || d.hidden_dim > 512) {
    reason(TMNN_PLAN_HIDDEN_DIM_UNSUPPORTED);
    return;
  }
  const ModelShape m = shape_of(d);
  const bool f16 = d.precision == TMNN_PRECISION_FP16;
  struct Elig {
    bool train = false, eval = false;
    KernelPlan tp;
  } fam[3];
  for (int f = 0; f < 3; ++f) {
    const bool ff16 = f == TMNN_FAMILY_SAFE_DEBUG ? false : f16;
    int why = 0, why_eval = 0;
    fam[f].train = size_plan(m, ff16, true, f, caps.lds_bytes_per_cu, fam[f].tp, &why);
    if (f == TMNN_FAMILY_FULLY_FUSED && fam[f].train && m.HP == kWideHP && !ff16) {
      // width-128 fp32 training: the layer's fp32 weight and gradient
      // operands do not fit one CU's LDS next to the activations (the fused
      // width-128 kernels train in fp16 only)
      fam[f].train = false;
      why = TMNN_PLAN_THREADGROUP_MEMORY_EXCEEDED;
    }
    KernelPlan ep;
    fam[f].eval = size_plan(m, false, false, f, caps.lds_bytes_per_cu, ep, &why_eval);
    if (f == TMNN_FAMILY_FULLY_FUSED && !fam[f].train && why) reason(why);
    if (fam[f].train && fam[f].eval) p.candidate_families |= 1u << f;
  }
  int sel = -1;
  if (d.forced_family == TMNN_FAMILY_SAFE_DEBUG) {
    reason(TMNN_PLAN_FORCED_SAFE_DEBUG);
    sel = TMNN_FAMILY_SAFE_DEBUG;
  } else if (d.forced_family == TMNN_FAMILY_TILED) {
    reason(TMNN_PLAN_FORCED_TILED);
    sel = TMNN_FAMILY_TILED;
  } else if (p.candidate_families & (1u << TMNN_FAMILY_FULLY_FUSED)) {
    sel = TMNN_FAMILY_FULLY_FUSED;
  } else if (p.candidate_families & (1u << TMNN_FAMILY_TILED)) {
    sel = TMNN_FAMILY_TILED;
  }
  if (sel < 0 || !(p.candidate_families & (1u << sel))) return;
  p.selected_family = sel;
  p.fused_train = sel == TMNN_FAMILY_FULLY_FUSED;
  {
    // the evaluator is fused when the family's forward kernel is specialised
    KernelPlan ep;
    int why = 0;
    p.fused_eval = sel == TMNN_FAMILY_FULLY_FUSED &&
                   size_plan(m, false, false, sel, caps.lds_bytes_per_cu, ep, &why) &&
                   (ep.wide || ep.xmem || ep.fn != select_kernel(m.HP, m.INP, false, false, m.D, m.F, m.NHL,
                                                      TMNN_FAMILY_TILED).fn);
  }
  p.train_lds_bytes = fam[sel].tp.lds;
  p.train_waves_per_block = fam[sel].tp.wpb;
}

// size_plan for the trainer's family, then the device side: the packed
// image buffer, the dynamic LDS attribute and the resident block count.
int plan_kernel(tmnn_trainer *tr, bool f16, bool train, KernelPlan &out) {
  int why = 0;
  if (!size_plan(shape_of(tr->d), f16, train, tr->family, kMaxLdsBytes, out, &why))
    return fail(TMNN_ERR_UNSUPPORTED,
                why == TMNN_PLAN_THREADGROUP_MEMORY_EXCEEDED ? "model does not fit in LDS"
                                                             : "no kernel for this geometry");
  if (out.layerwise) return TMNN_OK;  // no packed image, plain launches
  TMNN_HIP_TRY(hipMalloc(&out.image, out.image_bytes));
  TMNN_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void *>(out.fn),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, out.lds));
  int per_cu = 0;
  TMNN_HIP_TRY(hipOccupancyMaxActiveBlocksPerMultiprocessor(
      &per_cu, reinterpret_cast<const void *>(out.fn), 64 * out.wpb, out.lds));
  if (per_cu < 1) return fail(TMNN_ERR_UNSUPPORTED, "field kernel cannot be resident");
  out.max_blocks = per_cu * tr->ctx->cu_count;
  return TMNN_OK;
}

FieldArgs base_args(const tmnn_trainer *tr) {
  FieldArgs a{};
  a.D = tr->d.spatial_dims;
  a.L = tr->d.num_levels;
  a.F = tr->d.features_per_level;
  a.IN = tr->IN;
  a.H = tr->d.hidden_dim;
  a.NHL = tr->d.num_hidden_layers;
  a.M = tr->d.num_outputs;
  a.log2T = static_cast<uint32_t>(tr->d.log2_hashmap_size);
  a.loss_kind = tr->d.loss_kind;
  a.huber_delta = baked6(tr->d.huber_delta);
  a.loss_scale = 1.0f;
  a.inv_loss_scale = 1.0f;
  a.mlp_count = static_cast<int32_t>(tr->mlp_count);
  for (int l = 0; l < kMaxLevels; ++l) a.res[l] = tr->res[l];
  a.table = tr->params.as<float>();
  a.mlp = tr->params.as<float>() + tr->hash_count;
  return a;
}

// Rebuild a plan's packed LDS image if the weights changed since it was made.
int ensure_image(tmnn_trainer *tr, KernelPlan &plan) {
  if (plan.layerwise || plan.packed_version == tr->weights_version) return TMNN_OK;
  PackArgs p{};
  p.s = make_layout(tr->INP, tr->HP, tr->IN, tr->d.hidden_dim, tr->d.num_hidden_layers,
                    tr->d.num_outputs, static_cast<int>(tr->mlp_count), plan.f16, plan.train, 1);
  p.f16 = plan.f16 ? 1 : 0;
  p.L = tr->d.num_levels;
  for (int l = 0; l < kMaxLevels; ++l) p.res[l] = tr->res[l];
  p.mlp = tr->params.as<float>() + tr->hash_count;
  p.image = static_cast<unsigned char *>(plan.image);
  int n = 0, total = 0;
  auto add = [&](int kind, int layer, int count) {
    p.sec_kind[n] = kind;
    p.sec_layer[n] = layer;
    p.sec_start[n] = total;
    total += count;
    ++n;
  };
  const int NHL = tr->d.num_hidden_layers;
  for (int k = 0; k <= NHL; ++k) {
    const int kin = k == 0 ? tr->INP : tr->HP;
    const int mout = k == NHL ? 16 : tr->HP;
    add(kSecFwd, k, kin * mout);
    if (plan.train) add(kSecBwd, k, kin * (plan.f16 ? round_up(mout, 32) : mout));
    add(kSecBias, k, mout);
  }
  add(kSecRes, 0, kMaxLevels);
  p.nsec = n;
  p.sec_start[n] = total;
  hipLaunchKernelGGL(pack_image_kernel, dim3((total + 255) / 256), dim3(256), 0, tr->ctx->stream, p);
  TMNN_HIP_TRY(hipGetLastError());
  plan.packed_version = tr->weights_version;
  return TMNN_OK;
}

// Input features of n points at pos as X tiles in tr->xfeat; with perm,
// point i is pos[perm[i]] and its position is also written to pos_out[i].
// Hash-grid kernels walk the levels one at a time (level-major) when a
// level's slice of the table exceeds 8 MB (the scatter) or 2 MB (the
// encode), else all levels per point.
bool level_major(const tmnn_trainer *tr) {
  return (static_cast<size_t>(tr->d.features_per_level) * 4u << tr->d.log2_hashmap_size) >
         (8u << 20);
}

// The encode goes level-major from 2 MB slices on (C3's 4 MB levels: 450 ->
// 345 us; its scatter measured slower level-major there, so it keeps 8 MB).
bool encode_level_major(const tmnn_trainer *tr) {
  return (static_cast<size_t>(tr->d.features_per_level) * 4u << tr->d.log2_hashmap_size) >
         (2u << 20);
}

int launch_encode(tmnn_trainer *tr, const float *pos, int n, const uint32_t *perm = nullptr,
                  float *pos_out = nullptr) {
  EncodeArgs e{};
  e.n = n;
  e.n_pad = (n + kTilePts - 1) / kTilePts * kTilePts;
  // inference batches are not bounded by the training batch: size here
  TMNN_HIP_TRY(tr->xfeat.ensure(static_cast<size_t>(e.n_pad) * tr->INP * sizeof(float)));
  e.L = tr->d.num_levels;
  e.KT0 = tr->INP / 16;
  e.log2T = static_cast<uint32_t>(tr->d.log2_hashmap_size);
  for (int l = 0; l < kMaxLevels; ++l) e.res[l] = tr->res[l];
  e.pos = pos;
  e.perm = perm;
  e.pos_out = pos_out;
  e.table = tr->params.as<float>();
  e.xfeat = tr->xfeat.as<float>();
  hipStream_t st = tr->ctx->stream;
  // level-major for large tables (the scatter's rule), reading the positions
  // in place: through a sort permutation they are first gathered into sorted
  // order in pos_out (which the scatter reads anyway), since every level
  // re-reading them through the permutation at random measured slower than
  // point-major
  bool by_level = encode_level_major(tr);
  if (by_level && perm != nullptr) {
    if (pos_out == nullptr) {
      by_level = false;
    } else {
      const size_t elems = static_cast<size_t>(n) * tr->d.spatial_dims;
      hipLaunchKernelGGL(gather_rows_kernel, dim3(static_cast<uint32_t>((elems + 255) / 256)),
                         dim3(256), 0, st, pos, nullptr, perm, n, tr->d.spatial_dims, 0,
                         pos_out, nullptr);
      e.pos = pos_out;
      e.perm = nullptr;
      e.pos_out = nullptr;
    }
  }
  // point-major: a batch of fewer blocks than one full round (four per CU)
  // splits each point's feature quads over up to 4 * KT0 threads
  const uint32_t bx = static_cast<uint32_t>((e.n_pad + kEncodeThreads - 1) / kEncodeThreads);
  uint32_t split = 1;
  if (!by_level)
    while (split < static_cast<uint32_t>(4 * e.KT0) &&
           bx * split < static_cast<uint32_t>(tr->ctx->cu_count) * 4u)
      split *= 2;
  const dim3 grid(bx, by_level ? static_cast<uint32_t>(e.L) : split);
#define TMNN_ENCODE(d, f)                                                                     \
  if (by_level)                                                                               \
    launch_step_kernel(tr, kKernEncode, encode_level_kernel<d, f>, grid, dim3(kEncodeThreads), \
                       0, st, e);                                                             \
  else                                                                                        \
    launch_step_kernel(tr, kKernEncode, encode_features_kernel<d, f>, grid,                   \
                       dim3(kEncodeThreads), 0, st, e);
  switch (tr->d.spatial_dims * 8 + tr->d.features_per_level) {
    case 2 * 8 + 1: TMNN_ENCODE(2, 1) break;
    case 2 * 8 + 2: TMNN_ENCODE(2, 2) break;
    case 2 * 8 + 4: TMNN_ENCODE(2, 4) break;
    case 3 * 8 + 1: TMNN_ENCODE(3, 1) break;
    case 3 * 8 + 2: TMNN_ENCODE(3, 2) break;
    case 3 * 8 + 4: TMNN_ENCODE(3, 4) break;
    case 4 * 8 + 1: TMNN_ENCODE(4, 1) break;
    case 4 * 8 + 2: TMNN_ENCODE(4, 2) break;
    default: TMNN_ENCODE(4, 4) break;
  }
#undef TMNN_ENCODE
  TMNN_HIP_TRY(hipGetLastError());
  return TMNN_OK;
}

// Launches a plan's field kernel over n points; XMEM plans first encode a.pos
// into tr->xfeat (unless reuse_x: the features of these points are there
// already), with profile mark prof_after_encode (if >= 0) in between.
int launch_layerwise(tmnn_trainer *tr, KernelPlan &plan, FieldArgs a, int n,
                     int prof_after_encode, bool reuse_x, const uint32_t *perm, float *pos_out);

int launch_field(tmnn_trainer *tr, KernelPlan &plan, FieldArgs a, int n,
                 int prof_after_encode = -1, bool reuse_x = false,
                 const uint32_t *perm = nullptr, float *pos_out = nullptr) {
  if (plan.layerwise)
    return launch_layerwise(tr, plan, a, n, prof_after_encode, reuse_x, perm, pos_out);
  int rc = ensure_image(tr, plan);
  if (rc != TMNN_OK) return rc;
  if (plan.xmem) {
    if (!reuse_x && (rc = launch_encode(tr, a.pos, n, perm, pos_out)) != TMNN_OK) return rc;
    a.xfeat = tr->xfeat.as<float>();
  }
  if (prof_after_encode >= 0 && (rc = prof_mark(tr, prof_after_encode)) != TMNN_OK) return rc;
  a.image = static_cast<const unsigned char *>(plan.image);
  a.n = n;
  a.n_tiles = (n + kTilePts - 1) / kTilePts;
  a.waves_per_block = plan.wpb;
  a.dw_global = plan.dw_global ? 1 : 0;
  if (plan.wide) {
    a.wide_mask = tr->wide_mask.as<uint64_t>();
    a.wide_act = tr->wide_act.as<_Float16>();
  }
  const int need = (a.n_tiles + plan.wpb - 1) / plan.wpb;
  const int blocks = std::max(1, std::min(need, plan.max_blocks));
  launch_step_kernel(tr, kKernTrain, plan.fn, dim3(blocks), dim3(64 * plan.wpb),
                     static_cast<uint32_t>(plan.lds), tr->ctx->stream, a);
  TMNN_HIP_TRY(hipGetLastError());
  return blocks;
}

// The layer-wise path (layer_kernels.hpp) over n points: encode (unless
// reuse_x: the features and, in kModeInputGrad, the forward activations of
// these points are in place), one product per layer forward, and for the
// training modes the output gradient, the weight-gradient partial rows (one
// per batch chunk; returns their count) and the input-feature gradients into
// a.dx_out. fp32 throughout (the loss scale of the fp16 kernels is not needed).
int launch_layerwise(tmnn_trainer *tr, KernelPlan &plan, FieldArgs a, int n,
                     int prof_after_encode, bool reuse_x, const uint32_t *perm, float *pos_out) {
  int rc;
  const bool fwd_only = a.mode == kModeForward;
  const int IN = tr->IN, H = tr->d.hidden_dim, NHL = tr->d.num_hidden_layers;
  const int M = tr->d.num_outputs;
  const FieldLayout lay = make_layout(tr->INP, tr->HP, IN, H, NHL, M, 0, false, false, 1);
  hipStream_t st = tr->ctx->stream;
  auto gemm = [&](LwGemmArgs g, int chunks) -> int {
    if (g.R <= 0 || g.C <= 0) return TMNN_OK;
    // 16-byte operand loads and epilogue stores where rows are aligned
    g.a_vec = (g.a_mode == kLwARow || g.a_mode == kLwACol) && lw_vec_ok(g.A, g.lda);
    g.b_vec = lw_vec_ok(g.B, g.ldb);
    const bool bias_ok = g.bias && (reinterpret_cast<uintptr_t>(g.bias) & 15u) == 0;
    g.o_vec = lw_vec_ok(g.out, g.ldo) &&
              (g.epi == kLwEpiScale || (g.epi == kLwEpiHidden && bias_ok) ||
               (g.epi == kLwEpiMask && lw_vec_ok(g.mask, g.ldm)));
    if (lw_narrow_out_ok(g)) {
      const int groups = (g.R + 15) / 16;
      const int blocks = std::min((groups + 3) / 4, 8 * tr->ctx->cu_count);
      const int kr = (g.K + kLwNarrowKStep - 1) / kLwNarrowKStep * kLwNarrowKStep;
      const size_t lds = sizeof(float) * kLwNarrow * kr;
      hipLaunchKernelGGL(lw_narrow_out_kernel, dim3(blocks), dim3(256), lds, st, g);
      TMNN_HIP_TRY(hipGetLastError());
      return TMNN_OK;
    }
    if (lw_narrow_wgrad_ok(g)) {
      const dim3 grid((g.R + 63) / 64, 1, chunks);
      hipLaunchKernelGGL(lw_narrow_wgrad_kernel, grid, dim3(256), 0, st, g);
      TMNN_HIP_TRY(hipGetLastError());
      return TMNN_OK;
    }
    if (chunks == 1 && lw_narrow_mask_ok(g)) {
      const dim3 grid((g.R + kLwNarrowRows - 1) / kLwNarrowRows, (g.C + 255) / 256);
      hipLaunchKernelGGL(lw_narrow_mask_kernel, grid, dim3(256), 0, st, g);
      TMNN_HIP_TRY(hipGetLastError());
      return TMNN_OK;
    }
    const dim3 grid((g.R + kLwTile - 1) / kLwTile, (g.C + kLwTile - 1) / kLwTile, chunks);
    const LwGemmFn fn = lw_gemm_fn(g);
    if (!fn) return fail(TMNN_ERR_RUNTIME, "layer-wise product of an unexpected form");
    hipLaunchKernelGGL(fn, grid, dim3(256), 0, st, g);
    TMNN_HIP_TRY(hipGetLastError());
    return TMNN_OK;
  };
  LwGemmArgs base{};
  base.KT0 = tr->INP / 16;
  base.scale = 1.0f;
  if (fwd_only) {
    // Forward passes (inference has no batch cap) run in chunks of at most
    // kLwForwardChunk points through two ping-pong activation buffers, so
    // their memory is bounded whatever n is; the backward's buffers are not
    // touched. Every forward caller hands over positions in output order
    // (perm == nullptr) with an optional output row index.
    const int chunk = std::min(n, kLwForwardChunk);
    const size_t C = static_cast<size_t>(chunk);
    TMNN_HIP_TRY(tr->lw_act.ensure(2 * C * H * sizeof(float)));
    float *buf[2] = {tr->lw_act.as<float>(), tr->lw_act.as<float>() + C * H};
    for (int c0 = 0; c0 < n; c0 += chunk) {
      const int cn = std::min(chunk, n - c0);
      if ((rc = launch_encode(tr, a.pos + static_cast<size_t>(c0) * tr->d.spatial_dims, cn)) !=
          TMNN_OK)
        return rc;
      if (c0 == 0 && prof_after_encode >= 0 && (rc = prof_mark(tr, prof_after_encode)) != TMNN_OK)
        return rc;
      for (int k = 0; k <= NHL; ++k) {
        LwGemmArgs g = base;
        g.R = cn;
        g.K = k == 0 ? IN : H;
        g.C = k == NHL ? M : H;
        g.k_chunk = g.K;
        g.a_mode = k == 0 ? kLwAXTiles : kLwARow;
        g.A = k == 0 ? tr->xfeat.as<float>() : buf[(k - 1) & 1];
        g.lda = H;
        g.B = a.mlp + lay.w_off(k);
        g.ldb = g.C;
        g.bias = a.mlp + lay.b_off(k);
        if (k < NHL) {
          g.epi = kLwEpiHidden;
          g.out = buf[k & 1];
          g.ldo = H;
        } else {
          g.epi = kLwEpiOutput;
          g.out = a.out_index ? a.out : a.out + static_cast<size_t>(c0) * M;
          g.out_index = a.out_index ? a.out_index + c0 : nullptr;
          g.ldo = M;
        }
        if ((rc = gemm(g, 1)) != TMNN_OK) return rc;
      }
    }
    return 1;
  }
  if (!reuse_x && (rc = launch_encode(tr, a.pos, n, perm, pos_out)) != TMNN_OK) return rc;
  if (prof_after_encode >= 0 && (rc = prof_mark(tr, prof_after_encode)) != TMNN_OK) return rc;
  const size_t N = static_cast<size_t>(n);
  TMNN_HIP_TRY(tr->lw_act.ensure(N * H * NHL * sizeof(float)));
  TMNN_HIP_TRY(tr->lw_y.ensure(N * M * sizeof(float)));
  TMNN_HIP_TRY(tr->lw_g.ensure(N * M * sizeof(float)));
  TMNN_HIP_TRY(tr->lw_d.ensure(2 * N * std::max(H, 1) * sizeof(float)));
  float *act = tr->lw_act.as<float>();
  auto act_k = [&](int k) { return act + static_cast<size_t>(k) * N * H; };
  // ---- forward (kept when the caller re-runs the backward for another output)
  if (!(reuse_x && a.mode == kModeInputGrad)) {
    for (int k = 0; k <= NHL; ++k) {
      LwGemmArgs g = base;
      g.R = n;
      g.K = k == 0 ? IN : H;
      g.C = k == NHL ? M : H;
      g.k_chunk = g.K;
      g.a_mode = k == 0 ? kLwAXTiles : kLwARow;
      g.A = k == 0 ? tr->xfeat.as<float>() : act_k(k - 1);
      g.lda = H;
      g.B = a.mlp + lay.w_off(k);
      g.ldb = g.C;
      g.bias = a.mlp + lay.b_off(k);
      if (k < NHL) {
        g.epi = kLwEpiHidden;
        g.out = act_k(k);
        g.ldo = H;
      } else {
        g.epi = kLwEpiOutput;
        g.out = nullptr;
        g.out_index = a.out_index;
        g.ldo = M;
        g.out2 = tr->lw_y.as<float>();
        g.ldo2 = M;
      }
      if ((rc = gemm(g, 1)) != TMNN_OK) return rc;
    }
  }
  // ---- output gradient (and the loss), per batch chunk: chunks of at least
  // 512 points (2^16 points: 128 chunks; 256 points per chunk wrote twice the
  // partial rows for a slower step at every measured width)
  const int P = std::max(1, std::min(plan.max_blocks, (n + 511) / 512));
  const int chunk = (n + P - 1) / P;
  LwLossArgs la{};
  la.n = n;
  la.M = M;
  la.mode = a.mode;
  la.loss_kind = a.loss_kind;
  la.grad_output = a.grad_output;
  la.chunk = chunk;
  la.huber_delta = a.huber_delta;
  la.inv_n = a.inv_n;
  la.loss_scale = 1.0f;
  la.y = tr->lw_y.as<float>();
  la.target = a.target;
  la.tgt_index = a.tgt_index;
  la.out = a.out;
  la.out_index = a.out_index;
  la.g = tr->lw_g.as<float>();
  la.loss_partials = a.loss_partials;
  la.amax_partials = a.amax_partials;
  hipLaunchKernelGGL(lw_loss_kernel, dim3(P), dim3(256), 0, st, la);
  TMNN_HIP_TRY(hipGetLastError());
  // ---- backward: weight-gradient partial rows (training), deltas, dx
  const bool wgrads = a.mode != kModeInputGrad;
  const int64_t row = a.mlp_count;
  float *dbuf[2] = {tr->lw_d.as<float>(), tr->lw_d.as<float>() + N * H};
  // dW_k and b_k of one layer as one product: A's extra all-ones row (r = R)
  // writes the column sums of D into row R of the partial, which is b_k's
  // slot (b_off = w_off + R * C in the reference layout)
  auto partial_dw = [&](const float *A, int a_mode, int lda, int R, const float *D, int C,
                        int w_off) -> int {
    LwGemmArgs g = base;
    g.R = R + 1;
    g.ones_row = 1;
    g.C = C;
    g.K = n;
    g.k_chunk = chunk;
    g.a_mode = a_mode;
    g.A = A;
    g.lda = lda;
    g.B = D;
    g.ldb = C;
    g.epi = kLwEpiPartial;
    g.dst = a.grad_partials;
    g.dst_stride = row;
    g.dst_off = w_off;
    return gemm(g, P);
  };
  const float *dcur = tr->lw_g.as<float>();  // gradient at the current layer's output
  int dcols = M;
  for (int k = NHL; k >= 0; --k) {
    // layer k maps its input (X for k = 0, else h_{k-1}) to dcur
    if (wgrads) {
      if (k > 0)
        rc = partial_dw(act_k(k - 1), kLwACol, H, H, dcur, dcols, lay.w_off(k));
      else
        rc = partial_dw(tr->xfeat.as<float>(), kLwAXTilesT, 0, IN, dcur, dcols, lay.w_off(0));
      if (rc != TMNN_OK) return rc;
    }
    LwGemmArgs g = base;
    g.R = n;
    g.K = dcols;
    g.k_chunk = dcols;
    g.a_mode = kLwARow;
    g.A = dcur;
    g.lda = dcols;
    g.B = a.mlp + lay.w_off(k);  // W_k [in][dcols], read transposed
    g.b_trans = 1;
    g.ldb = dcols;
    if (k > 0) {
      float *dnext = dbuf[k & 1];
      g.C = H;
      g.epi = kLwEpiMask;  // times [h_{k-1} > 0]
      g.mask = act_k(k - 1);
      g.ldm = H;
      g.out = dnext;
      g.ldo = H;
      if ((rc = gemm(g, 1)) != TMNN_OK) return rc;
      dcur = dnext;
      dcols = H;
    } else {
      g.C = IN;
      g.epi = kLwEpiScale;
      g.out = a.dx_out;
      g.ldo = IN;
      if ((rc = gemm(g, 1)) != TMNN_OK) return rc;
    }
  }
  return P;
}

// Power-of-two loss scale for the fp16 backward: d_out carries 1/N, which
// puts it in fp16's subnormal range at large N; scaling by ~N keeps the
// backward operands normal and the rescale exact.
float loss_scale_for(int n, bool f16) {
  if (!f16 || n <= 1) return 1.0f;
  int e = 0;
  std::frexp(static_cast<float>(n), &e);
  return std::ldexp(1.0f, std::min(e, 24));
}

int ensure_batch(tmnn_trainer *tr, int n) {
  const size_t D = tr->d.spatial_dims, M = tr->d.num_outputs;
  TMNN_HIP_TRY(tr->in_pos.ensure(n * D * sizeof(float)));
  TMNN_HIP_TRY(tr->in_tgt.ensure(n * M * sizeof(float)));
  TMNN_HIP_TRY(tr->s_pos.ensure(n * D * sizeof(float)));
  TMNN_HIP_TRY(tr->s_tgt.ensure(n * M * sizeof(float)));
  TMNN_HIP_TRY(tr->keys0.ensure(n * sizeof(uint32_t)));
  TMNN_HIP_TRY(tr->keys1.ensure(n * sizeof(uint32_t)));
  TMNN_HIP_TRY(tr->vals0.ensure(n * sizeof(uint32_t)));
  TMNN_HIP_TRY(tr->vals1.ensure(n * sizeof(uint32_t)));
  size_t tmp = 0;
  TMNN_HIP_TRY(morton_sort_temp_bytes(n, &tmp));
  TMNN_HIP_TRY(tr->sort_tmp.ensure(std::max<size_t>(tmp, 256)));
  if (tr->d.morton_sort)
    for (auto &ss : tr->step_sort) {
      TMNN_HIP_TRY(ss.keys0.ensure(n * sizeof(uint32_t)));
      TMNN_HIP_TRY(ss.keys1.ensure(n * sizeof(uint32_t)));
      TMNN_HIP_TRY(ss.vals0.ensure(n * sizeof(uint32_t)));
      TMNN_HIP_TRY(ss.vals1.ensure(n * sizeof(uint32_t)));
      TMNN_HIP_TRY(ss.tmp.ensure(std::max<size_t>(tmp, 256)));
    }
  // dx rows for the whole last tile: the MLP train kernel stores unconditionally
  TMNN_HIP_TRY(tr->dx.ensure(static_cast<size_t>((n + kTilePts - 1) / kTilePts) * kTilePts *
                             tr->IN * sizeof(float)));
  TMNN_HIP_TRY(tr->xfeat.ensure(static_cast<size_t>((n + kTilePts - 1) / kTilePts) * kTilePts *
                                tr->INP * sizeof(float)));
  if (tr->train_plan.wide && tr->d.num_hidden_layers > 1) {
    const size_t tiles = static_cast<size_t>((n + kTilePts - 1) / kTilePts);
    const size_t layers = static_cast<size_t>(tr->d.num_hidden_layers - 1);
    TMNN_HIP_TRY(tr->wide_mask.ensure(layers * tiles * 64 * sizeof(uint64_t)));
    TMNN_HIP_TRY(tr->wide_act.ensure(layers * tiles * kWideHP * kTilePts * 2));
  }
  return TMNN_OK;
}

// Morton order of the batch: returns the permutation (sorted i -> original
// row), or nullptr when sorting is off. With gather, also the sorted copies
// of (pos, tgt) in s_pos / s_tgt (else *pos_out / *tgt_out are the inputs:
// the training path reads them through the permutation).
int sort_batch(tmnn_trainer *tr, const float *d_pos, const float *d_tgt,
               int tgt_dims, int n, const float **pos_out,
               const float **tgt_out, const uint32_t **perm_out, bool gather = true) {
  hipStream_t st = tr->ctx->stream;
  if (!tr->d.morton_sort || n <= 1) {
    *pos_out = d_pos;
    *tgt_out = d_tgt;
    *perm_out = nullptr;
    return TMNN_OK;
  }
  const int threads = 256;
  const uint32_t *sorted_keys = nullptr, *perm = nullptr;
  TMNN_HIP_TRY(morton_sort_batch(tr->sort_tmp.ptr, tr->sort_tmp.bytes, d_pos, tr->d.spatial_dims,
                                 tr->keys0.as<uint32_t>(), tr->keys1.as<uint32_t>(),
                                 tr->vals0.as<uint32_t>(), tr->vals1.as<uint32_t>(), n, st,
                                 &sorted_keys, &perm));
  if (!gather) {
    *pos_out = d_pos;
    *tgt_out = d_tgt;
    *perm_out = perm;
    return TMNN_OK;
  }
  const size_t elems = static_cast<size_t>(n) * (tr->d.spatial_dims + (d_tgt ? tgt_dims : 0));
  hipLaunchKernelGGL(gather_rows_kernel, dim3(static_cast<uint32_t>((elems + threads - 1) / threads)),
                     dim3(threads), 0, st, d_pos, d_tgt, perm, n, tr->d.spatial_dims, tgt_dims,
                     tr->s_pos.as<float>(), d_tgt ? tr->s_tgt.as<float>() : nullptr);
  TMNN_HIP_TRY(hipGetLastError());
  *pos_out = tr->s_pos.as<float>();
  *tgt_out = d_tgt ? tr->s_tgt.as<float>() : nullptr;
  *perm_out = perm;
  return TMNN_OK;
}

// Hash-grid backward of the dx the train kernel left in tr->dx for the n
// points at pos (same order): table gradients + visit flags.
int launch_scatter(tmnn_trainer *tr, const float *pos, int n) {
  ScatterArgs s{};
  s.n = n;
  s.IN = tr->IN;
  s.log2T = static_cast<uint32_t>(tr->d.log2_hashmap_size);
  for (int l = 0; l < kMaxLevels; ++l) s.res[l] = tr->res[l];
  s.pos = pos;
  s.dx = tr->dx.as<float>();
  s.grad_hash = tr->grad_hash.as<int32_t>();
  s.mask = tr->mask[tr->mask_cur].as<uint8_t>();
  // point-major while a level's slice of the table is cache-sized, else
  // level-major (one level's slice at a time). Point-major 3D splits a
  // point's levels over four threads (C3: 415 -> 378 us); 2D keeps one
  // thread per point (splitting measured slower at C2)
  const bool by_level = level_major(tr);
  const int split = tr->d.spatial_dims == 3 ? 4 : 1;
  const dim3 grid((n + kScatterThreads - 1) / kScatterThreads,
                  by_level ? tr->d.num_levels : split);
  hipStream_t st = tr->ctx->stream;
#define TMNN_SCATTER(d, f)                                                                   \
  if (by_level)                                                                              \
    launch_step_kernel(tr, kKernScatter, hash_scatter_level_kernel<d, f>, grid,              \
                       dim3(kScatterThreads), 0, st, s);                                     \
  else                                                                                       \
    launch_step_kernel(tr, kKernScatter, hash_scatter_kernel<d, f>, grid,                    \
                       dim3(kScatterThreads), 0, st, s);
  switch (tr->d.spatial_dims * 8 + tr->d.features_per_level) {
    case 2 * 8 + 1: TMNN_SCATTER(2, 1) break;
    case 2 * 8 + 2: TMNN_SCATTER(2, 2) break;
    case 2 * 8 + 4: TMNN_SCATTER(2, 4) break;
    case 3 * 8 + 1: TMNN_SCATTER(3, 1) break;
    case 3 * 8 + 2: TMNN_SCATTER(3, 2) break;
    case 3 * 8 + 4: TMNN_SCATTER(3, 4) break;
    case 4 * 8 + 1: TMNN_SCATTER(4, 1) break;
    case 4 * 8 + 2: TMNN_SCATTER(4, 2) break;
    default: TMNN_SCATTER(4, 4) break;
  }
#undef TMNN_SCATTER
  TMNN_HIP_TRY(hipGetLastError());
  return TMNN_OK;
}

// Flags of the events that order the side stream's sort and the main stream's
// step. Both streams run on this device, so the producer's release and the
// consumer's acquire only need device scope: without
// hipEventDisableSystemFence every record and wait adds a system-scope fence
// (cache write-back and invalidation), measured at C2 as 98.7 -> 94.6 us per
// step.
constexpr unsigned kSyncEventFlags = hipEventDisableTiming | hipEventDisableSystemFence;

// The fused step's Morton sort on the side stream into buffer set
// tr->sort_parity (see tmnn_trainer::step_sort): the side stream first waits
// until the step that last used the set has finished (and, when the batch
// was staged on the main stream, for that copy); the main stream then waits
// for the sort. The caller marks the set consumed after the step
// (sort_set_consumed). Returns the permutation in *perm_out.
int sort_batch_overlapped(tmnn_trainer *tr, const float *d_pos, int n, bool staged_on_main,
                          const uint32_t **perm_out) {
  hipStream_t st = tr->ctx->stream;
  if (!tr->side) {
    TMNN_HIP_TRY(hipStreamCreateWithFlags(&tr->side, hipStreamNonBlocking));
    for (int k = 0; k < tmnn_trainer::kSortSets; ++k) {
      TMNN_HIP_TRY(hipEventCreateWithFlags(&tr->ev_sorted[k], kSyncEventFlags));
      TMNN_HIP_TRY(hipEventCreateWithFlags(&tr->ev_consumed[k], kSyncEventFlags));
    }
  }
  const int k = tr->sort_parity;
  auto &ss = tr->step_sort[k];
  hipStream_t sd = tr->side;
  if (tr->consumed_recorded[k]) TMNN_HIP_TRY(hipStreamWaitEvent(sd, tr->ev_consumed[k], 0));
  if (tr->input_ready) TMNN_HIP_TRY(hipStreamWaitEvent(sd, tr->input_ready, 0));
  if (staged_on_main) {
    // the batch was copied in on the main stream: the sort reads it after
    // that (an event with the system-scope fence, as the copy came from host
    // memory)
    if (!tr->ev_staged) TMNN_HIP_TRY(hipEventCreateWithFlags(&tr->ev_staged, hipEventDisableTiming));
    TMNN_HIP_TRY(hipEventRecord(tr->ev_staged, st));
    TMNN_HIP_TRY(hipStreamWaitEvent(sd, tr->ev_staged, 0));
  }
  const uint32_t *sorted_keys = nullptr;
  TMNN_HIP_TRY(morton_sort_batch(ss.tmp.ptr, ss.tmp.bytes, d_pos, tr->d.spatial_dims,
                                 ss.keys0.as<uint32_t>(), ss.keys1.as<uint32_t>(),
                                 ss.vals0.as<uint32_t>(), ss.vals1.as<uint32_t>(), n, sd,
                                 &sorted_keys, perm_out));
  TMNN_HIP_TRY(hipEventRecord(tr->ev_sorted[k], sd));
  TMNN_HIP_TRY(hipStreamWaitEvent(st, tr->ev_sorted[k], 0));
  return TMNN_OK;
}

// After the last reader of the current sort set on the main stream: the set
// may be sorted into again (kSortSets steps later); the next step takes the
// next set.
int sort_set_consumed(tmnn_trainer *tr) {
  const int k = tr->sort_parity;
  TMNN_HIP_TRY(hipEventRecord(tr->ev_consumed[k], tr->ctx->stream));
  tr->consumed_recorded[k] = true;
  tr->sort_parity = (k + 1) % tmnn_trainer::kSortSets;
  return TMNN_OK;
}

// Fused forward/backward over n device-resident points, gradients
// accumulated into grad_hash / grad_mlp / mask. Returns the block count used
// (for the loss reduction) or a negative status.
int run_forward_backward(tmnn_trainer *tr, const float *d_pos, const float *d_tgt,
                         int n, bool external_grad, float *d_loss = nullptr,
                         bool reduce = true, int overlap_sort = 0) {
  const bool f16 = tr->d.precision == TMNN_PRECISION_FP16;
  const float *pos = d_pos, *tgt = d_tgt;
  const uint32_t *perm = nullptr;
  int rc = prof_mark(tr, 0);
  if (rc != TMNN_OK) return rc;
  // the packed weight image (rebuilt after every Adam step) counts with the sort
  if ((rc = ensure_image(tr, tr->train_plan)) != TMNN_OK) return rc;
  if (overlap_sort && tr->d.morton_sort && n > 1 && tr->train_plan.xmem) {
    // feature-tile plans read the batch through the permutation (no gather)
    rc = sort_batch_overlapped(tr, d_pos, n, overlap_sort > 1, &perm);
  } else {
    rc = sort_batch(tr, d_pos, d_tgt, tr->d.num_outputs, n, &pos, &tgt, &perm,
                    !tr->train_plan.xmem);
  }
  if (rc != TMNN_OK) return rc;
  if ((rc = prof_mark(tr, 1)) != TMNN_OK) return rc;
  FieldArgs a = base_args(tr);
  a.mode = external_grad ? kModeTrainExtGrad : kModeTrainLoss;
  a.inv_n = 1.0f / static_cast<float>(n);
  a.loss_scale = loss_scale_for(n, f16);
  a.inv_loss_scale = 1.0f / a.loss_scale;
  a.pos = pos;
  a.target = tgt;
  // feature-tile plans read the batch through the permutation: the encode
  // kernel writes the sorted positions (for the scatter), targets are indexed
  const bool indexed = tr->train_plan.xmem && perm != nullptr;
  a.tgt_index = indexed ? perm : nullptr;
  float *sorted_pos = indexed ? tr->s_pos.as<float>() : nullptr;
  a.grad_partials = tr->partials.as<float>();
  a.loss_partials = tr->loss_partials.as<float>();
  a.amax_partials = (!external_grad && tr->num_this_step) ? tr->amax_partials.as<float>() : nullptr;
  if (tr->dbg_step_out) {  // parity read-out: outputs in the caller's row order
    a.out = tr->dbg_step_out;
    a.out_index = perm;
  }
  a.dx_out = tr->dx.as<float>();
  const bool fused_scatter = tr->train_plan.tile_scatter;
  if (fused_scatter) {  // the training kernel runs the hash-grid backward per tile
    a.spos = indexed ? sorted_pos : pos;
    a.grad_hash = tr->grad_hash.as<int32_t>();
    a.mask = tr->mask[tr->mask_cur].as<uint8_t>();
  }
  const int blocks = launch_field(tr, tr->train_plan, a, n, 2, false, a.tgt_index, sorted_pos);
  if (blocks < 0) return blocks;
  if ((rc = prof_mark(tr, 3)) != TMNN_OK) return rc;
  if (!fused_scatter) {  // else the scatter phase is empty (no boundary event)
    if ((rc = launch_scatter(tr, indexed ? sorted_pos : pos, n)) != TMNN_OK) return rc;
    if ((rc = prof_mark(tr, 4)) != TMNN_OK) return rc;
  }
  if (!reduce) return blocks;  // finish_step_kernel reduces the rows and the loss
  // dW rows, plus (training steps) the loss in one extra block
  const uint32_t rblocks = (tr->mlp_count + kReduceCols - 1) / kReduceCols + (d_loss ? 1 : 0);
  hipLaunchKernelGGL(reduce_partials_kernel, dim3(rblocks), dim3(kReduceCols * kReduceGroups), 0,
                     tr->ctx->stream, tr->partials.as<float>(), blocks,
                     static_cast<int32_t>(tr->mlp_count), tr->grad_mlp.as<float>(),
                     tr->loss_partials.as<float>(), n, d_loss);
  TMNN_HIP_TRY(hipGetLastError());
  return blocks;
}

AdamArgs adam_args(tmnn_trainer *tr, bool clear_grads, bool clear_mask) {
  AdamArgs a{};
  a.params = tr->params.as<float>();
  a.m = tr->m.as<float>();
  a.v = tr->v.as<float>();
  a.grad_hash = tr->grad_hash.as<int32_t>();
  a.grad_mlp = tr->grad_mlp.as<float>();
  // Sparse hash Adam needs l1_reg == 0 (default_trainer.cpp:1868-1876).
  a.lazy = (tr->d.hash_adam_mode == TMNN_HASH_ADAM_LAZY && tr->d.l1_reg == 0.0f) ? 1 : 0;
  a.mask = tr->mask[tr->mask_cur].as<uint8_t>();
  a.mask_next = tr->mask[tr->mask_cur ^ 1].as<uint8_t>();
  a.partner_xor = tr->d.spatial_dims == 2 ? (kPrimeZ & ((1u << tr->d.log2_hashmap_size) - 1u)) : 0u;
  a.log2T = static_cast<uint32_t>(tr->d.log2_hashmap_size);
  a.hash_entries = tr->hash_entries;
  a.mlp_count = tr->mlp_count;
  a.lr_hash = tr->lr_enc;
  a.lr_mlp = tr->lr_net;
  a.beta1 = tr->d.beta1;
  a.beta2 = tr->d.beta2;
  a.eps = tr->d.epsilon;
  // adam_params.h:39-46: bc = 1 - pow(beta, step + 1) in fp32 on the host.
  const float s = static_cast<float>(tr->step + 1);
  a.bc1 = 1.0f - std::pow(tr->d.beta1, s);
  a.bc2 = 1.0f - std::pow(tr->d.beta2, s);
  a.l1_hash = tr->d.l1_reg;
  a.l2_mlp = tr->d.l2_reg;
  a.grad_clip = tr->d.grad_clip;
  a.weight_decay = tr->d.weight_decay;
  a.clear_grads = clear_grads ? 1 : 0;
  a.clear_mask = clear_mask ? 1 : 0;
  return a;
}

int run_adam(tmnn_trainer *tr, bool clear_grads, bool clear_mask) {
  const AdamArgs a = adam_args(tr, clear_grads, clear_mask);
  const uint32_t total = tr->hash_entries + tr->mlp_count;
  const uint32_t blocks = std::min<uint32_t>((total + 255) / 256,
                                             static_cast<uint32_t>(tr->ctx->cu_count) * 16u);
  switch (tr->d.features_per_level) {
    case 1: hipLaunchKernelGGL(adam_kernel<1>, dim3(blocks), dim3(256), 0, tr->ctx->stream, a); break;
    case 2: hipLaunchKernelGGL(adam_kernel<2>, dim3(blocks), dim3(256), 0, tr->ctx->stream, a); break;
    default: hipLaunchKernelGGL(adam_kernel<4>, dim3(blocks), dim3(256), 0, tr->ctx->stream, a); break;
  }
  TMNN_HIP_TRY(hipGetLastError());
  if (clear_mask) tr->mask_cur ^= 1;  // the zeroed buffer collects the next step
  ++tr->weights_version;
  return TMNN_OK;
}

// The end of a fused training step (finish_step_kernel): dW reduction of the
// part_blocks partial rows, the loss, Adam (grads and flags cleared), and the
// training plan's image updated in place when it was current.
int run_finish(tmnn_trainer *tr, int part_blocks, int n, float *d_loss) {
  FinishArgs f{};
  f.adam = adam_args(tr, true, true);
  f.partials = tr->partials.as<float>();
  f.part_blocks = part_blocks;
  f.loss_partials = tr->loss_partials.as<float>();
  f.n = n;
  f.loss_out = d_loss;
  f.mlp_blocks = static_cast<int32_t>((tr->mlp_count + kReduceCols - 1) / kReduceCols);
  KernelPlan &plan = tr->train_plan;
  const bool image_current = plan.image && plan.packed_version == tr->weights_version;
  f.s = make_layout(tr->INP, tr->HP, tr->IN, tr->d.hidden_dim, tr->d.num_hidden_layers,
                    tr->d.num_outputs, static_cast<int>(tr->mlp_count), plan.f16, plan.train, 1);
  f.f16 = plan.f16 ? 1 : 0;
  f.image = image_current ? static_cast<unsigned char *>(plan.image) : nullptr;
  const bool num = tr->num_this_step;
  f.amax_partials = tr->amax_partials.as<float>();
  f.num_rows = static_cast<float4 *>(tr->num_rows.ptr);
  // Hash blocks: large tables grid-stride over at most four blocks per CU;
  // a small table's blocks fill what the MLP and loss blocks leave of one
  // round of resident blocks (two 1024-thread blocks per CU) when that keeps
  // each thread at two entries or fewer (no second, partial round of blocks)
  const uint32_t needed = (tr->hash_entries + kFinishThreads - 1) / kFinishThreads;
  const uint32_t cap = static_cast<uint32_t>(tr->ctx->cu_count) * 4u;
  const uint32_t resident = static_cast<uint32_t>(tr->ctx->cu_count) * 2u;
  const uint32_t other = static_cast<uint32_t>(f.mlp_blocks) + 1u;
  const uint32_t room = resident > other ? resident - other : 0u;
  const uint32_t hash_blocks =
      needed > cap ? cap : std::max<uint32_t>({1u, std::min(needed, room), (needed + 1u) / 2u});
  const dim3 grid(static_cast<uint32_t>(f.mlp_blocks) + 1u + hash_blocks);
  if (num && tr->num_rows.bytes < grid.x * sizeof(float4))
    return fail(TMNN_ERR_RUNTIME, "numerics rows smaller than the finish grid");
  hipStream_t st = tr->ctx->stream;
#define TMNN_FINISH(ff)                                                                            \
  if (num)                                                                                         \
    launch_step_kernel(tr, kKernFinish, finish_step_kernel<ff, true>, grid, dim3(kFinishThreads),  \
                       0, st, f);                                                                  \
  else                                                                                             \
    launch_step_kernel(tr, kKernFinish, finish_step_kernel<ff, false>, grid, dim3(kFinishThreads), \
                       0, st, f);
  switch (tr->d.features_per_level) {
    case 1: TMNN_FINISH(1) break;
    case 2: TMNN_FINISH(2) break;
    default: TMNN_FINISH(4) break;
  }
#undef TMNN_FINISH
  TMNN_HIP_TRY(hipGetLastError());
  if (num) {
    tr->num_row_count = static_cast<int>(grid.x);
    tr->num_loss_row = f.mlp_blocks;
    tr->num_step = tr->step + 1;
    tr->num_batch = static_cast<uint32_t>(n);
  }
  tr->mask_cur ^= 1;  // the zeroed buffer collects the next step
  ++tr->weights_version;
  if (image_current) plan.packed_version = tr->weights_version;
  return TMNN_OK;
}

int zero_device(tmnn_trainer *tr, void *ptr, size_t bytes) {
  if (bytes == 0) return TMNN_OK;
  const size_t n16 = (bytes + 15) / 16;
  const uint32_t blocks = static_cast<uint32_t>(
      std::min<size_t>((n16 + 255) / 256, static_cast<size_t>(tr->ctx->cu_count) * 8));
  hipLaunchKernelGGL(zero_bytes_kernel, dim3(std::max<uint32_t>(blocks, 1)), dim3(256), 0,
                     tr->ctx->stream, static_cast<uint8_t *>(ptr), bytes);
  TMNN_HIP_TRY(hipGetLastError());
  return TMNN_OK;
}

// Releases the event set claimed for a step that failed before its last
// event was recorded (prof_collect would otherwise read unrecorded events).
void prof_abort(tmnn_trainer *tr) {
  if (tr->prof_cur >= 0) tr->prof_used = static_cast<size_t>(tr->prof_cur);
  tr->prof_cur = -1;
}

// NumericsGuard::should_sample (numerics_guard.cpp:12-36) for the step
// counter after the update.
bool numerics_should_sample(const tmnn_trainer *tr, uint32_t step) {
  const bool after_anomaly = tr->num_anomalies > 0 && step == tr->num_last_anomaly + 1;
  switch (tr->num_mode) {
    case TMNN_NUMERICS_DISABLED: return false;
    case TMNN_NUMERICS_FULL: return true;
    case TMNN_NUMERICS_PERIODIC:
      return after_anomaly || (step != 0 && step % tr->num_interval == 0);
    default:
      return step == 0 || step == 1 || after_anomaly || step % tr->num_interval == 0;
  }
}

// A report from the finish kernel's rows (host copies): the largest |output|
// and the loss from the loss block's row, max / sum / OR over the others.
void numerics_from_rows(const std::vector<float4> &rows, int loss_row, tmnn_step_result *out) {
  float gmax = 0.0f, umax = 0.0f;
  double g2 = 0.0;
  uint32_t bad = 0u;
  for (size_t b = 0; b < rows.size(); ++b) {
    if (static_cast<int>(b) == loss_row) continue;
    gmax = std::max(gmax, rows[b].x);
    g2 += static_cast<double>(rows[b].y);
    umax = std::max(umax, rows[b].z);
    uint32_t w;
    std::memcpy(&w, &rows[b].w, sizeof w);
    bad |= w;
  }
  tmnn_numerics_report &r = out->numerics;
  r = tmnn_numerics_report{};
  const float loss = rows[loss_row].y;
  r.finite_forward = std::isfinite(loss) ? 1 : 0;
  r.finite_backward = (bad & 1u) ? 0 : 1;
  r.finite_update = (r.finite_backward && !(bad & 2u)) ? 1 : 0;
  r.max_abs_activation = rows[loss_row].x;
  r.max_abs_gradient = gmax;
  r.max_abs_update = umax;
  r.first_bad_layer = 0u;
  out->grad_norm = static_cast<float>(std::sqrt(g2));
  out->numerics_reported = 1;
  out->has_numerics_anomaly = (r.finite_forward && r.finite_backward && r.finite_update) ? 0 : 1;
}

// Copies the rows of the last computed report (enqueued on the trainer's
// stream; the caller synchronizes).
int numerics_rows_download(tmnn_trainer *tr, std::vector<float4> &rows) {
  rows.resize(static_cast<size_t>(tr->num_row_count));
  TMNN_HIP_TRY(hipMemcpyAsync(rows.data(), tr->num_rows.ptr, rows.size() * sizeof(float4),
                              hipMemcpyDeviceToHost, tr->ctx->stream));
  return TMNN_OK;
}

// NumericsGuard::record_step: an anomaly makes the next step sampled.
void numerics_record(tmnn_trainer *tr, uint32_t step, const tmnn_step_result &r) {
  if (r.has_numerics_anomaly) {
    ++tr->num_anomalies;
    tr->num_last_anomaly = step;
  }
}

// overlap_sort: 0 sorts on the main stream (the step's buffers may be
// borrowed scratch); 1 sorts on the side stream (the caller's batch is
// ready); 2 as 1, the batch being staged on the main stream.
// num: the finish kernel also computes the step's numerics report (rows on
// the device). input_ready (nullable): an event of the caller's that every
// stream reading the batch waits for first.
int train_step_device(tmnn_trainer *tr, const float *d_pos, const float *d_tgt, int n,
                      float *d_loss, int overlap_sort = 1, bool num = false,
                      hipEvent_t input_ready = nullptr) {
  if (input_ready) TMNN_HIP_TRY(hipStreamWaitEvent(tr->ctx->stream, input_ready, 0));
  int rc = prof_begin_step(tr);
  if (rc != TMNN_OK) return rc;
  float *loss = d_loss ? d_loss : tr->loss_out.as<float>();
  const bool overlapped = overlap_sort && tr->d.morton_sort && n > 1 && tr->train_plan.xmem;
  tr->num_this_step = num;
  tr->input_ready = input_ready;
  const int blocks = run_forward_backward(tr, d_pos, d_tgt, n, false, loss, false, overlap_sort);
  tr->input_ready = nullptr;
  if (blocks < 0) {
    tr->num_this_step = false;
    prof_abort(tr);
    if (overlapped) (void)sort_set_consumed(tr);
    return blocks;
  }
  // dW reduction, loss and Adam in one kernel (the reduce phase is empty: no
  // boundary event)
  rc = run_finish(tr, blocks, n, loss);
  tr->num_this_step = false;
  if (rc != TMNN_OK || (rc = prof_mark(tr, 6)) != TMNN_OK) {
    prof_abort(tr);
    if (overlapped) (void)sort_set_consumed(tr);
    return rc;
  }
  if (overlapped && (rc = sort_set_consumed(tr)) != TMNN_OK) return rc;
  if (tr->prof_cur >= 0) tr->prof_acc.batch_size = static_cast<uint32_t>(n);
  tr->prof_cur = -1;
  ++tr->step;
  return TMNN_OK;
}

int zero_training_state(tmnn_trainer *tr) {
  int rc = zero_device(tr, tr->grad_hash.ptr, tr->hash_count * sizeof(int32_t));
  if (rc == TMNN_OK) rc = zero_device(tr, tr->grad_mlp.ptr, tr->mlp_count * sizeof(float));
  if (rc == TMNN_OK) rc = zero_device(tr, tr->mask[0].ptr, tr->hash_entries);
  if (rc == TMNN_OK) rc = zero_device(tr, tr->mask[1].ptr, tr->hash_entries);
  return rc;
}

int reset_moments(tmnn_trainer *tr) {
  const size_t total = (static_cast<size_t>(tr->hash_count) + tr->mlp_count) * sizeof(float);
  int rc = zero_device(tr, tr->m.ptr, total);
  if (rc == TMNN_OK) rc = zero_device(tr, tr->v.ptr, total);
  return rc;
}

int philox_fill(hipStream_t st, float *dst, uint32_t count, uint64_t seed, uint32_t base,
                float low, float high) {
  if (count == 0) return TMNN_OK;
  const uint32_t threads = (count + 3u) / 4u;
  hipLaunchKernelGGL(philox_uniform_kernel, dim3((threads + 255) / 256), dim3(256), 0, st, dst,
                     count, static_cast<uint32_t>(seed & 0xFFFFFFFFu),
                     static_cast<uint32_t>(seed >> 32), base, low, high);
  TMNN_HIP_TRY(hipGetLastError());
  return TMNN_OK;
}

// init_weights_with_config (default_trainer.cpp:1978-2180): one Philox
// stream; hash at counter 0, then per layer W (Kaiming uniform, ReLU gain)
// and b (U(+-1/sqrt(fan_in))), each advancing the counter by ceil(count/4).
int init_weights(tmnn_trainer *tr) {
  hipStream_t st = tr->ctx->stream;
  float *hash = tr->params.as<float>();
  const float r = tr->d.hash_init_range;
  int rc = philox_fill(st, hash, tr->hash_count, tr->d.seed, 0u, -r, r);
  if (rc != TMNN_OK) return rc;
  uint32_t ctr = (tr->hash_count + 3u) / 4u;
  const float gain = std::sqrt(2.0f);
  const int H = tr->d.hidden_dim, M = tr->d.num_outputs;
  struct Slice { int wc, bc, fan_in; };
  std::vector<Slice> layers;
  layers.push_back({tr->IN * H, H, tr->IN});
  for (int k = 1; k < tr->d.num_hidden_layers; ++k) layers.push_back({H * H, H, H});
  layers.push_back({H * M, M, H});
  float *dst = hash + tr->hash_count;
  for (const Slice &s : layers) {
    const float fin = static_cast<float>(s.fan_in);
    const float bw = gain * std::sqrt(3.0f / fin);
    rc = philox_fill(st, dst, static_cast<uint32_t>(s.wc), tr->d.seed, ctr, -bw, bw);
    if (rc != TMNN_OK) return rc;
    ctr += static_cast<uint32_t>((s.wc + 3) / 4);
    dst += s.wc;
    const float bb = 1.0f / std::sqrt(fin);
    rc = philox_fill(st, dst, static_cast<uint32_t>(s.bc), tr->d.seed, ctr, -bb, bb);
    if (rc != TMNN_OK) return rc;
    ctr += static_cast<uint32_t>((s.bc + 3) / 4);
    dst += s.bc;
  }
  ++tr->weights_version;
  return TMNN_OK;
}

void put_u32(uint8_t *p, uint32_t v) {
  p[0] = static_cast<uint8_t>(v & 0xFFu);
  p[1] = static_cast<uint8_t>((v >> 8) & 0xFFu);
  p[2] = static_cast<uint8_t>((v >> 16) & 0xFFu);
  p[3] = static_cast<uint8_t>((v >> 24) & 0xFFu);
}

uint32_t get_u32(const uint8_t *p) {
  return static_cast<uint32_t>(p[0]) | (static_cast<uint32_t>(p[1]) << 8) |
         (static_cast<uint32_t>(p[2]) << 16) | (static_cast<uint32_t>(p[3]) << 24);
}


// The synchronous step of the host-pointer entry points: the batch staged
// on the main stream, the fused device step, then the loss (and, on sampled
// steps or when the loss is not finite, the numerics rows) read back. The
// finish kernel computes the report on every such step, so a non-finite
// loss is reported in full as the reference's forced probe does
// (training_step_execution.cpp:1015-1043); only the read-back is sampled.
// dbg_out (host, nullable): the training kernel's outputs, caller row order.
int host_training_step(tmnn_trainer *tr, const float *input, const float *target, int32_t n,
                       tmnn_step_result *out, float *dbg_out) {
  if (!tr) return fail(TMNN_ERR_INVALID_ARGUMENT, "trainer is null");
  if (out && out->struct_size != sizeof(tmnn_step_result))
    return fail(TMNN_ERR_INVALID_ARGUMENT, "tmnn_step_result.struct_size mismatch");
  if (n <= 0) return fail(TMNN_ERR_INVALID_ARGUMENT, "training_step: N must be > 0");
  if (!input || !target) return fail(TMNN_ERR_INVALID_ARGUMENT, "input/target is null");
  TMNN_HIP_TRY(hipSetDevice(tr->ctx->device));
  const int bn = std::min(n, tr->d.batch_size);
  int rc = ensure_batch(tr, bn);
  if (rc != TMNN_OK) return rc;
  hipStream_t st = tr->ctx->stream;
  const size_t M = tr->d.num_outputs;
  if (dbg_out) TMNN_HIP_TRY(tr->out_buf.ensure(static_cast<size_t>(bn) * M * sizeof(float)));
  TMNN_HIP_TRY(hipMemcpyAsync(tr->in_pos.ptr, input,
                              static_cast<size_t>(bn) * tr->d.spatial_dims * sizeof(float),
                              hipMemcpyHostToDevice, st));
  TMNN_HIP_TRY(hipMemcpyAsync(tr->in_tgt.ptr, target, static_cast<size_t>(bn) * M * sizeof(float),
                              hipMemcpyHostToDevice, st));
  const uint32_t next = tr->step + 1;
  const bool sampled = numerics_should_sample(tr, next);
  tr->dbg_step_out = dbg_out ? tr->out_buf.as<float>() : nullptr;
  rc = train_step_device(tr, tr->in_pos.as<float>(), tr->in_tgt.as<float>(), bn,
                         tr->loss_out.as<float>(), 2, true);
  tr->dbg_step_out = nullptr;
  if (rc != TMNN_OK) return rc;
  float loss = 0.0f;
  TMNN_HIP_TRY(hipMemcpyAsync(&loss, tr->loss_out.ptr, sizeof(float), hipMemcpyDeviceToHost, st));
  std::vector<float4> rows;
  if (sampled && (rc = numerics_rows_download(tr, rows)) != TMNN_OK) return rc;
  if (dbg_out)
    TMNN_HIP_TRY(hipMemcpyAsync(dbg_out, tr->out_buf.ptr, static_cast<size_t>(bn) * M * sizeof(float),
                                hipMemcpyDeviceToHost, st));
  TMNN_HIP_TRY(hipStreamSynchronize(st));
  if (!sampled && !std::isfinite(loss)) {  // forced report of a non-finite loss
    if ((rc = numerics_rows_download(tr, rows)) != TMNN_OK) return rc;
    TMNN_HIP_TRY(hipStreamSynchronize(st));
  }
  tmnn_step_result r{};
  r.struct_size = sizeof r;
  r.loss = loss;
  r.step = tr->step;
  r.batch_n = static_cast<uint32_t>(bn);
  if (!rows.empty()) {
    numerics_from_rows(rows, tr->num_loss_row, &r);
    numerics_record(tr, r.step, r);
  }
  if (out) *out = r;
  return TMNN_OK;
}

}  // namespace

extern "C" {

const char *tmnn_last_error(void) { return g_last_error.c_str(); }

uint32_t tmnn_abi_version(void) { return kAbiVersion; }

int tmnn_context_create(int32_t device, tmnn_context **out) {
  if (!out) return fail(TMNN_ERR_INVALID_ARGUMENT, "out is null");
  *out = nullptr;
  int count = 0;
  TMNN_HIP_TRY(hipGetDeviceCount(&count));
  if (device < 0 || device >= count)
    return fail(TMNN_ERR_INVALID_ARGUMENT, "device ordinal out of range");
  TMNN_HIP_TRY(hipSetDevice(device));
  hipDeviceProp_t prop;
  TMNN_HIP_TRY(hipGetDeviceProperties(&prop, device));
  std::unique_ptr<tmnn_context> ctx(new (std::nothrow) tmnn_context());
  if (!ctx) return fail(TMNN_ERR_RUNTIME, "out of host memory");
  ctx->device = device;
  ctx->cu_count = prop.multiProcessorCount;
  ctx->mem_bytes = prop.totalGlobalMem;
  ctx->name = prop.gcnArchName;
  TMNN_HIP_TRY(hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking));
  {
    // This device's copy of the step scratch, with the device current, and
    // the event that orders its users. Only the allocation-free step needs
    // them: if either is unavailable the context is still created, and that
    // entry point reports the missing scratch.
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch.size() < static_cast<size_t>(count)) g_scratch.resize(count);
    ScratchDevice &sd = g_scratch[device];
    if (!sd.ptr) {
      void *p = nullptr;
      hipEvent_t ev = nullptr;
      if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) == hipSuccess && p &&
          hipEventCreateWithFlags(&ev, hipEventDisableTiming) == hipSuccess) {
        sd.ptr = static_cast<unsigned char *>(p);
        sd.done = ev;
      } else {
        (void)hipGetLastError();  // clear the sticky error of the failed lookup
      }
    }
    ctx->scratch = sd.ptr;
  }
  *out = ctx.release();
  return TMNN_OK;
}

int tmnn_context_destroy(tmnn_context *ctx) {
  if (!ctx) return TMNN_OK;
  (void)hipSetDevice(ctx->device);
  if (ctx->stream) {
    (void)hipStreamSynchronize(ctx->stream);
    (void)hipStreamDestroy(ctx->stream);
  }
  delete ctx;
  return TMNN_OK;
}

int tmnn_context_device_info(tmnn_context *ctx, int32_t *cu_count, uint64_t *global_mem_bytes,
                             char *name, size_t name_capacity) {
  if (!ctx) return fail(TMNN_ERR_INVALID_ARGUMENT, "context is null");
  if (cu_count) *cu_count = ctx->cu_count;
  if (global_mem_bytes) *global_mem_bytes = ctx->mem_bytes;
  if (name && name_capacity > 0) {
    std::strncpy(name, ctx->name.c_str(), name_capacity - 1);
    name[name_capacity - 1] = '\0';
  }
  return TMNN_OK;
}

// Reference defaults: factory_json_detail.h:159-290 (encoding/network),
// trainer.h:34-61 (optimizer), weight_init.h:113-141 (init).
void tmnn_model_desc_init(tmnn_model_desc *d) {
  if (!d) return;
  std::memset(d, 0, sizeof *d);
  d->struct_size = sizeof *d;
  d->spatial_dims = 3;
  d->num_levels = 16;
  d->features_per_level = 2;
  d->log2_hashmap_size = 19;
  d->base_resolution = 16.0f;
  d->per_level_scale = 1.447f;
  d->hidden_dim = 64;
  d->num_hidden_layers = 2;
  d->num_outputs = 1;
  d->loss_kind = TMNN_LOSS_L2;
  d->huber_delta = 1.0f;
  d->lr_encoding = 1e-2f;
  d->lr_network = 1e-3f;
  d->beta1 = 0.9f;
  d->beta2 = 0.99f;
  d->epsilon = 1e-15f;
  d->batch_size = 1024;
  d->precision = TMNN_PRECISION_FP32;
  d->hash_adam_mode = TMNN_HASH_ADAM_LAZY;
  d->morton_sort = 1;
  d->seed = 42u;
  d->hash_init_range = 1.0e-4f;
  d->forced_family = TMNN_FAMILY_AUTO;
}

void tmnn_device_caps_init(tmnn_device_caps *c) {
  if (!c) return;
  std::memset(c, 0, sizeof *c);
  c->struct_size = sizeof *c;
  c->gpu_available = 1;
  c->cu_count = 256;
  c->lds_bytes_per_cu = kMaxLdsBytes;
  c->wave_size = 64;
  c->has_mfma_f16 = 1;
  c->global_mem_bytes = 288ull << 30;
}

int tmnn_context_caps(tmnn_context *ctx, tmnn_device_caps *out) {
  if (!ctx || !out) return fail(TMNN_ERR_INVALID_ARGUMENT, "null argument");
  tmnn_device_caps_init(out);
  out->cu_count = ctx->cu_count;
  out->global_mem_bytes = ctx->mem_bytes;
  return TMNN_OK;
}

int tmnn_plan_network(const tmnn_device_caps *caps, const tmnn_model_desc *desc,
                      tmnn_network_plan *out) {
  if (!caps || !desc || !out) return fail(TMNN_ERR_INVALID_ARGUMENT, "null argument");
  if (caps->struct_size != sizeof(tmnn_device_caps))
    return fail(TMNN_ERR_INVALID_ARGUMENT, "tmnn_device_caps.struct_size mismatch");
  if (desc->struct_size != sizeof(tmnn_model_desc))
    return fail(TMNN_ERR_INVALID_ARGUMENT, "tmnn_model_desc.struct_size mismatch");
  std::string why;
  if (!desc_ok(desc, why)) return fail(TMNN_ERR_INVALID_ARGUMENT, "KernelSpec: " + why);
  plan_network_impl(*caps, *desc, *out);
  return TMNN_OK;
}

int tmnn_trainer_get_plan(tmnn_trainer *tr, tmnn_network_plan *out) {
  if (!tr || !out) return fail(TMNN_ERR_INVALID_ARGUMENT, "null argument");
  *out = tr->plan;
  return TMNN_OK;
}

int tmnn_trainer_create(tmnn_context *ctx, const tmnn_model_desc *desc, tmnn_trainer **out) {
  if (!ctx || !desc || !out) return fail(TMNN_ERR_INVALID_ARGUMENT, "null argument");
  *out = nullptr;
  if (desc->struct_size != sizeof(tmnn_model_desc))
    return fail(TMNN_ERR_INVALID_ARGUMENT, "tmnn_model_desc.struct_size mismatch");
  std::string why;
  if (!desc_ok(desc, why)) return fail(TMNN_ERR_INVALID_ARGUMENT, "KernelSpec: " + why);
  const int IN = desc->num_levels * desc->features_per_level;
  TMNN_HIP_TRY(hipSetDevice(ctx->device));

  // the planner decides the family the kernels come from
  tmnn_device_caps caps;
  int rc = tmnn_context_caps(ctx, &caps);
  if (rc != TMNN_OK) return rc;
  tmnn_network_plan plan;
  plan_network_impl(caps, *desc, plan);
  if (plan.selected_family < 0)
    return fail(TMNN_ERR_UNSUPPORTED, "planner: no network family can run this model (reasons mask " +
                                          std::to_string(plan.reasons) + ")");

  std::unique_ptr<tmnn_trainer> tr(new (std::nothrow) tmnn_trainer());
  if (!tr) return fail(TMNN_ERR_RUNTIME, "out of host memory");
  tr->ctx = ctx;
  tr->d = *desc;
  tr->plan = plan;
  tr->family = plan.selected_family;
  if (tr->family == TMNN_FAMILY_SAFE_DEBUG) {  // fp32 generic kernels, batches in input order
    tr->d.precision = TMNN_PRECISION_FP32;
    tr->d.morton_sort = 0;
  }
  tr->IN = IN;
  {
    const ModelShape ms = shape_of(*desc);
    tr->INP = ms.INP;
    tr->HP = ms.HP;
  }
  tr->lr_enc = desc->lr_encoding;
  tr->lr_net = desc->lr_network;
  tr->hash_count = static_cast<uint32_t>(desc->num_levels) *
                   (1u << desc->log2_hashmap_size) *
                   static_cast<uint32_t>(desc->features_per_level);
  const FieldLayout lay = make_layout(tr->INP, tr->HP, IN, desc->hidden_dim,
                                      desc->num_hidden_layers, desc->num_outputs, 0, false,
                                      false, 1);
  tr->mlp_count = static_cast<uint32_t>(lay.mlp_count());
  tr->hash_entries = tr->hash_count / static_cast<uint32_t>(desc->features_per_level);
  // Reference bit-mask layout: a bit per entry when F == 2, else per float.
  const uint32_t width = desc->features_per_level == 2 ? 2u : 1u;
  tr->mask_words = (tr->hash_count / width + 31u) / 32u;
  // One fp32 resolution table for every kernel: r_0 = b, r_l = r_{l-1} * s
  // (iterated product of the eval path, mlp_kernel_emitter.cpp:224,298).
  {
    float r = baked6(desc->base_resolution);
    const float s = baked6(desc->per_level_scale);
    for (int l = 0; l < desc->num_levels; ++l) {
      tr->res[l] = r;
      r = r * s;
    }
  }

  if ((rc = plan_kernel(tr.get(), tr->d.precision == TMNN_PRECISION_FP16, true,
                        tr->train_plan)) != TMNN_OK)
    return rc;
  if ((rc = plan_kernel(tr.get(), tr->d.precision == TMNN_PRECISION_FP16, false,
                        tr->fwd_plan)) != TMNN_OK)
    return rc;
  if ((rc = plan_kernel(tr.get(), false, false, tr->infer_plan)) != TMNN_OK) return rc;

  const size_t total = static_cast<size_t>(tr->hash_count) + tr->mlp_count;
  TMNN_HIP_TRY(tr->params.ensure(total * sizeof(float)));
  TMNN_HIP_TRY(tr->m.ensure(total * sizeof(float)));
  TMNN_HIP_TRY(tr->v.ensure(total * sizeof(float)));
  TMNN_HIP_TRY(tr->grad_hash.ensure(tr->hash_count * sizeof(int32_t)));
  TMNN_HIP_TRY(tr->grad_mlp.ensure(tr->mlp_count * sizeof(float)));
  TMNN_HIP_TRY(tr->mask[0].ensure(tr->hash_entries));
  TMNN_HIP_TRY(tr->mask[1].ensure(tr->hash_entries));
  TMNN_HIP_TRY(tr->partials.ensure(static_cast<size_t>(tr->train_plan.max_blocks) *
                                   tr->mlp_count * sizeof(float)));
  TMNN_HIP_TRY(tr->loss_partials.ensure(static_cast<size_t>(tr->train_plan.max_blocks) *
                                        sizeof(float)));
  TMNN_HIP_TRY(tr->loss_out.ensure(sizeof(float)));
  // numerics: one largest-|output| per training block, one row per finish
  // block (MLP column blocks, the loss block, at most four hash blocks per CU)
  TMNN_HIP_TRY(tr->amax_partials.ensure(static_cast<size_t>(tr->train_plan.max_blocks) *
                                        sizeof(float)));
  TMNN_HIP_TRY(tr->num_rows.ensure(
      ((tr->mlp_count + kReduceCols - 1) / kReduceCols + 1 + static_cast<size_t>(ctx->cu_count) * 4) *
      sizeof(float4)));
  if ((rc = init_weights(tr.get())) != TMNN_OK) return rc;
  if ((rc = reset_moments(tr.get())) != TMNN_OK) return rc;
  if ((rc = zero_training_state(tr.get())) != TMNN_OK) return rc;
  TMNN_HIP_TRY(hipStreamSynchronize(ctx->stream));
  *out = tr.release();
  return TMNN_OK;
}

int tmnn_trainer_destroy(tmnn_trainer *tr) {
  if (!tr) return TMNN_OK;
  (void)hipSetDevice(tr->ctx->device);
  (void)hipStreamSynchronize(tr->ctx->stream);
  delete tr;
  return TMNN_OK;
}

int tmnn_trainer_param_counts(tmnn_trainer *tr, uint32_t *hash_count, uint32_t *mlp_count) {
  if (!tr) return fail(TMNN_ERR_INVALID_ARGUMENT, "trainer is null");
  if (hash_count) *hash_count = tr->hash_count;
  if (mlp_count) *mlp_count = tr->mlp_count;
  return TMNN_OK;
}

int tmnn_trainer_inspect(tmnn_trainer *tr, tmnn_inspection *o) {
  if (!tr || !o) return fail(TMNN_ERR_INVALID_ARGUMENT, "null argument");
  std::memset(o, 0, sizeof *o);
  o->family = tr->family;
  o->precision = tr->d.precision;
  o->hidden_padded = tr->HP;
  o->input_padded = tr->INP;
  o->points_per_wave_tile = kTilePts;
  o->waves_per_block_train = tr->train_plan.wpb;
  o->blocks_train = tr->train_plan.max_blocks;
  o->lds_bytes_train = tr->train_plan.lds;
  o->lds_bytes_infer = tr->infer_plan.lds;
  o->cu_count = tr->ctx->cu_count;
  o->hash_param_count = tr->hash_count;
  o->mlp_param_count = tr->mlp_count;
  o->batch_size = static_cast<uint32_t>(tr->d.batch_size);
  o->train_fused_scatter = tr->train_plan.tile_scatter ? 1 : 0;
  return TMNN_OK;
}

int tmnn_training_step(tmnn_trainer *tr, const float *input, const float *target, int32_t n,
                       tmnn_step_result *out) {
  return host_training_step(tr, input, target, n, out, nullptr);
}

int tmnn_training_step_device(tmnn_trainer *tr, const float *d_input, const float *d_target,
                              int32_t n, float *d_loss_out) {
  return tmnn_training_step_device_after(tr, d_input, d_target, n, d_loss_out, nullptr);
}

int tmnn_training_step_device_after(tmnn_trainer *tr, const float *d_input,
                                    const float *d_target, int32_t n, float *d_loss_out,
                                    void *wait_event) {
  if (!tr) return fail(TMNN_ERR_INVALID_ARGUMENT, "trainer is null");
  if (n <= 0) return fail(TMNN_ERR_INVALID_ARGUMENT, "training_step: N must be > 0");
  if (!d_input || !d_target) return fail(TMNN_ERR_INVALID_ARGUMENT, "input/target is null");
  TMNN_HIP_TRY(hipSetDevice(tr->ctx->device));
  const int bn = std::min(n, tr->d.batch_size);
  const int rc = ensure_batch(tr, bn);
  if (rc != TMNN_OK) return rc;
  // device steps are sampled by step only: their losses are not read back
  return train_step_device(tr, d_input, d_target, bn, d_loss_out, 1,
                           numerics_should_sample(tr, tr->step + 1),
                           static_cast<hipEvent_t>(wait_event));
}

int tmnn_record_event(tmnn_trainer *tr, void *event) {
  if (!tr || !event) return fail(TMNN_ERR_INVALID_ARGUMENT, "null argument");
  TMNN_HIP_TRY(hipSetDevice(tr->ctx->device));
  TMNN_HIP_TRY(hipEventRecord(static_cast<hipEvent_t>(event), tr->ctx->stream));
  return TMNN_OK;
}

int tmnn_set_numerics_sampling(tmnn_trainer *tr, int32_t mode, uint32_t interval) {
  if (!tr) return fail(TMNN_ERR_INVALID_ARGUMENT, "trainer is null");
  if (mode < TMNN_NUMERICS_SAMPLED || mode > TMNN_NUMERICS_DISABLED)
    return fail(TMNN_ERR_INVALID_ARGUMENT, "unknown numerics sampling mode");
  tr->num_mode = mode;
  tr->num_interval = interval > 0 ? interval : 1u;  // NumericsGuard::set_sample_interval
  tr->num_anomalies = 0;
  tr->num_last_anomaly = 0;
  return TMNN_OK;
}

int tmnn_get_last_numerics(tmnn_trainer *tr, tmnn_step_result *out) {
  if (!tr || !out) return fail(TMNN_ERR_INVALID_ARGUMENT, "null argument");
  if (out->struct_size != sizeof(tmnn_step_result))
    return fail(TMNN_ERR_INVALID_ARGUMENT, "tmnn_step_result.struct_size mismatch");
  TMNN_HIP_TRY(hipSetDevice(tr->ctx->device));
  tmnn_step_result r{};
  r.struct_size = sizeof r;
  if (tr->num_step > 0) {
    std::vector<float4> rows;
    const int rc = numerics_rows_download(tr, rows);
    if (rc != TMNN_OK) return rc;
    TMNN_HIP_TRY(hipStreamSynchronize(tr->ctx->stream));
    r.loss = rows[tr->num_loss_row].y;
    r.step = tr->num_step;
    r.batch_n = tr->num_batch;
    numerics_from_rows(rows, tr->num_loss_row, &r);
  } else {
    TMNN_HIP_TRY(hipStreamSynchronize(tr->ctx->stream));
  }
  *out = r;
  return TMNN_OK;
}

int tmnn_debug_step_outputs(tmnn_trainer *tr, const float *input, const float *target,
                            int32_t n, float *outputs, tmnn_step_result *result) {
  if (!outputs) return fail(TMNN_ERR_INVALID_ARGUMENT, "outputs is null");
  return host_training_step(tr, input, target, n, result, outputs);
}

int tmnn_training_step_device_noalloc(tmnn_trainer *tr, const float *d_input,
                                      const float *d_target, int32_t n, float *d_loss_out) {
  if (!tr) return fail(TMNN_ERR_INVALID_ARGUMENT, "trainer is null");
  if (n <= 0) return fail(TMNN_ERR_INVALID_ARGUMENT, "training_step: N must be > 0");
  if (!d_input || !d_target) return fail(TMNN_ERR_INVALID_ARGUMENT, "input/target is null");
  if (!tr->ctx->scratch) return fail(TMNN_ERR_RUNTIME, "device scratch address unknown");
  if (tr->train_plan.wide || tr->train_plan.layerwise)
    return fail(TMNN_ERR_UNSUPPORTED,
                "the allocation-free step runs neither hidden width 128 nor the layer-wise "
                "path (their activation buffers exceed the scratch): use "
                "tmnn_training_step_device");
  TMNN_HIP_TRY(hipSetDevice(tr->ctx->device));
  const int bn = std::min(n, tr->d.batch_size);
  // carve the scratch: [keys0 | keys1 | vals0 | vals1 | sort tmp | s_pos | s_tgt | xfeat | dx]
  const size_t D = tr->d.spatial_dims, M = tr->d.num_outputs;
  const size_t n_pad = static_cast<size_t>((bn + kTilePts - 1) / kTilePts) * kTilePts;
  size_t sort_bytes = 0;
  TMNN_HIP_TRY(morton_sort_temp_bytes(bn, &sort_bytes));
  DevBuf *bufs[] = {&tr->keys0, &tr->keys1, &tr->vals0, &tr->vals1, &tr->sort_tmp,
                    &tr->s_pos, &tr->s_tgt, &tr->xfeat, &tr->dx};
  const size_t want[] = {bn * sizeof(uint32_t), bn * sizeof(uint32_t), bn * sizeof(uint32_t),
                         bn * sizeof(uint32_t), std::max<size_t>(sort_bytes, 256),
                         bn * D * sizeof(float), bn * M * sizeof(float),
                         n_pad * tr->INP * sizeof(float), n_pad * tr->IN * sizeof(float)};
  constexpr int kRegions = sizeof(want) / sizeof(want[0]);
  size_t off[kRegions], total = 0;
  for (int r = 0; r < kRegions; ++r) {
    off[r] = total;
    total += (want[r] + 255) / 256 * 256;
  }
  if (total > TMNN_NOALLOC_SCRATCH_BYTES)
    return fail(TMNN_ERR_INVALID_ARGUMENT,
                "training_step_device_noalloc: a batch of " + std::to_string(bn) +
                    " points needs " + std::to_string(total) + " bytes of scratch, above the " +
                    std::to_string(static_cast<size_t>(TMNN_NOALLOC_SCRATCH_BYTES)) +
                    "-byte maximum");
  // lend the regions to the step's buffers for this call, then give them back
  struct Saved {
    void *ptr;
    size_t bytes;
    bool borrowed;
  } saved[kRegions];
  for (int r = 0; r < kRegions; ++r) {
    saved[r] = {bufs[r]->ptr, bufs[r]->bytes, bufs[r]->borrowed};
    bufs[r]->ptr = tr->ctx->scratch + off[r];
    bufs[r]->bytes = want[r];
    bufs[r]->borrowed = true;
  }
  // steps of other contexts on this device may hold the scratch: this step's
  // kernels start after the last one's (the event is re-recorded under the
  // same lock, after this step's kernels)
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  ScratchDevice &sd = g_scratch[tr->ctx->device];
  if (!sd.done) return fail(TMNN_ERR_RUNTIME, "device scratch event unavailable");
  if (sd.recorded) TMNN_HIP_TRY(hipStreamWaitEvent(tr->ctx->stream, sd.done, 0));
  tr->prof_suspended = true;
  int rc = train_step_device(tr, d_input, d_target, bn, d_loss_out, 0,
                             numerics_should_sample(tr, tr->step + 1));
  tr->prof_suspended = false;
  for (int r = 0; r < kRegions; ++r) {
    bufs[r]->ptr = saved[r].ptr;
    bufs[r]->bytes = saved[r].bytes;
    bufs[r]->borrowed = saved[r].borrowed;
  }
  // recorded even after a failed enqueue: whatever was enqueued is ordered
  const hipError_t e = hipEventRecord(sd.done, tr->ctx->stream);
  if (e == hipSuccess)
    sd.recorded = true;
  else if (rc == TMNN_OK)
    rc = fail(TMNN_ERR_GPU, std::string("hipEventRecord: ") + hipGetErrorString(e));
  return rc;
}

int tmnn_inference_device(tmnn_trainer *tr, const float *d_positions, float *d_output,
                          int32_t n) {
  return tmnn_inference_device_after(tr, d_positions, d_output, n, nullptr);
}

int tmnn_inference_device_after(tmnn_trainer *tr, const float *d_positions, float *d_output,
                                int32_t n, void *wait_event) {
  if (!tr) return fail(TMNN_ERR_INVALID_ARGUMENT, "trainer is null");
  if (n < 0) return fail(TMNN_ERR_INVALID_ARGUMENT, "FieldEvaluator::evaluate: N must be non-negative");
  if (n == 0) return TMNN_OK;
  if (!d_positions || !d_output)
    return fail(TMNN_ERR_INVALID_ARGUMENT, "positions and output must be non-null when N > 0");
  TMNN_HIP_TRY(hipSetDevice(tr->ctx->device));
  if (wait_event)
    TMNN_HIP_TRY(hipStreamWaitEvent(tr->ctx->stream, static_cast<hipEvent_t>(wait_event), 0));
  FieldArgs a = base_args(tr);
  a.mode = kModeForward;
  a.pos = d_positions;
  a.out = d_output;
  std::array<hipEvent_t, 2> *ev = nullptr;
  int rc = prof_infer_begin(tr, &ev);
  if (rc != TMNN_OK) return rc;
  // the image repack (after weight changes) stays outside the timed pair
  if ((rc = ensure_image(tr, tr->infer_plan)) != TMNN_OK) return rc;
  if (ev) TMNN_HIP_TRY(hipEventRecord((*ev)[0], tr->ctx->stream));
  const int blocks = launch_field(tr, tr->infer_plan, a, n);
  if (blocks < 0) return blocks;
  if (ev) {
    TMNN_HIP_TRY(hipEventRecord((*ev)[1], tr->ctx->stream));
    ++tr->infer_used;
  }
  return TMNN_OK;
}

int tmnn_inference(tmnn_trainer *tr, const float *positions, float *output, int32_t n) {
  if (!tr) return fail(TMNN_ERR_INVALID_ARGUMENT, "trainer is null");
  if (n < 0) return fail(TMNN_ERR_INVALID_ARGUMENT, "FieldEvaluator::evaluate: N must be non-negative");
  if (n == 0) return TMNN_OK;
  if (!positions || !output)
    return fail(TMNN_ERR_INVALID_ARGUMENT, "positions and output must be non-null when N > 0");
  TMNN_HIP_TRY(hipSetDevice(tr->ctx->device));
  hipStream_t st = tr->ctx->stream;
  const size_t D = tr->d.spatial_dims, M = tr->d.num_outputs;
  TMNN_HIP_TRY(tr->in_pos.ensure(n * D * sizeof(float)));
  TMNN_HIP_TRY(tr->out_buf.ensure(n * M * sizeof(float)));
  TMNN_HIP_TRY(hipMemcpyAsync(tr->in_pos.ptr, positions, n * D * sizeof(float),
                              hipMemcpyHostToDevice, st));
  const int rc = tmnn_inference_device(tr, tr->in_pos.as<float>(), tr->out_buf.as<float>(), n);
  if (rc != TMNN_OK) return rc;
  TMNN_HIP_TRY(hipMemcpyAsync(output, tr->out_buf.ptr, n * M * sizeof(float),
                              hipMemcpyDeviceToHost, st));
  TMNN_HIP_TRY(hipStreamSynchronize(st));
  return TMNN_OK;
}

int tmnn_evaluate_with_gradient(tmnn_trainer *tr, const float *positions, float *output,
                                float *gradients, int32_t n) {
  if (!tr) return fail(TMNN_ERR_INVALID_ARGUMENT, "trainer is null");
  if (n < 0)
    return fail(TMNN_ERR_INVALID_ARGUMENT,
                "FieldEvaluator::evaluate_with_gradient: N must be non-negative");
  if (n == 0) return TMNN_OK;
  if (!positions || !output || !gradients)
    return fail(TMNN_ERR_INVALID_ARGUMENT,
                "positions, output, and gradients must be non-null when N > 0");
  TMNN_HIP_TRY(hipSetDevice(tr->ctx->device));
  int rc;
  if (!tr->grad_planned) {  // the evaluator's gradient kernel is fp32 (default_trainer.cpp:497-507)
    if ((rc = plan_kernel(tr, false, true, tr->grad_plan)) != TMNN_OK) return rc;
    TMNN_HIP_TRY(tr->partials.ensure(static_cast<size_t>(tr->grad_plan.max_blocks) *
                                     tr->mlp_count * sizeof(float)));
    TMNN_HIP_TRY(tr->loss_partials.ensure(static_cast<size_t>(tr->grad_plan.max_blocks) *
                                          sizeof(float)));
    tr->grad_planned = true;
  }
  hipStream_t st = tr->ctx->stream;
  const size_t D = tr->d.spatial_dims, M = tr->d.num_outputs;
  if ((rc = ensure_batch(tr, n)) != TMNN_OK) return rc;
  TMNN_HIP_TRY(tr->out_buf.ensure(n * M * sizeof(float)));
  TMNN_HIP_TRY(tr->grad_out.ensure(n * M * D * sizeof(float)));
  TMNN_HIP_TRY(hipMemcpyAsync(tr->in_pos.ptr, positions, n * D * sizeof(float),
                              hipMemcpyHostToDevice, st));
  PosGradArgs g{};
  g.n = n;
  g.L = tr->d.num_levels;
  g.F = tr->d.features_per_level;
  g.M = static_cast<int32_t>(M);
  g.log2T = static_cast<uint32_t>(tr->d.log2_hashmap_size);
  for (int l = 0; l < kMaxLevels; ++l) g.res[l] = tr->res[l];
  g.pos = tr->in_pos.as<float>();
  g.table = tr->params.as<float>();
  g.dx = tr->dx.as<float>();
  g.grads = tr->grad_out.as<float>();
  for (int m = 0; m < static_cast<int>(M); ++m) {
    // d out_m / d features for every point, then the position gradient
    FieldArgs a = base_args(tr);
    a.mode = kModeInputGrad;
    a.grad_output = m;
    a.pos = tr->in_pos.as<float>();
    a.out = m == 0 ? tr->out_buf.as<float>() : nullptr;
    a.dx_out = tr->dx.as<float>();
    a.grad_partials = tr->partials.as<float>();
    a.loss_partials = tr->loss_partials.as<float>();
    // the features of these points are the same for every output
    const int blocks = launch_field(tr, tr->grad_plan, a, n, -1, m > 0);
    if (blocks < 0) return blocks;
    g.m = m;
    const dim3 grid((n + 255) / 256);
    switch (tr->d.spatial_dims) {
      case 2: hipLaunchKernelGGL(pos_grad_kernel<2>, grid, dim3(256), 0, st, g); break;
      case 3: hipLaunchKernelGGL(pos_grad_kernel<3>, grid, dim3(256), 0, st, g); break;
      default: hipLaunchKernelGGL(pos_grad_kernel<4>, grid, dim3(256), 0, st, g); break;
    }
    TMNN_HIP_TRY(hipGetLastError());
  }
  TMNN_HIP_TRY(hipMemcpyAsync(output, tr->out_buf.ptr, n * M * sizeof(float),
                              hipMemcpyDeviceToHost, st));
  TMNN_HIP_TRY(hipMemcpyAsync(gradients, tr->grad_out.ptr, n * M * D * sizeof(float),
                              hipMemcpyDeviceToHost, st));
  TMNN_HIP_TRY(hipStreamSynchronize(st));
  return TMNN_OK;
}

int tmnn_forward_for_training(tmnn_trainer *tr, const float *input, float *output, int32_t n,
                              uint32_t *written) {
  if (!tr) return fail(TMNN_ERR_INVALID_ARGUMENT, "trainer is null");
  if (written) *written = 0;
  if (n <= 0)
    return fail(TMNN_ERR_INVALID_ARGUMENT, "Trainer::forward_for_training: N must be greater than zero");
  if (!input || !output) return fail(TMNN_ERR_INVALID_ARGUMENT, "input/output is null");
  TMNN_HIP_TRY(hipSetDevice(tr->ctx->device));
  const int bn = std::min(n, tr->d.batch_size);
  int rc = ensure_batch(tr, bn);
  if (rc != TMNN_OK) return rc;
  hipStream_t st = tr->ctx->stream;
  const size_t D = tr->d.spatial_dims, M = tr->d.num_outputs;
  TMNN_HIP_TRY(tr->out_buf.ensure(bn * M * sizeof(float)));
  TMNN_HIP_TRY(hipMemcpyAsync(tr->in_pos.ptr, input, bn * D * sizeof(float),
                              hipMemcpyHostToDevice, st));
  const float *pos = nullptr, *unused = nullptr;
  const uint32_t *perm = nullptr;
  rc = sort_batch(tr, tr->in_pos.as<float>(), nullptr, 0, bn, &pos, &unused, &perm);
  if (rc != TMNN_OK) return rc;
  FieldArgs a = base_args(tr);
  a.mode = kModeForward;
  a.pos = pos;
  a.out = tr->out_buf.as<float>();
  a.out_index = perm;  // write each sorted point back to its caller row
  const int blocks = launch_field(tr, tr->fwd_plan, a, bn);
  if (blocks < 0) return blocks;
  TMNN_HIP_TRY(hipMemcpyAsync(output, tr->out_buf.ptr, bn * M * sizeof(float),
                              hipMemcpyDeviceToHost, st));
  TMNN_HIP_TRY(hipStreamSynchronize(st));
  if (written) *written = static_cast<uint32_t>(bn * M);
  return TMNN_OK;
}

int tmnn_zero_gradients(tmnn_trainer *tr) {
  if (!tr) return fail(TMNN_ERR_INVALID_ARGUMENT, "trainer is null");
  TMNN_HIP_TRY(hipSetDevice(tr->ctx->device));
  const int rc = zero_training_state(tr);
  if (rc != TMNN_OK) return rc;
  TMNN_HIP_TRY(hipStreamSynchronize(tr->ctx->stream));
  return TMNN_OK;
}

int tmnn_backward_accumulate(tmnn_trainer *tr, const float *input, const float *d_output,
                             int32_t n) {
  if (!tr) return fail(TMNN_ERR_INVALID_ARGUMENT, "trainer is null");
  if (n <= 0) return fail(TMNN_ERR_INVALID_ARGUMENT, "backward_accumulate: N must be > 0");
  if (!input || !d_output) return fail(TMNN_ERR_INVALID_ARGUMENT, "input/d_output is null");
  TMNN_HIP_TRY(hipSetDevice(tr->ctx->device));
  const int bn = std::min(n, tr->d.batch_size);
  int rc = ensure_batch(tr, bn);
  if (rc != TMNN_OK) return rc;
  hipStream_t st = tr->ctx->stream;
  TMNN_HIP_TRY(hipMemcpyAsync(tr->in_pos.ptr, input,
                              static_cast<size_t>(bn) * tr->d.spatial_dims * sizeof(float),
                              hipMemcpyHostToDevice, st));
  TMNN_HIP_TRY(hipMemcpyAsync(tr->in_tgt.ptr, d_output,
                              static_cast<size_t>(bn) * tr->d.num_outputs * sizeof(float),
                              hipMemcpyHostToDevice, st));
  tr->prof_cur = -1;  // only fused steps are profiled
  const int blocks = run_forward_backward(tr, tr->in_pos.as<float>(), tr->in_tgt.as<float>(), bn,
                                          true);
  if (blocks < 0) return blocks;
  TMNN_HIP_TRY(hipStreamSynchronize(st));
  return TMNN_OK;
}

int tmnn_adam_step(tmnn_trainer *tr) {
  if (!tr) return fail(TMNN_ERR_INVALID_ARGUMENT, "trainer is null");
  TMNN_HIP_TRY(hipSetDevice(tr->ctx->device));
  // Split-path Adam keeps the accumulated gradients (they persist until the
  // next zero_gradients) and consumes the mask (default_trainer.cpp:1396-1443).
  const int rc = run_adam(tr, false, true);
  if (rc != TMNN_OK) return rc;
  TMNN_HIP_TRY(hipStreamSynchronize(tr->ctx->stream));
  ++tr->step;
  return TMNN_OK;
}

int tmnn_synchronize(tmnn_trainer *tr) {
  if (!tr) return fail(TMNN_ERR_INVALID_ARGUMENT, "trainer is null");
  TMNN_HIP_TRY(hipSetDevice(tr->ctx->device));
  TMNN_HIP_TRY(hipStreamSynchronize(tr->ctx->stream));
  return TMNN_OK;
}

int tmnn_get_step(tmnn_trainer *tr, uint32_t *step) {
  if (!tr || !step) return fail(TMNN_ERR_INVALID_ARGUMENT, "null argument");
  *step = tr->step;
  return TMNN_OK;
}

int tmnn_get_weights(tmnn_trainer *tr, float *hash, size_t hash_count, float *mlp,
                     size_t mlp_count) {
  if (!tr) return fail(TMNN_ERR_INVALID_ARGUMENT, "trainer is null");
  if (hash && hash_count != tr->hash_count)
    return fail(TMNN_ERR_INVALID_ARGUMENT, "hash_weights count mismatch");
  if (mlp && mlp_count != tr->mlp_count)
    return fail(TMNN_ERR_INVALID_ARGUMENT, "mlp_weights count mismatch");
  TMNN_HIP_TRY(hipSetDevice(tr->ctx->device));
  hipStream_t st = tr->ctx->stream;
  if (hash)
    TMNN_HIP_TRY(hipMemcpyAsync(hash, tr->params.ptr, hash_count * sizeof(float),
                                hipMemcpyDeviceToHost, st));
  if (mlp)
    TMNN_HIP_TRY(hipMemcpyAsync(mlp, tr->params.as<float>() + tr->hash_count,
                                mlp_count * sizeof(float), hipMemcpyDeviceToHost, st));
  TMNN_HIP_TRY(hipStreamSynchronize(st));
  return TMNN_OK;
}

int tmnn_set_initial_weights(tmnn_trainer *tr, const float *hash, size_t hash_count,
                             const float *mlp, size_t mlp_count) {
  if (!tr) return fail(TMNN_ERR_INVALID_ARGUMENT, "trainer is null");
  if (hash && hash_count != tr->hash_count)
    return fail(TMNN_ERR_RUNTIME, "set_initial_weights: hash_weights count mismatch: got " +
                                      std::to_string(hash_count) + " expected " +
                                      std::to_string(tr->hash_count));
  if (mlp && mlp_count != tr->mlp_count)
    return fail(TMNN_ERR_RUNTIME, "set_initial_weights: mlp_weights count mismatch: got " +
                                      std::to_string(mlp_count) + " expected " +
                                      std::to_string(tr->mlp_count));
  TMNN_HIP_TRY(hipSetDevice(tr->ctx->device));
  hipStream_t st = tr->ctx->stream;
  if (hash && hash_count)
    TMNN_HIP_TRY(hipMemcpyAsync(tr->params.ptr, hash, hash_count * sizeof(float),
                                hipMemcpyHostToDevice, st));
  if (mlp && mlp_count)
    TMNN_HIP_TRY(hipMemcpyAsync(tr->params.as<float>() + tr->hash_count, mlp,
                                mlp_count * sizeof(float), hipMemcpyHostToDevice, st));
  ++tr->weights_version;
  int rc = reset_moments(tr);
  if (rc != TMNN_OK) return rc;
  rc = zero_training_state(tr);
  if (rc != TMNN_OK) return rc;
  TMNN_HIP_TRY(hipStreamSynchronize(st));
  tr->step = 0;
  return TMNN_OK;
}

int tmnn_export_optimizer_state(tmnn_trainer *tr, uint32_t *version, uint32_t *step,
                                uint8_t *payload, size_t capacity, size_t *payload_len) {
  if (!tr || !payload_len) return fail(TMNN_ERR_INVALID_ARGUMENT, "null argument");
  const size_t hb = static_cast<size_t>(tr->hash_count) * sizeof(float);
  const size_t mb = static_cast<size_t>(tr->mlp_count) * sizeof(float);
  const size_t need = 4 * 4 + 2 * hb + 2 * mb;
  *payload_len = need;
  if (version) *version = kOptimizerBlobVersion;
  if (step) *step = tr->step;
  if (!payload) return TMNN_OK;
  if (capacity < need) return fail(TMNN_ERR_INVALID_ARGUMENT, "payload capacity too small");
  TMNN_HIP_TRY(hipSetDevice(tr->ctx->device));
  hipStream_t st = tr->ctx->stream;
  // sections: m_hash, v_hash, m_mlp, v_mlp (default_trainer.cpp:1656-1661)
  const struct { const DevBuf *buf; size_t off, bytes; } sec[4] = {
      {&tr->m, 0, hb}, {&tr->v, 0, hb}, {&tr->m, hb, mb}, {&tr->v, hb, mb}};
  uint8_t *cur = payload;
  for (const auto &s : sec) {
    put_u32(cur, static_cast<uint32_t>(s.bytes));
    cur += 4;
    if (s.bytes)
      TMNN_HIP_TRY(hipMemcpyAsync(cur, static_cast<const uint8_t *>(s.buf->ptr) + s.off, s.bytes,
                                  hipMemcpyDeviceToHost, st));
    cur += s.bytes;
  }
  TMNN_HIP_TRY(hipStreamSynchronize(st));
  return TMNN_OK;
}

int tmnn_import_optimizer_state(tmnn_trainer *tr, uint32_t version, uint32_t step,
                                const uint8_t *payload, size_t payload_len) {
  if (!tr) return fail(TMNN_ERR_INVALID_ARGUMENT, "trainer is null");
  if (version != kOptimizerBlobVersion)
    return fail(TMNN_ERR_RUNTIME, "DefaultRuntime: unsupported optimizer blob version");
  if (!payload && payload_len) return fail(TMNN_ERR_INVALID_ARGUMENT, "payload is null");
  const size_t hb = static_cast<size_t>(tr->hash_count) * sizeof(float);
  const size_t mb = static_cast<size_t>(tr->mlp_count) * sizeof(float);
  const size_t expect[4] = {hb, hb, mb, mb};
  const char *names[4] = {"adam_m_hash", "adam_v_hash", "adam_m_mlp", "adam_v_mlp"};
  const uint8_t *cur = payload;
  size_t remaining = payload_len;
  const uint8_t *data[4];
  for (int i = 0; i < 4; ++i) {
    if (remaining < 4) return fail(TMNN_ERR_RUNTIME, "DefaultRuntime: optimizer blob truncated");
    const uint32_t sz = get_u32(cur);
    cur += 4;
    remaining -= 4;
    if (remaining < sz)
      return fail(TMNN_ERR_RUNTIME, "DefaultRuntime: optimizer blob section truncated");
    if (sz != expect[i])
      return fail(TMNN_ERR_RUNTIME, std::string("DefaultRuntime: ") + names[i] + " size mismatch");
    data[i] = cur;
    cur += sz;
    remaining -= sz;
  }
  if (remaining != 0)
    return fail(TMNN_ERR_RUNTIME, "DefaultRuntime: optimizer blob has trailing bytes");
  TMNN_HIP_TRY(hipSetDevice(tr->ctx->device));
  hipStream_t st = tr->ctx->stream;
  uint8_t *mp = static_cast<uint8_t *>(tr->m.ptr);
  uint8_t *vp = static_cast<uint8_t *>(tr->v.ptr);
  if (hb) {
    TMNN_HIP_TRY(hipMemcpyAsync(mp, data[0], hb, hipMemcpyHostToDevice, st));
    TMNN_HIP_TRY(hipMemcpyAsync(vp, data[1], hb, hipMemcpyHostToDevice, st));
  }
  if (mb) {
    TMNN_HIP_TRY(hipMemcpyAsync(mp + hb, data[2], mb, hipMemcpyHostToDevice, st));
    TMNN_HIP_TRY(hipMemcpyAsync(vp + hb, data[3], mb, hipMemcpyHostToDevice, st));
  }
  const int rc = zero_training_state(tr);
  if (rc != TMNN_OK) return rc;
  TMNN_HIP_TRY(hipStreamSynchronize(st));
  tr->step = step;
  return TMNN_OK;
}

int tmnn_reset_optimizer(tmnn_trainer *tr) {
  if (!tr) return fail(TMNN_ERR_INVALID_ARGUMENT, "trainer is null");
  TMNN_HIP_TRY(hipSetDevice(tr->ctx->device));
  int rc = reset_moments(tr);
  if (rc != TMNN_OK) return rc;
  rc = zero_training_state(tr);
  if (rc != TMNN_OK) return rc;
  TMNN_HIP_TRY(hipStreamSynchronize(tr->ctx->stream));
  tr->step = 0;
  return TMNN_OK;
}

int tmnn_set_learning_rate(tmnn_trainer *tr, float lr_encoding, float lr_network) {
  if (!tr) return fail(TMNN_ERR_INVALID_ARGUMENT, "trainer is null");
  tr->lr_enc = lr_encoding;
  tr->lr_net = lr_network;
  return TMNN_OK;
}

int tmnn_set_step_profiling(tmnn_trainer *tr, int32_t enabled) {
  if (!tr) return fail(TMNN_ERR_INVALID_ARGUMENT, "trainer is null");
  if (enabled < 0) return fail(TMNN_ERR_INVALID_ARGUMENT, "profiling interval must be >= 0");
  TMNN_HIP_TRY(hipSetDevice(tr->ctx->device));
  const int rc = prof_collect(tr);  // drop what an earlier window recorded
  if (rc != TMNN_OK) return rc;
  tr->prof_acc = tmnn_step_profile{};
  tr->prof_samples.clear();
  tr->prof_every = enabled;
  tr->prof_seen = 0;
  tr->prof_infer_seen = 0;
  return TMNN_OK;
}

int tmnn_get_step_profile(tmnn_trainer *tr, tmnn_step_profile *out) {
  if (!tr || !out) return fail(TMNN_ERR_INVALID_ARGUMENT, "null argument");
  TMNN_HIP_TRY(hipSetDevice(tr->ctx->device));
  const int rc = prof_collect(tr);
  if (rc != TMNN_OK) return rc;
  *out = tr->prof_acc;
  return TMNN_OK;
}

int tmnn_debug_encode(tmnn_trainer *tr, const float *positions, int32_t n, float *features,
                      uint32_t *corner_index, float *corner_weight) {
  if (!tr) return fail(TMNN_ERR_INVALID_ARGUMENT, "trainer is null");
  if (n < 0) return fail(TMNN_ERR_INVALID_ARGUMENT, "N must be non-negative");
  if (n == 0) return TMNN_OK;
  if (!positions || !features) return fail(TMNN_ERR_INVALID_ARGUMENT, "null argument");
  TMNN_HIP_TRY(hipSetDevice(tr->ctx->device));
  hipStream_t st = tr->ctx->stream;
  const size_t D = tr->d.spatial_dims, L = tr->d.num_levels, F = tr->d.features_per_level;
  const size_t C = size_t(1) << D;
  TMNN_HIP_TRY(tr->in_pos.ensure(n * D * sizeof(float)));
  TMNN_HIP_TRY(tr->dbg_a.ensure(n * L * F * sizeof(float)));
  TMNN_HIP_TRY(tr->dbg_b.ensure(n * L * C * sizeof(uint32_t)));
  TMNN_HIP_TRY(tr->dbg_c.ensure(n * L * C * sizeof(float) + kMaxLevels * sizeof(float)));
  float *res_dev = reinterpret_cast<float *>(static_cast<uint8_t *>(tr->dbg_c.ptr) +
                                             n * L * C * sizeof(float));
  TMNN_HIP_TRY(hipMemcpyAsync(res_dev, tr->res, kMaxLevels * sizeof(float),
                              hipMemcpyHostToDevice, st));
  TMNN_HIP_TRY(hipMemcpyAsync(tr->in_pos.ptr, positions, n * D * sizeof(float),
                              hipMemcpyHostToDevice, st));
  const int64_t threads = static_cast<int64_t>(n) * static_cast<int64_t>(L);
  hipLaunchKernelGGL(encode_debug_kernel, dim3(static_cast<uint32_t>((threads + 255) / 256)),
                     dim3(256), 0, st, tr->params.as<float>(),
                     static_cast<uint32_t>(tr->d.log2_hashmap_size), tr->d.spatial_dims,
                     tr->d.features_per_level, tr->d.num_levels, res_dev, tr->in_pos.as<float>(),
                     n, tr->dbg_a.as<float>(), tr->dbg_b.as<uint32_t>(),
                     tr->dbg_c.as<float>());
  TMNN_HIP_TRY(hipGetLastError());
  TMNN_HIP_TRY(hipMemcpyAsync(features, tr->dbg_a.ptr, n * L * F * sizeof(float),
                              hipMemcpyDeviceToHost, st));
  if (corner_index)
    TMNN_HIP_TRY(hipMemcpyAsync(corner_index, tr->dbg_b.ptr, n * L * C * sizeof(uint32_t),
                                hipMemcpyDeviceToHost, st));
  if (corner_weight)
    TMNN_HIP_TRY(hipMemcpyAsync(corner_weight, tr->dbg_c.ptr, n * L * C * sizeof(float),
                                hipMemcpyDeviceToHost, st));
  TMNN_HIP_TRY(hipStreamSynchronize(st));
  return TMNN_OK;
}

// DefaultAuthority::parameter_layout (default_trainer.cpp:241-260): counts of
// the fused parameter buffer and the step's per-launch control data. The
// kernels of this library take the step parameters (N, loss scale, active
// levels) and Adam's hyper-parameters as launch arguments, so the reference's
// TrainParams / AdamParams device buffers have no counterpart (float counts 0,
// TrainParamsLayout indices as the reference's defaults, schema.h:29-35).
int tmnn_parameter_layout(tmnn_trainer *tr, tmnn_parameter_layout_t *out) {
  if (!tr || !out) return fail(TMNN_ERR_INVALID_ARGUMENT, "null argument");
  if (out->struct_size != sizeof(tmnn_parameter_layout_t))
    return fail(TMNN_ERR_INVALID_ARGUMENT, "tmnn_parameter_layout_t.struct_size mismatch");
  std::memset(out, 0, sizeof *out);
  out->struct_size = sizeof *out;
  out->hash_grid_float_count = tr->hash_count;
  out->mlp_weight_float_count = tr->mlp_count;
  out->train_params_float_count = 0;
  out->train_params_idx_n = 0;
  out->train_params_idx_unsigned_mode = 1;
  out->train_params_idx_loss_scale = 2;
  out->train_params_idx_num_active_levels = 3;
  out->adam_params_float_count = 0;
  out->config_header_float_count = 0;
  out->config_tail_float_count = 0;
  out->target_dims = static_cast<uint32_t>(tr->d.num_outputs);
  out->reduction_terms = 1;  // one loss partial per training block
  out->fused_adam = 1;       // Adam runs inside the step's last kernel
  return TMNN_OK;
}

// DefaultRuntime::batch_plan (default_trainer.cpp:2333-2360): one step lane
// (the trainer's stream runs one step at a time), no 65536 cap, and the
// training kernel's block geometry.
int tmnn_batch_plan(tmnn_trainer *tr, tmnn_batch_plan_t *out) {
  if (!tr || !out) return fail(TMNN_ERR_INVALID_ARGUMENT, "null argument");
  if (out->struct_size != sizeof(tmnn_batch_plan_t))
    return fail(TMNN_ERR_INVALID_ARGUMENT, "tmnn_batch_plan_t.struct_size mismatch");
  std::memset(out, 0, sizeof *out);
  out->struct_size = sizeof *out;
  const uint64_t B = static_cast<uint64_t>(tr->d.batch_size);
  out->max_batch_size = static_cast<uint32_t>(B);
  out->lane_count = 1;
  out->input_dims = static_cast<uint32_t>(tr->d.spatial_dims);
  out->target_dims = static_cast<uint32_t>(tr->d.num_outputs);
  out->reduction_terms = 1;
  out->positions_bytes_per_lane = B * out->input_dims * sizeof(float);
  out->targets_bytes_per_lane = B * out->target_dims * sizeof(float);
  out->reduction_bytes_per_lane = static_cast<uint64_t>(tr->train_plan.max_blocks) * sizeof(float);
  const int tile = tr->train_plan.wide ? kWideWaves * kTilePts : kTilePts;
  out->threadgroup_size = static_cast<uint32_t>(64 * tr->train_plan.wpb);
  out->points_per_threadgroup = static_cast<uint32_t>(
      tr->train_plan.layerwise ? kLwTile
                               : (tr->train_plan.wide ? tile : kTilePts * tr->train_plan.wpb));
  return TMNN_OK;
}

// RuntimeStoragePolicy (runtime_authority.h:57-66): every buffer is device
// memory (hipMalloc); host access goes through explicit copies.
int tmnn_storage_policy(tmnn_trainer *tr, tmnn_storage_policy_t *out) {
  if (!tr || !out) return fail(TMNN_ERR_INVALID_ARGUMENT, "null argument");
  if (out->struct_size != sizeof(tmnn_storage_policy_t))
    return fail(TMNN_ERR_INVALID_ARGUMENT, "tmnn_storage_policy_t.struct_size mismatch");
  std::memset(out, 0, sizeof *out);
  out->struct_size = sizeof *out;
  out->parameter_weights = TMNN_STORAGE_GPU_ONLY;
  out->gradients = TMNN_STORAGE_GPU_ONLY;
  out->optimizer_state = TMNN_STORAGE_GPU_ONLY;
  out->control_buffers = TMNN_STORAGE_GPU_ONLY;
  out->step_inputs = TMNN_LIFETIME_TRANSIENT;
  out->step_targets = TMNN_LIFETIME_TRANSIENT;
  out->step_reduction = TMNN_LIFETIME_TRANSIENT;
  out->requires_staging_uploads = 1;
  return TMNN_OK;
}

// DefaultAuthority::buffer(role) (default_trainer.cpp:263-297): the device
// range holding a role's data. Roles whose data this library passes as
// launch arguments (TrainParams, AdamParams) return an empty view, as the
// reference does for a buffer it does not have (RuntimeBufferView::valid()
// is false). ConfigWeights is the training kernel's packed weight image (its
// layout is this library's, not the reference's 8-float header + MLP copy).
int tmnn_runtime_buffer(tmnn_trainer *tr, int32_t role, tmnn_buffer_view *out) {
  if (!tr || !out) return fail(TMNN_ERR_INVALID_ARGUMENT, "null argument");
  if (out->struct_size != sizeof(tmnn_buffer_view))
    return fail(TMNN_ERR_INVALID_ARGUMENT, "tmnn_buffer_view.struct_size mismatch");
  std::memset(out, 0, sizeof *out);
  out->struct_size = sizeof *out;
  out->role = role;
  out->visibility = TMNN_STORAGE_GPU_ONLY;
  out->lifetime = TMNN_LIFETIME_PERSISTENT;
  const uint64_t hb = static_cast<uint64_t>(tr->hash_count) * sizeof(float);
  const uint64_t mb = static_cast<uint64_t>(tr->mlp_count) * sizeof(float);
  auto set = [&](void *base, uint64_t off, uint64_t bytes, int32_t elem) {
    out->gpu_buffer = base;
    out->offset = off;
    out->bytes = bytes;
    out->element_kind = elem;
    out->device_ptr = base ? static_cast<uint8_t *>(base) + off : nullptr;
  };
  switch (role) {
    case TMNN_BUFFER_CONFIG_WEIGHTS:
      set(tr->train_plan.image, 0, tr->train_plan.image_bytes, TMNN_ELEM_OPAQUE);
      break;
    case TMNN_BUFFER_HASH_WEIGHTS: set(tr->params.ptr, 0, hb, TMNN_ELEM_F32); break;
    case TMNN_BUFFER_MLP_WEIGHTS: set(tr->params.ptr, hb, mb, TMNN_ELEM_F32); break;
    case TMNN_BUFFER_GRAD_HASH:
      set(tr->grad_hash.ptr, 0, static_cast<uint64_t>(tr->hash_count) * sizeof(int32_t),
          tr->d.features_per_level == 2 ? TMNN_ELEM_I32_PACKED_PAIR : TMNN_ELEM_I32);
      break;
    case TMNN_BUFFER_GRAD_MLP: set(tr->grad_mlp.ptr, 0, mb, TMNN_ELEM_F32); break;
    case TMNN_BUFFER_TRAIN_PARAMS:
    case TMNN_BUFFER_ADAM_PARAMS:
      set(nullptr, 0, 0, TMNN_ELEM_F32);
      break;
    case TMNN_BUFFER_FUSED_WEIGHTS: set(tr->params.ptr, 0, hb + mb, TMNN_ELEM_F32); break;
    case TMNN_BUFFER_FUSED_FIRST_MOMENT: set(tr->m.ptr, 0, hb + mb, TMNN_ELEM_F32); break;
    case TMNN_BUFFER_FUSED_SECOND_MOMENT: set(tr->v.ptr, 0, hb + mb, TMNN_ELEM_F32); break;
    default: return fail(TMNN_ERR_INVALID_ARGUMENT, "unknown RuntimeBufferRole");
  }
  return TMNN_OK;
}

int tmnn_debug_encode_tiles(tmnn_trainer *tr, const float *positions, int32_t n, int32_t sorted,
                            float *features, uint32_t *perm_out, float *sorted_pos_out,
                            uint64_t *padding_nonzero) {
  if (!tr) return fail(TMNN_ERR_INVALID_ARGUMENT, "trainer is null");
  if (n < 0) return fail(TMNN_ERR_INVALID_ARGUMENT, "N must be non-negative");
  if (n == 0) return TMNN_OK;
  if (!positions || !features) return fail(TMNN_ERR_INVALID_ARGUMENT, "null argument");
  TMNN_HIP_TRY(hipSetDevice(tr->ctx->device));
  hipStream_t st = tr->ctx->stream;
  int rc = ensure_batch(tr, n);
  if (rc != TMNN_OK) return rc;
  const size_t D = tr->d.spatial_dims;
  TMNN_HIP_TRY(hipMemcpyAsync(tr->in_pos.ptr, positions, n * D * sizeof(float),
                              hipMemcpyHostToDevice, st));
  const float *pos = tr->in_pos.as<float>(), *unused = nullptr;
  const uint32_t *perm = nullptr;
  if (sorted) {
    rc = sort_batch(tr, tr->in_pos.as<float>(), nullptr, 0, n, &pos, &unused, &perm, false);
    if (rc != TMNN_OK) return rc;
  }
  float *pos_out = perm ? tr->s_pos.as<float>() : nullptr;
  if ((rc = launch_encode(tr, pos, n, perm, pos_out)) != TMNN_OK) return rc;
  const int n_pad = (n + kTilePts - 1) / kTilePts * kTilePts;
  const int KT0 = tr->INP / 16;
  std::vector<float> tiles(static_cast<size_t>(n_pad) * tr->INP);
  TMNN_HIP_TRY(hipMemcpyAsync(tiles.data(), tr->xfeat.ptr, tiles.size() * sizeof(float),
                              hipMemcpyDeviceToHost, st));
  if (perm_out && perm)
    TMNN_HIP_TRY(hipMemcpyAsync(perm_out, perm, n * sizeof(uint32_t), hipMemcpyDeviceToHost, st));
  if (sorted_pos_out && perm)
    TMNN_HIP_TRY(hipMemcpyAsync(sorted_pos_out, pos_out, n * D * sizeof(float),
                                hipMemcpyDeviceToHost, st));
  TMNN_HIP_TRY(hipStreamSynchronize(st));
  if (perm_out && !perm)
    for (int i = 0; i < n; ++i) perm_out[i] = static_cast<uint32_t>(i);
  if (sorted_pos_out && !perm)
    std::memcpy(sorted_pos_out, positions, n * D * sizeof(float));
  uint64_t pad = 0;
  for (int i = 0; i < n_pad; ++i)
    for (int f = 0; f < tr->INP; ++f) {
      const float x = tiles[xtile_offset(i, f / 4, KT0) + f % 4];
      if (i < n && f < tr->IN)
        features[static_cast<size_t>(i) * tr->IN + f] = x;
      else if (x != 0.0f)
        ++pad;
    }
  if (padding_nonzero) *padding_nonzero = pad;
  return TMNN_OK;
}

int tmnn_debug_hash_rates(tmnn_trainer *tr, const float *d_positions, int32_t n, int32_t sorted,
                          int32_t reps, double *gather_us, double *atomic_us, double *flag_us) {
  if (!tr || !d_positions) return fail(TMNN_ERR_INVALID_ARGUMENT, "null argument");
  if (n <= 0 || reps < 1) return fail(TMNN_ERR_INVALID_ARGUMENT, "N and reps must be >= 1");
  TMNN_HIP_TRY(hipSetDevice(tr->ctx->device));
  hipStream_t st = tr->ctx->stream;
  int rc = ensure_batch(tr, n);
  if (rc != TMNN_OK) return rc;
  const float *pos = d_positions, *unused = nullptr;
  const uint32_t *perm = nullptr;
  if (sorted && (rc = sort_batch(tr, d_positions, nullptr, 0, n, &pos, &unused, &perm)) != TMNN_OK)
    return rc;
  TMNN_HIP_TRY(tr->dbg_a.ensure(static_cast<size_t>(tr->hash_count) * sizeof(int32_t)));
  TMNN_HIP_TRY(tr->dbg_b.ensure(tr->hash_entries));
  TMNN_HIP_TRY(tr->dbg_c.ensure(static_cast<size_t>(n) * sizeof(float)));
  if ((rc = zero_device(tr, tr->dbg_a.ptr, static_cast<size_t>(tr->hash_count) * 4)) != TMNN_OK ||
      (rc = zero_device(tr, tr->dbg_b.ptr, tr->hash_entries)) != TMNN_OK)
    return rc;
  HashRateArgs ra{};
  ra.n = n;
  ra.L = tr->d.num_levels;
  ra.log2T = static_cast<uint32_t>(tr->d.log2_hashmap_size);
  for (int l = 0; l < kMaxLevels; ++l) ra.res[l] = tr->res[l];
  ra.pos = pos;
  ra.table = tr->params.as<float>();
  ra.out = tr->dbg_c.as<float>();
  ra.acc = tr->dbg_a.as<int32_t>();
  ra.flags = tr->dbg_b.as<uint8_t>();
  hipEvent_t e0 = nullptr, e1 = nullptr;
  TMNN_HIP_TRY(hipEventCreate(&e0));
  if (hipEventCreate(&e1) != hipSuccess) {
    (void)hipEventDestroy(e0);
    return fail(TMNN_ERR_GPU, "hipEventCreate failed");
  }
  double *dst[3] = {gather_us, atomic_us, flag_us};
  const dim3 grid((n + 255) / 256);
  // the level-major kernels where the trainer's encode (gather) or scatter
  // (atomic, flag) walks the levels one at a time
  const dim3 grid_l((n + 255) / 256, static_cast<uint32_t>(tr->d.num_levels));
  const bool lm_gather = encode_level_major(tr), lm_scatter = level_major(tr);
  hipError_t err = hipSuccess;
  for (int kind = 0; kind < 3 && err == hipSuccess; ++kind) {
    const bool lm = kind == kRateGather ? lm_gather : lm_scatter;
    err = hipEventRecord(e0, st);
    for (int r = 0; r < reps && err == hipSuccess; ++r) {
#define TMNN_RATE_KIND(DD, FF, KK)                                                               \
  if (lm)                                                                                        \
    hipLaunchKernelGGL((hash_rate_level_kernel<DD, FF, KK>), grid_l, dim3(256), 0, st, ra);      \
  else                                                                                           \
    hipLaunchKernelGGL((hash_rate_kernel<DD, FF, KK>), grid, dim3(256), 0, st, ra);
#define TMNN_RATE(DD, FF)                                                                        \
  if (tr->d.spatial_dims == DD && tr->d.features_per_level == FF) {                              \
    if (kind == kRateGather) {                                                                   \
      TMNN_RATE_KIND(DD, FF, kRateGather)                                                        \
    } else if (kind == kRateAtomic) {                                                            \
      TMNN_RATE_KIND(DD, FF, kRateAtomic)                                                        \
    } else {                                                                                     \
      TMNN_RATE_KIND(DD, FF, kRateFlag)                                                          \
    }                                                                                            \
  }
      TMNN_RATE(2, 1) TMNN_RATE(2, 2) TMNN_RATE(2, 4) TMNN_RATE(3, 1) TMNN_RATE(3, 2)
      TMNN_RATE(3, 4) TMNN_RATE(4, 1) TMNN_RATE(4, 2) TMNN_RATE(4, 4)
#undef TMNN_RATE
#undef TMNN_RATE_KIND
      err = hipGetLastError();
    }
    if (err == hipSuccess) err = hipEventRecord(e1, st);
    if (err == hipSuccess) err = hipEventSynchronize(e1);
    float ms = 0.0f;
    if (err == hipSuccess) err = hipEventElapsedTime(&ms, e0, e1);
    if (err == hipSuccess && dst[kind]) *dst[kind] = 1e3 * static_cast<double>(ms) / reps;
  }
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  if (err != hipSuccess) return fail(TMNN_ERR_GPU, std::string("hash rates: ") + hipGetErrorString(err));
  return TMNN_OK;
}

int tmnn_debug_lds_rate(tmnn_context *ctx, int32_t reps, double *bytes_per_s) {
  if (!ctx || !bytes_per_s) return fail(TMNN_ERR_INVALID_ARGUMENT, "null argument");
  if (reps < 1) return fail(TMNN_ERR_INVALID_ARGUMENT, "reps must be >= 1");
  TMNN_HIP_TRY(hipSetDevice(ctx->device));
  hipStream_t st = ctx->stream;
  // four resident 32 KB blocks per CU, two rounds of them
  const uint32_t blocks = static_cast<uint32_t>(ctx->cu_count) * 8u;
  const int32_t iters = 4096;
  uint32_t *sink = nullptr;
  TMNN_HIP_TRY(hipMalloc(&sink, blocks * sizeof(uint32_t)));
  hipEvent_t e0 = nullptr, e1 = nullptr;
  hipError_t err = hipEventCreate(&e0);
  if (err == hipSuccess) err = hipEventCreate(&e1);
  // one untimed launch, then reps timed ones
  for (int r = 0; r <= reps && err == hipSuccess; ++r) {
    if (r == 1) err = hipEventRecord(e0, st);
    if (err != hipSuccess) break;
    hipLaunchKernelGGL(lds_rate_kernel, dim3(blocks), dim3(kLdsRateThreads), 0, st, iters, sink);
    err = hipGetLastError();
  }
  if (err == hipSuccess) err = hipEventRecord(e1, st);
  if (err == hipSuccess) err = hipEventSynchronize(e1);
  float ms = 0.0f;
  if (err == hipSuccess) err = hipEventElapsedTime(&ms, e0, e1);
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  (void)hipFree(sink);
  if (err != hipSuccess) return fail(TMNN_ERR_GPU, std::string("lds rate: ") + hipGetErrorString(err));
  const double bytes = static_cast<double>(blocks) * kLdsRateThreads * 16.0 * kLdsRateSlots *
                       iters * reps;
  *bytes_per_s = bytes / (1e-3 * static_cast<double>(ms));
  return TMNN_OK;
}

int tmnn_get_step_profile_samples(tmnn_trainer *tr, float *out, uint32_t capacity,
                                  uint32_t *count) {
  if (!tr || !count) return fail(TMNN_ERR_INVALID_ARGUMENT, "null argument");
  TMNN_HIP_TRY(hipSetDevice(tr->ctx->device));
  const int rc = prof_collect(tr);
  if (rc != TMNN_OK) return rc;
  *count = static_cast<uint32_t>(tr->prof_samples.size());
  if (out) {
    const size_t k = std::min<size_t>(capacity, tr->prof_samples.size());
    for (size_t i = 0; i < k; ++i)
      std::memcpy(out + i * TMNN_PROFILE_COLUMNS, tr->prof_samples[i].data(),
                  TMNN_PROFILE_COLUMNS * sizeof(float));
  }
  return TMNN_OK;
}

int tmnn_debug_get_gradients(tmnn_trainer *tr, int32_t *grad_hash, size_t hash_count,
                             float *grad_mlp, size_t mlp_count) {
  if (!tr) return fail(TMNN_ERR_INVALID_ARGUMENT, "trainer is null");
  if (grad_hash && hash_count != tr->hash_count)
    return fail(TMNN_ERR_INVALID_ARGUMENT, "grad_hash count mismatch");
  if (grad_mlp && mlp_count != tr->mlp_count)
    return fail(TMNN_ERR_INVALID_ARGUMENT, "grad_mlp count mismatch");
  TMNN_HIP_TRY(hipSetDevice(tr->ctx->device));
  hipStream_t st = tr->ctx->stream;
  if (grad_hash)
    TMNN_HIP_TRY(hipMemcpyAsync(grad_hash, tr->grad_hash.ptr, hash_count * sizeof(int32_t),
                                hipMemcpyDeviceToHost, st));
  if (grad_mlp)
    TMNN_HIP_TRY(hipMemcpyAsync(grad_mlp, tr->grad_mlp.ptr, mlp_count * sizeof(float),
                                hipMemcpyDeviceToHost, st));
  TMNN_HIP_TRY(hipStreamSynchronize(st));
  // F == 2 entries hold one packed 64-bit sum; restore feature 1
  if (grad_hash && tr->d.features_per_level == 2)
    for (size_t e = 0; e + 1 < hash_count; e += 2)
      grad_hash[e + 1] = unpack_hi(grad_hash[e], grad_hash[e + 1]);
  return TMNN_OK;
}

int tmnn_debug_get_active_mask(tmnn_trainer *tr, uint32_t *words, size_t word_count) {
  if (!tr || !words) return fail(TMNN_ERR_INVALID_ARGUMENT, "null argument");
  if (word_count != tr->mask_words) return fail(TMNN_ERR_INVALID_ARGUMENT, "word count mismatch");
  TMNN_HIP_TRY(hipSetDevice(tr->ctx->device));
  std::vector<uint8_t> flags(tr->hash_entries);
  TMNN_HIP_TRY(hipMemcpyAsync(flags.data(), tr->mask[tr->mask_cur].ptr, flags.size(),
                              hipMemcpyDeviceToHost, tr->ctx->stream));
  TMNN_HIP_TRY(hipStreamSynchronize(tr->ctx->stream));
  // Reference layout (mlp_kernel_emitter.cpp:48-71): bit per entry (F == 2),
  // else bit per float, all F floats of a visited entry set; lifted 2D points
  // also set their z = 1 corners, the partners of the flagged z = 0 entries.
  std::memset(words, 0, word_count * sizeof(uint32_t));
  const uint32_t F = static_cast<uint32_t>(tr->d.features_per_level);
  const uint32_t per = F == 2 ? 1u : F;
  const uint32_t tmask = (1u << tr->d.log2_hashmap_size) - 1u;
  const uint32_t pxor = tr->d.spatial_dims == 2 ? (kPrimeZ & tmask) : 0u;
  for (uint32_t e = 0; e < tr->hash_entries; ++e) {
    const bool z1 = pxor != 0 && flags[(e & ~tmask) | ((e & tmask) ^ pxor)];
    if (!flags[e] && !z1) continue;
    for (uint32_t f = 0; f < per; ++f) {
      const uint32_t bit = e * per + f;
      words[bit >> 5] |= 1u << (bit & 31u);
    }
  }
  return TMNN_OK;
}

int tmnn_debug_morton_sort(tmnn_trainer *tr, const float *positions, int32_t n, uint32_t *codes,
                           uint32_t *perm) {
  if (!tr) return fail(TMNN_ERR_INVALID_ARGUMENT, "trainer is null");
  if (n < 0) return fail(TMNN_ERR_INVALID_ARGUMENT, "N must be non-negative");
  if (n == 0) return TMNN_OK;
  if (!positions || !codes || !perm) return fail(TMNN_ERR_INVALID_ARGUMENT, "null argument");
  TMNN_HIP_TRY(hipSetDevice(tr->ctx->device));
  hipStream_t st = tr->ctx->stream;
  int rc = ensure_batch(tr, n);
  if (rc != TMNN_OK) return rc;
  const size_t D = tr->d.spatial_dims;
  TMNN_HIP_TRY(hipMemcpyAsync(tr->in_pos.ptr, positions, n * D * sizeof(float),
                              hipMemcpyHostToDevice, st));
  const int threads = 256, blocks = (n + threads - 1) / threads;
  hipLaunchKernelGGL(morton_codes_kernel, dim3(blocks), dim3(threads), 0, st,
                     tr->in_pos.as<float>(), n, tr->d.spatial_dims, tr->keys0.as<uint32_t>());
  TMNN_HIP_TRY(hipGetLastError());
  TMNN_HIP_TRY(hipMemcpyAsync(codes, tr->keys0.ptr, n * sizeof(uint32_t), hipMemcpyDeviceToHost,
                              st));
  TMNN_HIP_TRY(hipStreamSynchronize(st));
  const float *sp = nullptr, *stg = nullptr;
  const uint32_t *p = nullptr;
  rc = sort_batch(tr, tr->in_pos.as<float>(), nullptr, 0, n, &sp, &stg, &p);
  if (rc != TMNN_OK) return rc;
  if (!p && n == 1) {
    perm[0] = 0u;  // a single point is its own order
    return TMNN_OK;
  }
  if (!p) return fail(TMNN_ERR_RUNTIME, "morton_sort is disabled for this trainer");
  TMNN_HIP_TRY(hipMemcpyAsync(perm, p, n * sizeof(uint32_t), hipMemcpyDeviceToHost, st));
  TMNN_HIP_TRY(hipStreamSynchronize(st));
  return TMNN_OK;
}

int tmnn_debug_get_resolutions(tmnn_trainer *tr, float *out, int32_t count) {
  if (!tr || !out) return fail(TMNN_ERR_INVALID_ARGUMENT, "null argument");
  if (count != tr->d.num_levels) return fail(TMNN_ERR_INVALID_ARGUMENT, "count must equal num_levels");
  for (int l = 0; l < count; ++l) out[l] = tr->res[l];
  return TMNN_OK;
}

int tmnn_debug_train_image(tmnn_trainer *tr, void *current, void *repacked, uint64_t *bytes) {
  if (!tr || !bytes) return fail(TMNN_ERR_INVALID_ARGUMENT, "null argument");
  KernelPlan &plan = tr->train_plan;
  if (!plan.image) return fail(TMNN_ERR_RUNTIME, "the trainer has no training plan image");
  *bytes = plan.image_bytes;
  if (!current && !repacked) return TMNN_OK;
  if (!current || !repacked) return fail(TMNN_ERR_INVALID_ARGUMENT, "null image buffer");
  TMNN_HIP_TRY(hipSetDevice(tr->ctx->device));
  hipStream_t st = tr->ctx->stream;
  TMNN_HIP_TRY(hipMemcpyAsync(current, plan.image, plan.image_bytes, hipMemcpyDeviceToHost, st));
  // repack into a copy (bytes the packer does not write stay as they are)
  KernelPlan tmp = plan;
  TMNN_HIP_TRY(hipMalloc(&tmp.image, plan.image_bytes));
  int rc = TMNN_OK;
  if (hipMemcpyAsync(tmp.image, plan.image, plan.image_bytes, hipMemcpyDeviceToDevice, st) !=
      hipSuccess) {
    rc = fail(TMNN_ERR_RUNTIME, "image copy failed");
  } else {
    tmp.packed_version = ~0ull;
    rc = ensure_image(tr, tmp);
    if (rc == TMNN_OK &&
        (hipMemcpyAsync(repacked, tmp.image, plan.image_bytes, hipMemcpyDeviceToHost, st) !=
             hipSuccess ||
         hipStreamSynchronize(st) != hipSuccess))
      rc = fail(TMNN_ERR_RUNTIME, "image readback failed");
  }
  if (hipStreamSynchronize(st) != hipSuccess && rc == TMNN_OK)
    rc = fail(TMNN_ERR_RUNTIME, "stream synchronize failed");
  if (hipFree(tmp.image) != hipSuccess && rc == TMNN_OK) rc = fail(TMNN_ERR_RUNTIME, "free failed");
  return rc;
}

int tmnn_debug_philox_uniform(tmnn_context *ctx, uint64_t seed, uint32_t counter_base,
                              uint32_t count, float low, float high, float *out) {
  if (!ctx || (!out && count)) return fail(TMNN_ERR_INVALID_ARGUMENT, "null argument");
  if (count == 0) return TMNN_OK;
  TMNN_HIP_TRY(hipSetDevice(ctx->device));
  float *dev = nullptr;
  TMNN_HIP_TRY(hipMalloc(&dev, count * sizeof(float)));
  int rc = philox_fill(ctx->stream, dev, count, seed, counter_base, low, high);
  if (rc == TMNN_OK) {
    hipError_t e = hipMemcpyAsync(out, dev, count * sizeof(float), hipMemcpyDeviceToHost,
                                  ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) rc = fail(TMNN_ERR_GPU, hipGetErrorString(e));
  }
  (void)hipFree(dev);
  return rc;
}

}  // extern "C"
