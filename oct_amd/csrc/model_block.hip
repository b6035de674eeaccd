// Resident model blocks and the compiled Z-Image session
// (internal/prometheus/native/reactor_api.h:666-1249, 2713-2821;
//  reactor_vulkan_model_block.c; reactors/PrometheusModelBlock.concept).
//
// The reference's contract, kept here:
//   * one model block and one session per runtime; ids are never reused;
//   * a create request is a closed program: the seven fixed steps, declared
//     weights (content/layout identity, byte count) and, for the Z-Image
//     families, the model lock's parameter-set aggregates and weight sizes
//     (reactor_vulkan_model_block.c:393-493);
//   * weights bind in one transaction: an initial upload invalidates the set
//     until every weight has landed; a rebind (replacement) uploads into a
//     second set and swaps at commit, so the old set stays valid on failure
//     (PrometheusModelBlock.concept:1140-1268); the binding generation
//     advances only at commit;
//   * block outputs stay resident and are versioned by output_generation; a
//     resident execution names the generation it consumes; audits copy a
//     completed output (or one stage) to the host;
//   * the session owns the PreparedImage, PreparedContext and JointWorking
//     streams; capture, compose and the MainTransformer's joint read/write are
//     generation-checked (PrometheusModelBlock.concept:860-1098);
//   * faults: the config's test_flags (FAIL_UPLOAD, FAIL_DOWNLOAD) and the
//     one-shot reduction_test_flags (command record, queue submit, completion
//     observation), consumed in execution order; an unobserved completion
//     quarantines the block until the next call reaps it.
//
// The MI355X design: Vulkan buffers, descriptor sets and command buffers
// become plain device allocations made once at create (nothing is allocated
// by an execution), work is queued on the runtime's HIP stream and completion
// is a stream synchronisation.  FP16 weights are widened to fp32 once, at
// upload, into the layouts the fp32 Z-Image block (zimage_f32.hip) reads; the
// W1 and W3 tensors land side by side in one [3840, 20480] matrix so the FFN
// up-projection is a single GEMM.
#include <string.h>

#include <new>

#include "reactor_internal.h"

namespace prom {

namespace {

constexpr uint32_t kShaderResident = 23u;  // the resident proof program (identity)
constexpr uint32_t kShaderNoise = 24u;     // NoiseRefiner (M1B ingress + block)
constexpr uint32_t kShaderContext = 25u;   // ContextRefiner
constexpr uint32_t kShaderMain = 40u;      // MainTransformer

constexpr int kWidth = 3840, kHeads = 30, kFfn = 10240;
constexpr int kImageTokens = 1024, kContextTokens = 32, kJointTokens = 1056;
constexpr float kEps = 1e-5f;
constexpr uint32_t kTransientAuditFloats = 64u;  // PROM_MODEL_BLOCK_M1C_TRANSIENT_AUDIT_FLOATS

// Device audit area of a Z-Image block, allocated at create: the audit-arena
// records (both lock arenas need fewer bytes), the summary job table, the
// M1C witness and a [T, D] scratch for the stages the chain does not keep.
constexpr size_t kAuditRecordBytes = 196608;
constexpr uint32_t kAuditMaxJobs = 32;
constexpr size_t kAuditJobOffset = kAuditRecordBytes;
constexpr size_t kAuditWitnessOffset = kAuditJobOffset + 4096;
constexpr size_t kAuditScratchOffset = kAuditWitnessOffset + 256;
constexpr size_t kAuditClockOffset = kAuditWitnessOffset - 64;  // device clock stamp of a timed execution
static_assert(kAuditJobOffset + kAuditMaxJobs * sizeof(ZImageAuditJob) <= kAuditClockOffset,
              "job table overlaps the clock stamp");
constexpr int kStageEvents = 16;  // ingress begin, the 14 stage boundaries, joint copy end
static_assert(PROM_ZIMAGE_TURBO_AUDIT_REQUIRED_BYTES <= kAuditRecordBytes, "NoiseRefiner arena records");
static_assert(kAuditMaxJobs * sizeof(ZImageAuditJob) <= 4096, "audit job table");

const uint32_t kSteps[PROM_MODEL_BLOCK_MAX_STEPS] = {1u, 2u, 3u, 4u, 5u, 6u, 7u};

// Cache-manifest lexical order of one NoiseRefiner / MainTransformer layer
// (reactor_vulkan_model_block.c:158-161) and of the unmodulated ContextRefiner
// (:198-200), whose tensor i is semantic slot i + 2.
const uint64_t kNoiseWeightBytes[13] = {30720ull,    7864320ull,  256ull,      29491200ull, 256ull,
                                        88473600ull, 7680ull,     7680ull,     78643200ull, 78643200ull,
                                        78643200ull, 7680ull,     7680ull};
const uint64_t kContextWeightBytes[11] = {256ull,       29491200ull, 256ull,       88473600ull,
                                          7680ull,      7680ull,     78643200ull,  78643200ull,
                                          78643200ull, 7680ull,     7680ull};

// Parameter-set aggregates and descriptor identities of the Z-Image Turbo lock
// (the reference's generated models/zimage-turbo/resolved_descriptor.h).
const uint64_t kNoiseAggregate[2] = {0xa1ba526898a2a752ull, 0x80c0cd75f44cc434ull};
const uint64_t kContextAggregate[2] = {0xc08b908a921a80e1ull, 0x30268c3b0d7a6fafull};
const uint64_t kNoiseMemoryPlan = 654891776ull;
const uint64_t kNoiseExecutionPlan = 6517444848718386192ull;
const uint64_t kContextMemoryPlan = 536870912ull;
const uint64_t kContextExecutionPlan = 0xa30b2ac6ff947b21ull;
const uint64_t kContextCanonical[2] = {0xd2b8167de614da25ull, 0x08377e8a46b65cffull};
const uint64_t kMainAggregate[30] = {
    0x48e987811885741aull, 0x7ec04d7363bb1ac0ull, 0x41b9b7985035fd20ull, 0x3ba944c7dd3bc787ull,
    0xc83fa21d17408859ull, 0xa643f7836a056d34ull, 0x6ee8d2ce1947fb66ull, 0xc00357c21617e910ull,
    0xfc1f557f75895368ull, 0xf3d59ef2a2f18d24ull, 0x7e79e59c29ee081bull, 0x3fef07f8f482453eull,
    0xa2067c05a569f2d5ull, 0xd4bcc84602cd9e77ull, 0xebc24a91474ac4d5ull, 0xa42866e4b7a055f8ull,
    0xdb0272f70aa50aa9ull, 0xf6aa44dcc9f59945ull, 0xf921c7aa36817102ull, 0x96a9d4e83e046880ull,
    0xc161dd253cfe99d7ull, 0x9638d4a676d163acull, 0x0e4070f7fda57719ull, 0x76813a3cc2486108ull,
    0xd64f21d7e6b80100ull, 0xe616bea34a39ed99ull, 0xf177c2e5179c53c4ull, 0x75700608176f4340ull,
    0x7750f6f142eeb066ull, 0xdb7de286ef1f507aull};
const uint64_t kStreamBytes[3] = {15728640ull, 491520ull, 16220160ull};  // image, context, joint

// fp32 destination of semantic weight slot s: [rows, cols] written with
// leading dimension ld at column offset col0 of the buffer of slot `owner`.
struct SlotShape {
  uint32_t rows, cols, ld, col0, owner;
};
const SlotShape kSlots[13] = {
    {1, 4 * kWidth, 4 * kWidth, 0, 0},           // adaLN bias
    {256, 4 * kWidth, 4 * kWidth, 0, 1},         // adaLN weight [256, 15360]
    {1, 128, 128, 0, 2},                         // k_norm
    {kWidth, kWidth, kWidth, 0, 3},              // attention.out [3840, 3840]
    {1, 128, 128, 0, 4},                         // q_norm
    {kWidth, 3 * kWidth, 3 * kWidth, 0, 5},      // attention.qkv [3840, 11520]
    {1, kWidth, kWidth, 0, 6},                   // attention_norm1
    {1, kWidth, kWidth, 0, 7},                   // attention_norm2
    {kWidth, kFfn, 2 * kFfn, 0, 8},              // w1 -> columns [0, F) of W13
    {kFfn, kWidth, kWidth, 0, 9},                // w2 [10240, 3840]
    {kWidth, kFfn, 2 * kFfn, kFfn, 8},           // w3 -> columns [F, 2F) of W13
    {1, kWidth, kWidth, 0, 11},                  // ffn_norm1
    {1, kWidth, kWidth, 0, 12}};                 // ffn_norm2

enum Program { kProgProof, kProgNoise, kProgContext, kProgMain };

uint64_t hash_u64(uint64_t h, uint64_t v) {  // FNV-1a over the 8 little-endian bytes
  for (int i = 0; i < 8; ++i) {
    h ^= (v >> (8 * i)) & 0xffu;
    h *= 1099511628211ull;
  }
  return h;
}

struct WeightSet {
  void* buf[13] = {};  // device buffers per slot (slot 10 aliases slot 8's W13)
  uint64_t bytes = 0;
  uint32_t allocations = 0;
};

// The PREFETCH profile's second weight window (reactor_vulkan_model_block.c:
// 4545-4715, PrometheusModelBlock.concept:1310-1485): a full Z-Image weight
// set filled from pinned host staging on a transfer stream of its own while
// the runtime stream executes with the active set.  A prefetch holds `mu`
// (taken after the device context's lock) for its whole transfer and never
// takes the device context's lock while holding it, so activation, reset and
// destroy wait for an in-flight transfer by taking `mu`.
struct PrefetchWindow {
  std::mutex mu;
  bool enabled = false;
  WeightSet set;
  void* host[2] = {};    // pinned staging, alternated so a memcpy overlaps the previous copy
  void* dev = nullptr;   // device staging the FP16 widening reads
  uint64_t staging_bytes = 0;
  hipStream_t stream = nullptr;
  hipEvent_t copied[2] = {};  // host[k] may be refilled once copied[k] has completed
  uint32_t state = PROM_MODEL_WEIGHT_WINDOW_EMPTY;
  uint32_t target_position = 0, family = 0, parameter_set = 0, count = 0;
  int program = 0;
  uint64_t aggregate = 0, generation = 0, transfer_ns = 0;
};

struct ModelBlock {
  bool created = false;
  bool shared = false;  // the compiled-model owner: retargeted through every family
  uint64_t id = 0;
  Program program = kProgProof;
  int tokens = 0;
  int alloc_tokens = 0;  // buffers are sized for this many tokens (the owner: the joint 1056)
  // declared program
  uint32_t family = 0, parameter_set = 0, shader_id = 0, weight_count = 0, step_count = 0;
  uint32_t steps[PROM_MODEL_BLOCK_MAX_STEPS] = {};
  uint64_t aggregate = 0, model_contract = 0, weight_identity = 0, shader_portfolio = 0, precision = 0,
           capability = 0, memory_ceiling = 0, ext_in = 0, ext_out = 0, declared_audit = 0;
  PrometheusModelBlockWeightDeclaration decl[PROM_MODEL_BLOCK_MAX_WEIGHTS] = {};
  // binding
  WeightSet active, candidate;
  PrefetchWindow* pf = nullptr;  // the owner's second window under PREFETCH (held by ModelState)
  uint64_t prefetch_bytes = 0;   // device bytes of that window's weight set
  uint32_t active_window = 0;    // flips at every activated prefetch
  bool binding_valid = false;
  uint32_t binding_phase = 0;  // 0 empty, 3 uploading, 7 failed (binding_state when not valid)
  uint64_t binding_generation = 0, descriptor_generation = 0;
  // device buffers, allocated at create
  void* staging = nullptr;  // raw upload bytes (largest declared weight)
  uint64_t staging_bytes = 0;
  float* x = nullptr;       // block input [T, D] (external ingress or resident boundary)
  float* out = nullptr;     // resident output [T, D]
  uint16_t* x_bf16 = nullptr;
  uint16_t* cond_bf16 = nullptr;
  float* cond = nullptr;    // [256]
  float* coords = nullptr;  // [T, 3]
  char* ws = nullptr;
  size_t ws_off[kZCount] = {};
  char* audit_dev = nullptr;  // Z-Image programs: audit records, job table, witness, scratch
  float* proof_in = nullptr;  // resident proof: input, output, audit
  float* proof_out = nullptr;
  float* proof_audit = nullptr;
  uint64_t reusable_bytes = 0, audit_alloc_bytes = 0;
  hipEvent_t ev_begin = nullptr, ev_end = nullptr;
  hipEvent_t stage_ev[kStageEvents] = {};  // Z-Image programs
  // per-stage timing of the last MainTransformer execution, in device wall-clock nanoseconds
  uint64_t total_begin_tick = 0, total_end_tick = 0, compute_begin_tick = 0, compute_end_tick = 0;
  uint64_t ingress_ns = 0, joint_copy_ns = 0;
  uint64_t stage_begin_tick[PROM_MODEL_BLOCK_MAIN_STAGE_COUNT] = {};
  uint64_t stage_end_tick[PROM_MODEL_BLOCK_MAIN_STAGE_COUNT] = {};
  uint64_t stage_ns[PROM_MODEL_BLOCK_MAIN_STAGE_COUNT] = {};
  // execution state
  bool quarantined = false, output_valid = false, audit_valid = false;
  uint64_t output_generation = 0, resident_input_generation = 0;
  uint64_t plan_identity = 0, replay_identity = 0, prefix_replay = 0;
  uint64_t m1b_prefix = 0;  // replay identity of the M1B whose pre-attention state the workspace holds
  uint64_t cold_allocations = 0, pipelines = 0, uploads = 0, executions = 0;
  uint64_t last_execution_ns = 0, gpu_total_ns = 0, gpu_compute_ns = 0, last_memcpy_ns = 0, last_readback_ns = 0;
  int32_t last_detail = 0;
};

struct Stream {
  uint64_t generation = 0, producer = 0, output = 0;
  bool valid = false;
};

struct ModelSession {
  bool created = false;
  uint64_t id = 0, lock = 0;
  uint32_t requested_profile = 0, requested_route = 0;
  uint32_t selected_profile = PROM_MODEL_EXECUTION_PROFILE_MINIMUM_MEMORY;  // decided at owner create
  uint32_t selected_route = 0, route_fallback = 0, route_shader = 0;
  float* buf[3] = {};  // image [1024, D], context [32, D], joint [1056, D]
  Stream streams[3];
  bool joint_writing = false;
  uint64_t joint_image_generation = 0, joint_context_generation = 0, compositions = 0;
  uint64_t active_block_id = 0, binding_generation = 0, replay = 0, cold_allocations = 0;
  // owner position: 0 NoiseRefiner 0, 1 NoiseRefiner 1, 2 ContextRefiner 0,
  // 3 ContextRefiner 1, 4 + i MainTransformer layer i
  uint32_t retarget_position = 0;
  uint64_t evaluation_generation = 0;
  uint32_t profile_fallback = 0;
  int32_t last_detail = 0;
};

}  // namespace

struct ModelState {
  ModelBlock block;
  ModelSession session;
  PrefetchWindow prefetch;
  uint64_t next_block_id = 1, next_session_id = 1;
};

namespace {

// ---------------------------------------------------------------- helpers

// One lane writes the device's constant-rate wall clock (the time base of the
// per-stage ticks in the evidence).
__global__ __launch_bounds__(64) void device_clock_kernel(uint64_t* __restrict__ dst) {
  if (threadIdx.x == 0) dst[0] = wall_clock64();
}

__global__ __launch_bounds__(256) void proof_kernel(const float* __restrict__ in, float* __restrict__ out, uint64_t n,
                                                    float* __restrict__ audit, uint64_t audit_n) {
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x) {
    const float v = in[i];
    out[i] = v;
    if (i < audit_n) audit[i] = v;
  }
}

// coords [T, 3] of the image grid (frame 33 = 15 text tokens + 17 padding + 1,
// row t/32, column t%32: zimage/canonical_contract.go:36-64) followed by the
// context tokens (frame 1 + i, 0, 0: context_refiner_reference.go:156-158).
__global__ void coords_kernel(float* __restrict__ c, int image, int context) {
  const int t = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (t >= image + context) return;
  if (t < image) {
    c[3 * t] = 33.0f;
    c[3 * t + 1] = (float)(t / 32);
    c[3 * t + 2] = (float)(t % 32);
  } else {
    c[3 * t] = (float)(t - image + 1);
    c[3 * t + 1] = 0.0f;
    c[3 * t + 2] = 0.0f;
  }
}

ModelState* state_of(Runtime* rt) {
  if (rt->model == nullptr) rt->model = new (std::nothrow) ModelState();
  return rt->model;
}

bool alloc_dev(ModelBlock* b, void** p, uint64_t bytes) {
  *p = nullptr;
  if (bytes == 0) return true;
  if (hipMalloc(p, (size_t)bytes) != hipSuccess) {
    *p = nullptr;
    return false;
  }
  ++b->cold_allocations;
  return true;
}

void free_dev(void* p) {
  if (p) (void)hipFree(p);
}

void free_set(WeightSet* s) {
  for (int i = 0; i < 13; ++i)
    if (i != 10) free_dev(s->buf[i]);  // slot 10 aliases slot 8 for the Z-Image programs
  *s = WeightSet{};
}

void free_set_proof(WeightSet* s) {
  for (int i = 0; i < 13; ++i) free_dev(s->buf[i]);
  *s = WeightSet{};
}

// Waits for an in-flight prefetch (its transfer holds pf->mu), then frees the window.
void release_prefetch(PrefetchWindow* pf) {
  std::lock_guard<std::mutex> window(pf->mu);
  if (pf->stream) (void)hipStreamSynchronize(pf->stream);
  free_set(&pf->set);
  free_dev(pf->dev);
  for (int k = 0; k < 2; ++k) {
    if (pf->host[k]) (void)hipHostFree(pf->host[k]);
    if (pf->copied[k]) (void)hipEventDestroy(pf->copied[k]);
    pf->host[k] = nullptr;
    pf->copied[k] = nullptr;
  }
  if (pf->stream) (void)hipStreamDestroy(pf->stream);
  pf->stream = nullptr;
  pf->dev = nullptr;
  pf->staging_bytes = 0;
  pf->enabled = false;
  pf->state = PROM_MODEL_WEIGHT_WINDOW_EMPTY;
  pf->target_position = pf->family = pf->parameter_set = pf->count = 0;
  pf->aggregate = pf->transfer_ns = 0;
}

void release_block(ModelBlock* b) {
  if (ctx().available) (void)hipStreamSynchronize(ctx().stream);
  if (b->pf) release_prefetch(b->pf);
  if (b->program == kProgProof) {
    free_set_proof(&b->active);
    free_set_proof(&b->candidate);
  } else {
    free_set(&b->active);
    free_set(&b->candidate);
  }
  void* ptrs[] = {b->staging, b->x,       b->out,      b->x_bf16,   b->cond_bf16,  b->cond,
                  b->coords,  b->ws,      b->audit_dev, b->proof_in, b->proof_out, b->proof_audit};
  for (void* p : ptrs) free_dev(p);
  if (b->ev_begin) (void)hipEventDestroy(b->ev_begin);
  if (b->ev_end) (void)hipEventDestroy(b->ev_end);
  for (hipEvent_t e : b->stage_ev)
    if (e) (void)hipEventDestroy(e);
  *b = ModelBlock{};
}

void release_session(ModelSession* s) {
  if (!s->created) return;
  if (ctx().available) (void)hipStreamSynchronize(ctx().stream);
  for (float* p : s->buf) free_dev(p);
  *s = ModelSession{};
}

// Drains work whose completion was not observed (reactor_vulkan_model_block.c:1045-1063).
bool reap(ModelBlock* b) {
  if (!b->quarantined) return true;
  if (hipStreamSynchronize(ctx().stream) != hipSuccess) return false;
  b->quarantined = false;
  b->output_valid = false;
  b->audit_valid = false;
  return true;
}

void mark_failure(ModelBlock* b, int32_t detail) {
  b->output_valid = false;
  b->audit_valid = false;
  b->last_detail = detail;
}

uint32_t binding_state(const ModelBlock* b) {
  if (b->quarantined) return PROM_NOISE_REFINER_BINDING_QUARANTINED;
  if (b->binding_valid) return PROM_NOISE_REFINER_BINDING_BOUND;
  return b->binding_phase;
}

void fill_evidence(const ModelBlock* b, int32_t detail, PrometheusModelBlockEvidence* ev) {
  if (ev == nullptr) return;
  memset(ev, 0, sizeof(*ev));
  ev->struct_size = (uint32_t)sizeof(*ev);
  ev->detail_code = detail;
  if (b == nullptr || !b->created) return;
  const uint64_t persistent = b->active.bytes + b->candidate.bytes + b->prefetch_bytes;
  const uint64_t audit = b->audit_alloc_bytes;
  ev->created = 1u;
  ev->weights_uploaded = b->binding_valid ? 1u : 0u;
  ev->quarantined = b->quarantined ? 1u : 0u;
  ev->output_valid = b->output_valid ? 1u : 0u;
  ev->audit_valid = b->audit_valid ? 1u : 0u;
  ev->fixed_step_count = b->step_count;
  ev->weight_count = b->weight_count;
  ev->persistent_bytes = persistent;
  ev->reusable_bytes = b->reusable_bytes;
  ev->audit_bytes = audit;
  ev->external_bytes = b->ext_in + b->ext_out;
  ev->total_committed_bytes = persistent + b->reusable_bytes + audit;
  ev->peak_plan_bytes = ev->total_committed_bytes;
  ev->cold_buffer_allocation_count = b->cold_allocations;
  ev->warm_buffer_allocation_count = 0;  // executions never allocate
  ev->pipeline_create_count = b->pipelines;
  ev->weight_upload_count = b->uploads;
  ev->execution_count = b->executions;
  ev->last_execution_ns = b->last_execution_ns;
  ev->execution_plan_identity = b->plan_identity;
  ev->replay_identity = b->replay_identity;
  ev->assembly_family = b->family;
  ev->parameter_set = b->parameter_set;
  ev->binding_state = binding_state(b);
  ev->active_weight_window = b->active_window;
  ev->parameter_set_aggregate_identity = b->aggregate;
  ev->binding_generation = b->binding_generation;
  ev->output_generation = b->output_generation;
  ev->descriptor_generation = b->descriptor_generation;
  ev->gpu_total_ns = b->gpu_total_ns;
  ev->gpu_compute_ns = b->gpu_compute_ns;
  ev->gpu_total_begin_tick = b->total_begin_tick;
  ev->gpu_total_end_tick = b->total_end_tick;
  ev->gpu_compute_begin_tick = b->compute_begin_tick;
  ev->gpu_compute_end_tick = b->compute_end_tick;
  ev->gpu_ingress_transfer_ns = b->ingress_ns;
  ev->gpu_joint_copy_ns = b->joint_copy_ns;
  for (uint32_t i = 0; i < PROM_MODEL_BLOCK_MAIN_STAGE_COUNT; ++i) {
    ev->main_stage_gpu_begin_tick[i] = b->stage_begin_tick[i];
    ev->main_stage_gpu_end_tick[i] = b->stage_end_tick[i];
    ev->main_stage_gpu_ns[i] = b->stage_ns[i];
  }
  ev->last_staging_memcpy_ns = b->last_memcpy_ns;
  ev->last_output_readback_ns = b->last_readback_ns;
}

void fill_session_evidence(const ModelSession* s, PrometheusCompiledModelSessionEvidence* ev, int32_t detail_if_null) {
  if (ev == nullptr) return;
  memset(ev, 0, sizeof(*ev));
  ev->struct_size = (uint32_t)sizeof(*ev);
  if (s == nullptr || !s->created) {
    ev->detail_code = detail_if_null;
    return;
  }
  ev->detail_code = s->last_detail;
  ev->created = 1u;
  ev->session_identity = s->id;
  ev->lock_identity = s->lock;
  ev->active_block_id = s->active_block_id;
  ev->binding_generation = s->binding_generation;
  ev->replay_identity = s->replay;
  ev->prepared_image_generation = s->streams[0].generation;
  ev->prepared_context_generation = s->streams[1].generation;
  ev->joint_generation = s->streams[2].generation;
  ev->joint_image_generation = s->joint_image_generation;
  ev->joint_context_generation = s->joint_context_generation;
  ev->prepared_image_bytes = kStreamBytes[0];
  ev->prepared_context_bytes = kStreamBytes[1];
  ev->joint_bytes = kStreamBytes[2];
  ev->cold_buffer_allocation_count = s->cold_allocations;
  ev->composition_count = s->compositions;
  ev->requested_execution_profile = s->requested_profile;
  ev->selected_execution_profile = s->selected_profile;
  ev->profile_fallback_reason = s->profile_fallback;
  ev->requested_main_attention_route = s->requested_route;
  ev->selected_main_attention_route = s->selected_route;
  ev->main_attention_fallback_reason = s->route_fallback;
  ev->main_attention_shader_id = s->route_shader;
}

bool add_bytes(uint64_t* total, uint64_t v) {
  if (v > UINT64_MAX - *total) return false;
  *total += v;
  return true;
}

bool steps_exact(const PrometheusModelBlockCreateRequest* r) {
  if (r->step_count != PROM_MODEL_BLOCK_MAX_STEPS) return false;
  for (uint32_t i = 0; i < PROM_MODEL_BLOCK_MAX_STEPS; ++i)
    if (r->steps[i] != kSteps[i]) return false;
  return true;
}

// reactor_vulkan_model_block.c:393-493
bool validate_create(const PrometheusModelBlockCreateRequest* r) {
  if (r == nullptr || r->struct_size != sizeof(*r) || r->model_contract_identity == 0 || r->weight_identity == 0 ||
      r->shader_portfolio_identity == 0 || r->precision_policy_identity == 0 || r->capability_route_identity == 0 ||
      r->memory_ceiling_bytes == 0 ||
      (r->shader_id != kShaderResident && r->shader_id != kShaderNoise && r->shader_id != kShaderContext &&
       r->shader_id != kShaderMain) ||
      r->weight_count == 0 || r->weight_count > PROM_MODEL_BLOCK_MAX_WEIGHTS || r->audit_bytes == 0 ||
      (r->external_input_bytes % 4) != 0 || (r->external_output_bytes % 4) != 0 || (r->audit_bytes % 4) != 0 ||
      !steps_exact(r))
    return false;
  if (r->shader_id != kShaderMain && r->external_input_bytes == 0) return false;
  if (r->shader_id == kShaderResident && r->external_output_bytes == 0) return false;
  const uint32_t f = r->assembly_family, p = r->parameter_set;
  if (f == PROM_NOISE_REFINER_FAMILY_Z_IMAGE_TURBO &&
      ((p != 1u && p != 2u) || r->parameter_set_aggregate_identity != kNoiseAggregate[p == 2u ? 1 : 0] ||
       r->shader_id != kShaderNoise))
    return false;
  if (f == PROM_CONTEXT_REFINER_FAMILY_Z_IMAGE_TURBO &&
      ((p != 1u && p != 2u) || r->parameter_set_aggregate_identity != kContextAggregate[p == 2u ? 1 : 0] ||
       r->shader_id != kShaderContext))
    return false;
  if (f == PROM_MAIN_TRANSFORMER_FAMILY_Z_IMAGE_TURBO &&
      (p == 0u || p > 30u || r->parameter_set_aggregate_identity != kMainAggregate[p - 1] || r->shader_id != kShaderMain))
    return false;
  if (f > PROM_MAIN_TRANSFORMER_FAMILY_Z_IMAGE_TURBO) return false;
  if (f == 0u && (p != 0u || r->parameter_set_aggregate_identity != 0u)) return false;
  if (r->shader_id == kShaderNoise &&
      (r->weight_count != 13u || r->external_input_bytes != (uint64_t)kImageTokens * kWidth * 2 ||
       r->external_output_bytes != 0 || r->audit_bytes > PROM_ZIMAGE_TURBO_AUDIT_ARENA_BYTES))
    return false;
  if (f == PROM_CONTEXT_REFINER_FAMILY_Z_IMAGE_TURBO &&
      (r->weight_count != 11u || r->external_input_bytes != (uint64_t)kContextTokens * kWidth * 4 ||
       r->external_output_bytes != 0 || r->audit_bytes > PROM_ZIMAGE_TURBO_AUDIT_ARENA_BYTES))
    return false;
  if (f == PROM_MAIN_TRANSFORMER_FAMILY_Z_IMAGE_TURBO &&
      (r->weight_count != 13u || r->external_input_bytes != 0 || r->external_output_bytes != 0 ||
       r->audit_bytes > PROM_ZIMAGE_TURBO_AUDIT_ARENA_BYTES))
    return false;
  uint64_t weights = 0, total = 0;
  for (uint32_t i = 0; i < r->weight_count; ++i) {
    const PrometheusModelBlockWeightDeclaration& w = r->weights[i];
    if (w.content_identity == 0 || w.layout_identity == 0 || w.byte_count == 0 || !add_bytes(&weights, w.byte_count))
      return false;
    if ((r->shader_id == kShaderNoise || f == PROM_MAIN_TRANSFORMER_FAMILY_Z_IMAGE_TURBO) &&
        w.byte_count != kNoiseWeightBytes[i])
      return false;
    if (f == PROM_CONTEXT_REFINER_FAMILY_Z_IMAGE_TURBO && w.byte_count != kContextWeightBytes[i]) return false;
  }
  uint64_t reserve = 0;
  if (r->shader_id == kShaderNoise) reserve = 128ull << 20;
  else if (f == PROM_CONTEXT_REFINER_FAMILY_Z_IMAGE_TURBO) reserve = 16ull << 20;
  else if (f == PROM_MAIN_TRANSFORMER_FAMILY_Z_IMAGE_TURBO) reserve = 192ull << 20;
  if (r->shader_id == kShaderNoise || f >= PROM_CONTEXT_REFINER_FAMILY_Z_IMAGE_TURBO) {
    total = weights;
    return add_bytes(&total, reserve) && total <= r->memory_ceiling_bytes;
  }
  return add_bytes(&total, weights) && add_bytes(&total, r->external_input_bytes) &&
         add_bytes(&total, r->external_input_bytes) && add_bytes(&total, r->external_output_bytes) &&
         add_bytes(&total, r->external_output_bytes) && add_bytes(&total, r->audit_bytes) &&
         add_bytes(&total, r->audit_bytes) && add_bytes(&total, weights) && total <= r->memory_ceiling_bytes;
}

// Program identity: the reference's field order (reactor_vulkan_model_block.c:495-522)
// followed, for the Z-Image programs, by this library's fixed kernel chain.
uint64_t plan_identity(const ModelBlock* b) {
  uint64_t h = 1469598103934665603ull;
  const uint64_t fields[] = {b->model_contract, b->family,       b->parameter_set, b->aggregate,
                             b->weight_identity, b->shader_portfolio, b->precision, b->capability,
                             b->shader_id,      b->ext_in,       b->ext_out,       b->declared_audit,
                             kTransientAuditFloats * 4ull, 3ull};
  for (uint64_t v : fields) h = hash_u64(h, v);
  for (uint32_t i = 0; i < b->weight_count; ++i) {
    h = hash_u64(h, b->decl[i].content_identity);
    h = hash_u64(h, b->decl[i].layout_identity);
    h = hash_u64(h, b->decl[i].byte_count);
  }
  for (uint32_t i = 0; i < b->step_count; ++i) h = hash_u64(h, b->steps[i]);
  if (b->program != kProgProof) {
    // adaln, norm_mod, qkv sgemm, qkv_split, flash attention, out sgemm,
    // resid_norm_mod, w13 sgemm, swiglu, w2 sgemm, final_resid
    for (uint64_t k = 1; k <= 11; ++k) h = hash_u64(h, 0x4d49333535100000ull | k);
    h = hash_u64(h, (uint64_t)b->tokens);
  }
  return h;
}

int slot_of(const ModelBlock* b, uint32_t index) { return b->program == kProgContext ? (int)index + 2 : (int)index; }

// Allocates the device buffers of one weight set (the Z-Image layout or the
// declared raw bytes of the resident proof).
bool alloc_set(ModelBlock* b, WeightSet* s) {
  *s = WeightSet{};
  if (b->program == kProgProof) {
    for (uint32_t i = 0; i < b->weight_count; ++i) {
      if (!alloc_dev(b, &s->buf[i], b->decl[i].byte_count)) return false;
      ++s->allocations;
      s->bytes += b->decl[i].byte_count;
    }
    return true;
  }
  for (uint32_t i = 0; i < b->weight_count; ++i) {
    const int slot = slot_of(b, i);
    if (slot == 10) continue;  // lands in W13 with slot 8
    const SlotShape& sh = kSlots[slot];
    const uint64_t bytes = (uint64_t)sh.rows * sh.ld * 4;
    if (!alloc_dev(b, &s->buf[slot], bytes)) return false;
    ++s->allocations;
    s->bytes += bytes;
  }
  if (s->buf[8]) s->buf[10] = s->buf[8];
  return true;
}

// Uploads weight i of `u` into set `s`: raw bytes, or FP16 widened to fp32.
hipError_t upload_one(ModelBlock* b, WeightSet* s, uint32_t i, const PrometheusModelBlockWeightUpload& u) {
  hipStream_t st = ctx().stream;
  if (b->program == kProgProof)
    return upload_host(s->buf[i], u.bytes, (size_t)u.byte_count, st);
  const int slot = slot_of(b, i);
  const SlotShape& sh = kSlots[slot];
  hipError_t e = upload_host(b->staging, u.bytes, (size_t)u.byte_count, st);
  if (e != hipSuccess) return e;
  float* dst = static_cast<float*>(s->buf[sh.owner]) + sh.col0;
  e = launch_widen_f16(static_cast<const uint16_t*>(b->staging), dst, sh.rows, sh.cols, sh.ld, st);
  if (e != hipSuccess) return e;
  return hipStreamSynchronize(st);  // the staging buffer is reused by the next weight
}

bool upload_matches(const ModelBlock* b, const PrometheusModelBlockWeightUpload* uploads, uint32_t count,
                    const uint64_t* sizes) {
  for (uint32_t i = 0; i < count; ++i) {
    const PrometheusModelBlockWeightUpload& u = uploads[i];
    if (u.binding_index != i || u.bytes == nullptr || u.byte_count > b->staging_bytes) return false;
    if (sizes != nullptr) {
      if (u.content_identity == 0 || u.layout_identity == 0 || u.byte_count != sizes[i]) return false;
    } else if (u.byte_count != b->decl[i].byte_count || u.content_identity != b->decl[i].content_identity ||
               u.layout_identity != b->decl[i].layout_identity) {
      return false;
    }
  }
  return true;
}

// The binding transaction (PrometheusModelBlock.concept:1140-1268 and
// reactor_vulkan_model_block.c:1065-1123).  replacement: upload into a second
// set and swap at commit; otherwise overwrite the active set in place.
bool change_weights(Runtime* rt, ModelBlock* b, const PrometheusModelBlockWeightUpload* uploads, uint32_t count,
                    bool replacement) {
  if (!reap(b)) {
    b->last_detail = PROM_MODEL_BLOCK_DETAIL_COMPLETION_UNCERTAIN;
    return false;
  }
  WeightSet* target = &b->active;
  if (replacement) {
    if (!alloc_set(b, &b->candidate)) {
      free_set(&b->candidate);
      b->last_detail = PROM_MODEL_BLOCK_DETAIL_RESOURCE_CREATE_FAILED;
      return false;
    }
    target = &b->candidate;
  } else {
    b->binding_valid = false;
    b->binding_phase = PROM_NOISE_REFINER_BINDING_UPLOADING;
  }
  const uint64_t t0 = wall_ns();
  for (uint32_t i = 0; i < count; ++i) {
    if ((rt->test_flags & PROM_TESTCFG_FAIL_UPLOAD) != 0u || upload_one(b, target, i, uploads[i]) != hipSuccess) {
      (void)hipStreamSynchronize(ctx().stream);
      if (replacement) {
        free_set(&b->candidate);
      } else {
        b->binding_phase = PROM_NOISE_REFINER_BINDING_FAILED_BEFORE_COMMIT;
      }
      b->last_detail = PROM_MODEL_BLOCK_DETAIL_UPLOAD_FAILED;
      mark_failure(b, PROM_MODEL_BLOCK_DETAIL_UPLOAD_FAILED);
      return false;
    }
    ++b->uploads;
  }
  if (hipStreamSynchronize(ctx().stream) != hipSuccess) {
    b->last_detail = PROM_MODEL_BLOCK_DETAIL_UPLOAD_FAILED;
    return false;
  }
  b->last_memcpy_ns = wall_ns() - t0;
  if (replacement) {
    free_set(&b->active);
    b->active = b->candidate;
    b->candidate = WeightSet{};
  }
  b->binding_valid = true;
  b->binding_phase = PROM_NOISE_REFINER_BINDING_BOUND;
  b->binding_generation += 1;
  b->descriptor_generation += 1;
  b->output_valid = false;
  b->audit_valid = false;
  b->resident_input_generation = 0;
  b->replay_identity = 0;
  b->prefix_replay = 0;
  b->last_detail = 0;
  return true;
}

ZImageBlockWeights weights_of(const ModelBlock* b) {
  const WeightSet& s = b->active;
  auto f = [&](int slot) { return static_cast<const float*>(s.buf[slot]); };
  ZImageBlockWeights w{};
  w.adaln_b = f(0);
  w.adaln_w = b->program == kProgContext ? nullptr : f(1);
  w.k_norm = f(2);
  w.w_out = f(3);
  w.q_norm = f(4);
  w.w_qkv = f(5);
  w.attn_norm1 = f(6);
  w.attn_norm2 = f(7);
  w.w_13 = f(8);
  w.w_2 = f(9);
  w.ffn_norm1 = f(11);
  w.ffn_norm2 = f(12);
  return w;
}

// One-shot faults of the runtime config, taken in execution order
// (reactor_concept_model_block_abi.c:184-202).  Returns the failing detail, or 0.
int32_t take_phase_fault(Runtime* rt, bool* unobserved) {
  *unobserved = false;
  if (rt->reduction_test_flags & PROM_REDUCTION_TESTCFG_FAIL_COMMAND_RECORD) {
    rt->reduction_test_flags &= ~(uint32_t)PROM_REDUCTION_TESTCFG_FAIL_COMMAND_RECORD;
    return PROM_MODEL_BLOCK_DETAIL_COMMAND_RECORD_FAILED;
  }
  if (rt->reduction_test_flags & PROM_REDUCTION_TESTCFG_FAIL_QUEUE_SUBMIT) {
    rt->reduction_test_flags &= ~(uint32_t)PROM_REDUCTION_TESTCFG_FAIL_QUEUE_SUBMIT;
    return PROM_MODEL_BLOCK_DETAIL_QUEUE_SUBMIT_FAILED;
  }
  if (rt->reduction_test_flags & PROM_REDUCTION_TESTCFG_FAIL_COMPLETION_OBSERVATION) {
    rt->reduction_test_flags &= ~(uint32_t)PROM_REDUCTION_TESTCFG_FAIL_COMPLETION_OBSERVATION;
    *unobserved = true;
  }
  return 0;
}

// Runs phases first..last of the Z-Image block of b on x -> out (1 through the
// Q/K/V split, 2 through the attention residual, 3 the FFN), timing them with
// events (stage_events: 14 more, at the boundaries of the 13 stages of a full
// run).  A run from phase 1 replaces the pre-attention state an M1B left.
// Returns 0 or a model-block detail; an injected unobserved completion leaves
// the work queued and quarantines the block.
int32_t run_block(Runtime* rt, ModelBlock* b, const float* x, float* out, int first_phase = 1, int last_phase = 3,
                  const hipEvent_t* stage_events = nullptr) {
  bool unobserved = false;
  const int32_t fault = take_phase_fault(rt, &unobserved);
  if (fault != 0) return fault;
  hipStream_t st = ctx().stream;
  const ZImageBlockWeights w = weights_of(b);
  if (first_phase == 1) b->m1b_prefix = 0;
  (void)hipEventRecord(b->ev_begin, st);
  uint32_t launches = 0;
  if (enqueue_zimage_block_f32(w, x, b->cond, out, b->ws, b->ws_off, b->tokens, kWidth, kFfn, kEps, st, &launches,
                               first_phase, last_phase, stage_events) != hipSuccess) {
    (void)hipStreamSynchronize(st);
    return PROM_MODEL_BLOCK_DETAIL_QUEUE_SUBMIT_FAILED;
  }
  (void)hipEventRecord(b->ev_end, st);
  if (unobserved) {
    b->quarantined = true;
    return PROM_MODEL_BLOCK_DETAIL_COMPLETION_UNCERTAIN;
  }
  if (hipStreamSynchronize(st) != hipSuccess) return PROM_MODEL_BLOCK_DETAIL_COMPLETION_UNCERTAIN;
  float ms = 0.f;
  if (hipEventElapsedTime(&ms, b->ev_begin, b->ev_end) == hipSuccess) b->gpu_compute_ns = (uint64_t)(ms * 1.0e6);
  b->gpu_total_ns = b->gpu_compute_ns;
  return 0;
}

// Opens a timed MainTransformer execution: stamps the device clock into the
// audit area, then records the ingress-begin event.
hipError_t begin_stage_timing(ModelBlock* b, hipStream_t st) {
  hipLaunchKernelGGL(device_clock_kernel, dim3(1), dim3(64), 0, st,
                     reinterpret_cast<uint64_t*>(b->audit_dev + kAuditClockOffset));
  const hipError_t e = hipGetLastError();
  return e != hipSuccess ? e : hipEventRecord(b->stage_ev[0], st);
}

// reactor_vulkan_model_block.c:3531-3565: resolves the 16 timestamps of a
// completed timed execution (0 ingress begin, 1..14 the stage boundaries, 15
// joint copy end) into the evidence's ticks and durations.  Ticks are
// nanoseconds of the device wall clock: the stamp read just before event 0
// plus each event's elapsed time from event 0, so every duration is the
// difference of its two ticks.  Leaves the previous timing on any failure.
void resolve_stage_timing(ModelBlock* b) {
  uint64_t clock = 0;
  int khz = 0;
  if (hipMemcpy(&clock, b->audit_dev + kAuditClockOffset, sizeof(clock), hipMemcpyDeviceToHost) != hipSuccess ||
      hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, ctx().device) != hipSuccess || khz <= 0)
    return;
  uint64_t t[kStageEvents];
  t[0] = (uint64_t)((double)clock * (1.0e6 / (double)khz) + 0.5);
  for (int i = 1; i < kStageEvents; ++i) {
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, b->stage_ev[0], b->stage_ev[i]) != hipSuccess || ms < 0.f) return;
    t[i] = std::max(t[i - 1], t[0] + (uint64_t)((double)ms * 1.0e6 + 0.5));
  }
  b->total_begin_tick = t[0];
  b->total_end_tick = t[15];
  b->compute_begin_tick = t[1];
  b->compute_end_tick = t[14];
  b->gpu_total_ns = t[15] - t[0];
  b->gpu_compute_ns = t[14] - t[1];
  b->ingress_ns = t[1] - t[0];
  b->joint_copy_ns = t[15] - t[14];
  for (uint32_t s = 0; s < PROM_MODEL_BLOCK_MAIN_STAGE_COUNT; ++s) {
    b->stage_begin_tick[s] = t[s + 1];
    b->stage_end_tick[s] = t[s + 2];
    b->stage_ns[s] = t[s + 2] - t[s + 1];
  }
}

// Allocates everything a block executes with (create time; executions never allocate).
bool alloc_block_buffers(ModelBlock* b) {
  uint64_t max_weight = 0;
  for (uint32_t i = 0; i < b->weight_count; ++i) max_weight = std::max(max_weight, b->decl[i].byte_count);
  b->staging_bytes = max_weight;
  if (hipEventCreate(&b->ev_begin) != hipSuccess || hipEventCreate(&b->ev_end) != hipSuccess) return false;
  if (b->program != kProgProof)
    for (hipEvent_t& e : b->stage_ev)
      if (hipEventCreate(&e) != hipSuccess) return false;
  if (b->program == kProgProof) {
    const bool ok = alloc_dev(b, reinterpret_cast<void**>(&b->proof_in), b->ext_in) &&
                    alloc_dev(b, reinterpret_cast<void**>(&b->proof_out), b->ext_out) &&
                    alloc_dev(b, reinterpret_cast<void**>(&b->proof_audit), b->declared_audit) &&
                    alloc_dev(b, &b->staging, max_weight);
    b->reusable_bytes = b->ext_in + b->ext_out + max_weight;
    b->audit_alloc_bytes = b->declared_audit;
    b->pipelines = 1;
    return ok && alloc_set(b, &b->active);
  }
  const int T = b->alloc_tokens;
  const size_t act = (size_t)T * kWidth * 4;
  const size_t ws_bytes = zimage_workspace_layout(T, kWidth, kHeads, kFfn, b->ws_off);
  const bool ok = alloc_dev(b, &b->staging, max_weight) && alloc_dev(b, reinterpret_cast<void**>(&b->x), act) &&
                  alloc_dev(b, reinterpret_cast<void**>(&b->out), act) &&
                  alloc_dev(b, reinterpret_cast<void**>(&b->x_bf16), (size_t)T * kWidth * 2) &&
                  alloc_dev(b, reinterpret_cast<void**>(&b->cond_bf16), kZImageConditionWidth * 2) &&
                  alloc_dev(b, reinterpret_cast<void**>(&b->cond), kZImageConditionWidth * 4) &&
                  alloc_dev(b, reinterpret_cast<void**>(&b->coords), (size_t)T * 3 * 4) &&
                  alloc_dev(b, reinterpret_cast<void**>(&b->ws), ws_bytes) &&
                  alloc_dev(b, reinterpret_cast<void**>(&b->audit_dev), kAuditScratchOffset + act) &&
                  hipMemset(b->cond, 0, kZImageConditionWidth * 4) == hipSuccess;
  b->reusable_bytes = max_weight + 2 * act + (uint64_t)T * kWidth * 2 + kZImageConditionWidth * 6 +
                      (uint64_t)T * 12 + ws_bytes;
  b->audit_alloc_bytes = kAuditScratchOffset + act;  // stage audits copy workspace buffers directly
  b->pipelines = 11;         // the fixed kernel chain of the block
  return ok && alloc_set(b, &b->active);
}

// Selects the Z-Image program (sequence length, workspace offsets inside the
// allocation, coordinates and RoPE table); the owner calls it on every retarget.
bool set_program(ModelBlock* b, Program program) {
  b->program = program;
  b->tokens = program == kProgNoise ? kImageTokens : (program == kProgContext ? kContextTokens : kJointTokens);
  (void)zimage_workspace_layout(b->tokens, kWidth, kHeads, kFfn, b->ws_off);
  hipStream_t st = ctx().stream;
  const int image = program == kProgContext ? 0 : kImageTokens;
  const int context = program == kProgNoise ? 0 : kContextTokens;
  hipLaunchKernelGGL(coords_kernel, dim3((b->tokens + 255) / 256), dim3(256), 0, st, b->coords, image, context);
  if (hipGetLastError() != hipSuccess) return false;
  if (launch_zimage_rope_table(b->coords, reinterpret_cast<float2*>(b->ws + b->ws_off[kZRope]), b->tokens, st) !=
      hipSuccess)
    return false;
  return hipStreamSynchronize(st) == hipSuccess;
}

// ---------------------------------------------------------------- create

int create_block(Runtime* rt, const PrometheusModelBlockCreateRequest* r, uint64_t* out_id,
                 PrometheusModelBlockEvidence* ev, bool shared = false) {
  if (out_id) *out_id = 0;
  if (!validate_create(r) || out_id == nullptr) {
    fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_INVALID_REQUEST, ev);
    return PROM_ERROR;
  }
  ModelState* ms = rt->available ? state_of(rt) : nullptr;
  if (ms == nullptr) {
    fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_RESOURCE_CREATE_FAILED, ev);
    return PROM_ERROR;
  }
  ModelBlock* b = &ms->block;
  if (b->created) {
    fill_evidence(b, PROM_MODEL_BLOCK_DETAIL_ALREADY_CREATED, ev);
    return PROM_ERROR;
  }
  *b = ModelBlock{};
  if (r->assembly_family == PROM_CONTEXT_REFINER_FAMILY_Z_IMAGE_TURBO) {
    b->program = kProgContext;
    b->tokens = kContextTokens;
  } else if (r->assembly_family == PROM_MAIN_TRANSFORMER_FAMILY_Z_IMAGE_TURBO) {
    b->program = kProgMain;
    b->tokens = kJointTokens;
  } else if (r->shader_id == kShaderNoise) {
    b->program = kProgNoise;
    b->tokens = kImageTokens;
  } else {
    b->program = kProgProof;
  }
  b->family = r->assembly_family;
  b->parameter_set = r->parameter_set;
  b->aggregate = r->parameter_set_aggregate_identity;
  b->model_contract = r->model_contract_identity;
  b->weight_identity = r->weight_identity;
  b->shader_portfolio = r->shader_portfolio_identity;
  b->precision = r->precision_policy_identity;
  b->capability = r->capability_route_identity;
  b->memory_ceiling = r->memory_ceiling_bytes;
  b->ext_in = r->external_input_bytes;
  b->ext_out = r->external_output_bytes;
  b->declared_audit = r->audit_bytes;
  b->shader_id = r->shader_id;
  b->weight_count = r->weight_count;
  b->step_count = r->step_count;
  memcpy(b->steps, r->steps, sizeof(b->steps));
  memcpy(b->decl, r->weights, sizeof(b->decl));
  b->shared = shared;
  b->alloc_tokens = shared ? kJointTokens : b->tokens;
  if ((rt->test_flags & PROM_TESTCFG_FAIL_BUFFER_ALLOC) != 0u || !alloc_block_buffers(b) ||
      (b->program != kProgProof && !set_program(b, b->program))) {
    release_block(b);
    fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_RESOURCE_CREATE_FAILED, ev);
    return PROM_ERROR;
  }
  b->created = true;
  b->id = ms->next_block_id++;
  b->plan_identity = plan_identity(b);
  *out_id = b->id;
  fill_evidence(b, 0, ev);
  return PROM_OK;
}

ModelBlock* find_block(Runtime* rt, uint64_t id) {
  if (rt->model == nullptr || !rt->model->block.created || rt->model->block.id != id) return nullptr;
  return &rt->model->block;
}

int upload_weights(Runtime* rt, uint64_t id, const PrometheusModelBlockWeightUpload* uploads, uint32_t count,
                   PrometheusModelBlockEvidence* ev) {
  if (uploads == nullptr) {
    fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_INVALID_REQUEST, ev);
    return PROM_ERROR;
  }
  ModelBlock* b = find_block(rt, id);
  if (b == nullptr) {
    fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_NOT_FOUND, ev);
    return PROM_ERROR;
  }
  if (!reap(b)) {
    fill_evidence(b, PROM_MODEL_BLOCK_DETAIL_COMPLETION_UNCERTAIN, ev);
    return PROM_ERROR;
  }
  if (b->binding_valid || count != b->weight_count) {
    mark_failure(b, PROM_MODEL_BLOCK_DETAIL_WEIGHT_MISMATCH);
    fill_evidence(b, b->last_detail, ev);
    return PROM_ERROR;
  }
  if ((rt->test_flags & PROM_TESTCFG_FAIL_UPLOAD) != 0u) {
    mark_failure(b, PROM_MODEL_BLOCK_DETAIL_UPLOAD_FAILED);
    fill_evidence(b, b->last_detail, ev);
    return PROM_ERROR;
  }
  if (!upload_matches(b, uploads, count, nullptr)) {
    mark_failure(b, PROM_MODEL_BLOCK_DETAIL_WEIGHT_MISMATCH);
    fill_evidence(b, b->last_detail, ev);
    return PROM_ERROR;
  }
  if (!change_weights(rt, b, uploads, count, false)) {
    fill_evidence(b, b->last_detail, ev);
    return PROM_ERROR;
  }
  fill_evidence(b, 0, ev);
  return PROM_OK;
}

// Facade create of the lock-selected ContextRefiner / MainTransformer: the
// closed create request is derived from the lock, then the initial payload
// binds atomically (reactor_vulkan_model_block.c:2305-2462).
int facade_create(Runtime* rt, const PrometheusContextRefinerCreateRequest* r, uint64_t* out_id,
                  PrometheusModelBlockEvidence* ev, bool main) {
  PrometheusModelBlockCreateRequest c;
  memset(&c, 0, sizeof(c));
  c.struct_size = sizeof(c);
  const uint32_t count = main ? 13u : 11u;
  for (uint32_t i = 0; i < count; ++i) {
    c.weights[i].content_identity = r->uploads[i].content_identity;
    c.weights[i].layout_identity = r->uploads[i].layout_identity;
    c.weights[i].byte_count = r->uploads[i].byte_count;
  }
  c.weight_count = count;
  c.step_count = PROM_MODEL_BLOCK_MAX_STEPS;
  memcpy(c.steps, kSteps, sizeof(c.steps));
  c.audit_bytes = PROM_ZIMAGE_TURBO_AUDIT_ARENA_BYTES;
  if (main) {
    c.assembly_family = PROM_MAIN_TRANSFORMER_FAMILY_Z_IMAGE_TURBO;
    c.parameter_set = r->model_local_block_id + 1u;
    c.parameter_set_aggregate_identity = kMainAggregate[r->model_local_block_id];
    c.model_contract_identity = PROM_ZIMAGE_TURBO_LOCK_ID;
    c.weight_identity = c.parameter_set_aggregate_identity;
    c.shader_portfolio_identity = PROM_ZIMAGE_TURBO_LOCK_ID;
    c.precision_policy_identity = PROM_ZIMAGE_TURBO_LOCK_ID;
    c.capability_route_identity = PROM_ZIMAGE_TURBO_LOCK_ID;
    c.memory_ceiling_bytes = PROM_ZIMAGE_TURBO_LOCK_ID;
    c.shader_id = kShaderMain;
  } else {
    c.assembly_family = PROM_CONTEXT_REFINER_FAMILY_Z_IMAGE_TURBO;
    c.parameter_set = PROM_CONTEXT_REFINER_PARAMETER_SET_0;
    c.parameter_set_aggregate_identity = kContextAggregate[0];
    c.model_contract_identity = PROM_ZIMAGE_TURBO_LOCK_ID;
    c.weight_identity = kContextAggregate[0];
    c.shader_portfolio_identity = kContextExecutionPlan;
    c.precision_policy_identity = PROM_ZIMAGE_TURBO_LOCK_ID;
    c.capability_route_identity = kContextCanonical[0];
    c.memory_ceiling_bytes = kContextMemoryPlan;
    c.external_input_bytes = (uint64_t)kContextTokens * kWidth * 4;
    c.shader_id = kShaderContext;
  }
  if (create_block(rt, &c, out_id, ev) != PROM_OK) return PROM_ERROR;
  if (upload_weights(rt, *out_id, r->uploads, r->upload_count, ev) != PROM_OK) {
    release_block(&rt->model->block);
    *out_id = 0;
    return PROM_ERROR;
  }
  return PROM_OK;
}

// Rebind to the next parameter set of the same family (replacement binding).
int rebind(Runtime* rt, uint64_t id, ModelBlock* b, const PrometheusModelBlockWeightUpload* uploads, uint32_t count,
           const uint64_t* sizes, uint32_t new_set, uint64_t new_aggregate, PrometheusModelBlockEvidence* ev) {
  (void)id;
  if (!upload_matches(b, uploads, count, sizes)) {
    fill_evidence(b, PROM_MODEL_BLOCK_DETAIL_WEIGHT_MISMATCH, ev);
    return PROM_ERROR;
  }
  if (!change_weights(rt, b, uploads, count, true)) {
    fill_evidence(b, b->last_detail, ev);
    return PROM_ERROR;
  }
  b->parameter_set = new_set;
  b->aggregate = new_aggregate;
  fill_evidence(b, 0, ev);
  return PROM_OK;
}

// Copies stage `count` floats (rows x cols with source pitch) of the last
// execution to the host.
bool copy_out(float* dst, const float* src, size_t rows, size_t cols, size_t src_ld) {
  hipStream_t st = ctx().stream;
  hipError_t e;
  if (cols == src_ld)
    e = download_host(dst, src, rows * cols * 4, st);
  else
    e = hipMemcpy2DAsync(dst, cols * 4, src, src_ld * 4, cols * 4, rows, hipMemcpyDeviceToHost, st);
  return e == hipSuccess && hipStreamSynchronize(st) == hipSuccess;
}

uint64_t audit_elements(uint32_t family, uint32_t stage, int T) {
  const uint64_t model = (uint64_t)T * kWidth;
  if (family == PROM_NOISE_REFINER_AUDIT_M1B) {
    if (stage == 3) return 4ull * kWidth;
    if (stage == 14) return (uint64_t)T * 3 * kWidth;
    if (stage == 2) return kZImageConditionWidth;
    if (stage >= 4 && stage <= 11) return kWidth;
    return model;
  }
  if (family == PROM_NOISE_REFINER_AUDIT_M1D && (stage == 3 || stage == 4 || stage == 5)) return (uint64_t)T * kFfn;
  return model;
}

// Copies one stage of the completed (or stopped) chain to the host
// (stage numbering: reactor_api.h:776-797, 988-992, 1085-1093).
bool copy_stage(ModelBlock* b, uint32_t family, uint32_t stage, float* dst) {
  const int T = b->tokens, H = kHeads, D = kWidth;
  hipStream_t st = ctx().stream;
  char* ws = b->ws;
  auto W = [&](int k) { return reinterpret_cast<float*>(ws + b->ws_off[k]); };
  const ZImageBlockWeights w = weights_of(b);
  const float2* tab = reinterpret_cast<const float2*>(ws + b->ws_off[kZRope]);
  float* scratch = W(kZO);  // free before attention (M1B) and reused only for audits
  if (family == PROM_NOISE_REFINER_AUDIT_M1B) {
    switch (stage) {
      case 1: return copy_out(dst, b->x, T, D, D);
      case 2: return copy_out(dst, b->cond, 1, kZImageConditionWidth, kZImageConditionWidth);
      case 3: return copy_out(dst, W(kZModRaw), 1, 4 * D, 4 * D);
      case 4: case 6: case 8: case 10: return copy_out(dst, W(kZModRaw) + (stage - 4) / 2 * D, 1, D, D);
      case 5: case 7: case 9: case 11: return copy_out(dst, W(kZMod) + (stage - 5) / 2 * D, 1, D, D);
      case 12:
        return launch_zimage_norm(b->x, w.attn_norm1, scratch, T, D, kEps, st) == hipSuccess &&
               copy_out(dst, scratch, T, D, D);
      case 13: return copy_out(dst, W(kZA), T, D, D);
      case 14: return copy_out(dst, W(kZQkv), T, 3 * D, 3 * D);
      case 15: case 16: case 17: return copy_out(dst, W(kZQkv) + (stage - 15) * D, T, D, 3 * D);
      case 18: case 19: case 20: case 21: {
        const int which = (stage == 18 || stage == 20) ? 0 : 1;
        const bool rope = stage >= 20;
        return launch_zimage_qk_audit(W(kZQkv), tab, which ? w.k_norm : w.q_norm, scratch, T, H, kEps, which, rope,
                                      st) == hipSuccess &&
               copy_out(dst, scratch, T, D, D);
      }
      default: return false;
    }
  }
  if (family == PROM_NOISE_REFINER_AUDIT_M1C) {
    if (stage == 1) return copy_out(dst, W(kZO), T, D, D);
    if (stage == 2) return copy_out(dst, W(kZProj), T, D, D);
    if (stage == 3) return copy_out(dst, W(kZR), T, D, D);
    return false;
  }
  switch (stage) {  // M1D
    case 1:
      return launch_zimage_norm(W(kZR), w.ffn_norm1, W(kZA), T, D, kEps, st) == hipSuccess &&
             copy_out(dst, W(kZA), T, D, D);
    case 2: return copy_out(dst, W(kZF), T, D, D);
    case 3: return copy_out(dst, W(kZG), T, kFfn, 2 * kFfn);
    case 4: return copy_out(dst, W(kZG) + kFfn, T, kFfn, 2 * kFfn);
    case 5: return copy_out(dst, W(kZH), T, kFfn, kFfn);
    case 6: return copy_out(dst, W(kZW2), T, D, D);
    case 7: return copy_out(dst, b->out, T, D, D);
    default: return false;
  }
}

// ---------------------------------------------------------------- NoiseRefiner

// External BF16 ingress of parameter set `required_set`
// (reactor_vulkan_model_block.c:2204-2289).
int noise_external(Runtime* rt, uint64_t id, const PrometheusNoiseRefiner0ExecuteRequest* r, uint32_t required_set,
                   PrometheusModelBlockEvidence* ev) {
  if (r == nullptr || r->struct_size != sizeof(*r) || r->model_input_bf16 == nullptr || r->timestep_bf16 == nullptr ||
      r->model_input_bytes != (uint64_t)kImageTokens * kWidth * 2 || r->timestep_bytes != kZImageConditionWidth * 2 ||
      r->input_identity == 0 || r->timestep_identity == 0 || r->output_identity == 0 || r->audit_enabled != 0) {
    fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_INVALID_REQUEST, ev);
    return PROM_ERROR;
  }
  ModelBlock* b = find_block(rt, id);
  if (b == nullptr || b->family != PROM_NOISE_REFINER_FAMILY_Z_IMAGE_TURBO || b->parameter_set != required_set ||
      binding_state(b) != PROM_NOISE_REFINER_BINDING_BOUND) {
    fill_evidence(b, PROM_MODEL_BLOCK_DETAIL_PARAMETER_SET_MISMATCH, ev);
    return PROM_ERROR;
  }
  if (!reap(b)) {
    mark_failure(b, PROM_MODEL_BLOCK_DETAIL_COMPLETION_UNCERTAIN);
    fill_evidence(b, b->last_detail, ev);
    return PROM_ERROR;
  }
  b->resident_input_generation = 0;  // an external ingress starts a new chain
  b->output_valid = false;
  b->audit_valid = false;
  const uint64_t t0 = wall_ns();
  hipStream_t st = ctx().stream;
  if (upload_host(b->x_bf16, r->model_input_bf16, (size_t)r->model_input_bytes, st) != hipSuccess ||
      hipMemcpyAsync(b->cond_bf16, r->timestep_bf16, (size_t)r->timestep_bytes, hipMemcpyHostToDevice, st) !=
          hipSuccess ||
      launch_widen_bf16(b->x_bf16, b->x, (size_t)kImageTokens * kWidth, st) != hipSuccess ||
      launch_widen_bf16(b->cond_bf16, b->cond, kZImageConditionWidth, st) != hipSuccess) {
    (void)hipStreamSynchronize(st);
    mark_failure(b, PROM_MODEL_BLOCK_DETAIL_INGRESS_DISPATCH_FAILED);
    fill_evidence(b, b->last_detail, ev);
    return PROM_ERROR;
  }
  const int32_t d = run_block(rt, b, b->x, b->out);
  if (d != 0) {
    mark_failure(b, d);
    fill_evidence(b, d, ev);
    return PROM_ERROR;
  }
  b->prefix_replay = hash_u64(hash_u64(hash_u64(hash_u64(b->family, b->parameter_set), b->binding_generation),
                                       r->input_identity),
                              r->timestep_identity);
  b->replay_identity = hash_u64(hash_u64(b->prefix_replay, r->output_identity), 3u);
  b->replay_identity = hash_u64(hash_u64(b->replay_identity, r->output_identity), 7u);
  b->output_valid = true;
  b->output_generation += 1;
  b->executions += 3;
  b->last_execution_ns = wall_ns() - t0;
  b->last_detail = 0;
  fill_evidence(b, 0, ev);
  return PROM_OK;
}

// Resident chain execution of parameter set 1 (reactor_vulkan_model_block.c:3274-3400).
int noise_resident(Runtime* rt, uint64_t id, const PrometheusNoiseRefinerResidentExecuteRequest* r,
                   PrometheusModelBlockEvidence* ev) {
  const bool bad_shape =
      r == nullptr || r->struct_size != sizeof(*r) || r->input_generation == 0 || r->output_identity == 0 ||
      r->audit_enabled > 1u ||
      (r->audit_enabled == 0 && (r->audit_family != PROM_NOISE_REFINER_AUDIT_NONE || r->audit_stage != 0 ||
                                 r->audit_output != nullptr || r->audit_element_capacity != 0)) ||
      (r->audit_enabled != 0 && (r->audit_family < PROM_NOISE_REFINER_AUDIT_M1B ||
                                 r->audit_family > PROM_NOISE_REFINER_AUDIT_M1D || r->audit_output == nullptr));
  if (bad_shape) {
    fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_INVALID_REQUEST, ev);
    return PROM_ERROR;
  }
  const uint32_t fam = r->audit_enabled ? r->audit_family : 0u;
  const uint32_t stage = r->audit_stage;
  if ((fam == PROM_NOISE_REFINER_AUDIT_M1B && (stage < 1 || stage > 21)) ||
      (fam == PROM_NOISE_REFINER_AUDIT_M1C && (stage < 1 || stage > 3)) ||
      (fam == PROM_NOISE_REFINER_AUDIT_M1D && (stage < 1 || stage > 7)) ||
      (fam != 0 && r->audit_element_capacity < audit_elements(fam, stage, kImageTokens))) {
    fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_INVALID_REQUEST, ev);
    return PROM_ERROR;
  }
  ModelBlock* b = find_block(rt, id);
  if (b == nullptr) {
    fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_NOT_FOUND, ev);
    return PROM_ERROR;
  }
  const bool first = b->resident_input_generation == 0;
  if (b->family != PROM_NOISE_REFINER_FAMILY_Z_IMAGE_TURBO || b->parameter_set != PROM_NOISE_REFINER_PARAMETER_SET_1 ||
      binding_state(b) != PROM_NOISE_REFINER_BINDING_BOUND ||
      (first ? r->input_generation != b->output_generation : r->input_generation != b->resident_input_generation) ||
      !reap(b)) {
    mark_failure(b, PROM_MODEL_BLOCK_DETAIL_STALE_OUTPUT);
    fill_evidence(b, b->last_detail, ev);
    return PROM_ERROR;
  }
  b->output_valid = false;
  b->audit_valid = false;
  b->prefix_replay =
      hash_u64(hash_u64(hash_u64(b->family, b->parameter_set), b->binding_generation), r->input_generation);
  const uint64_t t0 = wall_ns();
  hipStream_t st = ctx().stream;
  // The first resident execution takes the predecessor's resident output as
  // its boundary input; later ones re-run that same boundary.
  if (first && hipMemcpyAsync(b->x, b->out, (size_t)kImageTokens * kWidth * 4, hipMemcpyDeviceToDevice, st) !=
                   hipSuccess) {
    mark_failure(b, PROM_MODEL_BLOCK_DETAIL_QUEUE_SUBMIT_FAILED);
    fill_evidence(b, b->last_detail, ev);
    return PROM_ERROR;
  }
  const int stop = fam == PROM_NOISE_REFINER_AUDIT_M1B ? 1 : (fam == PROM_NOISE_REFINER_AUDIT_M1C ? 2 : 0);
  const int32_t d = run_block(rt, b, b->x, b->out, 1, stop == 0 ? 3 : stop);
  if (d != 0) {
    mark_failure(b, d);
    fill_evidence(b, d, ev);
    return PROM_ERROR;
  }
  if (fam != 0) {
    if (!copy_stage(b, fam, stage, r->audit_output)) {
      mark_failure(b, PROM_MODEL_BLOCK_DETAIL_AUDIT_FAILED);
      fill_evidence(b, b->last_detail, ev);
      return PROM_ERROR;
    }
    b->audit_valid = true;
  }
  if (stop != 0) {  // a stage audit ends the chain early and publishes no output
    b->executions += stop;
    b->last_execution_ns = wall_ns() - t0;
    b->replay_identity = hash_u64(b->prefix_replay, stage);
    b->last_detail = 0;
    fill_evidence(b, 0, ev);
    return PROM_OK;
  }
  if (first) b->resident_input_generation = r->input_generation;
  b->output_valid = true;
  b->output_generation += 1;
  b->executions += 3;
  b->last_execution_ns = wall_ns() - t0;
  b->replay_identity = hash_u64(hash_u64(b->prefix_replay, r->output_identity), b->aggregate);
  b->last_detail = 0;
  fill_evidence(b, 0, ev);
  return PROM_OK;
}

// Final audit egress of a completed resident output (reactor_vulkan_model_block.c:3402-3460).
int audit_final(Runtime* rt, uint64_t id, const PrometheusNoiseRefinerFinalAuditRequest* r, Program program,
                PrometheusModelBlockEvidence* ev) {
  const int T = program == kProgNoise ? kImageTokens : (program == kProgContext ? kContextTokens : kJointTokens);
  if (r == nullptr || r->struct_size != sizeof(*r) || r->output == nullptr || r->output_identity == 0 ||
      r->required_output_generation == 0 || r->output_element_capacity < (uint64_t)T * kWidth) {
    fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_INVALID_REQUEST, ev);
    return PROM_ERROR;
  }
  ModelBlock* b = find_block(rt, id);
  if (b == nullptr) {
    fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_NOT_FOUND, ev);
    return PROM_ERROR;
  }
  if (b->program != program || !b->output_valid || b->output_generation != r->required_output_generation ||
      !reap(b)) {
    mark_failure(b, PROM_MODEL_BLOCK_DETAIL_STALE_OUTPUT);
    fill_evidence(b, b->last_detail, ev);
    return PROM_ERROR;
  }
  const uint64_t t0 = wall_ns();
  if ((rt->test_flags & PROM_TESTCFG_FAIL_DOWNLOAD) != 0u || !copy_out(r->output, b->out, T, kWidth, kWidth)) {
    mark_failure(b, PROM_MODEL_BLOCK_DETAIL_AUDIT_FAILED);
    fill_evidence(b, b->last_detail, ev);
    return PROM_ERROR;
  }
  b->last_readback_ns = wall_ns() - t0;
  b->audit_valid = true;
  b->replay_identity = hash_u64(b->replay_identity, r->output_identity);
  b->last_detail = 0;
  fill_evidence(b, 0, ev);
  return PROM_OK;
}

// ---------------------------------------------------------------- ContextRefiner

// reactor_vulkan_model_block.c:2510-2583
int context_execute(Runtime* rt, uint64_t id, uint32_t required_set, const float* input, uint64_t input_bytes,
                    uint64_t input_generation, uint64_t input_identity, uint64_t output_identity,
                    uint32_t audit_enabled, bool resident, PrometheusModelBlockEvidence* ev) {
  if (output_identity == 0 || audit_enabled != 0 ||
      (!resident && (input == nullptr || input_identity == 0 ||
                     input_bytes != (uint64_t)kContextTokens * kWidth * 4))) {
    fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_INVALID_REQUEST, ev);
    return PROM_ERROR;
  }
  ModelBlock* b = find_block(rt, id);
  if (b == nullptr) {
    fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_NOT_FOUND, ev);
    return PROM_ERROR;
  }
  if (!reap(b)) {
    fill_evidence(b, PROM_MODEL_BLOCK_DETAIL_COMPLETION_UNCERTAIN, ev);
    return PROM_ERROR;
  }
  const bool first = resident && b->resident_input_generation == 0;
  if (b->program != kProgContext || b->parameter_set != required_set ||
      binding_state(b) != PROM_NOISE_REFINER_BINDING_BOUND ||
      (resident && (input_generation == 0 || (first ? input_generation != b->output_generation
                                                    : input_generation != b->resident_input_generation)))) {
    mark_failure(b, PROM_MODEL_BLOCK_DETAIL_STALE_OUTPUT);
    fill_evidence(b, b->last_detail, ev);
    return PROM_ERROR;
  }
  if ((uint32_t)(b->output_generation + 1u) == 0u) {
    fill_evidence(b, PROM_MODEL_BLOCK_DETAIL_INVALID_REQUEST, ev);
    return PROM_ERROR;
  }
  b->output_valid = false;
  b->audit_valid = false;
  const uint64_t t0 = wall_ns();
  hipStream_t st = ctx().stream;
  const size_t bytes = (size_t)kContextTokens * kWidth * 4;
  hipError_t e = hipSuccess;
  if (!resident) e = hipMemcpyAsync(b->x, input, bytes, hipMemcpyHostToDevice, st);
  else if (first) e = hipMemcpyAsync(b->x, b->out, bytes, hipMemcpyDeviceToDevice, st);
  if (e != hipSuccess) {
    mark_failure(b, PROM_MODEL_BLOCK_DETAIL_QUEUE_SUBMIT_FAILED);
    fill_evidence(b, b->last_detail, ev);
    return PROM_ERROR;
  }
  const int32_t d = run_block(rt, b, b->x, b->out);
  if (d != 0) {
    mark_failure(b, d);
    fill_evidence(b, d, ev);
    return PROM_ERROR;
  }
  b->output_valid = true;
  b->output_generation += 1;
  if (first) b->resident_input_generation = input_generation;
  b->executions += 1;
  b->last_execution_ns = wall_ns() - t0;
  b->replay_identity = hash_u64(b->plan_identity, resident ? input_generation : input_identity);
  b->replay_identity = hash_u64(b->replay_identity, output_identity);
  b->replay_identity = hash_u64(b->replay_identity, b->aggregate);
  b->last_detail = 0;
  fill_evidence(b, 0, ev);
  return PROM_OK;
}

// ---------------------------------------------------------------- session

bool joint_valid(const ModelSession* s) {
  return s->streams[2].valid && !s->joint_writing && s->streams[0].valid && s->streams[1].valid &&
         s->joint_image_generation == s->streams[0].generation &&
         s->joint_context_generation == s->streams[1].generation;
}

ModelSession* find_session(Runtime* rt, uint64_t id) {
  if (rt->model == nullptr || !rt->model->session.created || rt->model->session.id != id) return nullptr;
  return &rt->model->session;
}

// ---------------------------------------------------------------- compiled-model owner

struct Target {
  Program program;
  uint32_t family, parameter_set, count, local;
  uint64_t aggregate;
  const uint64_t* bytes;
};

// The block the owner binds at `position` (reactor_vulkan_model_block.c:4474-4503).
bool target_at(uint32_t position, Target* t) {
  if (position <= 1) {
    *t = Target{kProgNoise, PROM_NOISE_REFINER_FAMILY_Z_IMAGE_TURBO, position + 1, 13u, position,
                kNoiseAggregate[position], kNoiseWeightBytes};
    return true;
  }
  if (position <= 3) {
    *t = Target{kProgContext, PROM_CONTEXT_REFINER_FAMILY_Z_IMAGE_TURBO, position - 1, 11u, position - 2,
                kContextAggregate[position - 2], kContextWeightBytes};
    return true;
  }
  if (position < 34) {
    const uint32_t layer = position - 4;
    *t = Target{kProgMain, PROM_MAIN_TRANSFORMER_FAMILY_Z_IMAGE_TURBO, layer + 1, 13u, layer, kMainAggregate[layer],
                kNoiseWeightBytes};
    return true;
  }
  return false;
}

bool retarget_uploads_match(const ModelBlock* b, const PrometheusModelBlockWeightUpload* uploads, const Target& t) {
  for (uint32_t i = 0; i < t.count; ++i) {
    const PrometheusModelBlockWeightUpload& u = uploads[i];
    if (u.binding_index != i || u.bytes == nullptr || u.content_identity == 0 || u.layout_identity == 0 ||
        u.byte_count != t.bytes[i] || u.byte_count > b->staging_bytes)
      return false;
  }
  return true;
}

// The PREFETCH window of a freshly created owner (bound to NoiseRefiner 0, so
// alloc_set lays out all 13 slots, which also hold any ContextRefiner set):
// its weight set, two pinned staging buffers and a device staging buffer of
// the largest weight, a non-blocking stream at the default priority and two
// events (reactor_vulkan_model_block.c:1730-1741).
bool alloc_prefetch(ModelBlock* b, PrefetchWindow* pf) {
  std::lock_guard<std::mutex> window(pf->mu);
  b->pf = pf;  // release_block frees a partial window
  pf->staging_bytes = b->staging_bytes;
  if (!alloc_set(b, &pf->set) || !alloc_dev(b, &pf->dev, pf->staging_bytes) ||
      hipStreamCreateWithFlags(&pf->stream, hipStreamNonBlocking) != hipSuccess) {
    pf->stream = nullptr;
    return false;
  }
  for (int k = 0; k < 2; ++k) {
    if (hipHostMalloc(&pf->host[k], (size_t)pf->staging_bytes, hipHostMallocDefault) != hipSuccess) {
      pf->host[k] = nullptr;
      return false;
    }
    ++b->cold_allocations;
    if (hipEventCreateWithFlags(&pf->copied[k], hipEventDisableTiming) != hipSuccess) {
      pf->copied[k] = nullptr;
      return false;
    }
  }
  pf->enabled = true;
  pf->state = PROM_MODEL_WEIGHT_WINDOW_EMPTY;
  b->prefetch_bytes = pf->set.bytes;
  b->reusable_bytes += pf->staging_bytes;
  return true;
}

// One prefetch transfer (PrometheusModelBlock.concept:1370-1404): weight i is
// copied into pinned staging, sent to the device staging buffer and widened
// from FP16 into its slot of the window on the window's stream.  The caller
// holds pf->mu and not the device context's lock.  Returns 0 or a detail.
int32_t prefetch_transfer(PrefetchWindow* pf, const Target& t, const PrometheusModelBlockWeightUpload* uploads) {
  // The calling thread may never have used the device: make the library's
  // device current for it (the library runs on that one device only).
  if (hipSetDevice(ctx().device) != hipSuccess) return PROM_MODEL_BLOCK_DETAIL_COMMAND_RECORD_FAILED;
  for (uint32_t i = 0; i < t.count; ++i) {
    const int k = (int)(i & 1u);
    // the copy that last read host[k] (weight i - 2) must have completed
    if (i >= 2 && hipEventSynchronize(pf->copied[k]) != hipSuccess)
      return PROM_MODEL_BLOCK_DETAIL_COMPLETION_UNCERTAIN;
    const PrometheusModelBlockWeightUpload& u = uploads[i];
    memcpy(pf->host[k], u.bytes, (size_t)u.byte_count);
    const SlotShape& sh = kSlots[t.program == kProgContext ? i + 2u : i];
    float* dst = static_cast<float*>(pf->set.buf[sh.owner]) + sh.col0;
    if (hipMemcpyAsync(pf->dev, pf->host[k], (size_t)u.byte_count, hipMemcpyHostToDevice, pf->stream) != hipSuccess ||
        hipEventRecord(pf->copied[k], pf->stream) != hipSuccess ||
        launch_widen_f16(static_cast<const uint16_t*>(pf->dev), dst, sh.rows, sh.cols, sh.ld, pf->stream) !=
            hipSuccess) {
      (void)hipStreamSynchronize(pf->stream);
      return PROM_MODEL_BLOCK_DETAIL_QUEUE_SUBMIT_FAILED;
    }
  }
  return hipStreamSynchronize(pf->stream) == hipSuccess ? 0 : PROM_MODEL_BLOCK_DETAIL_COMPLETION_UNCERTAIN;
}


// ---------------------------------------------------------------- main attention route

// The MainTransformer attention route (reactor_sgemm.cpp:1479-1516).  The
// subgroup-owned route is defined on 32-lane subgroups; a CDNA wavefront has
// 64 lanes, so this library admits the serial-canonical route (its shader 41)
// only: AUTO falls back to it with reason SUBGROUP_SIZE and an explicit
// SUBGROUP_OWNED32 request is not admitted.
struct RouteDecision {
  bool admitted;
  uint32_t selected, fallback, shader;
};
constexpr uint32_t kShaderMainAttentionSerial = 41u;

RouteDecision decide_main_route(uint32_t requested) {
  if (requested == PROM_MAIN_ATTENTION_ROUTE_SERIAL_CANONICAL)
    return {true, PROM_MAIN_ATTENTION_ROUTE_SERIAL_CANONICAL, PROM_MAIN_ATTENTION_FALLBACK_NONE,
            kShaderMainAttentionSerial};
  if (requested == PROM_MAIN_ATTENTION_ROUTE_SUBGROUP_OWNED32)
    return {false, 0u, PROM_MAIN_ATTENTION_FALLBACK_SUBGROUP_SIZE, 0u};
  return {true, PROM_MAIN_ATTENTION_ROUTE_SERIAL_CANONICAL, PROM_MAIN_ATTENTION_FALLBACK_SUBGROUP_SIZE,
          kShaderMainAttentionSerial};
}

void reset_main_route(ModelSession* s) {
  s->selected_route = PROM_MAIN_ATTENTION_ROUTE_SERIAL_CANONICAL;
  s->route_fallback = PROM_MAIN_ATTENTION_FALLBACK_NONE;
  s->route_shader = kShaderMainAttentionSerial;
}

// ---------------------------------------------------------------- stage-split NoiseRefiner

bool stage_split_block(const ModelBlock* b) {
  return b->shader_id == kShaderNoise && b->program == kProgNoise && b->binding_valid;
}

// The 64-float attention witness of the workspace's last phase 2 into device
// memory `dst` (stream-ordered).
hipError_t enqueue_witness(ModelBlock* b, bool image_format, float* dst) {
  auto W = [&](int k) { return reinterpret_cast<const float*>(b->ws + b->ws_off[k]); };
  return launch_zimage_attention_witness(W(kZQ), W(kZKt), W(kZV), W(kZO), b->tokens, kHeads,
                                         1.0f / sqrtf((float)(kWidth / kHeads)), image_format, dst, ctx().stream);
}

// reactor_vulkan_model_block.c:1955-2057: BF16 ingress and the pre-attention
// phase; the workspace keeps Q, K, V, the gates and the residual input for M1C.
int m1b_execute(Runtime* rt, uint64_t id, const PrometheusModelBlockM1BExecuteRequest* r,
                PrometheusModelBlockEvidence* ev) {
  if (r == nullptr || r->struct_size != sizeof(*r) || r->model_input_bf16 == nullptr || r->timestep_bf16 == nullptr ||
      r->input_identity == 0 || r->timestep_identity == 0 || r->audit_enabled > 1u ||
      (r->audit_enabled == 0 && r->audit_stage != PROM_MODEL_BLOCK_M1B_AUDIT_NONE) ||
      (r->audit_enabled != 0 && (r->audit_stage < PROM_MODEL_BLOCK_M1B_AUDIT_INGRESS_INPUT ||
                                 r->audit_stage > PROM_MODEL_BLOCK_M1B_AUDIT_POSITIONED_K))) {
    fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_INVALID_REQUEST, ev);
    return PROM_ERROR;
  }
  ModelBlock* b = find_block(rt, id);
  if (b == nullptr) {
    fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_NOT_FOUND, ev);
    return PROM_ERROR;
  }
  auto fail = [&](int32_t d) {
    mark_failure(b, d);
    fill_evidence(b, d, ev);
    return PROM_ERROR;
  };
  if (r->model_input_bytes != (uint64_t)kImageTokens * kWidth * 2)
    return fail(PROM_MODEL_BLOCK_DETAIL_INGRESS_INPUT_SIZE_MISMATCH);
  if (r->timestep_bytes != kZImageConditionWidth * 2) return fail(PROM_MODEL_BLOCK_DETAIL_INGRESS_TIMESTEP_SIZE_MISMATCH);
  if (!stage_split_block(b)) return fail(PROM_MODEL_BLOCK_DETAIL_STALE_OUTPUT);
  if (!reap(b)) return fail(PROM_MODEL_BLOCK_DETAIL_COMPLETION_UNCERTAIN);
  const uint64_t audit_n =
      r->audit_enabled ? audit_elements(PROM_NOISE_REFINER_AUDIT_M1B, r->audit_stage, kImageTokens) : 0;
  if (r->audit_enabled != 0 &&
      (r->audit_output == nullptr || r->audit_element_capacity < audit_n || audit_n * 4 > b->declared_audit))
    return fail(PROM_MODEL_BLOCK_DETAIL_AUDIT_FAILED);
  b->output_valid = false;
  b->audit_valid = false;
  b->resident_input_generation = 0;  // the ingress buffer is also the resident boundary
  const uint64_t t0 = wall_ns();
  hipStream_t st = ctx().stream;
  if (upload_host(b->x_bf16, r->model_input_bf16, (size_t)r->model_input_bytes, st) != hipSuccess ||
      hipMemcpyAsync(b->cond_bf16, r->timestep_bf16, (size_t)r->timestep_bytes, hipMemcpyHostToDevice, st) !=
          hipSuccess ||
      launch_widen_bf16(b->x_bf16, b->x, (size_t)kImageTokens * kWidth, st) != hipSuccess ||
      launch_widen_bf16(b->cond_bf16, b->cond, kZImageConditionWidth, st) != hipSuccess) {
    (void)hipStreamSynchronize(st);
    return fail(PROM_MODEL_BLOCK_DETAIL_INGRESS_DISPATCH_FAILED);
  }
  const int32_t d = run_block(rt, b, b->x, b->out, 1, 1);
  if (d != 0) return fail(d);
  if ((rt->test_flags & PROM_TESTCFG_FAIL_DOWNLOAD) != 0u) return fail(PROM_MODEL_BLOCK_DETAIL_AUDIT_FAILED);
  if (r->audit_enabled != 0) {
    if (!copy_stage(b, PROM_NOISE_REFINER_AUDIT_M1B, r->audit_stage, r->audit_output))
      return fail(PROM_MODEL_BLOCK_DETAIL_AUDIT_FAILED);
    b->audit_valid = true;
  }
  b->output_valid = true;
  b->executions += 1;
  b->last_execution_ns = wall_ns() - t0;
  b->replay_identity = hash_u64(hash_u64(hash_u64(hash_u64(b->plan_identity, r->input_identity), r->timestep_identity),
                                         r->audit_enabled),
                                r->audit_stage);
  b->m1b_prefix = b->replay_identity;
  b->last_detail = 0;
  fill_evidence(b, 0, ev);
  return PROM_OK;
}

// reactor_vulkan_model_block.c:2059-2130: attention, projection and gated
// residual of the matching M1B prefix; one stage to the host with the witness.
int m1c_execute(Runtime* rt, uint64_t id, const PrometheusModelBlockM1CExecuteRequest* r,
                PrometheusModelBlockEvidence* ev) {
  const uint64_t model_n = (uint64_t)kImageTokens * kWidth;
  if (r == nullptr || r->struct_size != sizeof(*r) || r->output == nullptr || r->output_identity == 0 ||
      r->m1b_prefix_replay_identity == 0 || r->output_element_capacity < model_n ||
      r->audit_stage < PROM_MODEL_BLOCK_M1C_AUDIT_ATTENTION || r->audit_stage > PROM_MODEL_BLOCK_M1C_AUDIT_RESIDUAL) {
    fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_INVALID_REQUEST, ev);
    return PROM_ERROR;
  }
  ModelBlock* b = find_block(rt, id);
  if (b == nullptr) {
    fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_NOT_FOUND, ev);
    return PROM_ERROR;
  }
  auto fail = [&](int32_t d) {
    mark_failure(b, d);
    fill_evidence(b, d, ev);
    return PROM_ERROR;
  };
  if (!stage_split_block(b) || b->m1b_prefix != r->m1b_prefix_replay_identity || b->declared_audit < model_n * 4)
    return fail(PROM_MODEL_BLOCK_DETAIL_STALE_OUTPUT);
  if (!reap(b)) return fail(PROM_MODEL_BLOCK_DETAIL_COMPLETION_UNCERTAIN);
  b->output_valid = false;
  b->audit_valid = false;
  b->resident_input_generation = 0;
  const uint64_t t0 = wall_ns();
  const int32_t d = run_block(rt, b, b->x, b->out, 2, 2);
  if (d != 0) return fail(d);
  if ((rt->test_flags & PROM_TESTCFG_FAIL_DOWNLOAD) != 0u) return fail(PROM_MODEL_BLOCK_DETAIL_AUDIT_FAILED);
  float witness[kTransientAuditFloats];
  float* dev_witness = reinterpret_cast<float*>(b->audit_dev + kAuditWitnessOffset);
  if (enqueue_witness(b, true, dev_witness) != hipSuccess ||
      !copy_out(witness, dev_witness, 1, kTransientAuditFloats, kTransientAuditFloats))
    return fail(PROM_MODEL_BLOCK_DETAIL_AUDIT_FAILED);
  // both selected softmax denominators must be finite and positive
  if (witness[30] != 1.0f || witness[62] != 1.0f) return fail(PROM_MODEL_BLOCK_DETAIL_M1C_SOFTMAX_INVALID);
  if (r->transient_audit != nullptr && r->transient_audit_element_capacity >= kTransientAuditFloats)
    memcpy(r->transient_audit, witness, sizeof(witness));
  if (!copy_stage(b, PROM_NOISE_REFINER_AUDIT_M1C, r->audit_stage, r->output))
    return fail(PROM_MODEL_BLOCK_DETAIL_AUDIT_FAILED);
  b->output_valid = true;
  b->executions += 1;
  b->last_execution_ns = wall_ns() - t0;
  b->replay_identity = hash_u64(hash_u64(b->m1b_prefix, r->output_identity), r->audit_stage);
  b->last_detail = 0;
  fill_evidence(b, 0, ev);
  return PROM_OK;
}

// reactor_vulkan_model_block.c:2132-2199: the FFN and final residual of the
// matching M1C; one stage to the host (the final output stays resident).
int m1d_execute(Runtime* rt, uint64_t id, const PrometheusModelBlockM1DExecuteRequest* r,
                PrometheusModelBlockEvidence* ev) {
  const bool hidden = r != nullptr && (r->audit_stage == PROM_MODEL_BLOCK_M1D_AUDIT_W1 ||
                                       r->audit_stage == PROM_MODEL_BLOCK_M1D_AUDIT_W3 ||
                                       r->audit_stage == PROM_MODEL_BLOCK_M1D_AUDIT_GATED_HIDDEN);
  const uint64_t required = (uint64_t)kImageTokens * (hidden ? kFfn : kWidth);
  if (r == nullptr || r->struct_size != sizeof(*r) || r->output == nullptr || r->output_identity == 0 ||
      r->m1c_prefix_replay_identity == 0 || r->output_element_capacity < required ||
      r->audit_stage < PROM_MODEL_BLOCK_M1D_AUDIT_FFN_NORM || r->audit_stage > PROM_MODEL_BLOCK_M1D_AUDIT_FINAL_OUTPUT) {
    fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_INVALID_REQUEST, ev);
    return PROM_ERROR;
  }
  ModelBlock* b = find_block(rt, id);
  if (b == nullptr) {
    fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_NOT_FOUND, ev);
    return PROM_ERROR;
  }
  auto fail = [&](int32_t d) {
    mark_failure(b, d);
    fill_evidence(b, d, ev);
    return PROM_ERROR;
  };
  if (!stage_split_block(b) || b->replay_identity != r->m1c_prefix_replay_identity ||
      b->declared_audit < required * 4)
    return fail(PROM_MODEL_BLOCK_DETAIL_STALE_OUTPUT);
  if (!reap(b)) return fail(PROM_MODEL_BLOCK_DETAIL_COMPLETION_UNCERTAIN);
  b->output_valid = false;
  b->audit_valid = false;
  const uint64_t t0 = wall_ns();
  const int32_t d = run_block(rt, b, b->x, b->out, 3, 3);
  if (d != 0) return fail(d);
  if ((rt->test_flags & PROM_TESTCFG_FAIL_DOWNLOAD) != 0u ||
      !copy_stage(b, PROM_NOISE_REFINER_AUDIT_M1D, r->audit_stage, r->output))
    return fail(PROM_MODEL_BLOCK_DETAIL_AUDIT_FAILED);
  b->output_valid = true;
  b->audit_valid = true;
  b->executions += 1;
  b->last_execution_ns = wall_ns() - t0;
  b->replay_identity = hash_u64(hash_u64(r->m1c_prefix_replay_identity, r->output_identity), r->audit_stage);
  b->last_detail = 0;
  fill_evidence(b, 0, ev);
  return PROM_OK;
}

// ---------------------------------------------------------------- static audits

// Sources of the lock's audit schedules in this library's workspace.  The
// first six recomputed ones are stages the chain does not keep: the norms
// before modulation and the head norms with and without RoPE.
enum AuditSource : uint8_t {
  kAsAttnNorm, kAsQNorm, kAsKNorm, kAsQRope, kAsKRope, kAsFfnNorm,
  kAsInput, kAsModRaw, kAsMod, kAsA, kAsQkv, kAsQ, kAsK, kAsV, kAsO, kAsProj, kAsR, kAsF, kAsW1, kAsW3, kAsGated,
  kAsW2, kAsOut
};
bool recomputed(uint8_t s) { return s <= kAsFfnNorm; }

// Projection keys of a stage, by the shape of its view (N = T * 3840, NH =
// T * 10240): a row view takes {0, N-1, N/2, 3839}, a head view {0, N-1, N/2,
// 127, 128}, a rotated head view adds the pair boundary {63, 64}, the fused
// QKV {0, 3N-1, 3N/2, N-1, N, 2N}, the FFN hidden {0, NH-1, NH/2, 10239}; the
// NoiseRefiner schedule adds the first element of the last row (and 2N-1 to
// the fused QKV).  These are the projection keys of the lock's generated
// schedule (resolved_audit_schedule.h:14-30, 71-81).
enum AuditKeys : uint8_t { kKeysNone, kKeysRow, kKeysHead, kKeysRope, kKeysFused, kKeysHidden };

uint32_t audit_keys(uint8_t kind, uint32_t T, bool tail, uint32_t* k) {
  const uint32_t D = kWidth, N = T * kWidth, NH = T * kFfn;
  uint32_t n = 0;
  switch (kind) {
    case kKeysRow:
      for (uint32_t v : {0u, N - 1, N / 2, D - 1}) k[n++] = v;
      if (tail) k[n++] = N - D;
      break;
    case kKeysHead:
    case kKeysRope:
      for (uint32_t v : {0u, N - 1, N / 2}) k[n++] = v;
      if (kind == kKeysRope) k[n++] = 63u, k[n++] = 64u;
      k[n++] = 127u;
      k[n++] = 128u;
      if (tail) k[n++] = N - D;
      break;
    case kKeysFused:
      for (uint32_t v : {0u, 3 * N - 1, 3 * N / 2, N - 1, N}) k[n++] = v;
      if (tail) k[n++] = 2 * N - 1;
      k[n++] = 2 * N;
      break;
    case kKeysHidden:
      for (uint32_t v : {0u, NH - 1, NH / 2, (uint32_t)kFfn - 1}) k[n++] = v;
      if (tail) k[n++] = NH - kFfn;
      break;
    default:
      break;
  }
  return n;
}

// One stage of a schedule: a full copy of `count` elements of the source from
// `base`, or a 256-byte summary record, at byte `dest` of the arena.
struct AuditStage {
  uint8_t stage, source, keys;
  uint32_t dest;
  bool full;
  uint32_t base, count;
};

// resolved_audit_schedule.h:20-50 (NoiseRefiner, witness at 189440; the
// schedule's resource of each stage in the comment).
const AuditStage kNoiseAudit[29] = {
    {1, kAsModRaw, kKeysNone, 0, true, 0, 4 * kWidth},            // ADALN: timestep_linear
    {2, kAsModRaw, kKeysNone, 61440, true, 0, kWidth},            // ADALN: attention_scale_raw
    {3, kAsMod, kKeysNone, 76800, true, 0, kWidth},               // ATTENTION_SCALE
    {4, kAsModRaw, kKeysNone, 92160, true, kWidth, kWidth},       // ADALN: attention_gate_raw
    {5, kAsMod, kKeysNone, 107520, true, kWidth, kWidth},         // ATTENTION_GATE (tanh)
    {6, kAsModRaw, kKeysNone, 122880, true, 2 * kWidth, kWidth},  // ADALN: mlp_scale_raw
    {7, kAsMod, kKeysNone, 138240, true, 2 * kWidth, kWidth},     // MLP_SCALE
    {8, kAsModRaw, kKeysNone, 153600, true, 3 * kWidth, kWidth},  // ADALN: mlp_gate_raw
    {9, kAsMod, kKeysNone, 168960, true, 3 * kWidth, kWidth},     // MLP_GATE (tanh)
    {10, kAsAttnNorm, kKeysRow, 184320, false, 0, 0},             // NORM: attention_norm
    {11, kAsA, kKeysRow, 184576, false, 0, 0},                    // MODULATED
    {12, kAsQkv, kKeysFused, 184832, false, 0, 0},                // QKV
    {13, kAsQ, kKeysHead, 185088, false, 0, 0},                   // QKV: q
    {14, kAsK, kKeysHead, 185344, false, 0, 0},                   // QKV: k
    {15, kAsV, kKeysHead, 185600, false, 0, 0},                   // QKV: v
    {16, kAsQNorm, kKeysHead, 185856, false, 0, 0},               // NORM: q_norm
    {17, kAsKNorm, kKeysHead, 186112, false, 0, 0},               // NORM: k_norm
    {18, kAsQRope, kKeysRope, 186368, false, 0, 0},               // QKV: q_rope
    {19, kAsKRope, kKeysRope, 186624, false, 0, 0},               // QKV: k_rope
    {20, kAsO, kKeysHead, 186880, false, 0, 0},                   // ATTENTION: aggregation
    {21, kAsProj, kKeysRow, 187136, false, 0, 0},                 // ATTENTION_PROJECTION
    {22, kAsR, kKeysRow, 187392, false, 0, 0},                    // ATTENTION_RESIDUAL
    {23, kAsFfnNorm, kKeysRow, 187648, false, 0, 0},              // NORM: ffn_norm
    {24, kAsF, kKeysRow, 187904, false, 0, 0},                    // MODULATED: ffn_modulated
    {25, kAsW1, kKeysHidden, 188160, false, 0, 0},                // w1
    {26, kAsW3, kKeysHidden, 188416, false, 0, 0},                // w3
    {27, kAsGated, kKeysHidden, 188672, false, 0, 0},             // ffn_gated_hidden
    {28, kAsW2, kKeysRow, 188928, false, 0, 0},                   // w2
    {29, kAsOut, kKeysRow, 189184, false, 0, 0}};                 // final_output

// resolved_audit_schedule.h:84-101 (ContextRefiner, witness at 4096; with no
// adaLN its ffn_norm stage is the FFN input).
const AuditStage kContextAudit[16] = {
    {1, kAsInput, kKeysRow, 0, false, 0, 0},        {2, kAsAttnNorm, kKeysRow, 256, false, 0, 0},
    {3, kAsQkv, kKeysFused, 512, false, 0, 0},      {4, kAsQNorm, kKeysHead, 768, false, 0, 0},
    {5, kAsKNorm, kKeysHead, 1024, false, 0, 0},    {6, kAsQRope, kKeysRope, 1280, false, 0, 0},
    {7, kAsKRope, kKeysRope, 1536, false, 0, 0},    {8, kAsO, kKeysHead, 1792, false, 0, 0},
    {9, kAsProj, kKeysRow, 2048, false, 0, 0},      {10, kAsR, kKeysRow, 2304, false, 0, 0},
    {11, kAsF, kKeysRow, 2560, false, 0, 0},        {12, kAsW1, kKeysHidden, 2816, false, 0, 0},
    {13, kAsW3, kKeysHidden, 3072, false, 0, 0},    {14, kAsGated, kKeysHidden, 3328, false, 0, 0},
    {15, kAsW2, kKeysRow, 3584, false, 0, 0},       {16, kAsOut, kKeysRow, 3840, false, 0, 0}};

struct AuditView {
  const float* src;
  uint32_t count, cols, ld;  // v[e] = src[(e / cols) * ld + e % cols]
};

AuditView view_of(const ModelBlock* b, uint8_t source, const float* scratch) {
  const uint32_t T = (uint32_t)b->tokens, D = kWidth, F = kFfn;
  auto W = [&](int k) { return reinterpret_cast<const float*>(b->ws + b->ws_off[k]); };
  switch (source) {
    case kAsInput: return {b->x, T * D, D, D};
    case kAsModRaw: return {W(kZModRaw), 4 * D, 4 * D, 4 * D};
    case kAsMod: return {W(kZMod), 4 * D, 4 * D, 4 * D};
    case kAsA: return {W(kZA), T * D, D, D};
    case kAsQkv: return {W(kZQkv), 3 * T * D, 3 * D, 3 * D};
    case kAsQ: case kAsK: case kAsV: return {W(kZQkv) + (source - kAsQ) * D, T * D, D, 3 * D};
    case kAsO: return {W(kZO), T * D, D, D};
    case kAsProj: return {W(kZProj), T * D, D, D};
    case kAsR: return {W(kZR), T * D, D, D};
    case kAsF: return {W(kZF), T * D, D, D};
    case kAsW1: return {W(kZG), T * F, F, 2 * F};
    case kAsW3: return {W(kZG) + F, T * F, F, 2 * F};
    case kAsGated: return {W(kZH), T * F, F, F};
    case kAsW2: return {W(kZW2), T * D, D, D};
    case kAsOut: return {b->out, T * D, D, D};
    default: return {scratch, T * D, D, D};  // recomputed into the scratch
  }
}

hipError_t recompute(ModelBlock* b, uint8_t source, float* scratch) {
  hipStream_t st = ctx().stream;
  const ZImageBlockWeights w = weights_of(b);
  const float* qkv = reinterpret_cast<const float*>(b->ws + b->ws_off[kZQkv]);
  const float* R = reinterpret_cast<const float*>(b->ws + b->ws_off[kZR]);
  const float2* tab = reinterpret_cast<const float2*>(b->ws + b->ws_off[kZRope]);
  const int T = b->tokens;
  switch (source) {
    case kAsAttnNorm: return launch_zimage_norm(b->x, w.attn_norm1, scratch, T, kWidth, kEps, st);
    case kAsFfnNorm: return launch_zimage_norm(R, w.ffn_norm1, scratch, T, kWidth, kEps, st);
    case kAsQNorm: return launch_zimage_qk_audit(qkv, tab, w.q_norm, scratch, T, kHeads, kEps, 0, false, st);
    case kAsKNorm: return launch_zimage_qk_audit(qkv, tab, w.k_norm, scratch, T, kHeads, kEps, 1, false, st);
    case kAsQRope: return launch_zimage_qk_audit(qkv, tab, w.q_norm, scratch, T, kHeads, kEps, 0, true, st);
    case kAsKRope: return launch_zimage_qk_audit(qkv, tab, w.k_norm, scratch, T, kHeads, kEps, 1, true, st);
    default: return hipSuccess;
  }
}

// Fills the device records of one schedule from the completed chain: the full
// copies, one summary launch over the stages the workspace keeps, then each
// recomputed stage (recompute into the scratch, summarise), and the attention
// witness at byte `witness_offset`.  Stream-ordered.
bool record_schedule(ModelBlock* b, const AuditStage* sched, uint32_t n, bool tail, uint32_t generation,
                     uint32_t witness_offset, bool image_format) {
  hipStream_t st = ctx().stream;
  char* dev = b->audit_dev;
  float* scratch = reinterpret_cast<float*>(dev + kAuditScratchOffset);
  ZImageAuditJob* djobs = reinterpret_cast<ZImageAuditJob*>(dev + kAuditJobOffset);
  ZImageAuditJob jobs[kAuditMaxJobs];
  uint8_t later_source[kAuditMaxJobs];
  memset(jobs, 0, sizeof(jobs));
  uint32_t live = 0, later = 0;  // live jobs fill the table from the front, recomputed ones from the back
  if (hipMemsetAsync(dev, 0, kAuditRecordBytes, st) != hipSuccess) return false;
  for (uint32_t i = 0; i < n; ++i) {
    const AuditStage& a = sched[i];
    const AuditView v = view_of(b, a.source, scratch);
    if (a.full) {
      if (a.base + a.count > v.count ||
          hipMemcpyAsync(dev + a.dest, v.src + a.base, (size_t)a.count * 4, hipMemcpyDeviceToDevice, st) != hipSuccess)
        return false;
      continue;
    }
    if (live + later >= kAuditMaxJobs || a.dest + 256u > kAuditRecordBytes) return false;
    const uint32_t slot = recomputed(a.source) ? kAuditMaxJobs - 1 - later : live;
    ZImageAuditJob& j = jobs[slot];
    j.src = v.src;
    j.count = v.count;
    j.cols = v.cols;
    j.ld = v.ld;
    j.stage_id = a.stage;
    j.generation = generation;
    j.dest_word = a.dest / 4;
    j.key_count = audit_keys(a.keys, (uint32_t)b->tokens, tail, j.keys);
    if (recomputed(a.source)) later_source[later++] = a.source;
    else ++live;
  }
  // the table is read by the launches below; the copy completes before the host array goes away
  if (hipMemcpyAsync(djobs, jobs, sizeof(jobs), hipMemcpyHostToDevice, st) != hipSuccess ||
      hipStreamSynchronize(st) != hipSuccess ||
      launch_zimage_audit_summary(djobs, live, reinterpret_cast<uint32_t*>(dev), st) != hipSuccess)
    return false;
  for (uint32_t r = 0; r < later; ++r) {
    if (recompute(b, later_source[r], scratch) != hipSuccess ||
        launch_zimage_audit_summary(djobs + (kAuditMaxJobs - 1 - r), 1, reinterpret_cast<uint32_t*>(dev), st) !=
            hipSuccess)
      return false;
  }
  return enqueue_witness(b, image_format, reinterpret_cast<float*>(dev + witness_offset)) == hipSuccess;
}

// Copies `bytes` of device memory into the caller's arena after zeroing its
// bytes [bytes, clear_to).
bool arena_out(void* arena, uint64_t clear_to, const void* src, uint64_t bytes) {
  if (clear_to > bytes) memset(static_cast<char*>(arena) + bytes, 0, (size_t)(clear_to - bytes));
  return hipMemcpyAsync(arena, src, (size_t)bytes, hipMemcpyDeviceToHost, ctx().stream) == hipSuccess &&
         hipStreamSynchronize(ctx().stream) == hipSuccess;
}

// reactor_vulkan_model_block.c:3212-3272: one resident NoiseRefiner 1
// execution (first-resident rules as execute_resident) with the arena.
int noise_static_audit(Runtime* rt, uint64_t id, const PrometheusNoiseRefinerStaticAuditRequest* r,
                       PrometheusModelBlockEvidence* ev) {
  if (r == nullptr || r->struct_size != sizeof(*r) || r->lock_identity != PROM_ZIMAGE_TURBO_AUDIT_LOCK_ID ||
      r->input_generation == 0 || r->output_identity == 0 || r->audit_arena == nullptr ||
      r->audit_arena_capacity_bytes < PROM_ZIMAGE_TURBO_AUDIT_ARENA_BYTES) {
    fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_INVALID_REQUEST, ev);
    return PROM_ERROR;
  }
  ModelBlock* b = find_block(rt, id);
  if (b == nullptr) {
    fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_NOT_FOUND, ev);
    return PROM_ERROR;
  }
  auto fail = [&](int32_t d) {
    mark_failure(b, d);
    fill_evidence(b, d, ev);
    return PROM_ERROR;
  };
  const bool first = b->resident_input_generation == 0;
  if (b->program != kProgNoise || b->family != PROM_NOISE_REFINER_FAMILY_Z_IMAGE_TURBO ||
      b->parameter_set != PROM_NOISE_REFINER_PARAMETER_SET_1 || binding_state(b) != PROM_NOISE_REFINER_BINDING_BOUND ||
      (first ? r->input_generation != b->output_generation : r->input_generation != b->resident_input_generation) ||
      !reap(b) || b->declared_audit != PROM_ZIMAGE_TURBO_AUDIT_ARENA_BYTES)
    return fail(PROM_MODEL_BLOCK_DETAIL_STALE_OUTPUT);
  const uint32_t generation = (uint32_t)(b->output_generation + 1u);
  if (generation == 0u) {
    fill_evidence(b, PROM_MODEL_BLOCK_DETAIL_INVALID_REQUEST, ev);
    return PROM_ERROR;
  }
  b->output_valid = false;
  b->audit_valid = false;
  const uint64_t t0 = wall_ns();
  hipStream_t st = ctx().stream;
  if (first && hipMemcpyAsync(b->x, b->out, (size_t)kImageTokens * kWidth * 4, hipMemcpyDeviceToDevice, st) !=
                   hipSuccess)
    return fail(PROM_MODEL_BLOCK_DETAIL_QUEUE_SUBMIT_FAILED);
  const int32_t d = run_block(rt, b, b->x, b->out);
  if (d != 0) return fail(d);
  if (!record_schedule(b, kNoiseAudit, 29, true, generation, PROM_ZIMAGE_TURBO_AUDIT_TRANSIENT_ATTENTION_OFFSET,
                       true) ||
      !arena_out(r->audit_arena, PROM_ZIMAGE_TURBO_AUDIT_ARENA_BYTES, b->audit_dev,
                 PROM_ZIMAGE_TURBO_AUDIT_REQUIRED_BYTES))
    return fail(PROM_MODEL_BLOCK_DETAIL_AUDIT_FAILED);
  if (first) b->resident_input_generation = r->input_generation;
  b->output_valid = true;
  b->audit_valid = true;
  b->output_generation = generation;
  b->executions += 1;
  b->last_execution_ns = wall_ns() - t0;
  b->replay_identity = hash_u64(hash_u64(PROM_ZIMAGE_TURBO_AUDIT_LOCK_ID, r->output_identity), generation);
  b->last_detail = 0;
  fill_evidence(b, 0, ev);
  return PROM_OK;
}

// reactor_vulkan_model_block.c:2671-2735: parameter set 0 re-runs the
// external input, set 1 the resident boundary, with the ContextRefiner arena.
int context_static_audit(Runtime* rt, uint64_t id, const PrometheusContextRefinerStaticAuditRequest* r,
                         PrometheusModelBlockEvidence* ev) {
  if (r == nullptr || r->struct_size != sizeof(*r) || r->lock_identity != PROM_ZIMAGE_TURBO_AUDIT_LOCK_ID ||
      r->input_generation == 0 || r->output_identity == 0 || r->audit_arena == nullptr ||
      r->audit_arena_capacity_bytes < PROM_ZIMAGE_TURBO_CONTEXT_AUDIT_ARENA_BYTES) {
    fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_INVALID_REQUEST, ev);
    return PROM_ERROR;
  }
  ModelBlock* b = find_block(rt, id);
  if (b == nullptr) {
    fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_NOT_FOUND, ev);
    return PROM_ERROR;
  }
  auto fail = [&](int32_t d) {
    mark_failure(b, d);
    fill_evidence(b, d, ev);
    return PROM_ERROR;
  };
  const bool set1 = b->parameter_set == PROM_CONTEXT_REFINER_PARAMETER_SET_1;
  const bool first = set1 && b->resident_input_generation == 0;
  if (b->program != kProgContext || binding_state(b) != PROM_NOISE_REFINER_BINDING_BOUND ||
      (!set1 && r->input_generation != b->output_generation) ||
      (set1 && (first ? r->input_generation != b->output_generation
                      : r->input_generation != b->resident_input_generation)) ||
      !reap(b))
    return fail(PROM_MODEL_BLOCK_DETAIL_STALE_OUTPUT);
  const uint32_t generation = (uint32_t)(b->output_generation + 1u);
  if (generation == 0u) {
    fill_evidence(b, PROM_MODEL_BLOCK_DETAIL_INVALID_REQUEST, ev);
    return PROM_ERROR;
  }
  b->output_valid = false;
  b->audit_valid = false;
  const uint64_t t0 = wall_ns();
  hipStream_t st = ctx().stream;
  if (first && hipMemcpyAsync(b->x, b->out, (size_t)kContextTokens * kWidth * 4, hipMemcpyDeviceToDevice, st) !=
                   hipSuccess)
    return fail(PROM_MODEL_BLOCK_DETAIL_QUEUE_SUBMIT_FAILED);
  const int32_t d = run_block(rt, b, b->x, b->out);
  if (d != 0) return fail(d);
  if (!record_schedule(b, kContextAudit, 16, false, generation,
                       PROM_ZIMAGE_TURBO_CONTEXT_AUDIT_TRANSIENT_ATTENTION_OFFSET, false) ||
      !arena_out(r->audit_arena, r->audit_arena_capacity_bytes, b->audit_dev,
                 PROM_ZIMAGE_TURBO_CONTEXT_AUDIT_REQUIRED_BYTES))
    return fail(PROM_MODEL_BLOCK_DETAIL_AUDIT_FAILED);
  b->output_valid = true;
  b->audit_valid = true;
  if (first) b->resident_input_generation = r->input_generation;
  b->output_generation = generation;
  b->executions += 1;
  b->last_execution_ns = wall_ns() - t0;
  b->replay_identity = hash_u64(b->replay_identity, r->output_identity);
  b->last_detail = 0;
  fill_evidence(b, 0, ev);
  return PROM_OK;
}

// reactor_vulkan_model_block.c:4020-4131: MainTransformer layer 0 re-run on
// the session's JointWorking stream with the timestep it last took; the
// session is not advanced and the arena receives the [1056, 3840] output.
int main_static_audit(Runtime* rt, uint64_t id, const PrometheusMainTransformerStaticAuditRequest* r,
                      PrometheusModelBlockEvidence* ev) {
  const uint64_t out_bytes = (uint64_t)kJointTokens * kWidth * 4;
  if (r == nullptr || r->struct_size != sizeof(*r) || r->lock_identity != PROM_ZIMAGE_TURBO_AUDIT_LOCK_ID ||
      r->model_local_block_id != 0u || r->session_identity == 0 || r->required_image_generation == 0 ||
      r->required_context_generation == 0 || r->required_joint_generation == 0 || r->output_identity == 0 ||
      r->audit_arena == nullptr || r->audit_arena_capacity_bytes < out_bytes) {
    fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_INVALID_REQUEST, ev);
    return PROM_ERROR;
  }
  ModelBlock* b = find_block(rt, id);
  if (b == nullptr) {
    fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_NOT_FOUND, ev);
    return PROM_ERROR;
  }
  if (!reap(b)) {
    fill_evidence(b, PROM_MODEL_BLOCK_DETAIL_COMPLETION_UNCERTAIN, ev);
    return PROM_ERROR;
  }
  auto fail = [&](int32_t d) {
    mark_failure(b, d);
    fill_evidence(b, d, ev);
    return PROM_ERROR;
  };
  const ModelSession* s = &rt->model->session;
  if (b->program != kProgMain || b->parameter_set != 1u || b->aggregate != kMainAggregate[0] ||
      binding_state(b) != PROM_NOISE_REFINER_BINDING_BOUND || !s->created || s->id != r->session_identity ||
      s->lock != r->lock_identity || !joint_valid(s) || s->streams[0].generation != r->required_image_generation ||
      s->streams[1].generation != r->required_context_generation ||
      s->streams[2].generation != r->required_joint_generation)
    return fail(PROM_MODEL_BLOCK_DETAIL_STALE_OUTPUT);
  b->output_valid = false;
  b->audit_valid = false;
  const uint64_t t0 = wall_ns();
  const int32_t d = run_block(rt, b, s->buf[2], b->out);
  if (d != 0) return fail(d);
  if (!arena_out(r->audit_arena, r->audit_arena_capacity_bytes, b->out, out_bytes))
    return fail(PROM_MODEL_BLOCK_DETAIL_AUDIT_FAILED);
  b->output_valid = true;
  b->audit_valid = true;
  b->output_generation += 1;
  b->executions += 1;
  b->last_execution_ns = wall_ns() - t0;
  b->replay_identity = hash_u64(b->replay_identity, r->output_identity);
  b->last_detail = 0;
  fill_evidence(b, 0, ev);
  return PROM_OK;
}

}  // namespace

void model_release(Runtime* rt) {
  if (rt == nullptr || rt->model == nullptr) return;
  std::lock_guard<std::mutex> lock(ctx().mu);
  release_block(&rt->model->block);
  release_session(&rt->model->session);
  delete rt->model;
  rt->model = nullptr;
}

}  // namespace prom

using namespace prom;

namespace {

// Runs `body` with the device context locked and the handle resolved; an
// unknown handle reports the invalid-request evidence.
template <typename F>
int with_runtime(void* handle, PrometheusModelBlockEvidence* ev, F body) {
  Runtime* rt = lookup(handle);
  if (rt == nullptr) {
    fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_INVALID_REQUEST, ev);
    return PROM_ERROR;
  }
  std::lock_guard<std::mutex> lock(ctx().mu);
  return body(rt);
}

template <typename F>
int with_session_runtime(void* handle, PrometheusCompiledModelSessionEvidence* ev, F body) {
  Runtime* rt = lookup(handle);
  if (rt == nullptr) {
    fill_session_evidence(nullptr, ev, PROM_MODEL_SESSION_DETAIL_INVALID_REQUEST);
    return PROM_ERROR;
  }
  std::lock_guard<std::mutex> lock(ctx().mu);
  return body(rt);
}

}  // namespace

extern "C" {

PROM_REACTOR_API int prometheus_reactor_runtime_model_block_create(void* handle,
                                                                   const PrometheusModelBlockCreateRequest* request,
                                                                   uint64_t* out_block_id,
                                                                   PrometheusModelBlockEvidence* out_evidence) {
  if (out_block_id) *out_block_id = 0;
  return with_runtime(handle, out_evidence,
                      [&](Runtime* rt) -> int { return create_block(rt, request, out_block_id, out_evidence); });
}

PROM_REACTOR_API int prometheus_reactor_runtime_model_block_upload_weights(
    void* handle, uint64_t block_id, const PrometheusModelBlockWeightUpload* uploads, uint32_t upload_count,
    PrometheusModelBlockEvidence* out_evidence) {
  return with_runtime(handle, out_evidence, [&](Runtime* rt) -> int {
    return upload_weights(rt, block_id, uploads, upload_count, out_evidence);
  });
}

// reactor_vulkan_model_block.c:1884-1953: the resident proof program.
PROM_REACTOR_API int prometheus_reactor_runtime_model_block_execute(void* handle, uint64_t block_id,
                                                                    const PrometheusModelBlockExecuteRequest* request,
                                                                    PrometheusModelBlockEvidence* out_evidence) {
  return with_runtime(handle, out_evidence, [&](Runtime* rt) -> int {
    const PrometheusModelBlockExecuteRequest* r = request;
    if (r == nullptr || r->struct_size != sizeof(*r) || r->input == nullptr || r->output == nullptr ||
        r->input_identity == 0 || r->audit_enabled > 1u || r->element_count == 0 ||
        r->element_count > UINT64_MAX / 4) {
      fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_INVALID_REQUEST, out_evidence);
      return PROM_ERROR;
    }
    ModelBlock* b = find_block(rt, block_id);
    if (b == nullptr) {
      fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_NOT_FOUND, out_evidence);
      return PROM_ERROR;
    }
    const uint64_t bytes = r->element_count * 4;
    if (b->program != kProgProof || !b->binding_valid || bytes != b->ext_in || bytes != b->ext_out ||
        r->element_count > 4194304u) {
      mark_failure(b, PROM_MODEL_BLOCK_DETAIL_STALE_OUTPUT);
      fill_evidence(b, b->last_detail, out_evidence);
      return PROM_ERROR;
    }
    if (!reap(b)) {
      mark_failure(b, PROM_MODEL_BLOCK_DETAIL_COMPLETION_UNCERTAIN);
      fill_evidence(b, b->last_detail, out_evidence);
      return PROM_ERROR;
    }
    const uint64_t audit_n = b->declared_audit / 4;
    if (r->audit_enabled && (r->audit_output == nullptr || r->audit_element_capacity * 4 < b->declared_audit)) {
      mark_failure(b, PROM_MODEL_BLOCK_DETAIL_AUDIT_FAILED);
      fill_evidence(b, b->last_detail, out_evidence);
      return PROM_ERROR;
    }
    b->output_valid = false;
    b->audit_valid = false;
    const uint64_t t0 = wall_ns();
    bool unobserved = false;
    const int32_t fault = take_phase_fault(rt, &unobserved);
    if (fault != 0) {
      mark_failure(b, fault);
      fill_evidence(b, fault, out_evidence);
      return PROM_ERROR;
    }
    hipStream_t st = ctx().stream;
    (void)hipEventRecord(b->ev_begin, st);
    hipError_t e = upload_host(b->proof_in, r->input, (size_t)bytes, st);
    if (e == hipSuccess) {
      const unsigned blocks = (unsigned)std::min<uint64_t>(4096, (r->element_count + 255) / 256);
      hipLaunchKernelGGL(proof_kernel, dim3(blocks), dim3(256), 0, st, b->proof_in, b->proof_out, r->element_count,
                         b->proof_audit, r->audit_enabled ? std::min(audit_n, r->element_count) : 0ull);
      e = hipGetLastError();
    }
    (void)hipEventRecord(b->ev_end, st);
    if (e != hipSuccess) {
      (void)hipStreamSynchronize(st);
      mark_failure(b, PROM_MODEL_BLOCK_DETAIL_QUEUE_SUBMIT_FAILED);
      fill_evidence(b, b->last_detail, out_evidence);
      return PROM_ERROR;
    }
    if (unobserved) {
      b->quarantined = true;
      mark_failure(b, PROM_MODEL_BLOCK_DETAIL_COMPLETION_UNCERTAIN);
      fill_evidence(b, b->last_detail, out_evidence);
      return PROM_ERROR;
    }
    if ((rt->test_flags & PROM_TESTCFG_FAIL_DOWNLOAD) != 0u) {
      (void)hipStreamSynchronize(st);
      mark_failure(b, PROM_MODEL_BLOCK_DETAIL_AUDIT_FAILED);
      fill_evidence(b, b->last_detail, out_evidence);
      return PROM_ERROR;
    }
    e = download_host(r->output, b->proof_out, (size_t)b->ext_out, st);
    if (e == hipSuccess && r->audit_enabled)
      e = hipMemcpyAsync(r->audit_output, b->proof_audit, (size_t)b->declared_audit, hipMemcpyDeviceToHost, st);
    if (e != hipSuccess || hipStreamSynchronize(st) != hipSuccess) {
      mark_failure(b, PROM_MODEL_BLOCK_DETAIL_AUDIT_FAILED);
      fill_evidence(b, b->last_detail, out_evidence);
      return PROM_ERROR;
    }
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, b->ev_begin, b->ev_end) == hipSuccess) b->gpu_compute_ns = (uint64_t)(ms * 1.0e6);
    b->gpu_total_ns = b->gpu_compute_ns;
    b->output_valid = true;
    b->audit_valid = r->audit_enabled != 0;
    b->executions += 1;
    b->last_execution_ns = wall_ns() - t0;
    b->replay_identity = hash_u64(hash_u64(b->plan_identity, r->input_identity), r->audit_enabled);
    b->last_detail = 0;
    fill_evidence(b, 0, out_evidence);
    return PROM_OK;
  });
}

PROM_REACTOR_API int prometheus_reactor_runtime_model_block_execute_m1b(
    void* handle, uint64_t block_id, const PrometheusModelBlockM1BExecuteRequest* request,
    PrometheusModelBlockEvidence* out_evidence) {
  return with_runtime(handle, out_evidence,
                      [&](Runtime* rt) -> int { return m1b_execute(rt, block_id, request, out_evidence); });
}

PROM_REACTOR_API int prometheus_reactor_runtime_model_block_execute_m1c(
    void* handle, uint64_t block_id, const PrometheusModelBlockM1CExecuteRequest* request,
    PrometheusModelBlockEvidence* out_evidence) {
  return with_runtime(handle, out_evidence,
                      [&](Runtime* rt) -> int { return m1c_execute(rt, block_id, request, out_evidence); });
}

PROM_REACTOR_API int prometheus_reactor_runtime_model_block_execute_m1d(
    void* handle, uint64_t block_id, const PrometheusModelBlockM1DExecuteRequest* request,
    PrometheusModelBlockEvidence* out_evidence) {
  return with_runtime(handle, out_evidence,
                      [&](Runtime* rt) -> int { return m1d_execute(rt, block_id, request, out_evidence); });
}

PROM_REACTOR_API int prometheus_reactor_runtime_noise_refiner0_execute(
    void* handle, uint64_t block_id, const PrometheusNoiseRefiner0ExecuteRequest* request,
    PrometheusModelBlockEvidence* out_evidence) {
  return with_runtime(handle, out_evidence, [&](Runtime* rt) -> int {
    return noise_external(rt, block_id, request, PROM_NOISE_REFINER_PARAMETER_SET_0, out_evidence);
  });
}

PROM_REACTOR_API int prometheus_reactor_runtime_noise_refiner1_execute(
    void* handle, uint64_t block_id, const PrometheusNoiseRefiner1ExecuteRequest* request,
    PrometheusModelBlockEvidence* out_evidence) {
  return with_runtime(handle, out_evidence, [&](Runtime* rt) -> int {
    return noise_external(rt, block_id, request, PROM_NOISE_REFINER_PARAMETER_SET_1, out_evidence);
  });
}

// reactor_vulkan_model_block.c:1831-1882
PROM_REACTOR_API int prometheus_reactor_runtime_noise_refiner_rebind(void* handle, uint64_t block_id,
                                                                     const PrometheusNoiseRefinerRebindRequest* request,
                                                                     PrometheusModelBlockEvidence* out_evidence) {
  return with_runtime(handle, out_evidence, [&](Runtime* rt) -> int {
    const PrometheusNoiseRefinerRebindRequest* r = request;
    if (r == nullptr || r->struct_size != sizeof(*r) || r->uploads == nullptr || r->upload_count != 13u ||
        r->lock_identity != PROM_ZIMAGE_TURBO_LOCK_ID || r->model_local_block_id != 1u) {
      fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_INVALID_REQUEST, out_evidence);
      return PROM_ERROR;
    }
    ModelBlock* b = find_block(rt, block_id);
    if (b == nullptr) {
      fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_NOT_FOUND, out_evidence);
      return PROM_ERROR;
    }
    if (b->family != PROM_NOISE_REFINER_FAMILY_Z_IMAGE_TURBO || b->parameter_set != PROM_NOISE_REFINER_PARAMETER_SET_0 ||
        !b->binding_valid) {
      fill_evidence(b, PROM_MODEL_BLOCK_DETAIL_REBIND_FAILED, out_evidence);
      return PROM_ERROR;
    }
    return rebind(rt, block_id, b, r->uploads, 13u, kNoiseWeightBytes, PROM_NOISE_REFINER_PARAMETER_SET_1,
                  kNoiseAggregate[1], out_evidence);
  });
}

PROM_REACTOR_API int prometheus_reactor_runtime_noise_refiner_execute_resident(
    void* handle, uint64_t block_id, const PrometheusNoiseRefinerResidentExecuteRequest* request,
    PrometheusModelBlockEvidence* out_evidence) {
  return with_runtime(handle, out_evidence,
                      [&](Runtime* rt) -> int { return noise_resident(rt, block_id, request, out_evidence); });
}

PROM_REACTOR_API int prometheus_reactor_runtime_noise_refiner_execute_static_audit(
    void* handle, uint64_t block_id, const PrometheusNoiseRefinerStaticAuditRequest* request,
    PrometheusModelBlockEvidence* out_evidence) {
  return with_runtime(handle, out_evidence,
                      [&](Runtime* rt) -> int { return noise_static_audit(rt, block_id, request, out_evidence); });
}

PROM_REACTOR_API int prometheus_reactor_runtime_noise_refiner_audit_final(
    void* handle, uint64_t block_id, const PrometheusNoiseRefinerFinalAuditRequest* request,
    PrometheusModelBlockEvidence* out_evidence) {
  return with_runtime(handle, out_evidence,
                      [&](Runtime* rt) -> int { return audit_final(rt, block_id, request, kProgNoise, out_evidence); });
}

// reactor_vulkan_model_block.c:2305-2367
PROM_REACTOR_API int prometheus_reactor_runtime_context_refiner_create(
    void* handle, const PrometheusContextRefinerCreateRequest* request, uint64_t* out_block_id,
    PrometheusModelBlockEvidence* out_evidence) {
  if (out_block_id) *out_block_id = 0;
  return with_runtime(handle, out_evidence, [&](Runtime* rt) -> int {
    const PrometheusContextRefinerCreateRequest* r = request;
    if (r == nullptr || out_block_id == nullptr || r->struct_size != sizeof(*r) || r->uploads == nullptr ||
        r->upload_count != 11u || r->lock_identity != PROM_ZIMAGE_TURBO_LOCK_ID || r->model_local_block_id != 0u) {
      fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_INVALID_REQUEST, out_evidence);
      return PROM_ERROR;
    }
    return facade_create(rt, r, out_block_id, out_evidence, false);
  });
}

// reactor_vulkan_model_block.c:2464-2508
PROM_REACTOR_API int prometheus_reactor_runtime_context_refiner_rebind(
    void* handle, uint64_t block_id, const PrometheusContextRefinerRebindRequest* request,
    PrometheusModelBlockEvidence* out_evidence) {
  return with_runtime(handle, out_evidence, [&](Runtime* rt) -> int {
    const PrometheusContextRefinerRebindRequest* r = request;
    if (r == nullptr || r->uploads == nullptr || r->struct_size != sizeof(*r) || r->upload_count != 11u ||
        r->lock_identity != PROM_ZIMAGE_TURBO_LOCK_ID || r->model_local_block_id != 1u) {
      fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_INVALID_REQUEST, out_evidence);
      return PROM_ERROR;
    }
    ModelBlock* b = find_block(rt, block_id);
    if (b == nullptr) {
      fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_NOT_FOUND, out_evidence);
      return PROM_ERROR;
    }
    if (b->program != kProgContext || b->parameter_set != PROM_CONTEXT_REFINER_PARAMETER_SET_0 || !b->binding_valid) {
      fill_evidence(b, PROM_MODEL_BLOCK_DETAIL_REBIND_FAILED, out_evidence);
      return PROM_ERROR;
    }
    return rebind(rt, block_id, b, r->uploads, 11u, kContextWeightBytes, PROM_CONTEXT_REFINER_PARAMETER_SET_1,
                  kContextAggregate[1], out_evidence);
  });
}

PROM_REACTOR_API int prometheus_reactor_runtime_context_refiner0_execute(
    void* handle, uint64_t block_id, const PrometheusContextRefiner0ExecuteRequest* request,
    PrometheusModelBlockEvidence* out_evidence) {
  return with_runtime(handle, out_evidence, [&](Runtime* rt) -> int {
    if (request == nullptr || request->struct_size != sizeof(*request)) {
      fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_INVALID_REQUEST, out_evidence);
      return PROM_ERROR;
    }
    return context_execute(rt, block_id, PROM_CONTEXT_REFINER_PARAMETER_SET_0, request->context_input,
                           request->context_input_bytes, 0, request->input_identity, request->output_identity,
                           request->audit_enabled, false, out_evidence);
  });
}

PROM_REACTOR_API int prometheus_reactor_runtime_context_refiner_execute_resident(
    void* handle, uint64_t block_id, const PrometheusContextRefinerResidentExecuteRequest* request,
    PrometheusModelBlockEvidence* out_evidence) {
  return with_runtime(handle, out_evidence, [&](Runtime* rt) -> int {
    if (request == nullptr || request->struct_size != sizeof(*request)) {
      fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_INVALID_REQUEST, out_evidence);
      return PROM_ERROR;
    }
    return context_execute(rt, block_id, PROM_CONTEXT_REFINER_PARAMETER_SET_1, nullptr, 0, request->input_generation,
                           0, request->output_identity, request->audit_enabled, true, out_evidence);
  });
}

PROM_REACTOR_API int prometheus_reactor_runtime_context_refiner_execute_static_audit(
    void* handle, uint64_t block_id, const PrometheusContextRefinerStaticAuditRequest* request,
    PrometheusModelBlockEvidence* out_evidence) {
  return with_runtime(handle, out_evidence,
                      [&](Runtime* rt) -> int { return context_static_audit(rt, block_id, request, out_evidence); });
}

PROM_REACTOR_API int prometheus_reactor_runtime_context_refiner_audit_final(
    void* handle, uint64_t block_id, const PrometheusContextRefinerFinalAuditRequest* request,
    PrometheusModelBlockEvidence* out_evidence) {
  return with_runtime(handle, out_evidence,
                      [&](Runtime* rt) -> int { return audit_final(rt, block_id, request, kProgContext, out_evidence); });
}

// reactor_vulkan_model_block.c:2369-2462: needs a session of the same lock.
PROM_REACTOR_API int prometheus_reactor_runtime_main_transformer_create(
    void* handle, const PrometheusMainTransformerCreateRequest* request, uint64_t* out_block_id,
    PrometheusModelBlockEvidence* out_evidence) {
  if (out_block_id) *out_block_id = 0;
  return with_runtime(handle, out_evidence, [&](Runtime* rt) -> int {
    const PrometheusMainTransformerCreateRequest* r = request;
    if (r == nullptr || out_block_id == nullptr || r->struct_size != sizeof(*r) || r->uploads == nullptr ||
        r->upload_count != 13u || r->lock_identity != PROM_ZIMAGE_TURBO_LOCK_ID || r->model_local_block_id >= 30u) {
      fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_INVALID_REQUEST, out_evidence);
      return PROM_ERROR;
    }
    if (rt->model == nullptr || !rt->model->session.created || rt->model->session.lock != r->lock_identity) {
      fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_RESOURCE_CREATE_FAILED, out_evidence);
      return PROM_ERROR;
    }
    ModelSession* s = &rt->model->session;
    const RouteDecision route = decide_main_route(s->requested_route);
    if (!route.admitted) {  // reactor_vulkan_model_block.c:2419-2430
      fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_RESOURCE_CREATE_FAILED, out_evidence);
      return PROM_ERROR;
    }
    s->selected_route = route.selected;
    s->route_fallback = route.fallback;
    s->route_shader = route.shader;
    return facade_create(rt, r, out_block_id, out_evidence, true);
  });
}

// reactor_vulkan_model_block.c:3833-3881: only the lock's immediate successor layer.
PROM_REACTOR_API int prometheus_reactor_runtime_main_transformer_rebind(
    void* handle, uint64_t block_id, const PrometheusMainTransformerRebindRequest* request,
    PrometheusModelBlockEvidence* out_evidence) {
  return with_runtime(handle, out_evidence, [&](Runtime* rt) -> int {
    const PrometheusMainTransformerRebindRequest* r = request;
    if (r == nullptr || r->uploads == nullptr || r->struct_size != sizeof(*r) || r->upload_count != 13u ||
        r->lock_identity != PROM_ZIMAGE_TURBO_LOCK_ID || r->model_local_block_id >= 30u) {
      fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_INVALID_REQUEST, out_evidence);
      return PROM_ERROR;
    }
    ModelBlock* b = find_block(rt, block_id);
    if (b == nullptr) {
      fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_NOT_FOUND, out_evidence);
      return PROM_ERROR;
    }
    const uint32_t set = r->model_local_block_id + 1u;
    if (b->program != kProgMain || set != b->parameter_set + 1u || !b->binding_valid) {
      fill_evidence(b, PROM_MODEL_BLOCK_DETAIL_REBIND_FAILED, out_evidence);
      return PROM_ERROR;
    }
    return rebind(rt, block_id, b, r->uploads, 13u, kNoiseWeightBytes, set, kMainAggregate[set - 1], out_evidence);
  });
}

// reactor_vulkan_model_block.c:3883-4024
PROM_REACTOR_API int prometheus_reactor_runtime_main_transformer_execute(
    void* handle, uint64_t block_id, const PrometheusMainTransformerExecuteRequest* request,
    PrometheusModelBlockEvidence* out_evidence) {
  return with_runtime(handle, out_evidence, [&](Runtime* rt) -> int {
    const PrometheusMainTransformerExecuteRequest* r = request;
    if (r == nullptr || r->struct_size != sizeof(*r) || r->audit_enabled != 0 || r->resident_chain_mode > 1u ||
        r->lock_identity != PROM_ZIMAGE_TURBO_LOCK_ID || r->timestep_bf16 == nullptr ||
        r->timestep_bytes != kZImageConditionWidth * 2 || r->timestep_identity == 0 || r->output_identity == 0 ||
        r->required_image_generation == 0 || r->required_context_generation == 0 ||
        r->required_joint_generation == 0 || r->model_local_block_id >= 30u) {
      fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_INVALID_REQUEST, out_evidence);
      return PROM_ERROR;
    }
    ModelBlock* b = find_block(rt, block_id);
    if (b == nullptr) {
      fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_NOT_FOUND, out_evidence);
      return PROM_ERROR;
    }
    if (!reap(b)) {
      fill_evidence(b, PROM_MODEL_BLOCK_DETAIL_COMPLETION_UNCERTAIN, out_evidence);
      return PROM_ERROR;
    }
    ModelSession* s = &rt->model->session;
    const uint32_t set = r->model_local_block_id + 1u;
    if (b->program != kProgMain || b->parameter_set != set || b->aggregate != kMainAggregate[set - 1] ||
        binding_state(b) != PROM_NOISE_REFINER_BINDING_BOUND || !s->created || s->id != r->session_identity ||
        s->lock != r->lock_identity || !s->streams[0].valid || !s->streams[1].valid || !joint_valid(s) ||
        s->streams[0].generation != r->required_image_generation ||
        s->streams[1].generation != r->required_context_generation ||
        s->streams[2].generation != r->required_joint_generation) {
      mark_failure(b, PROM_MODEL_BLOCK_DETAIL_STALE_OUTPUT);
      fill_evidence(b, b->last_detail, out_evidence);
      return PROM_ERROR;
    }
    if (b->output_generation == UINT32_MAX || s->streams[2].generation == UINT64_MAX) {
      mark_failure(b, PROM_MODEL_BLOCK_DETAIL_STALE_OUTPUT);
      fill_evidence(b, PROM_MODEL_BLOCK_DETAIL_STALE_OUTPUT, out_evidence);
      return PROM_ERROR;
    }
    const bool chain = r->resident_chain_mode != 0;
    if (chain) {  // PromSessionBeginJoint: the joint is being rewritten
      s->streams[2].valid = false;
      s->joint_writing = true;
    }
    b->output_valid = false;
    b->audit_valid = false;
    const uint64_t t0 = wall_ns();
    hipStream_t st = ctx().stream;
    hipError_t e = begin_stage_timing(b, st);
    if (e == hipSuccess)
      e = hipMemcpyAsync(b->cond_bf16, r->timestep_bf16, (size_t)r->timestep_bytes, hipMemcpyHostToDevice, st);
    if (e == hipSuccess) e = launch_widen_bf16(b->cond_bf16, b->cond, kZImageConditionWidth, st);
    b->last_memcpy_ns = wall_ns() - t0;
    int32_t d = e == hipSuccess ? run_block(rt, b, s->buf[2], b->out, 1, 3, b->stage_ev + 1)
                                : PROM_MODEL_BLOCK_DETAIL_QUEUE_SUBMIT_FAILED;
    if (d == 0 && ((chain && hipMemcpyAsync(s->buf[2], b->out, (size_t)kStreamBytes[2], hipMemcpyDeviceToDevice,
                                            st) != hipSuccess) ||
                   hipEventRecord(b->stage_ev[15], st) != hipSuccess || hipStreamSynchronize(st) != hipSuccess))
      d = PROM_MODEL_BLOCK_DETAIL_COMPLETION_UNCERTAIN;
    if (d == 0) resolve_stage_timing(b);
    if (d != 0) {
      if (chain) {  // PromSessionEndJoint(commit = false)
        s->joint_writing = false;
        s->streams[2].valid = d != PROM_MODEL_BLOCK_DETAIL_COMPLETION_UNCERTAIN;
      }
      mark_failure(b, d);
      fill_evidence(b, d, out_evidence);
      return PROM_ERROR;
    }
    if (chain) {  // PromSessionEndJoint(commit = true)
      s->joint_writing = false;
      s->streams[2] = Stream{s->streams[2].generation + 1, block_id, b->output_generation + 1, true};
    }
    b->output_valid = true;
    b->output_generation += 1;
    b->executions += 1;
    b->last_execution_ns = wall_ns() - t0;
    uint64_t h = hash_u64(r->lock_identity, r->session_identity);
    h = hash_u64(h, r->required_image_generation);
    h = hash_u64(h, r->required_context_generation);
    h = hash_u64(h, r->required_joint_generation);
    h = hash_u64(h, b->aggregate);
    h = hash_u64(h, r->timestep_identity);
    b->replay_identity = hash_u64(h, r->output_identity);
    s->active_block_id = block_id;
    s->binding_generation = b->binding_generation;
    s->replay = hash_u64(s->replay, b->replay_identity);
    b->last_detail = 0;
    fill_evidence(b, 0, out_evidence);
    return PROM_OK;
  });
}

PROM_REACTOR_API int prometheus_reactor_runtime_main_transformer_execute_static_audit(
    void* handle, uint64_t block_id, const PrometheusMainTransformerStaticAuditRequest* request,
    PrometheusModelBlockEvidence* out_evidence) {
  return with_runtime(handle, out_evidence,
                      [&](Runtime* rt) -> int { return main_static_audit(rt, block_id, request, out_evidence); });
}

PROM_REACTOR_API int prometheus_reactor_runtime_main_transformer_audit_final(
    void* handle, uint64_t block_id, const PrometheusMainTransformerFinalAuditRequest* request,
    PrometheusModelBlockEvidence* out_evidence) {
  return with_runtime(handle, out_evidence,
                      [&](Runtime* rt) -> int { return audit_final(rt, block_id, request, kProgMain, out_evidence); });
}

PROM_REACTOR_API int prometheus_reactor_runtime_model_block_get_evidence(void* handle, uint64_t block_id,
                                                                         PrometheusModelBlockEvidence* out_evidence) {
  if (out_evidence == nullptr) return PROM_ERROR;
  return with_runtime(handle, out_evidence, [&](Runtime* rt) -> int {
    ModelBlock* b = find_block(rt, block_id);
    if (b == nullptr) {
      fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_NOT_FOUND, out_evidence);
      return PROM_ERROR;
    }
    fill_evidence(b, b->last_detail, out_evidence);
    return PROM_OK;
  });
}

PROM_REACTOR_API int prometheus_reactor_runtime_model_block_destroy(void* handle, uint64_t block_id) {
  return with_runtime(handle, nullptr, [&](Runtime* rt) -> int {
    ModelBlock* b = find_block(rt, block_id);
    if (b == nullptr) return PROM_ERROR;
    release_block(b);
    return PROM_OK;
  });
}

// reactor_vulkan_model_block.c:3654-3731
PROM_REACTOR_API int prometheus_reactor_runtime_compiled_model_session_create(
    void* handle, const PrometheusCompiledModelSessionCreateRequest* request, uint64_t* out_session_id,
    PrometheusCompiledModelSessionEvidence* out_evidence) {
  if (out_session_id) *out_session_id = 0;
  return with_session_runtime(handle, out_evidence, [&](Runtime* rt) -> int {
    const PrometheusCompiledModelSessionCreateRequest* r = request;
    if (r == nullptr || out_session_id == nullptr || r->struct_size != sizeof(*r) ||
        r->lock_identity != PROM_ZIMAGE_TURBO_LOCK_ID ||
        (r->execution_profile != PROM_MODEL_EXECUTION_PROFILE_MINIMUM_MEMORY &&
         r->execution_profile != PROM_MODEL_EXECUTION_PROFILE_PREFETCH) ||
        (r->main_attention_route_policy < PROM_MAIN_ATTENTION_ROUTE_AUTO ||
         r->main_attention_route_policy > PROM_MAIN_ATTENTION_ROUTE_SUBGROUP_OWNED32)) {
      fill_session_evidence(nullptr, out_evidence, PROM_MODEL_SESSION_DETAIL_INVALID_REQUEST);
      return PROM_ERROR;
    }
    ModelState* ms = rt->available ? state_of(rt) : nullptr;
    if (ms == nullptr || ms->session.created) {
      fill_session_evidence(ms ? &ms->session : nullptr, out_evidence, PROM_MODEL_SESSION_DETAIL_INVALID_REQUEST);
      return PROM_ERROR;
    }
    ModelSession* s = &ms->session;
    *s = ModelSession{};
    for (int i = 0; i < 3; ++i) {
      if ((rt->test_flags & PROM_TESTCFG_FAIL_BUFFER_ALLOC) != 0u ||
          hipMalloc(reinterpret_cast<void**>(&s->buf[i]), (size_t)kStreamBytes[i]) != hipSuccess) {
        s->buf[i] = nullptr;
        for (float* p : s->buf) free_dev(p);
        *s = ModelSession{};
        fill_session_evidence(nullptr, out_evidence, PROM_MODEL_BLOCK_DETAIL_RESOURCE_CREATE_FAILED);
        return PROM_ERROR;
      }
    }
    s->cold_allocations = 3;
    s->lock = r->lock_identity;
    s->requested_profile = r->execution_profile;
    s->requested_route = r->main_attention_route_policy;
    reset_main_route(s);  // the MainTransformer create decides the route
    s->id = ms->next_session_id++;
    s->created = true;
    *out_session_id = s->id;
    fill_session_evidence(s, out_evidence, 0);
    return PROM_OK;
  });
}

// reactor_vulkan_model_block.c:3733-3792: NoiseRefiner set 1 -> PreparedImage,
// ContextRefiner set 1 -> PreparedContext (PrometheusModelBlock.concept:920-1000).
PROM_REACTOR_API int prometheus_reactor_runtime_compiled_model_session_capture_completed(
    void* handle, uint64_t session_id, uint64_t completed_block_id,
    const PrometheusCompiledModelSessionCaptureRequest* request, PrometheusCompiledModelSessionEvidence* out_evidence) {
  return with_session_runtime(handle, out_evidence, [&](Runtime* rt) -> int {
    if (request == nullptr || request->struct_size != sizeof(*request) || rt->model == nullptr) {
      fill_session_evidence(nullptr, out_evidence, PROM_MODEL_SESSION_DETAIL_INVALID_REQUEST);
      return PROM_ERROR;
    }
    ModelSession* s = &rt->model->session;
    ModelBlock* b = &rt->model->block;
    if (!s->created || s->id != session_id || !b->created || b->id != completed_block_id || !b->output_valid ||
        b->output_generation != request->source_output_generation || !reap(b)) {
      s->last_detail = PROM_MODEL_SESSION_DETAIL_STALE_STREAM;
      fill_session_evidence(s->created && s->id == session_id ? s : nullptr, out_evidence,
                            PROM_MODEL_SESSION_DETAIL_INVALID_REQUEST);
      return PROM_ERROR;
    }
    int role;
    if (b->family == PROM_NOISE_REFINER_FAMILY_Z_IMAGE_TURBO && b->parameter_set == PROM_NOISE_REFINER_PARAMETER_SET_1)
      role = 0;
    else if (b->program == kProgContext && b->parameter_set == PROM_CONTEXT_REFINER_PARAMETER_SET_1)
      role = 1;
    else {
      s->last_detail = PROM_MODEL_SESSION_DETAIL_STREAM_MISMATCH;
      fill_session_evidence(s, out_evidence, 0);
      return PROM_ERROR;
    }
    if (s->joint_writing || s->streams[role].generation == UINT64_MAX) {
      s->last_detail = PROM_MODEL_SESSION_DETAIL_STALE_STREAM;
      fill_session_evidence(s, out_evidence, 0);
      return PROM_ERROR;
    }
    hipStream_t st = ctx().stream;
    s->streams[role].valid = false;
    if (hipMemcpyAsync(s->buf[role], b->out, (size_t)kStreamBytes[role], hipMemcpyDeviceToDevice, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess) {
      s->last_detail = PROM_MODEL_SESSION_DETAIL_COMPLETION_UNCERTAIN;
      fill_session_evidence(s, out_evidence, 0);
      return PROM_ERROR;
    }
    s->streams[role] = Stream{s->streams[role].generation + 1, completed_block_id, b->output_generation, true};
    s->active_block_id = completed_block_id;
    s->binding_generation = b->binding_generation;
    s->replay = hash_u64(s->replay == 0 ? s->lock : s->replay, completed_block_id);
    s->replay = hash_u64(s->replay, s->streams[role].generation);
    s->last_detail = 0;
    fill_session_evidence(s, out_evidence, 0);
    return PROM_OK;
  });
}

// reactor_vulkan_model_block.c:3794-3831: JointWorking = PreparedImage | PreparedContext.
PROM_REACTOR_API int prometheus_reactor_runtime_compiled_model_session_compose_joint(
    void* handle, uint64_t session_id, const PrometheusCompiledModelSessionComposeRequest* request,
    PrometheusCompiledModelSessionEvidence* out_evidence) {
  return with_session_runtime(handle, out_evidence, [&](Runtime* rt) -> int {
    ModelSession* s = find_session(rt, session_id);
    if (request == nullptr || request->struct_size != sizeof(*request) || s == nullptr) {
      fill_session_evidence(nullptr, out_evidence, PROM_MODEL_SESSION_DETAIL_INVALID_REQUEST);
      return PROM_ERROR;
    }
    if (!reap(&rt->model->block)) {
      s->last_detail = PROM_MODEL_SESSION_DETAIL_COMPLETION_UNCERTAIN;
      fill_session_evidence(s, out_evidence, 0);
      return PROM_ERROR;
    }
    const uint64_t ig = request->required_image_generation, cg = request->required_context_generation;
    if (s->joint_writing || !s->streams[0].valid || !s->streams[1].valid || ig == 0 || cg == 0 ||
        ig != s->streams[0].generation || cg != s->streams[1].generation || s->streams[2].generation == UINT64_MAX) {
      s->last_detail = PROM_MODEL_SESSION_DETAIL_STALE_STREAM;
      fill_session_evidence(s, out_evidence, 0);
      return PROM_ERROR;
    }
    hipStream_t st = ctx().stream;
    s->streams[2].valid = false;
    char* joint = reinterpret_cast<char*>(s->buf[2]);
    if (hipMemcpyAsync(joint, s->buf[0], (size_t)kStreamBytes[0], hipMemcpyDeviceToDevice, st) != hipSuccess ||
        hipMemcpyAsync(joint + kStreamBytes[0], s->buf[1], (size_t)kStreamBytes[1], hipMemcpyDeviceToDevice, st) !=
            hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess) {
      s->last_detail = PROM_MODEL_SESSION_DETAIL_COMPLETION_UNCERTAIN;
      fill_session_evidence(s, out_evidence, 0);
      return PROM_ERROR;
    }
    s->streams[2] = Stream{s->streams[2].generation + 1, 0, 0, true};
    s->joint_image_generation = ig;
    s->joint_context_generation = cg;
    s->compositions += 1;
    s->replay = hash_u64(s->replay, s->joint_image_generation);
    s->replay = hash_u64(s->replay, s->joint_context_generation);
    s->replay = hash_u64(s->replay, s->streams[2].generation);
    s->last_detail = 0;
    fill_session_evidence(s, out_evidence, 0);
    return PROM_OK;
  });
}

PROM_REACTOR_API int prometheus_reactor_runtime_compiled_model_session_get_evidence(
    void* handle, uint64_t session_id, PrometheusCompiledModelSessionEvidence* out_evidence) {
  if (out_evidence == nullptr) return PROM_ERROR;
  return with_session_runtime(handle, out_evidence, [&](Runtime* rt) -> int {
    ModelSession* s = find_session(rt, session_id);
    if (s == nullptr) {
      fill_session_evidence(nullptr, out_evidence, PROM_MODEL_SESSION_DETAIL_INVALID_REQUEST);
      return PROM_ERROR;
    }
    fill_session_evidence(s, out_evidence, 0);
    return PROM_OK;
  });
}

// reactor_vulkan_model_block.c:4229-4251
PROM_REACTOR_API int prometheus_reactor_runtime_compiled_model_session_set_main_attention_route(
    void* handle, uint64_t session_id, uint32_t main_attention_route_policy,
    PrometheusCompiledModelSessionEvidence* out_evidence) {
  if (out_evidence == nullptr || main_attention_route_policy < PROM_MAIN_ATTENTION_ROUTE_AUTO ||
      main_attention_route_policy > PROM_MAIN_ATTENTION_ROUTE_SUBGROUP_OWNED32 || lookup(handle) == nullptr)
    return PROM_ERROR;
  return with_session_runtime(handle, out_evidence, [&](Runtime* rt) -> int {
    ModelSession* s = find_session(rt, session_id);
    if (s == nullptr || rt->model->block.created) {  // the route is fixed once a block exists
      fill_session_evidence(rt->model ? &rt->model->session : nullptr, out_evidence,
                            PROM_MODEL_SESSION_DETAIL_INVALID_REQUEST);
      return PROM_ERROR;
    }
    s->requested_route = main_attention_route_policy;
    reset_main_route(s);
    fill_session_evidence(s, out_evidence, 0);
    return PROM_OK;
  });
}

PROM_REACTOR_API int prometheus_reactor_runtime_compiled_model_session_destroy(void* handle, uint64_t session_id) {
  return with_session_runtime(handle, nullptr, [&](Runtime* rt) -> int {
    ModelSession* s = find_session(rt, session_id);
    if (s == nullptr || !reap(&rt->model->block)) return PROM_ERROR;
    release_session(s);
    return PROM_OK;
  });
}

// reactor_vulkan_model_block.c:4348-4450: the shared owner, bound to NoiseRefiner 0.
PROM_REACTOR_API int prometheus_reactor_runtime_compiled_model_owner_create(
    void* handle, const PrometheusNoiseRefinerRebindRequest* request, uint64_t* out_block_id,
    PrometheusModelBlockEvidence* out_evidence) {
  if (out_block_id) *out_block_id = 0;
  return with_runtime(handle, out_evidence, [&](Runtime* rt) -> int {
    const PrometheusNoiseRefinerRebindRequest* r = request;
    if (r == nullptr || out_block_id == nullptr || r->struct_size != sizeof(*r) || r->model_local_block_id != 0u ||
        r->uploads == nullptr || r->upload_count != 13u || r->lock_identity != PROM_ZIMAGE_TURBO_LOCK_ID ||
        rt->model == nullptr || rt->model->block.created || !rt->model->session.created ||
        rt->model->session.lock != r->lock_identity) {
      fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_INVALID_REQUEST, out_evidence);
      return PROM_ERROR;
    }
    ModelSession* s = &rt->model->session;
    // reactor_vulkan_model_block.c:4364-4380: PREFETCH needs a transfer queue
    // independent of compute; a second HIP stream always is one, so the
    // requested profile is selected without a fallback.
    s->selected_profile = s->requested_profile == PROM_MODEL_EXECUTION_PROFILE_PREFETCH
                              ? PROM_MODEL_EXECUTION_PROFILE_PREFETCH
                              : PROM_MODEL_EXECUTION_PROFILE_MINIMUM_MEMORY;
    s->profile_fallback = 0u;
    const RouteDecision route = decide_main_route(s->requested_route);  // reactor_vulkan_model_block.c:4381-4408
    s->selected_route = route.selected;
    s->route_fallback = route.fallback;
    s->route_shader = route.shader;
    if (!route.admitted) {
      s->last_detail = PROM_MODEL_SESSION_DETAIL_MAIN_ATTENTION_ROUTE_REJECTED;
      fill_evidence(nullptr, PROM_MODEL_SESSION_DETAIL_MAIN_ATTENTION_ROUTE_REJECTED, out_evidence);
      return PROM_ERROR;
    }
    PrometheusModelBlockCreateRequest c;
    memset(&c, 0, sizeof(c));
    c.struct_size = sizeof(c);
    c.assembly_family = PROM_NOISE_REFINER_FAMILY_Z_IMAGE_TURBO;
    c.parameter_set = PROM_NOISE_REFINER_PARAMETER_SET_0;
    c.parameter_set_aggregate_identity = kNoiseAggregate[0];
    c.model_contract_identity = PROM_ZIMAGE_TURBO_LOCK_ID;
    c.weight_identity = kNoiseAggregate[0];
    c.shader_portfolio_identity = kNoiseExecutionPlan;
    c.precision_policy_identity = PROM_ZIMAGE_TURBO_LOCK_ID;
    c.capability_route_identity = PROM_ZIMAGE_TURBO_LOCK_ID;
    c.memory_ceiling_bytes = kNoiseMemoryPlan + (uint64_t)kImageTokens * kWidth * 4 + (uint64_t)kContextTokens * kFfn * 4;
    c.external_input_bytes = (uint64_t)kImageTokens * kWidth * 2;
    c.audit_bytes = PROM_ZIMAGE_TURBO_AUDIT_ARENA_BYTES;
    c.shader_id = kShaderNoise;
    c.weight_count = 13u;
    c.step_count = PROM_MODEL_BLOCK_MAX_STEPS;
    memcpy(c.steps, kSteps, sizeof(c.steps));
    for (uint32_t i = 0; i < 13u; ++i) {
      c.weights[i].content_identity = r->uploads[i].content_identity;
      c.weights[i].layout_identity = r->uploads[i].layout_identity;
      c.weights[i].byte_count = r->uploads[i].byte_count;
    }
    if (create_block(rt, &c, out_block_id, out_evidence, true) != PROM_OK) return PROM_ERROR;
    if (s->selected_profile == PROM_MODEL_EXECUTION_PROFILE_PREFETCH &&
        !alloc_prefetch(&rt->model->block, &rt->model->prefetch)) {
      release_block(&rt->model->block);
      *out_block_id = 0;
      fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_RESOURCE_CREATE_FAILED, out_evidence);
      return PROM_ERROR;
    }
    if (upload_weights(rt, *out_block_id, r->uploads, 13u, out_evidence) != PROM_OK) {
      release_block(&rt->model->block);
      *out_block_id = 0;
      return PROM_ERROR;
    }
    s->evaluation_generation = 1;
    s->retarget_position = 1;
    s->active_block_id = *out_block_id;
    s->binding_generation = rt->model->block.binding_generation;
    return PROM_OK;
  });
}

// reactor_vulkan_model_block.c:4452-4543: the owner moves to the block its
// position names; the weights are overwritten in place.
PROM_REACTOR_API int prometheus_reactor_runtime_compiled_model_retarget(
    void* handle, const PrometheusCompiledModelRetargetRequest* request, PrometheusModelBlockEvidence* out_evidence) {
  return with_runtime(handle, out_evidence, [&](Runtime* rt) -> int {
    const PrometheusCompiledModelRetargetRequest* r = request;
    if (r == nullptr || r->struct_size != sizeof(*r) || r->uploads == nullptr ||
        r->lock_identity != PROM_ZIMAGE_TURBO_LOCK_ID || rt->model == nullptr) {
      fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_INVALID_REQUEST, out_evidence);
      return PROM_ERROR;
    }
    ModelBlock* b = &rt->model->block;
    ModelSession* s = &rt->model->session;
    if (!b->created || !b->shared || !s->created || s->id != r->session_identity || s->lock != r->lock_identity ||
        !reap(b)) {
      if (b->created) {
        mark_failure(b, b->quarantined ? PROM_MODEL_BLOCK_DETAIL_COMPLETION_UNCERTAIN
                                       : PROM_MODEL_BLOCK_DETAIL_REBIND_FAILED);
        fill_evidence(b, b->last_detail, out_evidence);
      } else {
        fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_NOT_FOUND, out_evidence);
      }
      return PROM_ERROR;
    }
    Target t;
    if (!target_at(s->retarget_position, &t) || r->model_local_block_id != t.local || r->upload_count != t.count ||
        !retarget_uploads_match(b, r->uploads, t)) {
      fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_INVALID_REQUEST, out_evidence);
      return PROM_ERROR;
    }
    if (b->program != t.program && !set_program(b, t.program)) {
      mark_failure(b, PROM_MODEL_BLOCK_DETAIL_RESOURCE_CREATE_FAILED);
      fill_evidence(b, b->last_detail, out_evidence);
      return PROM_ERROR;
    }
    b->family = t.family;
    b->weight_count = t.count;
    if (!change_weights(rt, b, r->uploads, t.count, false)) {
      fill_evidence(b, b->last_detail, out_evidence);
      return PROM_ERROR;
    }
    b->parameter_set = t.parameter_set;
    b->aggregate = t.aggregate;
    s->retarget_position += 1;
    s->active_block_id = b->id;
    s->binding_generation = b->binding_generation;
    fill_evidence(b, 0, out_evidence);
    return PROM_OK;
  });
}

// reactor_vulkan_model_block.c:4545-4641: under the PREFETCH profile, uploads
// the weights of the block the session's position names into the owner's
// second window.  The transfer runs on the window's stream without the device
// context's lock, so a caller may execute the active block on another thread
// meanwhile (tools/prometheus_zimage_bridge/reactor_windows.go:510-531); the
// evidence of a successful prefetch reports only `created`, because the block's
// counters belong to that other thread.
PROM_REACTOR_API int prometheus_reactor_runtime_compiled_model_prefetch(
    void* handle, const PrometheusCompiledModelPrefetchRequest* request, PrometheusModelBlockEvidence* out_evidence) {
  Runtime* rt = lookup(handle);
  const PrometheusCompiledModelPrefetchRequest* r = request;
  if (rt == nullptr || r == nullptr || r->struct_size != sizeof(*r) || r->uploads == nullptr ||
      r->lock_identity != PROM_ZIMAGE_TURBO_LOCK_ID) {
    fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_INVALID_REQUEST, out_evidence);
    return PROM_ERROR;
  }
  std::unique_lock<std::mutex> lock(ctx().mu);
  ModelState* ms = rt->model;
  if (ms == nullptr || !ms->block.created || !ms->session.created || ms->session.id != r->session_identity ||
      ms->session.selected_profile != PROM_MODEL_EXECUTION_PROFILE_PREFETCH || ms->block.pf == nullptr ||
      !ms->prefetch.enabled) {
    fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_REBIND_FAILED, out_evidence);
    return PROM_ERROR;
  }
  const uint32_t position = ms->session.retarget_position;
  Target t;
  if (position == 0u || !target_at(position, &t) || r->model_local_block_id != t.local ||
      r->upload_count != t.count || !retarget_uploads_match(&ms->block, r->uploads, t)) {
    fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_INVALID_REQUEST, out_evidence);
    return PROM_ERROR;
  }
  PrefetchWindow* pf = &ms->prefetch;
  // PrometheusModelBlock.concept:1348-1352: a window that holds a prepared set
  // (or is being filled by another call) is not begun again.
  std::unique_lock<std::mutex> window(pf->mu, std::try_to_lock);
  if (!window.owns_lock() || pf->state == PROM_MODEL_WEIGHT_WINDOW_DEVICE_READY) {
    fill_evidence(nullptr, PROM_MODEL_BLOCK_DETAIL_REBIND_FAILED, out_evidence);
    return PROM_ERROR;
  }
  pf->state = PROM_MODEL_WEIGHT_WINDOW_UPLOAD_SUBMITTED;
  pf->target_position = 0;
  lock.unlock();  // compute may proceed; destroy, reset and activation wait on pf->mu
  const uint64_t t0 = wall_ns();
  const int32_t detail = prefetch_transfer(pf, t, r->uploads);
  if (detail != 0) {
    pf->state = PROM_MODEL_WEIGHT_WINDOW_UNCERTAIN;
    fill_evidence(nullptr, detail, out_evidence);
    return PROM_ERROR;
  }
  pf->transfer_ns = wall_ns() - t0;
  pf->state = PROM_MODEL_WEIGHT_WINDOW_DEVICE_READY;
  pf->program = (int)t.program;
  pf->family = t.family;
  pf->parameter_set = t.parameter_set;
  pf->count = t.count;
  pf->aggregate = t.aggregate;
  pf->target_position = position;
  pf->generation += 1;
  fill_evidence(nullptr, 0, out_evidence);
  if (out_evidence) out_evidence->created = 1u;
  return PROM_OK;
}

// reactor_vulkan_model_block.c:4643-4715: swaps the prepared window in as the
// owner's active weights when it holds the block the session's position names
// (waiting for a transfer still in flight), and advances the position.
PROM_REACTOR_API int prometheus_reactor_runtime_compiled_model_activate_prefetch(
    void* handle, uint64_t session_id, PrometheusModelBlockEvidence* out_evidence) {
  return with_runtime(handle, out_evidence, [&](Runtime* rt) -> int {
    ModelState* ms = rt->model;
    ModelBlock* b = ms && ms->block.created ? &ms->block : nullptr;
    ModelSession* s = ms ? &ms->session : nullptr;
    if (b == nullptr || !s->created || s->id != session_id ||
        s->selected_profile != PROM_MODEL_EXECUTION_PROFILE_PREFETCH || b->pf == nullptr) {
      fill_evidence(b, PROM_MODEL_BLOCK_DETAIL_REBIND_FAILED, out_evidence);
      return PROM_ERROR;
    }
    PrefetchWindow* pf = b->pf;
    std::lock_guard<std::mutex> window(pf->mu);
    if (pf->target_position != s->retarget_position) {
      fill_evidence(b, PROM_MODEL_BLOCK_DETAIL_REBIND_FAILED, out_evidence);
      return PROM_ERROR;
    }
    if (!reap(b)) {
      fill_evidence(b, PROM_MODEL_BLOCK_DETAIL_COMPLETION_UNCERTAIN, out_evidence);
      return PROM_ERROR;
    }
    if (pf->state != PROM_MODEL_WEIGHT_WINDOW_DEVICE_READY) {  // PrometheusModelBlock.concept:1406-1409
      fill_evidence(b, PROM_MODEL_BLOCK_DETAIL_REBIND_FAILED, out_evidence);
      return PROM_ERROR;
    }
    const Program program = (Program)pf->program;
    if (b->program != program && !set_program(b, program)) {
      fill_evidence(b, PROM_MODEL_BLOCK_DETAIL_DESCRIPTOR_UPDATE_FAILED, out_evidence);
      return PROM_ERROR;
    }
    // PrometheusModelBlock.concept:1428-1448: the windows trade places.
    std::swap(b->active, pf->set);
    b->family = pf->family;
    b->parameter_set = pf->parameter_set;
    b->weight_count = pf->count;
    b->aggregate = pf->aggregate;
    b->uploads += pf->count;
    b->last_memcpy_ns = pf->transfer_ns;
    b->binding_valid = true;
    b->binding_phase = PROM_NOISE_REFINER_BINDING_BOUND;
    b->binding_generation += 1;
    b->descriptor_generation += 1;
    b->output_valid = false;
    b->audit_valid = false;
    b->resident_input_generation = 0;
    b->replay_identity = 0;
    b->prefix_replay = 0;
    b->active_window ^= 1u;
    b->last_detail = 0;
    pf->state = PROM_MODEL_WEIGHT_WINDOW_EMPTY;
    pf->target_position = 0;
    pf->count = 0;
    s->retarget_position += 1;
    s->active_block_id = b->id;
    s->binding_generation = b->binding_generation;
    fill_evidence(b, 0, out_evidence);
    return PROM_OK;
  });
}

// reactor_vulkan_model_block.c:4717-4752 and PromSessionReset
// (PrometheusModelBlock.concept:1080-1088): a new evaluation starts at NoiseRefiner 0.
PROM_REACTOR_API int prometheus_reactor_runtime_compiled_model_evaluation_reset(
    void* handle, uint64_t session_id, PrometheusCompiledModelSessionEvidence* out_evidence) {
  return with_session_runtime(handle, out_evidence, [&](Runtime* rt) -> int {
    ModelSession* s = find_session(rt, session_id);
    ModelBlock* b = rt->model ? &rt->model->block : nullptr;
    if (s == nullptr || b == nullptr || !b->created || !b->shared || s->joint_writing || !reap(b)) {
      fill_session_evidence(nullptr, out_evidence, PROM_MODEL_SESSION_DETAIL_INVALID_REQUEST);
      return PROM_ERROR;
    }
    if (b->pf != nullptr) {  // reactor_vulkan_model_block.c:4731-4734: waits for and drops a prefetch
      std::lock_guard<std::mutex> window(b->pf->mu);
      b->pf->state = PROM_MODEL_WEIGHT_WINDOW_EMPTY;
      b->pf->target_position = 0;
      b->pf->count = 0;
    }
    for (Stream& st : s->streams) st = Stream{st.generation, 0, 0, false};
    s->joint_image_generation = 0;
    s->joint_context_generation = 0;
    s->evaluation_generation += 1;
    s->retarget_position = 0;
    s->active_block_id = 0;
    s->binding_generation = 0;
    s->replay = 0;
    b->output_valid = false;
    b->audit_valid = false;
    b->replay_identity = 0;
    s->last_detail = 0;
    fill_session_evidence(s, out_evidence, 0);
    return PROM_OK;
  });
}

}  // extern "C"
