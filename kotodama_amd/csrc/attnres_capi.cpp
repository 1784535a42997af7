// Host side of libattnres_hip.so: the C ABI declared in include/attnres.h.
//
// The gfx950 kernels are compiled ahead of time into code-object parts that
// are linked into this library as bytes (attnres_blob.S).  On first use of a
// device the parts are loaded with hipModuleLoadData; every call validates
// its arguments on the host, fills one kernel-argument block
// (attnres_params.h) and launches with hipModuleLaunchKernel on the caller's
// stream.  No allocation, no synchronisation, no state beyond the per-device
// module and function caches.

#include <hip/hip_runtime.h>

#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>

#include "attnres.h"
#include "attnres_params.h"

// Code-object parts (attnres_blob.S).
extern "C" const unsigned char attnres_hsaco_part0[];
extern "C" const unsigned char attnres_hsaco_part1[];
extern "C" const unsigned char attnres_hsaco_part2[];
extern "C" const unsigned char attnres_hsaco_part3[];
extern "C" const unsigned char attnres_hsaco_part4[];
extern "C" const unsigned char attnres_hsaco_part5[];
extern "C" const unsigned char attnres_hsaco_part6[];
extern "C" const unsigned char attnres_hsaco_part7[];
extern "C" const unsigned char attnres_hsaco_part8[];
extern "C" const unsigned char attnres_hsaco_part9[];
extern "C" const unsigned char attnres_hsaco_part10[];

namespace {

constexpr int kParts = 11;
constexpr int kMaxDevices = 64;
constexpr int kMaxThreads = 512;  // __launch_bounds__ of every kernel

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(ATTNRES_ERR_HIP, "%s failed: %s (%d)", what, hipGetErrorString(e), (int)e);
}

// Route kernel variants: type combo x S x V x (single/multi query).
enum TypeCombo { kBfDot2 = 0, kBfFma = 1, kF32Fma = 2, kTypeCombos = 3 };
constexpr int kNumS = ATTNRES_KMAX_SOURCES + 1;
constexpr int kRouteFuncs = kTypeCombos * kNumS * 2 * 2;
constexpr int kMergeFuncs = 4 * 2;
constexpr int kStreamMaxChunks = 8;  // rows of up to 8 KiB
constexpr int kStreamWaves = 4;      // waves per workgroup of the streaming kernels
// combo x out dtype x KiB x variant (plain / pointer table / fused / fused with the pointer table)
constexpr int kStreamFuncs = kTypeCombos * 2 * kStreamMaxChunks * 4;
constexpr int kBwdFuncs = 4 * kNumS * 2;  // (source, grad_out) dtype pairs x S x V
constexpr int kBwdMaxPerCu = 4;           // workgroups per CU the backward grid may use (workspace bound)
constexpr size_t kBwdStaticLds = 2 * ATTNRES_KMAX_WAVES * 48 * sizeof(float);  // reduction buffer, S = 16
constexpr size_t kQgStaticLds = 2 * ATTNRES_KMAX_WAVES * 72 * sizeof(float);   // batched-query reduction buffer
constexpr size_t kMqgStaticLds = 2 * ATTNRES_KMAX_WAVES * 72 * sizeof(float);  // its backward's (S <= 8)

// One kernel on one device.  Its handle is looked up once, under g_mu, and
// published with a release store; it never changes afterwards, so finding it
// again is one acquire load and no lock.  `static_lds` is written before the
// handle is published.  The resident-workgroup count depends on the launch's
// block size and dynamic LDS; it is cached in one packed word (valid bit,
// block, LDS bytes, workgroups per CU), read without a lock by launches of
// the same shape and recomputed for another shape (the value is a function
// of the shape, so two threads racing on it store the same word).
struct KernelSlot {
  std::atomic<hipFunction_t> fn{nullptr};
  std::atomic<uint64_t> occ{0};
  int static_lds = 0;
};

// Query-gradient reduction kernels: one launch (`cols`), or two (`stage`
// then `fin`) where the one-launch form's 32-bit offsets would not fit.
struct ReduceFns {
  hipFunction_t stage = nullptr;
  hipFunction_t fin = nullptr;
  hipFunction_t cols = nullptr;
};

struct DeviceState {
  std::atomic<bool> loaded{false};
  hipModule_t mods[kParts] = {};
  int num_cus = 0;
  int max_lds = 0;  // bytes of LDS one workgroup may use
  KernelSlot route[kRouteFuncs];
  KernelSlot route_qg[kNumS * 2];  // batched-query kernels: S x V
  KernelSlot stream[kStreamFuncs];
  KernelSlot merge[kMergeFuncs];
  KernelSlot merge_stream[2 * kStreamMaxChunks];  // row-per-wave merge: query path x row KiB
  KernelSlot bwd[kBwdFuncs];
  KernelSlot bwd_stream[2 * 10];  // row-per-wave backward: rows of 6 / 8 KiB x S (1..9)
  KernelSlot bwd_add[kBwdFuncs];   // the same with addend rows (_add)
  KernelSlot bwd_stream_add[2 * 10];
  KernelSlot reduce_stage, reduce_cols, reduce_fin;
  KernelSlot merge_bwd[kMergeFuncs];
  KernelSlot bwd_mq[kBwdFuncs];  // batched-query backward: (source, grad_out) dtypes x S x V
  KernelSlot bwd_dqw[4];         // source dtype x V
  KernelSlot bwd_mqg[2 * 9];     // batched-query backward on the matrix cores: query groups x S
  KernelSlot bwd_defer[4 * 10];  // row-per-wave backward with deferred block gradients: row width x S
  KernelSlot gather_seg[4 * ATTNRES_SEG_MAX_BLOCKS];  // segment sums: row width x blocks
};

DeviceState g_dev[kMaxDevices];
std::mutex g_mu;
std::atomic<int> g_policy{ATTNRES_POLICY_AUTO};

// Measurement knobs, read once and only when ATTNRES_TUNING=1 is set (so a
// stray variable cannot change kernel selection in a user's process; the
// defaults are the measured choices): ATTNRES_V forces chunks per thread (1 or
// 2) of the row-per-workgroup kernels, ATTNRES_STREAM /
// ATTNRES_STREAM_MIN_TOKENS choose when the row-per-wave streaming kernels
// run, ATTNRES_GRID_MULT scales the resident-workgroup grid,
// ATTNRES_STREAM_PER_CU sets the streaming kernels' workgroups per CU (0: the
// occupancy limit; by default by row width), ATTNRES_BWD_PER_CU caps the backward kernels' (at most
// kBwdMaxPerCu, the bound its workspace size assumes), ATTNRES_QG=0 turns off
// the batched-query kernel, ATTNRES_MQG=0 the matrix-core batched backward,
// ATTNRES_OUT_BATCH caps the streaming kernels' staged output rows per wave
// (1: store each row at once), ATTNRES_OUT_BATCH_MIN_S sets the source count
// from which they stage, ATTNRES_REDUCE_TWO_STAGE=1 reduces the query
// gradients in two launches always, ATTNRES_MERGE_STREAM=0 keeps the merge on
// its row-per-workgroup kernel, ATTNRES_GATHER_PER_CU sets the deferred-gradient
// sums' workgroups per CU (1..4).
struct Tuning {
  int force_v = 0;
  int qg = 1;
  int stream = -1;  // -1: by size, 0: never, 1: whenever the shape allows
  int64_t stream_min_tokens = 2048;
  double grid_mult = 1.0;
  double stream_per_cu = -1.0;  // workgroups per CU of the streaming kernels (< 0: by row width)
  int bwd_per_cu = 0;          // > 0: resident workgroups per CU of the routing backward
  int mqg = 1;                 // 0: the batched-query backward never uses the matrix-core kernel
  int out_batch = 0;           // > 0: at most this many staged output rows per streaming wave (1: none)
  int out_batch_min_s = 3;     // sources from which the streaming kernels stage output rows
  int stream_waves = 0;        // > 0: waves per workgroup of the streaming kernels (1..4); 0: by S
  int reduce_two_stage = 0;    // 1: the query-gradient reduction in two launches
  int merge_stream = 1;        // 0: the merge never uses the row-per-wave kernel
  int gather_per_cu = 0;       // > 0: workgroups per CU of the deferred-gradient sums
  Tuning() {
    const char* on = std::getenv("ATTNRES_TUNING");
    if (on == nullptr || std::strcmp(on, "1") != 0) return;
    if (const char* v = std::getenv("ATTNRES_MQG")) mqg = std::atoi(v);
    if (const char* v = std::getenv("ATTNRES_OUT_BATCH")) out_batch = std::atoi(v);
    if (const char* v = std::getenv("ATTNRES_OUT_BATCH_MIN_S")) out_batch_min_s = std::atoi(v);
    if (const char* v = std::getenv("ATTNRES_REDUCE_TWO_STAGE")) reduce_two_stage = std::atoi(v);
    if (const char* v = std::getenv("ATTNRES_MERGE_STREAM")) merge_stream = std::atoi(v);
    if (const char* v = std::getenv("ATTNRES_STREAM_WAVES")) {
      const int w = std::atoi(v);
      if (w >= 1 && w <= kStreamWaves) stream_waves = w;
    }
    if (const char* v = std::getenv("ATTNRES_BWD_PER_CU")) {
      bwd_per_cu = std::atoi(v);
      if (bwd_per_cu > kBwdMaxPerCu) bwd_per_cu = kBwdMaxPerCu;
    }
    if (const char* v = std::getenv("ATTNRES_STREAM_PER_CU")) stream_per_cu = std::atof(v);
    if (const char* v = std::getenv("ATTNRES_GATHER_PER_CU")) {
      gather_per_cu = std::atoi(v);
      if (gather_per_cu < 1) gather_per_cu = 1;
      if (gather_per_cu > 4) gather_per_cu = 4;
    }
    if (const char* v = std::getenv("ATTNRES_V")) force_v = std::atoi(v);
    if (const char* v = std::getenv("ATTNRES_QG")) qg = std::atoi(v);
    if (const char* v = std::getenv("ATTNRES_STREAM")) stream = std::atoi(v);
    if (const char* v = std::getenv("ATTNRES_STREAM_MIN_TOKENS")) stream_min_tokens = std::atoll(v);
    if (const char* g = std::getenv("ATTNRES_GRID_MULT")) {
      const double m = std::atof(g);
      if (m > 0.0) grid_mult = m;
    }
  }
};
const Tuning& tuning() {
  static Tuning t;
  return t;
}

int ensure_loaded(DeviceState** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(ATTNRES_ERR_HIP, "device ordinal %d out of range", dev);
  DeviceState& st = g_dev[dev];
  if (!st.loaded.load(std::memory_order_acquire)) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!st.loaded.load(std::memory_order_relaxed)) {
      const unsigned char* blobs[kParts] = {attnres_hsaco_part0, attnres_hsaco_part1, attnres_hsaco_part2,
                                            attnres_hsaco_part3, attnres_hsaco_part4, attnres_hsaco_part5,
                                            attnres_hsaco_part6, attnres_hsaco_part7, attnres_hsaco_part8,
                                            attnres_hsaco_part9, attnres_hsaco_part10};
      // On a failure nothing stays half-loaded: the next call starts over.
      auto unload = [&st](int n) {
        for (int j = 0; j < n; ++j) {
          (void)hipModuleUnload(st.mods[j]);
          st.mods[j] = nullptr;
        }
      };
      for (int i = 0; i < kParts; ++i) {
        e = hipModuleLoadData(&st.mods[i], blobs[i]);
        if (e != hipSuccess) {
          st.mods[i] = nullptr;
          unload(i);
          return hip_fail(e, "hipModuleLoadData");
        }
      }
      e = hipDeviceGetAttribute(&st.num_cus, hipDeviceAttributeMultiprocessorCount, dev);
      if (e == hipSuccess) e = hipDeviceGetAttribute(&st.max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
      if (e != hipSuccess) {
        unload(kParts);
        return hip_fail(e, "hipDeviceGetAttribute");
      }
      st.loaded.store(true, std::memory_order_release);
    }
  }
  *out = &st;
  return ATTNRES_OK;
}

// Code-object part holding the route kernels for S sources (the split of the
// ATTNRES_PART blocks in attnres_kernels.hip); merge kernels live in part 3.
int part_of_route(int s) { return s <= 5 ? 0 : s <= 9 ? 1 : s <= 13 ? 2 : 3; }
constexpr int kMergePart = 3;

int find_function(DeviceState& st, int part, const char* name, hipFunction_t* f) {
  hipError_t e = hipModuleGetFunction(f, st.mods[part], name);
  if (e != hipSuccess) {
    (void)hipGetLastError();  // do not leave a sticky error for the caller's runtime
    return fail(ATTNRES_ERR_HIP, "kernel %s not found in code-object part %d: %s", name, part, hipGetErrorString(e));
  }
  return ATTNRES_OK;
}

// The slot's kernel handle, looked up by `name` in code-object `part` on first use.
int slot_function(DeviceState& st, KernelSlot& k, int part, const char* name, hipFunction_t* f) {
  hipFunction_t fn = k.fn.load(std::memory_order_acquire);
  if (fn == nullptr) {
    std::lock_guard<std::mutex> lk(g_mu);
    fn = k.fn.load(std::memory_order_relaxed);
    if (fn == nullptr) {
      int rc = find_function(st, part, name, &fn);
      if (rc != ATTNRES_OK) return rc;
      int slds = 0;
      hipError_t e = hipFuncGetAttribute(&slds, HIP_FUNC_ATTRIBUTE_SHARED_SIZE_BYTES, fn);
      if (e != hipSuccess) return hip_fail(e, "hipFuncGetAttribute(SHARED_SIZE_BYTES)");
      k.static_lds = slds;
      k.fn.store(fn, std::memory_order_release);
    }
  }
  *f = fn;
  return ATTNRES_OK;
}

// Resident workgroups per CU of the slot's kernel for `block` threads and
// `lds` bytes of dynamic LDS (at least 1).
int slot_occupancy(KernelSlot& k, hipFunction_t fn, int block, size_t lds, int* bpc) {
  const uint64_t key = ((uint64_t)1 << 63) | ((uint64_t)(block & 0x7fff) << 48) | ((uint64_t)(lds & 0xffffffffu) << 16);
  const uint64_t o = k.occ.load(std::memory_order_acquire);
  if ((o & ~(uint64_t)0xffff) == key) {
    *bpc = (int)(o & 0xffff);
    return ATTNRES_OK;
  }
  int nb = 0;
  hipError_t e = hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&nb, fn, block, lds);
  if (e != hipSuccess) return hip_fail(e, "hipModuleOccupancyMaxActiveBlocksPerMultiprocessor");
  if (nb < 1) nb = 1;
  if (nb > 0xffff) nb = 0xffff;
  k.occ.store(key | (uint64_t)nb, std::memory_order_release);
  *bpc = nb;
  return ATTNRES_OK;
}

// Handle and occupancy together.
int slot_get(DeviceState& st, KernelSlot& k, int part, const char* name, int block, size_t lds, hipFunction_t* f,
             int* bpc) {
  int rc = slot_function(st, k, part, name, f);
  if (rc != ATTNRES_OK) return rc;
  return slot_occupancy(k, *f, block, lds, bpc);
}

int part_of_stream(int nch) { return nch <= 4 ? 2 : 1; }

enum StreamVariant { kStreamPlain = 0, kStreamTable = 1, kStreamFused = 2, kStreamFusedTable = 3 };
constexpr int kStreamVariants = 4;
const char* const kStreamVariantNames[kStreamVariants] = {"plain", "table", "fused", "fusedtable"};

int get_stream(DeviceState& st, int combo, bool out_bf, int nch, int variant, hipFunction_t* f, int* bpc,
               int* static_lds) {
  const int idx = ((combo * 2 + (out_bf ? 0 : 1)) * kStreamMaxChunks + (nch - 1)) * kStreamVariants + variant;
  static const char* combo_names[kTypeCombos] = {"bf_d2", "bf_fm", "f32_fm"};
  char name[96];
  snprintf(name, sizeof(name), "attnres_stream_%s_o%s_c%d_%s", combo_names[combo], out_bf ? "bf" : "f32", nch,
           kStreamVariantNames[variant]);
  KernelSlot& k = st.stream[idx];
  int rc = slot_get(st, k, part_of_stream(nch), name, 64 * kStreamWaves, 0, f, bpc);
  if (rc != ATTNRES_OK) return rc;
  *static_lds = k.static_lds;
  return ATTNRES_OK;
}

// Output rows a streaming-kernel wave stages in LDS and stores together
// (attnres_route_params.out_batch).  With several sources per row, stores in
// bursts run the read-heavy stream far faster (the store-only access pattern
// at the 3B shape: S = 4 83% -> 90%, S = 8 79% -> 91% of peak with batches of
// 8).  At S = 2 the batches measured slower (84.4% -> 83.3%) and at S = 3
// faster once they reached 10 rows (83.9% -> 85.4%), so they start at S = 3.
// As many rows as the LDS left over by the kernel's own arrays holds, at most
// 8; the plain and table kernels add rows held in registers to each batch (4
// up to 6 KiB rows, 2 above).
constexpr int kOutBatchMax = 8;
int stream_out_batch(int num_sources, int64_t out_row_bytes, int static_lds, int max_lds, int waves) {
  const int min_s = tuning().out_batch_min_s;
  if (num_sources < min_s || out_row_bytes <= 0) return 1;
  int64_t cap = ((int64_t)max_lds - static_lds) / ((int64_t)waves * out_row_bytes);
  const int limit = tuning().out_batch > 0 ? tuning().out_batch : kOutBatchMax;
  if (cap > limit) cap = limit;
  return cap >= 2 ? (int)cap : 1;
}

int route_index(int combo, int s, int v, bool multiq) { return ((combo * kNumS + s) * 2 + (v - 1)) * 2 + (multiq ? 1 : 0); }

int get_route(DeviceState& st, int combo, int s, int v, bool multiq, int block, hipFunction_t* f, int* bpc) {
  static const char* combo_names[kTypeCombos] = {"bf_d2", "bf_fm", "f32_fm"};
  char name[96];
  snprintf(name, sizeof(name), "attnres_route_%s_s%d_v%d_%s", combo_names[combo], s, v, multiq ? "qn" : "q1");
  return slot_get(st, st.route[route_index(combo, s, v, multiq)], part_of_route(s), name, block, 0, f, bpc);
}

// Batched-query kernel (bf16 sources and parameters, Q >= 2) with `lds` bytes
// of dynamic LDS for the staged queries.
int get_route_qg(DeviceState& st, int s, int v, int block, size_t lds, hipFunction_t* f, int* bpc) {
  char name[96];
  snprintf(name, sizeof(name), "attnres_route_bf_d2_s%d_v%d_qg", s, v);
  return slot_get(st, st.route_qg[s * 2 + (v - 1)], part_of_route(s), name, block, lds, f, bpc);
}

// Row-per-wave merge (code-object part 3): bf16 rows of nch KiB, the query on
// the v_dot2 path (bf16 parameter) or in fp32.
int get_merge_stream(DeviceState& st, bool d2, int nch, hipFunction_t* f) {
  char name[96];
  snprintf(name, sizeof(name), "attnres_merge_stream_%s_c%d", d2 ? "d2" : "fm", nch);
  return slot_function(st, st.merge_stream[(d2 ? 0 : kStreamMaxChunks) + (nch - 1)], kMergePart, name, f);
}

int get_merge(DeviceState& st, bool pbf, bool ibf, int v, int block, hipFunction_t* f, int* bpc) {
  char name[96];
  snprintf(name, sizeof(name), "attnres_merge_%s_%s_v%d", pbf ? "bf" : "f32", ibf ? "bf" : "f32", v);
  return slot_get(st, st.merge[((pbf ? 0 : 2) + (ibf ? 0 : 1)) * 2 + (v - 1)], kMergePart, name, block, 0, f, bpc);
}

// Backward kernels: S <= 8 and the column reduce in part 4, S >= 9 in part 5.
int part_of_bwd(int s) { return s <= 8 ? 4 : 5; }
constexpr int kReducePart = 4;

// Kernels with addend rows (_add): parts 8 (S <= 4 and the row-per-wave ones) and 9.
int part_of_bwd_add(int s) { return s <= 4 ? 8 : 9; }
constexpr int kBwdStreamAddPart = 8;

int get_bwd(DeviceState& st, bool bf, bool gbf, int s, int v, int block, size_t lds, hipFunction_t* f, int* bpc,
            bool add = false) {
  const int idx = (((bf ? 0 : 2) + (gbf ? 0 : 1)) * kNumS + s) * 2 + (v - 1);
  char name[96];
  snprintf(name, sizeof(name), "attnres_route_bwd_%s_g%s_s%d_v%d%s", bf ? "bf" : "f32", gbf ? "bf" : "f32", s, v,
           add ? "_add" : "");
  return slot_get(st, add ? st.bwd_add[idx] : st.bwd[idx], add ? part_of_bwd_add(s) : part_of_bwd(s), name, block,
                  lds, f, bpc);
}

// Row-per-wave backward (code-object part 4): bf16 sources and output
// gradients, rows of 6 KiB (hidden 3072, S <= 8, source rows kept in
// registers) or 8 KiB (hidden 4096, S <= 9; from S = 7 the first S - 6 rows
// kept in LDS); a grid of one 4-wave workgroup per CU.  Chosen by the kernel
// policy; under AUTO for 6 KiB rows and at least 64 rows per CU (16 per
// wave).  Against the row-per-workgroup kernel it measured 1-7% faster at
// every S at 128 rows per CU (the 3B prefill shape), even to 3.5% faster at
// 64, mixed at 32 (up to 5% slower at S <= 5) and up to 6% slower at 16; at
// 8 KiB rows the same within 1-2% and 19% slower at S = 2, so AUTO keeps the
// workgroup kernel there.
constexpr int kBwdStreamWaves = 4;
// the query (nch * 2 KiB) and the LDS-kept rows, or at the end the waves' query-gradient rows
size_t bwd_stream_lds(int nch, int num_sources) {
  const size_t kl = num_sources > 48 / nch ? (size_t)(num_sources - 48 / nch) : 0;
  const size_t run = (size_t)nch * 2048 + (size_t)kBwdStreamWaves * kl * (size_t)nch * 1024;
  const size_t end = (size_t)kBwdStreamWaves * (size_t)nch * 2048;
  return run > end ? run : end;
}
// Row KiB of the row-per-wave backward for this call, or 0 for the
// row-per-workgroup kernel (also when its dynamic LDS exceeds the device's
// per-workgroup limit, so that the launch and the kernel-name query agree).
int bwd_stream_nch(bool bf, bool gbf, int num_sources, int hidden, int64_t num_tokens, int num_cus, int max_lds) {
  if (!bf || !gbf || hidden % 512 != 0) return 0;
  const int nch = hidden / 512;
  if ((nch != 6 && nch != 8) || num_sources < 1 || num_sources > (nch == 6 ? 8 : 9)) return 0;
  if (num_tokens >= (int64_t)1 << 31) return 0;  // 32-bit row counters
  if (bwd_stream_lds(nch, num_sources) > (size_t)max_lds) return 0;
  const int policy = g_policy.load(std::memory_order_relaxed);
  const int want = policy == ATTNRES_POLICY_STREAM ? 1 : policy == ATTNRES_POLICY_WORKGROUP ? 0 : tuning().stream;
  return want == 1 || (want < 0 && nch == 6 && num_tokens >= 64LL * num_cus) ? nch : 0;
}

int get_bwd_stream(DeviceState& st, int nch, int s, hipFunction_t* f, bool add = false) {
  char name[96];
  snprintf(name, sizeof(name), "attnres_route_bwd_stream_c%d_s%d%s", nch, s, add ? "_add" : "");
  const int idx = (nch == 8 ? 10 : 0) + s;
  return slot_function(st, add ? st.bwd_stream_add[idx] : st.bwd_stream[idx], add ? kBwdStreamAddPart : 4, name, f);
}

// Deferred block gradients (code-object part 10): the row-per-wave backward
// forming only the partial's gradient (attnres_route_bwd_stream_c<NCH>_s<S>_defer,
// S >= 2) and the sums of the blocks' terms
// (attnres_route_bwd_gather_seg_c<NCH>_b<NB>).
constexpr int kDeferPart = 10;
// The row widths of the deferred path: hidden 3072, 4096, 1024 and 512 (rows of
// 6, 8, 2 and 1 KiB), the reference's 3B, 8B, 1B and proxy models.
bool defer_hidden(int hidden) { return hidden == 3072 || hidden == 4096 || hidden == 1024 || hidden == 512; }
int defer_width(int nch) { return nch == 6 ? 0 : nch == 8 ? 1 : nch == 2 ? 2 : 3; }
int get_bwd_defer(DeviceState& st, int nch, int s, hipFunction_t* f) {
  char name[96];
  snprintf(name, sizeof(name), "attnres_route_bwd_stream_c%d_s%d_defer", nch, s);
  return slot_function(st, st.bwd_defer[defer_width(nch) * 10 + s], kDeferPart, name, f);
}
int get_gather_seg(DeviceState& st, int nch, int nb, hipFunction_t* f) {
  char name[96];
  snprintf(name, sizeof(name), "attnres_route_bwd_gather_seg_c%d_b%d", nch, nb);
  return slot_function(st, st.gather_seg[defer_width(nch) * ATTNRES_SEG_MAX_BLOCKS + nb - 1], kDeferPart, name, f);
}
// Row parts per token of the segment kernel (each wave takes one) and the
// waves per SIMD each instance is compiled for (workgroups per CU), as the
// instances in attnres_kernels.hip.
// Parts per row and workgroups per CU of the segment kernel for (nch, nb),
// from the instance table the kernels are compiled from.
int gather_seg_parts(int nch, int nb) {
#define ATTNRES_SEG_PARTS(NCH, NB, CPW, DEPTH, WPE) \
  if (nch == NCH && nb == NB) return NCH / CPW;
  ATTNRES_SEG_INSTANCES(ATTNRES_SEG_PARTS)
#undef ATTNRES_SEG_PARTS
  return 0;
}
int gather_seg_per_cu(int nch, int nb) {
#define ATTNRES_SEG_WPE(NCH, NB, CPW, DEPTH, WPE) \
  if (nch == NCH && nb == NB) return WPE;
  ATTNRES_SEG_INSTANCES(ATTNRES_SEG_WPE)
#undef ATTNRES_SEG_WPE
  return 1;
}
// Row KiB of the deferred backward for this call, or 0 when it has no kernel
// (bf16 sources, output gradients and parameters; rows of 6 KiB with S <= 8
// or 8 KiB with S <= 9; at least one committed source).
int bwd_defer_nch(int src_dtype, int grad_out_dtype, int param_dtype, int num_sources, int hidden,
                  int64_t num_tokens) {
  if (src_dtype != ATTNRES_DTYPE_BF16 || grad_out_dtype != ATTNRES_DTYPE_BF16 || param_dtype != ATTNRES_DTYPE_BF16)
    return 0;
  if (!defer_hidden(hidden)) return 0;
  const int nch = hidden / 512;
  if (num_sources < 2 || num_sources > (nch == 8 ? 9 : 8)) return 0;
  if (num_tokens >= (int64_t)1 << 31) return 0;
  return nch;
}

// Batched-query backward kernels (code-object part 6).  Source-gradient
// accumulators are S * VEC * V fp32 registers per thread; the kernels exist
// where that stays within 72.
constexpr int kBwdMqPart = 6;
constexpr int kBwdMqgPart = 7;  // the matrix-core batched backward and query-gradient pass
bool bwd_mq_available(bool bf, int s, int v) {
  const int vec = bf ? 8 : 4;
  return s >= 1 && s <= ATTNRES_KMAX_SOURCES && (v == 1 || v == 2) && s * vec * v <= 72;
}

int get_bwd_mq(DeviceState& st, bool bf, bool gbf, int s, int v, int block, hipFunction_t* f, int* bpc) {
  const int idx = (((bf ? 0 : 2) + (gbf ? 0 : 1)) * kNumS + s) * 2 + (v - 1);
  char name[96];
  snprintf(name, sizeof(name), "attnres_route_bwd_mq_%s_g%s_s%d_v%d", bf ? "bf" : "f32", gbf ? "bf" : "f32", s, v);
  return slot_get(st, st.bwd_mq[idx], kBwdMqPart, name, block, 0, f, bpc);
}

// bf16 sources: the matrix-core variant (part 7) unless ATTNRES_MQG=0.
int get_bwd_dqw(DeviceState& st, bool bf, int v, int block, hipFunction_t* f, int* bpc) {
  char name[96];
  const bool mfma = bf && tuning().mqg != 0;
  if (mfma) {
    snprintf(name, sizeof(name), "attnres_route_bwd_dqwm_bf_v%d", v);
  } else {
    snprintf(name, sizeof(name), "attnres_route_bwd_dqw_%s_v%d", bf ? "bf" : "f32", v);
  }
  return slot_get(st, st.bwd_dqw[(bf ? 0 : 2) + (v - 1)], mfma ? kBwdMqgPart : kBwdMqPart, name, block, 0, f, bpc);
}

// Batched-query backward on the matrix cores (code-object part 7): bf16
// sources, output gradients and parameters, 1 <= S <= 8, Q <= 8, two chunks
// per thread in workgroups of at most 256 threads, the Q folded queries in
// `lds` bytes of dynamic LDS.
constexpr int kBwdMqgMaxThreads = 256;
bool bwd_mqg_shape(bool bf, bool gbf, bool pbf, int s, int nq, int nchunk) {
  return tuning().mqg != 0 && bf && gbf && pbf && s >= 1 && s <= 8 && nq >= 1 && nq <= 8 &&
         ((nchunk + 1) / 2 + 63) / 64 * 64 <= kBwdMqgMaxThreads;
}

int get_bwd_mqg(DeviceState& st, int s, int nq4, int block, size_t lds, hipFunction_t* f, int* bpc) {
  char name[96];
  snprintf(name, sizeof(name), "attnres_route_bwd_mqg_s%d_q%d", s, nq4);
  return slot_get(st, st.bwd_mqg[(nq4 - 1) * 9 + s], kBwdMqgPart, name, block, lds, f, bpc);
}

int get_merge_bwd(DeviceState& st, bool pbf, bool ibf, int v, int block, hipFunction_t* f, int* bpc) {
  char name[96];
  snprintf(name, sizeof(name), "attnres_merge_bwd_%s_%s_v%d", pbf ? "bf" : "f32", ibf ? "bf" : "f32", v);
  return slot_get(st, st.merge_bwd[((pbf ? 0 : 2) + (ibf ? 0 : 1)) * 2 + (v - 1)], kReducePart, name, block, 0, f,
                  bpc);
}

int get_reduce(DeviceState& st, ReduceFns* out) {
  int rc = slot_function(st, st.reduce_stage, kReducePart, "attnres_reduce_dqw_stage", &out->stage);
  if (rc == ATTNRES_OK) rc = slot_function(st, st.reduce_cols, kReducePart, "attnres_reduce_dqw_cols", &out->cols);
  if (rc == ATTNRES_OK) rc = slot_function(st, st.reduce_fin, kReducePart, "attnres_reduce_dqw", &out->fin);
  return rc;
}

inline int round64(int64_t t) { return (int)(((t + 63) / 64) * 64); }
inline int round16(int64_t t) { return (int)(((t + 15) / 16) * 16); }

// Dynamic LDS of the batched-query matrix-core backward: the folded queries in
// query slots of four, chunks in blocks of 16 ([chunk/16][slot][chunk%16]).
inline size_t mqg_lds_bytes(int num_queries, int nchunk) {
  return (size_t)((num_queries + 3) / 4 * 4) * (size_t)round16(nchunk) * 16;
}

// Chunks per thread V and the workgroup size for a row of `nchunk` 16-byte
// chunks.  Returns 0 when no variant fits in kMaxThreads.
int pick_v(int64_t n_tokens, int nchunk, int num_cus, int* block) {
  const int t1 = round64(nchunk);
  const int t2 = round64((nchunk + 1) / 2);
  const bool ok1 = t1 <= kMaxThreads, ok2 = t2 <= kMaxThreads;
  int v = 0;
  const int force = tuning().force_v;
  if (force == 1 && ok1) v = 1;
  else if (force == 2 && ok2) v = 2;
  else if (!ok1) v = ok2 ? 2 : 0;
  else if (!ok2) v = 1;
  else if (n_tokens < 2LL * num_cus) v = 1;  // few rows (decode): more threads per row
  else v = (t2 >= 128) ? 2 : 1;              // prefill: two chunks per thread if >= 2 waves remain
  *block = v == 1 ? t1 : t2;
  return v;
}

int grid_for(int64_t n_tokens, int num_cus, int bpc) {
  double g = (double)num_cus * bpc * tuning().grid_mult;
  int64_t grid = (int64_t)g;
  if (grid < 1) grid = 1;
  if (grid > n_tokens) grid = n_tokens;
  if (grid > 0x7fffffff) grid = 0x7fffffff;
  return (int)grid;
}

// Chunks per thread of the single-query backward: one where the row fits in
// one workgroup, except 5 <= S <= 8 over many rows of at most 384 chunks:
// there two (half the waves per row) measured 2-4% faster per call at the 3B
// prefill shape (32768 rows), while at 8192 rows and for 512-chunk rows two
// measured 1-2% slower (and the two-chunk instances spill from S = 12).
// ATTNRES_V=1 / 2 force one or two.
int bwd_chunks_per_thread(int nchunk, int num_sources, int64_t num_tokens, int num_cus) {
  const bool fits1 = round64(nchunk) <= kMaxThreads;
  int v = fits1 ? 1 : 2;
  if (v == 1 && num_sources >= 5 && num_sources <= 8 && nchunk <= 384 && num_tokens >= 64LL * num_cus) v = 2;
  if (tuning().force_v == 2) v = 2;
  if (tuning().force_v == 1 && fits1) v = 1;
  return v;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

bool valid_dtype(int d) { return d == ATTNRES_DTYPE_F32 || d == ATTNRES_DTYPE_BF16; }

int esize(int d) { return d == ATTNRES_DTYPE_BF16 ? 2 : 4; }

template <typename Params>
int launch(hipFunction_t f, int grid, int block, Params& P, void* stream, int grid_y = 1, size_t lds = 0) {
  size_t sz = sizeof(Params);
  void* cfg[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, &P, HIP_LAUNCH_PARAM_BUFFER_SIZE, &sz, HIP_LAUNCH_PARAM_END};
  hipError_t e = hipModuleLaunchKernel(f, (unsigned)grid, (unsigned)grid_y, 1, (unsigned)block, 1, 1, (unsigned)lds,
                                       (hipStream_t)stream, nullptr, cfg);
  if (e != hipSuccess) return hip_fail(e, "hipModuleLaunchKernel");
  return ATTNRES_OK;
}

// Which kernel a routing call runs: the row-per-wave streaming kernel (one
// query, S >= 1, a row of whole KiB up to 8 KiB, enough rows to give every
// wave of the chip several, or forced by the policy) or the row-per-workgroup
// kernel with V chunks per thread.
struct RouteChoice {
  bool stream = false;
  int combo = 0;
  int nch = 0;    // streaming: KiB per row
  int variant = kStreamPlain;  // streaming: plain / pointer table / fused
  int v = 0;      // workgroup: chunks per thread (0: no shape fits)
  int block = 0;  // threads per workgroup
  size_t qg_lds = 0;  // > 0: the batched-query kernel, with this much dynamic LDS
};

// The batched-query kernel takes Q >= 2 queries over bf16 sources with bf16
// parameters and a bf16 output, with the Q folded queries staged in LDS.
void choose_qg(RouteChoice& ch, int num_sources, int num_queries, int hidden, int out_dtype, int mode, int max_lds) {
  if (ch.stream || ch.v == 0 || ch.combo != kBfDot2 || num_queries < 2 || num_sources < 1 ||
      out_dtype != ATTNRES_DTYPE_BF16 || mode != ATTNRES_MODE_PLAIN || tuning().qg == 0)
    return;
  const size_t lds = (size_t)num_queries * (size_t)(hidden / 8) * 16;
  if (lds + kQgStaticLds <= (size_t)max_lds) ch.qg_lds = lds;
}

// Waves per workgroup of the streaming kernels (one workgroup per CU), one
// per SIMD.  Each wave requests its next row only once the current one has
// arrived, so a CU keeps one row per wave in flight, and the HBM serves this
// stream best with about 24-28 KiB per CU in flight: four waves up to 7 KiB
// rows (3B shape, S = 8: 86.3% of peak against 79.5% with three; 7 KiB rows
// at S = 9: 82.0% against 80.4%; 5 KiB 80.2% against 67%), three for
// 8 KiB rows (8B shape, S = 9: 84.8% against 80.6%).  The fused variants
// keep four at 8 KiB (8B schedule arena prefill 11.39 against 11.44 ms).
// (An earlier pipeline that requested the next row before the current one
// arrived kept up to two rows per wave in flight and ran best with three
// waves from S = 6.)
int stream_waves_for(int row_kib, bool fused) {
  if (tuning().stream_waves > 0) return tuning().stream_waves;
  return !fused && row_kib >= 8 ? 3 : kStreamWaves;
}

// Workgroups per CU of a streaming launch (0: the occupancy limit).  One
// 4-wave workgroup per CU is best from 6 KiB rows (above), but a wave of a
// narrow row keeps too few bytes in flight: bf16 routing steps (S = 2 and 8,
// 8192-131072 rows) ran at 2.3-2.7 TB/s with one workgroup per CU at 1 KiB
// rows and 5.0-6.6 TB/s with eight; at 2 KiB rows 3.8-4.3 TB/s against
// 5.3-6.3 with two to four (four best for the fused steps at 8192-32768
// rows, two for the others); at 3-4 KiB rows the fused steps gained 5-35%
// with two, while the routing calls that stage their output rows lost 1-6%.
double stream_per_cu_for(int row_kib, bool fused) {
  if (tuning().stream_per_cu >= 0.0) return tuning().stream_per_cu;
  if (row_kib <= 1) return 8.0;
  if (row_kib == 2) return fused ? 4.0 : 2.0;
  if (row_kib <= 4) return fused ? 2.0 : 1.0;
  return 1.0;
}

RouteChoice choose_route(int num_sources, int64_t num_tokens, int hidden, int src_dtype, int param_dtype,
                         int num_queries, int num_cus, bool stream_ok, bool fused) {
  RouteChoice ch;
  const bool bf = src_dtype == ATTNRES_DTYPE_BF16;
  ch.combo = bf ? (param_dtype == ATTNRES_DTYPE_BF16 ? kBfDot2 : kBfFma) : kF32Fma;
  const int64_t row_bytes = (int64_t)hidden * esize(src_dtype);
  ch.nch = (int)(row_bytes / 1024);
  // The streaming kernel uses 32-bit row/item counters.
  const bool stream_shape = num_queries == 1 && num_sources >= 1 && row_bytes % 1024 == 0 && ch.nch >= 1 &&
                            ch.nch <= kStreamMaxChunks && stream_ok &&
                            num_tokens * (int64_t)num_sources < (int64_t)1 << 31;
  const int policy = g_policy.load(std::memory_order_relaxed);
  const int want_stream = policy == ATTNRES_POLICY_STREAM      ? 1
                          : policy == ATTNRES_POLICY_WORKGROUP ? 0
                                                               : tuning().stream;
  ch.stream = stream_shape && (want_stream == 1 || (want_stream < 0 && num_tokens >= tuning().stream_min_tokens));
  if (ch.stream) {
    ch.block = 64 * stream_waves_for(ch.nch, fused);
  } else {
    ch.v = pick_v(num_tokens, hidden / (bf ? 8 : 4), num_cus, &ch.block);
  }
  return ch;
}

// The whole kernel choice of one routing call (family, streaming variant,
// chunks per thread, batched-query kernel), shared by the launch and the
// kernel-name query.  The streaming kernel addresses equally spaced sources
// as base + s*stride and any others through the kernel-argument pointer table;
// it shares one delta buffer between its two pipeline slots, which needs
// S >= 2 when accumulating into the partial (S = 1 accumulate calls run the
// workgroup kernel).
RouteChoice plan_route(int num_sources, int64_t num_tokens, int hidden, int src_dtype, int param_dtype,
                       int out_dtype, int num_queries, int mode, bool equally_spaced, const DeviceState& st) {
  const bool stream_ok = !(mode == ATTNRES_MODE_ACCUM && num_sources < 2);
  RouteChoice ch = choose_route(num_sources, num_tokens, hidden, src_dtype, param_dtype, num_queries, st.num_cus,
                                stream_ok, mode != ATTNRES_MODE_PLAIN);
  if (ch.stream) {
    const bool spaced = equally_spaced || num_sources < 2;
    ch.variant = mode != ATTNRES_MODE_PLAIN ? (spaced ? kStreamFused : kStreamFusedTable)
                 : spaced ? kStreamPlain
                          : kStreamTable;
  } else if (ch.v != 0) {
    choose_qg(ch, num_sources, num_queries, hidden, out_dtype, mode, st.max_lds);
  }
  return ch;
}

void kernel_name_of(const RouteChoice& ch, int num_sources, int num_queries, bool out_bf, char* buf, size_t n) {
  static const char* combo_names[kTypeCombos] = {"bf_d2", "bf_fm", "f32_fm"};
  if (ch.stream) {
    snprintf(buf, n, "attnres_stream_%s_o%s_c%d_%s", combo_names[ch.combo], out_bf ? "bf" : "f32", ch.nch,
             kStreamVariantNames[ch.variant]);
  } else {
    snprintf(buf, n, "attnres_route_%s_s%d_v%d_%s", combo_names[ch.combo], num_sources, ch.v,
             ch.qg_lds > 0 ? "qg" : num_queries > 1 ? "qn" : "q1");
  }
}

// Shared validation + launch of the route kernel.  `mode`/`delta` are the
// fused partial-update inputs of attnres_block_step.
// The kernel choice of one merge call, shared by the launch and the name
// query: the row-per-wave kernel for bf16 rows of whole 1 KiB chunks (at most
// kStreamMaxChunks) over enough rows (the routing kernels' policy and
// threshold), one workgroup of four waves per CU; else one workgroup per row.
struct MergeChoice {
  bool stream = false;
  int nch = 0;    // row KiB (row-per-wave kernel)
  int v = 0;      // chunks per thread (row-per-workgroup kernel); 0: no launch shape
  int block = 0;  // threads per workgroup
};
MergeChoice plan_merge(int64_t num_tokens, int hidden, int partial_dtype, int inter_dtype, const DeviceState& st) {
  MergeChoice ch;
  const bool pbf = partial_dtype == ATTNRES_DTYPE_BF16, ibf = inter_dtype == ATTNRES_DTYPE_BF16;
  const int64_t row_bytes = (int64_t)hidden * 2;
  ch.nch = (int)(row_bytes / 1024);
  const bool stream_shape = tuning().merge_stream != 0 && pbf && ibf && row_bytes % 1024 == 0 && ch.nch >= 1 &&
                            ch.nch <= kStreamMaxChunks && num_tokens < (int64_t)1 << 31;
  const int policy = g_policy.load(std::memory_order_relaxed);
  const int want_stream = policy == ATTNRES_POLICY_STREAM      ? 1
                          : policy == ATTNRES_POLICY_WORKGROUP ? 0
                                                               : tuning().stream;
  ch.stream = stream_shape && (want_stream == 1 || (want_stream < 0 && num_tokens >= tuning().stream_min_tokens));
  if (ch.stream) {
    ch.block = 64 * (tuning().stream_waves > 0 ? tuning().stream_waves : kStreamWaves);
  } else {
    ch.v = pick_v(num_tokens, hidden / (pbf ? 8 : 4), st.num_cus, &ch.block);
  }
  return ch;
}

int route_launch(const void* const* sources, int num_sources, int64_t num_tokens, int hidden, int64_t src_ld,
                 int src_dtype, const void* query, const void* gain, int num_queries, int param_dtype, float eps,
                 void* out, int out_dtype, int64_t out_ld, int64_t out_qstride, float* weights, float* lse,
                 float* inv_rms, float* logits, int mode, const void* delta, int64_t delta_ld, void* stream,
                 void* partial_out = nullptr) {
  if (num_sources < 0 || num_sources > ATTNRES_MAX_SOURCES)
    return fail(ATTNRES_ERR_UNSUPPORTED, "num_sources=%d outside [0, %d]", num_sources, ATTNRES_MAX_SOURCES);
  if (num_sources > 0 && sources == nullptr) return fail(ATTNRES_ERR_ARG, "sources is NULL");
  if (num_tokens < 0) return fail(ATTNRES_ERR_ARG, "num_tokens=%lld < 0", (long long)num_tokens);
  if (hidden <= 0) return fail(ATTNRES_ERR_ARG, "hidden=%d <= 0", hidden);
  if (!valid_dtype(src_dtype) || !valid_dtype(param_dtype) || !valid_dtype(out_dtype))
    return fail(ATTNRES_ERR_ARG, "unknown dtype code (src=%d param=%d out=%d)", src_dtype, param_dtype, out_dtype);
  if (query == nullptr) return fail(ATTNRES_ERR_ARG, "query is NULL");
  if (num_queries < 1) return fail(ATTNRES_ERR_ARG, "num_queries=%d < 1", num_queries);
  if (out == nullptr) return fail(ATTNRES_ERR_ARG, "out is NULL");
  if (!std::isfinite(eps)) return fail(ATTNRES_ERR_ARG, "eps is not finite");
  const bool bf = src_dtype == ATTNRES_DTYPE_BF16;
  const int vec = bf ? 8 : 4;
  if (hidden % vec != 0)
    return fail(ATTNRES_ERR_UNSUPPORTED, "hidden=%d is not a multiple of %d (16-byte chunks)", hidden, vec);
  const int nchunk = hidden / vec;
  if (round64((nchunk + 1) / 2) > kMaxThreads)
    return fail(ATTNRES_ERR_UNSUPPORTED, "hidden=%d exceeds the largest supported row (%d elements)", hidden,
                2 * kMaxThreads * vec);
  if (src_ld < hidden) return fail(ATTNRES_ERR_ARG, "src_ld=%lld < hidden=%d", (long long)src_ld, hidden);
  if ((src_ld * esize(src_dtype)) % 16 != 0) return fail(ATTNRES_ERR_ALIGN, "source row stride not 16-byte aligned");
  for (int s = 0; s < num_sources; ++s) {
    if (sources[s] == nullptr) return fail(ATTNRES_ERR_ARG, "sources[%d] is NULL", s);
    if (!aligned16(sources[s])) return fail(ATTNRES_ERR_ALIGN, "sources[%d] not 16-byte aligned", s);
  }
  if (out_ld < hidden) return fail(ATTNRES_ERR_ARG, "out_ld=%lld < hidden=%d", (long long)out_ld, hidden);
  const int out_es = esize(out_dtype);
  const int out_chunk_bytes = vec * out_es;  // bytes of one output chunk
  const int out_align = out_chunk_bytes >= 16 ? 16 : out_chunk_bytes;
  if (((uintptr_t)out % out_align) != 0 || ((out_ld * out_es) % out_align) != 0)
    return fail(ATTNRES_ERR_ALIGN, "out rows not %d-byte aligned", out_align);
  if (num_queries > 1) {
    if (out_qstride < num_tokens * out_ld)
      return fail(ATTNRES_ERR_ARG, "out_qstride=%lld overlaps query outputs", (long long)out_qstride);
    if ((out_qstride * out_es) % out_align != 0) return fail(ATTNRES_ERR_ALIGN, "out_qstride not aligned");
  }
  if (mode != ATTNRES_MODE_PLAIN) {
    if (num_sources < 1 || num_queries != 1) return fail(ATTNRES_ERR_ARG, "partial update needs S >= 1 and one query");
    if (delta == nullptr) return fail(ATTNRES_ERR_ARG, "delta is NULL");
    if (!aligned16(delta) || (delta_ld * esize(src_dtype)) % 16 != 0)
      return fail(ATTNRES_ERR_ALIGN, "delta rows not 16-byte aligned");
    if (partial_out != nullptr && !aligned16(partial_out))
      return fail(ATTNRES_ERR_ALIGN, "partial_out not 16-byte aligned");
  }
  if (num_tokens == 0) return ATTNRES_OK;

  DeviceState* st = nullptr;
  int rc = ensure_loaded(&st);
  if (rc != ATTNRES_OK) return rc;

  // Equally spaced sources (stacked buffers, arenas) get one base + stride.
  int64_t src_stride = 0;
  bool equally_spaced = true;
  if (num_sources >= 2) {
    src_stride = (int64_t)((uintptr_t)sources[1] - (uintptr_t)sources[0]);
    for (int s = 2; s < num_sources && equally_spaced; ++s)
      equally_spaced = (int64_t)((uintptr_t)sources[s] - (uintptr_t)sources[0]) == src_stride * s;
  }
  const RouteChoice ch = plan_route(num_sources, num_tokens, hidden, src_dtype, param_dtype, out_dtype, num_queries,
                                    mode, equally_spaced, *st);
  if (!ch.stream && ch.v == 0) return fail(ATTNRES_ERR_UNSUPPORTED, "hidden=%d has no launch shape", hidden);

  hipFunction_t f = nullptr;
  int bpc = 1;
  int block = ch.block;
  int64_t work_units = num_tokens;  // rows per workgroup-slot of the grid
  int out_batch = 1;
  size_t stream_lds = 0;
  if (ch.stream) {
    int slds = 0;
    rc = get_stream(*st, ch.combo, out_dtype == ATTNRES_DTYPE_BF16, ch.nch, ch.variant, &f, &bpc, &slds);
    if (rc != ATTNRES_OK) return rc;
    const int waves = block / 64;
    work_units = (num_tokens + waves - 1) / waves;
    const int64_t out_row_bytes = (int64_t)hidden * esize(out_dtype);
    // the fused variants write their partial rows back as they go: batching
    // the output rows alone measured 1-2% slower there
    out_batch = (ch.variant == kStreamFused || ch.variant == kStreamFusedTable)
                    ? 1
                    : stream_out_batch(num_sources, out_row_bytes, slds, st->max_lds, waves);
    if (out_batch > 1) stream_lds = (size_t)waves * out_batch * out_row_bytes;
  } else if (ch.qg_lds > 0) {
    rc = get_route_qg(*st, num_sources, ch.v, block, ch.qg_lds, &f, &bpc);
    if (rc != ATTNRES_OK) return rc;
  } else {
    rc = get_route(*st, ch.combo, num_sources, ch.v, num_queries > 1, block, &f, &bpc);
    if (rc != ATTNRES_OK) return rc;
  }

  attnres_route_params P;
  std::memset(&P, 0, sizeof(P));
  for (int s = 0; s < num_sources; ++s) P.src[s] = sources[s];
  P.query = query;
  P.gain = gain;
  P.delta = delta;
  P.partial_out = partial_out;
  P.out = out;
  P.weights = weights;
  P.lse = lse;
  P.inv_rms = inv_rms;
  P.logits = logits;
  P.n_tokens = num_tokens;
  P.src_ld = src_ld;
  P.delta_ld = delta_ld;
  P.out_ld = out_ld;
  P.out_qstride = out_qstride;
  P.src_stride = src_stride;
  P.d = hidden;
  P.nchunk = nchunk;
  P.num_queries = num_queries;
  P.param_bf16 = param_dtype == ATTNRES_DTYPE_BF16;
  P.out_bf16 = out_dtype == ATTNRES_DTYPE_BF16;
  P.mode = mode;
  P.num_sources = num_sources;
  P.block = block;
  P.out_batch = out_batch;
  P.eps = eps;
  P.inv_d = 1.0f / (float)hidden;
  // The streaming kernels run one 4-wave workgroup per CU from 6 KiB rows: at
  // the occupancy limit (up to four per CU) four times the requests are in
  // flight and the same traffic measured 4-6% slower; narrower rows run more
  // (stream_per_cu_for).
  int grid = grid_for(work_units, st->num_cus, bpc);
  const double per_cu =
      ch.stream ? stream_per_cu_for(ch.nch, ch.variant == kStreamFused || ch.variant == kStreamFusedTable) : 0.0;
  if (per_cu > 0.0) {
    int64_t g = (int64_t)(st->num_cus * (per_cu < bpc ? per_cu : (double)bpc));
    if (g < 1) g = 1;
    if (g > work_units) g = work_units;
    grid = (int)g;
  }
  return launch(f, grid, block, P, stream, 1, ch.stream ? stream_lds : ch.qg_lds);
}

// Query/gain gradients from `nparts` per-workgroup partial rows in
// `workspace`: summed in 64-row blocks (stage 1, in place), then the block
// sums (final stage); a fixed order, so the result is deterministic.
int reduce_launch(const ReduceFns& fn, void* workspace, int nparts, int hidden, const void* query,
                  const void* gain, int param_dtype, void* grad_query, void* grad_gain, void* stream,
                  int num_queries = 1) {
  attnres_reduce_params R;
  std::memset(&R, 0, sizeof(R));
  R.part = static_cast<float*>(workspace);
  R.query = query;
  R.gain = gain;
  R.dquery = grad_query;
  R.dgain = grad_gain;
  R.nparts = nparts;
  R.part_step = 1;
  R.d = hidden;
  R.param_bf16 = param_dtype == ATTNRES_DTYPE_BF16;
  R.num_queries = num_queries;
  const int64_t width = (int64_t)hidden * num_queries;
  // one launch (32 columns per 1024-thread workgroup) for up to four queries
  // where its byte offsets, up to 1024 rows past the last partial row, fit in
  // 32 bits; else two
  if (!tuning().reduce_two_stage && num_queries <= 4 && (int64_t)(nparts + 1024) * width * 4 < (int64_t)1 << 32)
    return launch(fn.cols, (hidden + 31) / 32, 1024, R, stream);
  if (nparts > 64) {
    int rc = launch(fn.stage, (int)((width + 63) / 64), 256, R, stream, (nparts + 63) / 64);
    if (rc != ATTNRES_OK) return rc;
    R.part_step = 64;
  }
  return launch(fn.fin, (hidden + 255) / 256, 256, R, stream);
}

}  // namespace

// Device address of the no-alloc entry point's scratch array on the current
// device, resolved once per device (attnres_noalloc.hip).
extern "C" int attnres_internal_scratch_setup(void);

extern "C" {

// Sets attnres_last_error() for attnres_noalloc.hip; returns `code`.
__attribute__((visibility("hidden"))) int attnres_internal_fail(int code, const char* msg) {
  return fail(code, "%s", msg);
}

int attnres_version(void) { return 10000; }

int attnres_max_sources(void) { return ATTNRES_MAX_SOURCES; }

const char* attnres_last_error(void) { return g_err.c_str(); }

int attnres_route_kernel_name(int num_sources, int64_t num_tokens, int hidden, int src_dtype, int param_dtype,
                              int out_dtype, int num_queries, int fused, int equally_spaced, char* buf,
                              int buf_len) {
  if (buf == nullptr || buf_len < 1) return fail(ATTNRES_ERR_ARG, "no output buffer");
  if (!valid_dtype(src_dtype) || !valid_dtype(param_dtype) || !valid_dtype(out_dtype))
    return fail(ATTNRES_ERR_ARG, "unknown dtype code");
  if (num_sources < 0 || num_sources > ATTNRES_MAX_SOURCES || hidden <= 0 || num_queries < 1)
    return fail(ATTNRES_ERR_ARG, "bad shape");
  if (fused < 0 || fused > 2) return fail(ATTNRES_ERR_ARG, "fused=%d is not 0, 1 or 2", fused);
  DeviceState* st = nullptr;
  int rc = ensure_loaded(&st);
  if (rc != ATTNRES_OK) return rc;
  const int mode = fused == 0 ? ATTNRES_MODE_PLAIN : fused == 1 ? ATTNRES_MODE_ACCUM : ATTNRES_MODE_SET;
  const RouteChoice ch = plan_route(num_sources, num_tokens, hidden, src_dtype, param_dtype, out_dtype, num_queries,
                                    mode, equally_spaced != 0, *st);
  if (!ch.stream && ch.v == 0) return fail(ATTNRES_ERR_UNSUPPORTED, "hidden=%d has no launch shape", hidden);
  kernel_name_of(ch, num_sources, num_queries, out_dtype == ATTNRES_DTYPE_BF16, buf, (size_t)buf_len);
  return ATTNRES_OK;
}

int attnres_merge_kernel_name(int64_t num_tokens, int hidden, int partial_dtype, int param_dtype, int inter_dtype,
                              char* buf, int buf_len) {
  if (buf == nullptr || buf_len < 1) return fail(ATTNRES_ERR_ARG, "no output buffer");
  if (!valid_dtype(partial_dtype) || !valid_dtype(param_dtype) || !valid_dtype(inter_dtype))
    return fail(ATTNRES_ERR_ARG, "unknown dtype code");
  if (num_tokens < 0 || hidden <= 0) return fail(ATTNRES_ERR_ARG, "bad shape");
  const int vec = partial_dtype == ATTNRES_DTYPE_BF16 ? 8 : 4;
  if (hidden % vec != 0) return fail(ATTNRES_ERR_UNSUPPORTED, "hidden=%d is not a multiple of %d", hidden, vec);
  if (num_tokens == 0) {  // attnres_merge_fwd launches nothing
    buf[0] = '\0';
    return ATTNRES_OK;
  }
  DeviceState* st = nullptr;
  int rc = ensure_loaded(&st);
  if (rc != ATTNRES_OK) return rc;
  const MergeChoice ch = plan_merge(num_tokens, hidden, partial_dtype, inter_dtype, *st);
  if (ch.stream) {
    snprintf(buf, (size_t)buf_len, "attnres_merge_stream_%s_c%d", param_dtype == ATTNRES_DTYPE_BF16 ? "d2" : "fm",
             ch.nch);
  } else if (ch.v != 0) {
    snprintf(buf, (size_t)buf_len, "attnres_merge_%s_%s_v%d", partial_dtype == ATTNRES_DTYPE_BF16 ? "bf" : "f32",
             inter_dtype == ATTNRES_DTYPE_BF16 ? "bf" : "f32", ch.v);
  } else {
    buf[0] = '\0';
  }
  return ATTNRES_OK;
}

int attnres_route_bwd_kernel_name(int num_sources, int64_t num_tokens, int hidden, int src_dtype, int grad_out_dtype,
                                  char* buf, int buf_len) {
  if (buf == nullptr || buf_len < 1) return fail(ATTNRES_ERR_ARG, "no output buffer");
  if (!valid_dtype(src_dtype) || !valid_dtype(grad_out_dtype)) return fail(ATTNRES_ERR_ARG, "unknown dtype code");
  if (num_sources < 1 || num_sources > ATTNRES_MAX_SOURCES || hidden <= 0 || num_tokens < 0)
    return fail(ATTNRES_ERR_ARG, "bad shape");
  const bool bf = src_dtype == ATTNRES_DTYPE_BF16;
  const int vec = bf ? 8 : 4;
  if (hidden % vec != 0) return fail(ATTNRES_ERR_UNSUPPORTED, "hidden=%d is not a multiple of %d", hidden, vec);
  DeviceState* st = nullptr;
  int rc = ensure_loaded(&st);
  if (rc != ATTNRES_OK) return rc;
  const int nch =
      bwd_stream_nch(bf, grad_out_dtype == ATTNRES_DTYPE_BF16, num_sources, hidden, num_tokens, st->num_cus,
                     st->max_lds);
  if (nch > 0) {
    snprintf(buf, (size_t)buf_len, "attnres_route_bwd_stream_c%d_s%d", nch, num_sources);
    return ATTNRES_OK;
  }
  const int v = bwd_chunks_per_thread(hidden / vec, num_sources, num_tokens, st->num_cus);
  snprintf(buf, (size_t)buf_len, "attnres_route_bwd_%s_g%s_s%d_v%d", bf ? "bf" : "f32",
           grad_out_dtype == ATTNRES_DTYPE_BF16 ? "bf" : "f32", num_sources, v);
  return ATTNRES_OK;
}

int attnres_route_bwd_queries_kernel_name(int num_sources, int hidden, int src_dtype, int param_dtype,
                                          int grad_out_dtype, int num_queries, char* buf, int buf_len) {
  if (buf == nullptr || buf_len < 1) return fail(ATTNRES_ERR_ARG, "no output buffer");
  if (!valid_dtype(src_dtype) || !valid_dtype(param_dtype) || !valid_dtype(grad_out_dtype))
    return fail(ATTNRES_ERR_ARG, "unknown dtype code");
  if (num_sources < 1 || num_sources > ATTNRES_MAX_SOURCES || hidden <= 0 || num_queries < 1)
    return fail(ATTNRES_ERR_ARG, "bad shape");
  const bool bf = src_dtype == ATTNRES_DTYPE_BF16;
  const int vec = bf ? 8 : 4;
  if (hidden % vec != 0) return fail(ATTNRES_ERR_UNSUPPORTED, "hidden=%d is not a multiple of %d", hidden, vec);
  DeviceState* st = nullptr;
  int rc = ensure_loaded(&st);
  if (rc != ATTNRES_OK) return rc;
  const int nchunk = hidden / vec;
  const int v = round64(nchunk) <= kMaxThreads ? 1 : 2;
  const bool gbf = grad_out_dtype == ATTNRES_DTYPE_BF16;
  const size_t lds = mqg_lds_bytes(num_queries, nchunk);
  if (bwd_mqg_shape(bf, gbf, param_dtype == ATTNRES_DTYPE_BF16, num_sources, num_queries, nchunk) &&
      lds + kMqgStaticLds <= (size_t)st->max_lds) {
    snprintf(buf, (size_t)buf_len, "attnres_route_bwd_mqg_s%d_q%d", num_sources, (num_queries + 3) / 4);
  } else if (bwd_mq_available(bf, num_sources, v)) {
    snprintf(buf, (size_t)buf_len, "attnres_route_bwd_mq_%s_g%s_s%d_v%d", bf ? "bf" : "f32", gbf ? "bf" : "f32",
             num_sources, v);
  } else {
    buf[0] = '\0';  // no batched kernel: attnres_route_bwd_queries returns ATTNRES_ERR_UNSUPPORTED
  }
  return ATTNRES_OK;
}

int attnres_set_kernel_policy(int policy) {
  if (policy != ATTNRES_POLICY_AUTO && policy != ATTNRES_POLICY_WORKGROUP && policy != ATTNRES_POLICY_STREAM)
    return fail(ATTNRES_ERR_ARG, "unknown kernel policy %d", policy);
  return g_policy.exchange(policy);
}

int attnres_init(void) {
  DeviceState* st = nullptr;
  int rc = ensure_loaded(&st);
  if (rc != ATTNRES_OK) return rc;
  return attnres_internal_scratch_setup();
}

int attnres_route_fwd(const void* const* sources, int num_sources, int64_t num_tokens, int hidden, int64_t src_ld,
                      int src_dtype, const void* query, const void* gain, int num_queries, int param_dtype, float eps,
                      void* out, int out_dtype, int64_t out_ld, int64_t out_qstride, float* weights, float* lse,
                      float* inv_rms, float* logits, void* stream) {
  return route_launch(sources, num_sources, num_tokens, hidden, src_ld, src_dtype, query, gain, num_queries,
                      param_dtype, eps, out, out_dtype, out_ld, out_qstride, weights, lse, inv_rms, logits,
                      ATTNRES_MODE_PLAIN, nullptr, 0, stream);
}

int attnres_merge_fwd(const void* partial, int64_t num_tokens, int hidden, int partial_dtype, const void* query,
                      int param_dtype, const void* inter, int inter_dtype, const float* inter_lse, float eps,
                      void* out, float* logit, float* inv_rms, void* stream) {
  if (partial == nullptr || query == nullptr || inter == nullptr || inter_lse == nullptr || out == nullptr)
    return fail(ATTNRES_ERR_ARG, "merge: partial, query, inter, inter_lse and out are required");
  if (num_tokens < 0) return fail(ATTNRES_ERR_ARG, "num_tokens=%lld < 0", (long long)num_tokens);
  if (hidden <= 0) return fail(ATTNRES_ERR_ARG, "hidden=%d <= 0", hidden);
  if (!valid_dtype(partial_dtype) || !valid_dtype(param_dtype) || !valid_dtype(inter_dtype))
    return fail(ATTNRES_ERR_ARG, "unknown dtype code");
  if (!std::isfinite(eps)) return fail(ATTNRES_ERR_ARG, "eps is not finite");
  const bool pbf = partial_dtype == ATTNRES_DTYPE_BF16;
  const bool ibf = inter_dtype == ATTNRES_DTYPE_BF16;
  const int vec = pbf ? 8 : 4;
  if (hidden % vec != 0)
    return fail(ATTNRES_ERR_UNSUPPORTED, "hidden=%d is not a multiple of %d (16-byte chunks)", hidden, vec);
  const int nchunk = hidden / vec;
  if (round64((nchunk + 1) / 2) > kMaxThreads)
    return fail(ATTNRES_ERR_UNSUPPORTED, "hidden=%d exceeds the largest supported row", hidden);
  const int inter_align = (vec * esize(inter_dtype)) >= 16 ? 16 : vec * esize(inter_dtype);
  if (!aligned16(partial) || ((uintptr_t)inter % inter_align) != 0 || ((uintptr_t)out % inter_align) != 0 ||
      ((int64_t)hidden * esize(inter_dtype)) % inter_align != 0)
    return fail(ATTNRES_ERR_ALIGN, "merge rows not aligned");
  if (num_tokens == 0) return ATTNRES_OK;

  DeviceState* st = nullptr;
  int rc = ensure_loaded(&st);
  if (rc != ATTNRES_OK) return rc;
  const MergeChoice ch = plan_merge(num_tokens, hidden, partial_dtype, inter_dtype, *st);
  if (!ch.stream && ch.v == 0) return fail(ATTNRES_ERR_UNSUPPORTED, "hidden=%d has no launch shape", hidden);
  const bool use_stream = ch.stream;
  const int block = ch.block;
  hipFunction_t f = nullptr;
  int bpc = 1;
  rc = use_stream ? get_merge_stream(*st, param_dtype == ATTNRES_DTYPE_BF16, ch.nch, &f)
                  : get_merge(*st, pbf, ibf, ch.v, block, &f, &bpc);
  if (rc != ATTNRES_OK) return rc;

  attnres_merge_params P;
  std::memset(&P, 0, sizeof(P));
  P.partial = partial;
  P.query = query;
  P.inter = inter;
  P.inter_lse = inter_lse;
  P.out = out;
  P.logit = logit;
  P.inv_rms = inv_rms;
  P.n_tokens = num_tokens;
  P.partial_ld = hidden;
  P.inter_ld = hidden;
  P.out_ld = hidden;
  P.d = hidden;
  P.nchunk = nchunk;
  P.param_bf16 = param_dtype == ATTNRES_DTYPE_BF16;
  P.inter_bf16 = ibf;
  P.block = block;
  P.eps = eps;
  P.inv_d = 1.0f / (float)hidden;
  if (use_stream) {
    // one workgroup per CU, fewer when there are fewer rows than waves
    const int64_t need = (num_tokens + block / 64 - 1) / (block / 64);
    return launch(f, (int)(need < st->num_cus ? need : st->num_cus), block, P, stream);
  }
  return launch(f, grid_for(num_tokens, st->num_cus, bpc), block, P, stream);
}

int attnres_block_step(void* arena, int num_slots, int64_t slot_stride, int n_committed, int commit,
                       const void* delta, int64_t num_tokens, int hidden, int dtype, const void* query,
                       const void* gain, int param_dtype, float eps, void* out, float* weights, float* lse,
                       void* stream) {
  if (arena == nullptr) return fail(ATTNRES_ERR_ARG, "arena is NULL");
  if (num_slots < 1) return fail(ATTNRES_ERR_ARG, "num_slots=%d < 1", num_slots);
  if (commit != 0 && commit != 1) return fail(ATTNRES_ERR_ARG, "commit=%d is not 0 or 1", commit);
  if (n_committed < 0) return fail(ATTNRES_ERR_ARG, "n_committed=%d < 0", n_committed);
  const int S = n_committed + commit + 1;
  if (S > num_slots)
    return fail(ATTNRES_ERR_ARG, "partial slot %d outside the arena (%d slots)", S - 1, num_slots);
  if (S > ATTNRES_MAX_SOURCES)
    return fail(ATTNRES_ERR_UNSUPPORTED, "%d sources exceed the maximum %d", S, ATTNRES_MAX_SOURCES);
  if (commit && delta == nullptr) return fail(ATTNRES_ERR_ARG, "a commit needs the new partial block (delta)");
  if (!valid_dtype(dtype)) return fail(ATTNRES_ERR_ARG, "unknown dtype code %d", dtype);
  if (num_tokens < 0 || hidden <= 0) return fail(ATTNRES_ERR_ARG, "bad num_tokens/hidden");
  if (slot_stride < num_tokens * (int64_t)hidden)
    return fail(ATTNRES_ERR_ARG, "slot_stride=%lld smaller than a slot", (long long)slot_stride);
  if ((slot_stride * esize(dtype)) % 16 != 0) return fail(ATTNRES_ERR_ALIGN, "slot_stride not 16-byte aligned");
  const void* srcs[ATTNRES_MAX_SOURCES];
  const char* base = static_cast<const char*>(arena);
  for (int s = 0; s < S; ++s) srcs[s] = base + (int64_t)s * slot_stride * esize(dtype);
  const int mode = commit ? ATTNRES_MODE_SET : (delta ? ATTNRES_MODE_ACCUM : ATTNRES_MODE_PLAIN);
  return route_launch(srcs, S, num_tokens, hidden, hidden, dtype, query, gain, 1, param_dtype, eps, out, dtype,
                      hidden, (int64_t)num_tokens * hidden, weights, lse, nullptr, nullptr, mode, delta, hidden,
                      stream);
}

int attnres_route_step(const void* const* committed, int num_committed, const void* partial, const void* delta,
                       void* partial_out, int64_t num_tokens, int hidden, int dtype, const void* query,
                       const void* gain, int param_dtype, float eps, void* out, float* weights, float* lse,
                       void* stream) {
  if (num_committed < 0) return fail(ATTNRES_ERR_ARG, "num_committed=%d < 0", num_committed);
  if (num_committed > 0 && committed == nullptr) return fail(ATTNRES_ERR_ARG, "committed is NULL");
  if (partial == nullptr || delta == nullptr || partial_out == nullptr)
    return fail(ATTNRES_ERR_ARG, "partial/delta/partial_out is NULL");
  const int S = num_committed + 1;
  if (S > ATTNRES_MAX_SOURCES)
    return fail(ATTNRES_ERR_UNSUPPORTED, "%d sources exceed the maximum %d", S, ATTNRES_MAX_SOURCES);
  if (!valid_dtype(dtype)) return fail(ATTNRES_ERR_ARG, "unknown dtype code %d", dtype);
  if (num_tokens < 0 || hidden <= 0) return fail(ATTNRES_ERR_ARG, "bad num_tokens/hidden");
  const char* po = static_cast<const char*>(partial_out);
  const int64_t bytes = num_tokens * (int64_t)hidden * esize(dtype);
  auto overlaps = [&](const void* p) {
    const char* q = static_cast<const char*>(p);
    return q < po + bytes && po < q + bytes;
  };
  const void* srcs[ATTNRES_MAX_SOURCES];
  for (int s = 0; s < num_committed; ++s) {
    srcs[s] = committed[s];
    if (srcs[s] != nullptr && bytes > 0 && overlaps(srcs[s]))
      return fail(ATTNRES_ERR_ARG, "partial_out overlaps committed[%d]", s);
  }
  if (bytes > 0 && (overlaps(partial) || overlaps(delta)))
    return fail(ATTNRES_ERR_ARG, "partial_out overlaps partial or delta");
  srcs[num_committed] = partial;
  return route_launch(srcs, S, num_tokens, hidden, hidden, dtype, query, gain, 1, param_dtype, eps, out, dtype, hidden,
                      (int64_t)num_tokens * hidden, weights, lse, nullptr, nullptr, ATTNRES_MODE_ACCUM, delta, hidden,
                      stream, partial_out);
}

int attnres_route_bwd_workspace_size(int64_t num_tokens, int hidden, int64_t* bytes) {
  if (bytes == nullptr) return fail(ATTNRES_ERR_ARG, "bytes is NULL");
  if (num_tokens < 0 || hidden <= 0) return fail(ATTNRES_ERR_ARG, "bad num_tokens/hidden");
  DeviceState* st = nullptr;
  int rc = ensure_loaded(&st);
  if (rc != ATTNRES_OK) return rc;
  int64_t parts = (int64_t)st->num_cus * kBwdMaxPerCu;
  if (parts > num_tokens) parts = num_tokens;
  *bytes = parts * (int64_t)hidden * (int64_t)sizeof(float);
  return ATTNRES_OK;
}

// The launch of a routing backward kernel (either family) over `grid`
// workgroups, each writing one query-gradient partial row to the workspace,
// then the column reduction of those rows into grad_query / grad_gain.
static int route_bwd_finish(hipFunction_t f, int grid, int block, size_t lds, DeviceState& st, int nchunk,
                     const void* const* sources, int num_sources, int64_t num_tokens, int hidden, int64_t src_ld,
                     const void* query, const void* gain, int param_dtype, float eps, const void* grad_out,
                     int grad_out_dtype, int64_t grad_out_ld, const float* grad_lse, void* const* grad_sources,
                     int64_t grad_ld, void* workspace, int64_t workspace_bytes, void* grad_query, void* grad_gain,
                     void* stream, const void* const* grad_addend, float* coef = nullptr,
                     void* qfold = nullptr) {
  int rc = ATTNRES_OK;
  const int64_t need = (int64_t)grid * (int64_t)hidden * (int64_t)sizeof(float);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(ATTNRES_ERR_ARG, "workspace of %lld bytes is smaller than the %lld needed", (long long)workspace_bytes,
                (long long)need);
  if (!aligned16(workspace)) return fail(ATTNRES_ERR_ALIGN, "workspace not 16-byte aligned");
  ReduceFns redfns;
  const ReduceFns* red = nullptr;
  if (grad_query != nullptr || grad_gain != nullptr) {
    rc = get_reduce(st, &redfns);
    red = &redfns;
    if (rc != ATTNRES_OK) return rc;
  }

  attnres_route_bwd_params P;
  std::memset(&P, 0, sizeof(P));
  for (int s = 0; s < num_sources; ++s) {
    P.src[s] = sources[s];
    P.dsrc[s] = grad_sources[s];
    P.dadd[s] = grad_addend != nullptr ? grad_addend[s] : nullptr;
  }
  P.query = query;
  P.gain = gain;
  P.grad_out = grad_out;
  P.grad_lse = grad_lse;
  P.dqw_part = static_cast<float*>(workspace);
  P.coef = coef;
  P.qfold = qfold;
  P.n_tokens = num_tokens;
  P.src_ld = src_ld;
  P.dsrc_ld = grad_ld;
  P.gout_ld = grad_out_ld;
  P.d = hidden;
  P.nchunk = nchunk;
  P.param_bf16 = param_dtype == ATTNRES_DTYPE_BF16;
  P.gout_bf16 = grad_out_dtype == ATTNRES_DTYPE_BF16;
  P.eps = eps;
  P.inv_d = 1.0f / (float)hidden;
  rc = launch(f, (int)grid, block, P, stream, 1, lds);
  if (rc != ATTNRES_OK || red == nullptr) return rc;

  return reduce_launch(*red, workspace, (int)grid, hidden, query, gain, param_dtype, grad_query, grad_gain, stream);
}

static int route_bwd_impl(const void* const* sources, int num_sources, int64_t num_tokens, int hidden,
                          int64_t src_ld, int src_dtype, const void* query, const void* gain, int param_dtype,
                          float eps, const void* grad_out, int grad_out_dtype, int64_t grad_out_ld,
                          const float* grad_lse, void* const* grad_sources, int64_t grad_ld, void* workspace,
                          int64_t workspace_bytes, void* grad_query, void* grad_gain, void* stream,
                          const void* const* grad_addend) {
  if (num_sources < 1 || num_sources > ATTNRES_MAX_SOURCES)
    return fail(ATTNRES_ERR_UNSUPPORTED, "backward: num_sources=%d outside [1, %d]", num_sources,
                ATTNRES_MAX_SOURCES);
  if (sources == nullptr || grad_sources == nullptr) return fail(ATTNRES_ERR_ARG, "sources/grad_sources is NULL");
  if (num_tokens < 0) return fail(ATTNRES_ERR_ARG, "num_tokens=%lld < 0", (long long)num_tokens);
  if (hidden <= 0) return fail(ATTNRES_ERR_ARG, "hidden=%d <= 0", hidden);
  if (!valid_dtype(src_dtype) || !valid_dtype(param_dtype) || !valid_dtype(grad_out_dtype))
    return fail(ATTNRES_ERR_ARG, "unknown dtype code");
  if (query == nullptr || grad_out == nullptr) return fail(ATTNRES_ERR_ARG, "query/grad_out is NULL");
  if (gain == nullptr && grad_gain != nullptr) return fail(ATTNRES_ERR_ARG, "grad_gain given without gain");
  if (!std::isfinite(eps)) return fail(ATTNRES_ERR_ARG, "eps is not finite");
  const bool bf = src_dtype == ATTNRES_DTYPE_BF16;
  const int vec = bf ? 8 : 4;
  if (hidden % vec != 0)
    return fail(ATTNRES_ERR_UNSUPPORTED, "hidden=%d is not a multiple of %d (16-byte chunks)", hidden, vec);
  const int nchunk = hidden / vec;
  if (round64((nchunk + 1) / 2) > kMaxThreads)
    return fail(ATTNRES_ERR_UNSUPPORTED, "hidden=%d exceeds the largest supported row (%d elements)", hidden,
                2 * kMaxThreads * vec);
  // grad_out chunks are read as 16 bytes (bf16 rows as 8-byte halves when
  // the sources are fp32): rows must be aligned to that.
  const int gvec_bytes = vec * esize(grad_out_dtype);
  const int galign = gvec_bytes >= 16 ? 16 : gvec_bytes;
  if (src_ld < hidden || grad_ld < hidden || grad_out_ld < hidden)
    return fail(ATTNRES_ERR_ARG, "a row stride is smaller than hidden=%d", hidden);
  if ((src_ld * esize(src_dtype)) % 16 != 0 || (grad_ld * esize(src_dtype)) % 16 != 0)
    return fail(ATTNRES_ERR_ALIGN, "source / gradient row stride not 16-byte aligned");
  if (((uintptr_t)grad_out % galign) != 0 || ((grad_out_ld * esize(grad_out_dtype)) % galign) != 0)
    return fail(ATTNRES_ERR_ALIGN, "grad_out rows not %d-byte aligned", galign);
  for (int s = 0; s < num_sources; ++s) {
    if (sources[s] == nullptr || grad_sources[s] == nullptr)
      return fail(ATTNRES_ERR_ARG, "sources[%d] or grad_sources[%d] is NULL", s, s);
    if (!aligned16(sources[s]) || !aligned16(grad_sources[s]))
      return fail(ATTNRES_ERR_ALIGN, "sources[%d] or grad_sources[%d] not 16-byte aligned", s, s);
  }
  bool add = false;
  if (grad_addend != nullptr) {
    for (int s = 0; s < num_sources; ++s) {
      if (grad_addend[s] == nullptr) continue;
      if (!aligned16(grad_addend[s])) return fail(ATTNRES_ERR_ALIGN, "grad_addend[%d] not 16-byte aligned", s);
      add = true;
    }
    if (add && bf != (grad_out_dtype == ATTNRES_DTYPE_BF16))
      return fail(ATTNRES_ERR_UNSUPPORTED, "addend rows need grad_out in the source dtype");
  }
  if (num_tokens == 0) return ATTNRES_OK;  // no tokens: the query gradients are not written

  DeviceState* st = nullptr;
  int rc = ensure_loaded(&st);
  if (rc != ATTNRES_OK) return rc;
  const void* const* addend = add ? grad_addend : nullptr;
  const int snch =
      bwd_stream_nch(bf, grad_out_dtype == ATTNRES_DTYPE_BF16, num_sources, hidden, num_tokens, st->num_cus,
                     st->max_lds);
  if (snch > 0) {
    hipFunction_t f = nullptr;
    rc = get_bwd_stream(*st, snch, num_sources, &f, add);
    if (rc != ATTNRES_OK) return rc;
    const int64_t need_wg = (num_tokens + kBwdStreamWaves - 1) / kBwdStreamWaves;
    const int64_t cap = (int64_t)st->num_cus * (tuning().bwd_per_cu > 0 ? tuning().bwd_per_cu : 1);
    const int grid = (int)(need_wg < cap ? need_wg : cap);
    return route_bwd_finish(f, grid, 64 * kBwdStreamWaves, bwd_stream_lds(snch, num_sources), *st, nchunk, sources,
                            num_sources, num_tokens, hidden, src_ld, query, gain, param_dtype, eps, grad_out,
                            grad_out_dtype, grad_out_ld, grad_lse, grad_sources, grad_ld, workspace, workspace_bytes,
                            grad_query, grad_gain, stream, addend);
  }
  const int v = bwd_chunks_per_thread(nchunk, num_sources, num_tokens, st->num_cus);
  const int block = v == 1 ? round64(nchunk) : round64((nchunk + 1) / 2);
  hipFunction_t f = nullptr;
  int bpc = 1;
  // dynamic LDS (S >= 5): each thread's qw chunks and, with one chunk per
  // thread, its query-gradient sums (fp32), a slot for every chunk index the
  // block touches (v * block of them; those past the row end hold zeros)
  const size_t lds = num_sources >= 5 ? (size_t)(v == 1 ? 2 : 1) * (size_t)(v * block) * vec * sizeof(float) : 0;
  if (lds + kBwdStaticLds > (size_t)st->max_lds)
    return fail(ATTNRES_ERR_UNSUPPORTED, "hidden=%d needs %zu bytes of LDS per workgroup (device limit %d)", hidden,
                lds + kBwdStaticLds, st->max_lds);
  rc = get_bwd(*st, bf, grad_out_dtype == ATTNRES_DTYPE_BF16, num_sources, v, block, lds, &f, &bpc, add);
  if (rc != ATTNRES_OK) return rc;
  // Resident workgroups per CU: more than two (where registers allow three or
  // four) measured 4-12% slower for S >= 2 at the 3B shapes; S = 1 gains
  // from a third.
  const int per_cu = tuning().bwd_per_cu > 0 ? tuning().bwd_per_cu : num_sources == 1 ? 3 : 2;
  int64_t grid = (int64_t)st->num_cus * (bpc < per_cu ? bpc : per_cu);
  if (grid > num_tokens) grid = num_tokens;
  return route_bwd_finish(f, (int)grid, block, lds, *st, nchunk, sources, num_sources, num_tokens, hidden, src_ld, query,
                          gain, param_dtype, eps, grad_out, grad_out_dtype, grad_out_ld, grad_lse, grad_sources,
                          grad_ld, workspace, workspace_bytes, grad_query, grad_gain, stream, addend);
}

int attnres_route_bwd(const void* const* sources, int num_sources, int64_t num_tokens, int hidden, int64_t src_ld,
                      int src_dtype, const void* query, const void* gain, int param_dtype, float eps,
                      const void* grad_out, int grad_out_dtype, int64_t grad_out_ld, const float* grad_lse,
                      void* const* grad_sources, int64_t grad_ld, void* workspace, int64_t workspace_bytes,
                      void* grad_query, void* grad_gain, void* stream) {
  return route_bwd_impl(sources, num_sources, num_tokens, hidden, src_ld, src_dtype, query, gain, param_dtype, eps,
                        grad_out, grad_out_dtype, grad_out_ld, grad_lse, grad_sources, grad_ld, workspace,
                        workspace_bytes, grad_query, grad_gain, stream, nullptr);
}

int attnres_route_bwd_add(const void* const* sources, int num_sources, int64_t num_tokens, int hidden,
                          int64_t src_ld, int src_dtype, const void* query, const void* gain, int param_dtype,
                          float eps, const void* grad_out, int grad_out_dtype, int64_t grad_out_ld,
                          const float* grad_lse, void* const* grad_sources, const void* const* grad_addend,
                          int64_t grad_ld, void* workspace, int64_t workspace_bytes, void* grad_query,
                          void* grad_gain, void* stream) {
  return route_bwd_impl(sources, num_sources, num_tokens, hidden, src_ld, src_dtype, query, gain, param_dtype, eps,
                        grad_out, grad_out_dtype, grad_out_ld, grad_lse, grad_sources, grad_ld, workspace,
                        workspace_bytes, grad_query, grad_gain, stream, grad_addend);
}

int attnres_route_bwd_defer(const void* const* sources, int num_sources, int64_t num_tokens, int hidden,
                            int64_t src_ld, int src_dtype, const void* query, const void* gain, int param_dtype,
                            float eps, const void* grad_out, int grad_out_dtype, int64_t grad_out_ld,
                            const float* grad_lse, void* grad_partial, const void* grad_partial_addend,
                            int64_t grad_ld, float* coef, void* qfold, void* workspace, int64_t workspace_bytes,
                            void* grad_query, void* grad_gain, void* stream) {
  if (num_sources < 1 || num_sources > ATTNRES_MAX_SOURCES)
    return fail(ATTNRES_ERR_ARG, "deferred backward: num_sources=%d outside [1, %d]", num_sources,
                ATTNRES_MAX_SOURCES);
  if (sources == nullptr || grad_partial == nullptr || coef == nullptr || qfold == nullptr)
    return fail(ATTNRES_ERR_ARG, "sources, grad_partial, coef or qfold is NULL");
  if (num_tokens < 0) return fail(ATTNRES_ERR_ARG, "num_tokens=%lld < 0", (long long)num_tokens);
  if (hidden <= 0) return fail(ATTNRES_ERR_ARG, "hidden=%d <= 0", hidden);
  if (!valid_dtype(src_dtype) || !valid_dtype(param_dtype) || !valid_dtype(grad_out_dtype))
    return fail(ATTNRES_ERR_ARG, "unknown dtype code");
  if (query == nullptr || grad_out == nullptr) return fail(ATTNRES_ERR_ARG, "query/grad_out is NULL");
  if (gain == nullptr && grad_gain != nullptr) return fail(ATTNRES_ERR_ARG, "grad_gain given without gain");
  if (!std::isfinite(eps)) return fail(ATTNRES_ERR_ARG, "eps is not finite");
  const int nch = bwd_defer_nch(src_dtype, grad_out_dtype, param_dtype, num_sources, hidden, num_tokens);
  if (nch == 0)
    return fail(ATTNRES_ERR_UNSUPPORTED,
                "deferred backward: no kernel for %d sources, hidden=%d and these dtypes (bf16, hidden 512, 1024 "
                "or 3072 with 2..8 sources, 4096 with 2..9)",
                num_sources, hidden);
  if (src_ld < hidden || grad_ld < hidden || grad_out_ld < hidden)
    return fail(ATTNRES_ERR_ARG, "a row stride is smaller than hidden=%d", hidden);
  if ((src_ld * 2) % 16 != 0 || (grad_ld * 2) % 16 != 0 || (grad_out_ld * 2) % 16 != 0)
    return fail(ATTNRES_ERR_ALIGN, "row strides not 16-byte aligned");
  if (!aligned16(grad_out) || !aligned16(grad_partial) || !aligned16(coef) || !aligned16(qfold) ||
      (grad_partial_addend != nullptr && !aligned16(grad_partial_addend)))
    return fail(ATTNRES_ERR_ALIGN, "grad_out, grad_partial, its addend, coef or qfold not 16-byte aligned");
  for (int s = 0; s < num_sources; ++s) {
    if (sources[s] == nullptr) return fail(ATTNRES_ERR_ARG, "sources[%d] is NULL", s);
    if (!aligned16(sources[s])) return fail(ATTNRES_ERR_ALIGN, "sources[%d] not 16-byte aligned", s);
  }
  if (num_tokens == 0) return ATTNRES_OK;
  DeviceState* st = nullptr;
  int rc = ensure_loaded(&st);
  if (rc != ATTNRES_OK) return rc;
  if (bwd_stream_lds(nch, num_sources) > (size_t)st->max_lds)
    return fail(ATTNRES_ERR_UNSUPPORTED, "deferred backward: %zu bytes of LDS exceed the device's %d",
                bwd_stream_lds(nch, num_sources), st->max_lds);
  const size_t lds = bwd_stream_lds(nch, num_sources);
  hipFunction_t f = nullptr;
  rc = get_bwd_defer(*st, nch, num_sources, &f);
  if (rc != ATTNRES_OK) return rc;
  void* grads[ATTNRES_MAX_SOURCES] = {};
  const void* adds[ATTNRES_MAX_SOURCES] = {};
  grads[num_sources - 1] = grad_partial;
  adds[num_sources - 1] = grad_partial_addend;
  const int64_t need_wg = (num_tokens + kBwdStreamWaves - 1) / kBwdStreamWaves;
  // rows of 1-2 KiB: more waves per CU to keep the memory system busy
  const int per_cu = tuning().bwd_per_cu > 0 ? tuning().bwd_per_cu : nch <= 2 ? kBwdMaxPerCu : 1;
  const int64_t cap = (int64_t)st->num_cus * per_cu;
  const int grid = (int)(need_wg < cap ? need_wg : cap);
  return route_bwd_finish(f, grid, 64 * kBwdStreamWaves, lds, *st, hidden / 8, sources, num_sources, num_tokens,
                          hidden, src_ld, query, gain, param_dtype, eps, grad_out, grad_out_dtype, grad_out_ld,
                          grad_lse, grads, grad_ld, workspace, workspace_bytes, grad_query, grad_gain, stream, adds,
                          coef, qfold);
}

constexpr int kGatherWaves = 4;  // waves per workgroup of the segment kernels

// Fill the launch parameters of the segment kernel for terms [j0, j0 + nt).
static void seg_terms(attnres_route_bwd_gather_seg_params& P, int j0, int nt, const void* const* grad_outs,
                      const float* const* coefs, const int64_t* coef_lds, const void* const* qfolds) {
  P.num_terms = nt;
  for (int j = 0; j < nt; ++j) {
    P.term[j].grad_out = grad_outs[j0 + j];
    P.term[j].coef = coefs[j0 + j];
    P.term[j].qfold = qfolds[j0 + j];
    P.term[j].coef_ld = coef_lds[j0 + j];
  }
}

// Grid of the segment kernel for (nch, nb): its workgroups per CU, at most one
// wave per row part.
static int seg_grid(const DeviceState& st, int nch, int nb, int64_t num_tokens) {
  const int per_cu = tuning().gather_per_cu > 0 ? tuning().gather_per_cu : gather_seg_per_cu(nch, nb);
  const int64_t need_wg = (num_tokens * gather_seg_parts(nch, nb) + kGatherWaves - 1) / kGatherWaves;
  const int64_t cap = (int64_t)st.num_cus * per_cu;
  return (int)(need_wg < cap ? need_wg : cap);
}

// One block's sum of deferred gradient terms: the segment kernel with one
// block (no running sum in), one launch per ATTNRES_SEG_MAX_TERMS terms, each
// finishing the block (its own c2 sum times x) onto the one before (the
// caller's addend for the first).
int attnres_route_bwd_gather(const void* x, int64_t num_tokens, int hidden, int64_t x_ld, int dtype, int num_terms,
                             const void* const* grad_outs, int64_t grad_out_ld, const float* const* coefs,
                             const int64_t* coef_lds, const void* const* qfolds, const void* addend, void* out,
                             int64_t out_ld, void* stream) {
  if (x == nullptr || out == nullptr) return fail(ATTNRES_ERR_ARG, "x/out is NULL");
  if (num_tokens < 0 || hidden <= 0) return fail(ATTNRES_ERR_ARG, "bad num_tokens/hidden");
  if (num_terms < 0) return fail(ATTNRES_ERR_ARG, "num_terms=%d < 0", num_terms);
  if (num_terms > 0 && (grad_outs == nullptr || coefs == nullptr || coef_lds == nullptr || qfolds == nullptr))
    return fail(ATTNRES_ERR_ARG, "term arrays are NULL");
  if (!valid_dtype(dtype)) return fail(ATTNRES_ERR_ARG, "unknown dtype code");
  if (dtype != ATTNRES_DTYPE_BF16 || !defer_hidden(hidden))
    return fail(ATTNRES_ERR_UNSUPPORTED, "gather: bf16 rows of hidden 512, 1024, 3072 or 4096 only (hidden=%d)",
                hidden);
  if (x_ld < hidden || out_ld < hidden || (num_terms > 0 && grad_out_ld < hidden))
    return fail(ATTNRES_ERR_ARG, "a row stride is smaller than hidden=%d", hidden);
  if ((x_ld * 2) % 16 != 0 || (out_ld * 2) % 16 != 0 || (num_terms > 0 && (grad_out_ld * 2) % 16 != 0))
    return fail(ATTNRES_ERR_ALIGN, "row strides not 16-byte aligned");
  if (!aligned16(x) || !aligned16(out) || (addend != nullptr && !aligned16(addend)))
    return fail(ATTNRES_ERR_ALIGN, "x, out or addend not 16-byte aligned");
  for (int j = 0; j < num_terms; ++j) {
    if (grad_outs[j] == nullptr || coefs[j] == nullptr || qfolds[j] == nullptr)
      return fail(ATTNRES_ERR_ARG, "term %d has a NULL pointer", j);
    if (!aligned16(grad_outs[j]) || !aligned16(coefs[j]) || !aligned16(qfolds[j]))
      return fail(ATTNRES_ERR_ALIGN, "term %d: grad_out, coef or qfold not 16-byte aligned", j);
    if (coef_lds[j] < 4 || coef_lds[j] % 4 != 0)
      return fail(ATTNRES_ERR_ARG, "term %d: coef_ld=%lld is not a positive multiple of 4", j,
                  (long long)coef_lds[j]);
  }
  if (num_tokens == 0) return ATTNRES_OK;
  const int nch = hidden / 512;
  if (num_tokens * gather_seg_parts(nch, 1) >= ((int64_t)1 << 31))
    return fail(ATTNRES_ERR_UNSUPPORTED, "num_tokens too large");
  DeviceState* st = nullptr;
  int rc = ensure_loaded(&st);
  if (rc != ATTNRES_OK) return rc;
  hipFunction_t f = nullptr;
  rc = get_gather_seg(*st, nch, 1, &f);
  if (rc != ATTNRES_OK) return rc;
  const int grid = seg_grid(*st, nch, 1, num_tokens);
  attnres_route_bwd_gather_seg_params P;
  int j0 = 0;
  do {
    const int nt = num_terms - j0 < ATTNRES_SEG_MAX_TERMS ? num_terms - j0 : ATTNRES_SEG_MAX_TERMS;
    std::memset(&P, 0, sizeof(P));
    P.x = x;
    P.addend = j0 == 0 ? addend : out;
    P.n_tokens = num_tokens;
    P.x_ld = x_ld;
    P.gout_ld = grad_out_ld;
    P.out_ld = out_ld;
    P.d = hidden;
    P.block = 64 * kGatherWaves;
    P.final_block = 1;
    seg_terms(P, j0, nt, grad_outs, coefs, coef_lds, qfolds);
    P.blk[0].part_out = out;
    rc = launch(f, grid, 64 * kGatherWaves, P, stream, 1, 0);
    if (rc != ATTNRES_OK) return rc;
    j0 += nt;
  } while (j0 < num_terms);
  return ATTNRES_OK;
}

int attnres_route_bwd_gather_seg(int num_blocks, int64_t num_tokens, int hidden, int dtype, int num_terms,
                                 const void* const* grad_outs, int64_t grad_out_ld, const float* const* coefs,
                                 const int64_t* coef_lds, const void* const* qfolds, const void* const* part_in,
                                 const float* const* csum_in, void* const* part_out, float* const* csum_out,
                                 const void* x, int64_t x_ld, const void* addend, int64_t out_ld, void* stream) {
  if (num_blocks < 1 || num_blocks > ATTNRES_SEG_MAX_BLOCKS)
    return fail(ATTNRES_ERR_UNSUPPORTED, "segment sum: num_blocks=%d outside [1, %d]", num_blocks,
                ATTNRES_SEG_MAX_BLOCKS);
  if (num_terms < 1) return fail(ATTNRES_ERR_ARG, "segment sum: num_terms=%d < 1", num_terms);
  if (grad_outs == nullptr || coefs == nullptr || coef_lds == nullptr || qfolds == nullptr || part_out == nullptr ||
      x == nullptr)
    return fail(ATTNRES_ERR_ARG, "segment sum: a required pointer array or x is NULL");
  if (num_tokens < 0 || hidden <= 0) return fail(ATTNRES_ERR_ARG, "bad num_tokens/hidden");
  if (!valid_dtype(dtype)) return fail(ATTNRES_ERR_ARG, "unknown dtype code");
  if (dtype != ATTNRES_DTYPE_BF16 || !defer_hidden(hidden))
    return fail(ATTNRES_ERR_UNSUPPORTED,
                "segment sum: bf16 rows of hidden 512, 1024, 3072 or 4096 only (hidden=%d)", hidden);
  if (x_ld < hidden || out_ld < hidden || grad_out_ld < hidden)
    return fail(ATTNRES_ERR_ARG, "a row stride is smaller than hidden=%d", hidden);
  if ((x_ld * 2) % 16 != 0 || (out_ld * 2) % 16 != 0 || (grad_out_ld * 2) % 16 != 0)
    return fail(ATTNRES_ERR_ALIGN, "row strides not 16-byte aligned");
  if (!aligned16(x) || (addend != nullptr && !aligned16(addend)))
    return fail(ATTNRES_ERR_ALIGN, "x or addend not 16-byte aligned");
  for (int j = 0; j < num_terms; ++j) {
    if (grad_outs[j] == nullptr || coefs[j] == nullptr || qfolds[j] == nullptr)
      return fail(ATTNRES_ERR_ARG, "term %d has a NULL pointer", j);
    if (!aligned16(grad_outs[j]) || !aligned16(coefs[j]) || !aligned16(qfolds[j]))
      return fail(ATTNRES_ERR_ALIGN, "term %d: grad_out, coef or qfold not 16-byte aligned", j);
    if (coef_lds[j] < 4 * (int64_t)num_blocks || coef_lds[j] % 4 != 0)
      return fail(ATTNRES_ERR_ARG, "term %d: coef_ld=%lld holds fewer than %d records", j, (long long)coef_lds[j],
                  num_blocks);
  }
  for (int k = 0; k < num_blocks; ++k) {
    if (part_out[k] == nullptr) return fail(ATTNRES_ERR_ARG, "part_out[%d] is NULL", k);
    if (!aligned16(part_out[k]) || (part_in != nullptr && part_in[k] != nullptr && !aligned16(part_in[k])))
      return fail(ATTNRES_ERR_ALIGN, "block %d: running sum rows not 16-byte aligned", k);
    // the last block's csum_out carries its sum between launches of more than ATTNRES_SEG_MAX_TERMS terms
    const bool need = k < num_blocks - 1 || num_terms > ATTNRES_SEG_MAX_TERMS;
    if (need && (csum_out == nullptr || csum_out[k] == nullptr))
      return fail(ATTNRES_ERR_ARG, "csum_out[%d] is NULL", k);
  }
  if (num_tokens == 0) return ATTNRES_OK;
  const int nch = hidden / 512;
  const int parts = gather_seg_parts(nch, num_blocks);
  if (num_tokens * parts >= ((int64_t)1 << 31)) return fail(ATTNRES_ERR_UNSUPPORTED, "num_tokens too large");
  DeviceState* st = nullptr;
  int rc = ensure_loaded(&st);
  if (rc != ATTNRES_OK) return rc;
  hipFunction_t f = nullptr;
  rc = get_gather_seg(*st, nch, num_blocks, &f);
  if (rc != ATTNRES_OK) return rc;
  const int grid = seg_grid(*st, nch, num_blocks, num_tokens);
  attnres_route_bwd_gather_seg_params P;
  int j0 = 0;
  do {
    const int nt = num_terms - j0 < ATTNRES_SEG_MAX_TERMS ? num_terms - j0 : ATTNRES_SEG_MAX_TERMS;
    const bool last = j0 + nt == num_terms;
    std::memset(&P, 0, sizeof(P));
    P.x = x;
    P.addend = addend;
    P.n_tokens = num_tokens;
    P.x_ld = x_ld;
    P.gout_ld = grad_out_ld;
    P.out_ld = out_ld;
    P.d = hidden;
    P.block = 64 * kGatherWaves;
    P.final_block = last ? 1 : 0;
    seg_terms(P, j0, nt, grad_outs, coefs, coef_lds, qfolds);
    for (int k = 0; k < num_blocks; ++k) {
      // later launches continue from the running sums the earlier ones stored
      P.blk[k].part_in = j0 == 0 ? (part_in != nullptr ? part_in[k] : nullptr) : part_out[k];
      P.blk[k].csum_in = j0 == 0 ? (csum_in != nullptr ? csum_in[k] : nullptr) : csum_out[k];
      P.blk[k].part_out = part_out[k];
      P.blk[k].csum_out = csum_out != nullptr ? csum_out[k] : nullptr;
    }
    rc = launch(f, grid, 64 * kGatherWaves, P, stream, 1, 0);
    if (rc != ATTNRES_OK) return rc;
    j0 += nt;
  } while (j0 < num_terms);
  return ATTNRES_OK;
}

// Workspace of the batched-query backward: c1 coefficients (num_tokens, Q, S)
// fp32, then the per-workgroup query-gradient partials (grid, Q, hidden).
constexpr int kBwdDqwPerCu = 2;
static int64_t bwd_mq_c1_bytes(int64_t num_tokens, int num_sources, int num_queries) {
  const int64_t b = num_tokens * (int64_t)num_queries * num_sources * (int64_t)sizeof(float);
  return (b + 255) / 256 * 256;
}

int attnres_route_bwd_queries_workspace_size(int64_t num_tokens, int hidden, int num_sources, int num_queries,
                                             int64_t* bytes) {
  if (bytes == nullptr) return fail(ATTNRES_ERR_ARG, "bytes is NULL");
  if (num_tokens < 0 || hidden <= 0 || num_sources < 1 || num_sources > ATTNRES_MAX_SOURCES || num_queries < 1)
    return fail(ATTNRES_ERR_ARG, "bad num_tokens/hidden/num_sources/num_queries");
  DeviceState* st = nullptr;
  int rc = ensure_loaded(&st);
  if (rc != ATTNRES_OK) return rc;
  int64_t parts = (int64_t)st->num_cus * kBwdDqwPerCu;
  if (parts > num_tokens) parts = num_tokens;
  *bytes = bwd_mq_c1_bytes(num_tokens, num_sources, num_queries) +
           parts * (int64_t)num_queries * hidden * (int64_t)sizeof(float);
  return ATTNRES_OK;
}

int attnres_route_bwd_queries(const void* const* sources, int num_sources, int64_t num_tokens, int hidden,
                              int64_t src_ld, int src_dtype, const void* query, const void* gain, int num_queries,
                              int param_dtype, float eps, const void* grad_out, int grad_out_dtype,
                              int64_t grad_out_ld, int64_t grad_out_qstride, const float* grad_lse,
                              void* const* grad_sources, int64_t grad_ld, void* workspace, int64_t workspace_bytes,
                              void* grad_query, void* grad_gain, void* stream) {
  if (num_sources < 1 || num_sources > ATTNRES_MAX_SOURCES)
    return fail(ATTNRES_ERR_UNSUPPORTED, "backward: num_sources=%d outside [1, %d]", num_sources,
                ATTNRES_MAX_SOURCES);
  if (num_queries < 1) return fail(ATTNRES_ERR_ARG, "num_queries=%d < 1", num_queries);
  if (sources == nullptr || grad_sources == nullptr) return fail(ATTNRES_ERR_ARG, "sources/grad_sources is NULL");
  if (num_tokens < 0) return fail(ATTNRES_ERR_ARG, "num_tokens=%lld < 0", (long long)num_tokens);
  if (hidden <= 0) return fail(ATTNRES_ERR_ARG, "hidden=%d <= 0", hidden);
  if (!valid_dtype(src_dtype) || !valid_dtype(param_dtype) || !valid_dtype(grad_out_dtype))
    return fail(ATTNRES_ERR_ARG, "unknown dtype code");
  if (query == nullptr || grad_out == nullptr) return fail(ATTNRES_ERR_ARG, "query/grad_out is NULL");
  if (gain == nullptr && grad_gain != nullptr) return fail(ATTNRES_ERR_ARG, "grad_gain given without gain");
  if (!std::isfinite(eps)) return fail(ATTNRES_ERR_ARG, "eps is not finite");
  const bool bf = src_dtype == ATTNRES_DTYPE_BF16;
  const int vec = bf ? 8 : 4;
  if (hidden % vec != 0)
    return fail(ATTNRES_ERR_UNSUPPORTED, "hidden=%d is not a multiple of %d (16-byte chunks)", hidden, vec);
  const int nchunk = hidden / vec;
  if (round64((nchunk + 1) / 2) > kMaxThreads)
    return fail(ATTNRES_ERR_UNSUPPORTED, "hidden=%d exceeds the largest supported row (%d elements)", hidden,
                2 * kMaxThreads * vec);
  const int v = round64(nchunk) <= kMaxThreads ? 1 : 2;
  const size_t mqg_lds = mqg_lds_bytes(num_queries, nchunk);
  const bool mqg_shape = bwd_mqg_shape(bf, grad_out_dtype == ATTNRES_DTYPE_BF16,
                                       param_dtype == ATTNRES_DTYPE_BF16, num_sources, num_queries, nchunk);
  if (!mqg_shape && !bwd_mq_available(bf, num_sources, v))
    return fail(ATTNRES_ERR_UNSUPPORTED,
                "batched backward of S=%d sources with %d chunks per thread is not built; call attnres_route_bwd "
                "once per query",
                num_sources, v);
  const int gvec_bytes = vec * esize(grad_out_dtype);
  const int galign = gvec_bytes >= 16 ? 16 : gvec_bytes;
  if (src_ld < hidden || grad_ld < hidden || grad_out_ld < hidden)
    return fail(ATTNRES_ERR_ARG, "a row stride is smaller than hidden=%d", hidden);
  if (num_queries > 1 && grad_out_qstride < num_tokens * grad_out_ld)
    return fail(ATTNRES_ERR_ARG, "grad_out_qstride=%lld overlaps query rows", (long long)grad_out_qstride);
  if ((src_ld * esize(src_dtype)) % 16 != 0 || (grad_ld * esize(src_dtype)) % 16 != 0)
    return fail(ATTNRES_ERR_ALIGN, "source / gradient row stride not 16-byte aligned");
  if (((uintptr_t)grad_out % galign) != 0 || ((grad_out_ld * esize(grad_out_dtype)) % galign) != 0 ||
      ((grad_out_qstride * esize(grad_out_dtype)) % galign) != 0)
    return fail(ATTNRES_ERR_ALIGN, "grad_out rows not %d-byte aligned", galign);
  for (int s = 0; s < num_sources; ++s) {
    if (sources[s] == nullptr || grad_sources[s] == nullptr)
      return fail(ATTNRES_ERR_ARG, "sources[%d] or grad_sources[%d] is NULL", s, s);
    if (!aligned16(sources[s]) || !aligned16(grad_sources[s]))
      return fail(ATTNRES_ERR_ALIGN, "sources[%d] or grad_sources[%d] not 16-byte aligned", s, s);
  }
  if (num_tokens == 0) return ATTNRES_OK;  // no tokens: the query gradients are not written

  DeviceState* st = nullptr;
  int rc = ensure_loaded(&st);
  if (rc != ATTNRES_OK) return rc;
  // the matrix-core kernel where its staged queries fit in LDS
  const bool mqg = mqg_shape && mqg_lds + kMqgStaticLds <= (size_t)st->max_lds;
  if (!mqg && !bwd_mq_available(bf, num_sources, v))
    return fail(ATTNRES_ERR_UNSUPPORTED,
                "batched backward of S=%d sources: %zu bytes of staged queries exceed the LDS and the VALU kernel "
                "is not built for %d chunks per thread; call attnres_route_bwd once per query",
                num_sources, mqg_lds, v);
  const int block = v == 1 ? round64(nchunk) : round64((nchunk + 1) / 2);
  const int mqg_block = round64((nchunk + 1) / 2);
  hipFunction_t f = nullptr, fq = nullptr;
  int bpc = 1, bpcq = 1;
  if (mqg) {
    rc = get_bwd_mqg(*st, num_sources, (num_queries + 3) / 4, mqg_block, mqg_lds, &f, &bpc);
  } else {
    rc = get_bwd_mq(*st, bf, grad_out_dtype == ATTNRES_DTYPE_BF16, num_sources, v, block, &f, &bpc);
  }
  if (rc != ATTNRES_OK) return rc;
  const bool want_q = grad_query != nullptr || grad_gain != nullptr;
  ReduceFns redfns;
  const ReduceFns* red = nullptr;
  int64_t grid_q = 0;
  if (want_q) {
    rc = get_bwd_dqw(*st, bf, v, block, &fq, &bpcq);
    if (rc != ATTNRES_OK) return rc;
    rc = get_reduce(*st, &redfns);
    red = &redfns;
    if (rc != ATTNRES_OK) return rc;
    grid_q = (int64_t)st->num_cus * (bpcq < kBwdDqwPerCu ? bpcq : kBwdDqwPerCu);
    if (grid_q > num_tokens) grid_q = num_tokens;
  }
  const int64_t c1_bytes = bwd_mq_c1_bytes(num_tokens, num_sources, num_queries);
  const int64_t need = c1_bytes + grid_q * (int64_t)num_queries * hidden * (int64_t)sizeof(float);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(ATTNRES_ERR_ARG, "workspace of %lld bytes is smaller than the %lld needed", (long long)workspace_bytes,
                (long long)need);
  if (!aligned16(workspace)) return fail(ATTNRES_ERR_ALIGN, "workspace not 16-byte aligned");
  float* c1 = static_cast<float*>(workspace);
  float* part = reinterpret_cast<float*>(static_cast<char*>(workspace) + c1_bytes);

  attnres_route_bwd_mq_params P;
  std::memset(&P, 0, sizeof(P));
  for (int s = 0; s < num_sources; ++s) {
    P.src[s] = sources[s];
    P.dsrc[s] = grad_sources[s];
  }
  P.query = query;
  P.gain = gain;
  P.grad_out = grad_out;
  P.grad_lse = grad_lse;
  P.c1 = c1;
  P.n_tokens = num_tokens;
  P.src_ld = src_ld;
  P.dsrc_ld = grad_ld;
  P.gout_ld = grad_out_ld;
  P.gout_qstride = grad_out_qstride;
  P.d = hidden;
  P.nchunk = nchunk;
  P.num_queries = num_queries;
  P.param_bf16 = param_dtype == ATTNRES_DTYPE_BF16;
  P.block = mqg ? mqg_block : block;
  P.eps = eps;
  P.inv_d = 1.0f / (float)hidden;
  // two resident workgroups per CU, as the single-query backward; the
  // matrix-core kernel at its occupancy limit
  int per_cu = mqg ? bpc : (bpc < 2 ? bpc : 2);
  if (tuning().bwd_per_cu > 0 && tuning().bwd_per_cu < per_cu) per_cu = tuning().bwd_per_cu;
  int64_t grid = (int64_t)st->num_cus * per_cu;
  if (grid > num_tokens) grid = num_tokens;
  rc = mqg ? launch(f, (int)grid, mqg_block, P, stream, 1, mqg_lds) : launch(f, (int)grid, block, P, stream);
  if (rc != ATTNRES_OK || !want_q) return rc;

  attnres_route_bwd_dqw_params Q;
  std::memset(&Q, 0, sizeof(Q));
  for (int s = 0; s < num_sources; ++s) Q.src[s] = sources[s];
  Q.c1 = c1;
  Q.part = part;
  Q.n_tokens = num_tokens;
  Q.src_ld = src_ld;
  Q.d = hidden;
  Q.nchunk = nchunk;
  Q.num_sources = num_sources;
  Q.num_queries = num_queries;
  Q.block = block;
  for (int q0 = 0; q0 < num_queries; q0 += 8) {  // eight queries per pass over the sources
    Q.q0 = q0;
    rc = launch(fq, (int)grid_q, block, Q, stream);
    if (rc != ATTNRES_OK) return rc;
  }
  return reduce_launch(*red, part, (int)grid_q, hidden, query, gain, param_dtype, grad_query, grad_gain, stream,
                       num_queries);
}

int attnres_merge_bwd(const void* partial, int64_t num_tokens, int hidden, int partial_dtype, const void* query,
                      int param_dtype, const void* inter, int inter_dtype, const float* inter_lse, float eps,
                      const void* grad_out, void* grad_partial, void* grad_inter, float* grad_inter_lse,
                      void* workspace, int64_t workspace_bytes, void* grad_query, void* stream) {
  if (partial == nullptr || query == nullptr || inter == nullptr || inter_lse == nullptr || grad_out == nullptr ||
      grad_partial == nullptr || grad_inter == nullptr)
    return fail(ATTNRES_ERR_ARG, "merge backward: partial, query, inter, inter_lse, grad_out, grad_partial and "
                                 "grad_inter are required");
  if (num_tokens < 0) return fail(ATTNRES_ERR_ARG, "num_tokens=%lld < 0", (long long)num_tokens);
  if (hidden <= 0) return fail(ATTNRES_ERR_ARG, "hidden=%d <= 0", hidden);
  if (!valid_dtype(partial_dtype) || !valid_dtype(param_dtype) || !valid_dtype(inter_dtype))
    return fail(ATTNRES_ERR_ARG, "unknown dtype code");
  if (!std::isfinite(eps)) return fail(ATTNRES_ERR_ARG, "eps is not finite");
  const bool pbf = partial_dtype == ATTNRES_DTYPE_BF16;
  const bool ibf = inter_dtype == ATTNRES_DTYPE_BF16;
  const int vec = pbf ? 8 : 4;
  if (hidden % vec != 0)
    return fail(ATTNRES_ERR_UNSUPPORTED, "hidden=%d is not a multiple of %d (16-byte chunks)", hidden, vec);
  const int nchunk = hidden / vec;
  if (round64((nchunk + 1) / 2) > kMaxThreads)
    return fail(ATTNRES_ERR_UNSUPPORTED, "hidden=%d exceeds the largest supported row", hidden);
  const int ialign = (vec * esize(inter_dtype)) >= 16 ? 16 : vec * esize(inter_dtype);
  if (!aligned16(partial) || !aligned16(grad_partial) || ((uintptr_t)inter % ialign) != 0 ||
      ((uintptr_t)grad_out % ialign) != 0 || ((uintptr_t)grad_inter % ialign) != 0 ||
      ((int64_t)hidden * esize(inter_dtype)) % ialign != 0)
    return fail(ATTNRES_ERR_ALIGN, "merge backward rows not aligned");
  if (num_tokens == 0) return ATTNRES_OK;  // no tokens: grad_query is not written

  DeviceState* st = nullptr;
  int rc = ensure_loaded(&st);
  if (rc != ATTNRES_OK) return rc;
  // two chunks per thread where that leaves at least two waves per row
  // (measured 5% faster at D = 3072 than one chunk per thread)
  int v = round64(nchunk) > kMaxThreads || round64((nchunk + 1) / 2) >= 128 ? 2 : 1;
  if (tuning().force_v == 1 && round64(nchunk) <= kMaxThreads) v = 1;  // measurement knob (ATTNRES_V)
  const int block = v == 1 ? round64(nchunk) : round64((nchunk + 1) / 2);
  hipFunction_t f = nullptr;
  int bpc = 1;
  rc = get_merge_bwd(*st, pbf, ibf, v, block, &f, &bpc);
  if (tuning().bwd_per_cu > 0 && tuning().bwd_per_cu < bpc) bpc = tuning().bwd_per_cu;
  if (rc != ATTNRES_OK) return rc;
  int64_t grid = (int64_t)st->num_cus * (bpc < kBwdMaxPerCu ? bpc : kBwdMaxPerCu);
  if (grid > num_tokens) grid = num_tokens;
  const int64_t need = grid * (int64_t)hidden * (int64_t)sizeof(float);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(ATTNRES_ERR_ARG, "workspace of %lld bytes is smaller than the %lld needed", (long long)workspace_bytes,
                (long long)need);
  if (!aligned16(workspace)) return fail(ATTNRES_ERR_ALIGN, "workspace not 16-byte aligned");
  ReduceFns redfns;
  const ReduceFns* red = nullptr;
  if (grad_query != nullptr) {
    rc = get_reduce(*st, &redfns);
    red = &redfns;
    if (rc != ATTNRES_OK) return rc;
  }

  attnres_merge_bwd_params P;
  std::memset(&P, 0, sizeof(P));
  P.partial = partial;
  P.query = query;
  P.inter = inter;
  P.inter_lse = inter_lse;
  P.grad_out = grad_out;
  P.grad_partial = grad_partial;
  P.grad_inter = grad_inter;
  P.grad_lse = grad_inter_lse;
  P.dq_part = static_cast<float*>(workspace);
  P.n_tokens = num_tokens;
  P.d = hidden;
  P.nchunk = nchunk;
  P.param_bf16 = param_dtype == ATTNRES_DTYPE_BF16;
  P.eps = eps;
  P.inv_d = 1.0f / (float)hidden;
  rc = launch(f, (int)grid, block, P, stream);
  if (rc != ATTNRES_OK || red == nullptr) return rc;
  return reduce_launch(*red, workspace, (int)grid, hidden, query, nullptr, param_dtype, grad_query, nullptr, stream);
}

}  // extern "C"
