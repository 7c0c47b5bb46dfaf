// C ABI of libflexattn.so: argument validation, tile-config selection and
// kernel launches.  See include/flexattn.h for the contract.
#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include <cstdlib>
#include <cstring>
#include <initializer_list>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/flexattn.h"
#include "launch.h"
#include "problem.h"
#include "mask_build.h"

// Kernels compiled at run time for one set of user mods (user_mods.h),
// loaded on one GPU.
struct fa_mods {
  hipModule_t module = nullptr;
  hipFunction_t fwd = nullptr, dq = nullptr, dkdv = nullptr;
  int dtype = 0, D = 0, flags = 0, device = -1;
};

namespace {

using fa::BwdArgs;
using fa::cdiv;
using fa::FwdArgs;
using fa::fwd_items;
using fa::interval_masks;
using fa::launch_status;
using fa::Problem;
using fa::Tiles;
using fa::build_problem;
using fa::choose_pack;
using fa::choose_splits;
using fa::default_tiles;
using fa::dkdv_query_tile;
using fa::split_bytes;

// ------------------------------------------------ allocation-free bwd ----
// fa_bwd_noalloc keeps its Delta rows (B * Hq * Sq floats) in this array
// instead of a caller workspace: 32 MiB per GPU, held from the library's
// first use on that GPU until the process ends.  In host code `scratch` is
// only a handle: its device address on the current GPU comes from
// hipGetSymbolAddress, taken once per device and kept in scratch_ptr.  Every
// launching entry point resolves it on its first call on a device, so a
// caller that captures fa_bwd_noalloc into a HIP graph has already resolved
// it (with the forward, or any other launch, made before the capture).
constexpr size_t kScratchFloats = size_t(8) << 20;
static __device__ __align__(256) float scratch[kScratchFloats];

constexpr int kMaxDevices = 64;
std::mutex scratch_mu;
float* scratch_ptr[kMaxDevices] = {nullptr};

// Device address of this device's scratch array (nullptr on failure).
float* device_scratch() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (!scratch_ptr[dev]) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return nullptr;
    scratch_ptr[dev] = static_cast<float*>(ptr);
  }
  return scratch_ptr[dev];
}

// Tensor rows are read and written 16 bytes per lane.
bool aligned16(std::initializer_list<const void*> ptrs) {
  for (const void* x : ptrs)
    if (reinterpret_cast<uintptr_t>(x) & 15) return false;
  return true;
}

// ------------------------------------------------------------- forward ----
template <typename T, bool M>
int fwd_d(const FwdArgs& a, int D, const Tiles& t, hipStream_t s) {
  switch (D) {
    case 32: return fa::launch_fwd<T, 32, M>(a, t, s);
    case 64: return fa::launch_fwd<T, 64, M>(a, t, s);
    default: return fa::launch_fwd<T, 128, M>(a, t, s);
  }
}

bool has_mods(const Problem& p) { return p.alibi != nullptr || p.softcap > 0.f; }

enum { kStageDelta = 1, kStageDkdv = 2, kStageDq = 4, kStageAll = 7 };


template <typename T, int D, bool M>
int bwd_all(const BwdArgs& a, const Tiles& t, int stages, hipStream_t s) {
  int rc = FA_OK;
  if (stages == kStageAll && sizeof(T) == 2 && interval_masks(a.p)) {
    // the bf16 dQ tile kernel computes Delta from O and dO and writes it, so
    // the whole backward is two launches: dQ, then dK/dV reading that Delta
    BwdArgs f = a;
    f.fuse_delta = 1;
    rc = fa::launch_dq<T, D, M>(f, t, s);
    if (!rc) rc = fa::launch_dkdv<T, D, M>(a, t, s);
    return rc;
  }
  if (stages & kStageDelta) rc = fa::launch_delta<T, D>(a, s);
  if (!rc && (stages & kStageDkdv)) rc = fa::launch_dkdv<T, D, M>(a, t, s);
  if (!rc && (stages & kStageDq)) rc = fa::launch_dq<T, D, M>(a, t, s);
  return rc;
}

template <typename T, bool M>
int bwd_d(const BwdArgs& a, int D, const Tiles& t, int stages, hipStream_t s) {
  switch (D) {
    case 32: return bwd_all<T, 32, M>(a, t, stages, s);
    case 64: return bwd_all<T, 64, M>(a, t, stages, s);
    default: return bwd_all<T, 128, M>(a, t, stages, s);
  }
}

// Validates the params for the requested backward stages and launches them.
int bwd_stages(const fa_params* p, BwdArgs& a, int stages, hipStream_t s) {
  if (!p) return FA_ERR_NULL;
  (void)device_scratch();
  if (p->dtype == FA_DTYPE_FP8_E4M3) return FA_ERR_DTYPE;  // the fp8 path is forward-only
  Tiles t;
  int rc = default_tiles(p, &t);
  if (rc) return rc;
  rc = build_problem(p, t, &a.p);
  if (rc) return rc;
  rc = dkdv_query_tile(p, a.p, &t);
  if (rc) return rc;
  if (a.p.has_tables && (stages & (kStageDkdv | kStageDq))) {
    if (a.p.mblk_q % t.bm || a.p.mblk_kv % t.bn || a.p.mblk_kv % t.bkv || a.p.mblk_q % t.bq)
      return FA_ERR_TABLES;
    if ((stages & kStageDq) && !a.p.kv_num && !a.p.full_kv_num) return FA_ERR_TABLES;
    if ((stages & kStageDkdv) && !a.p.q_num && !a.p.full_q_num) return FA_ERR_TABLES;
  }
  const bool m = has_mods(a.p);
  if (p->dtype == FA_DTYPE_BF16)
    return m ? bwd_d<uint16_t, true>(a, p->D, t, stages, s) : bwd_d<uint16_t, false>(a, p->D, t, stages, s);
  return m ? bwd_d<float, true>(a, p->D, t, stages, s) : bwd_d<float, false>(a, p->D, t, stages, s);
}

size_t delta_bytes(const fa_params* p) {
  return ((size_t)p->B * p->Hq * p->Sq * sizeof(float) + 255) & ~(size_t)255;
}

// ------------------------------------------------------ block masks ----
struct MaskLayout {
  int nq, nk;
  size_t flags_bytes, qdoc_off, kdoc_off, total;
};

int mask_layout(const fa_mask_build* m, MaskLayout* L) {
  if (!m) return FA_ERR_NULL;
  if (m->abi_version != FA_ABI_VERSION) return FA_ERR_VERSION;
  if (m->rows < 1 || m->q_len < 1 || m->kv_len < 1 || m->block < 1 || m->block > fa::kMaxMaskBlock)
    return FA_ERR_SHAPE;
  if (m->doc_ids && m->doc_len < (m->q_len > m->kv_len ? m->q_len : m->kv_len)) return FA_ERR_SHAPE;
  if (!m->doc_ids && m->rows != 1) return FA_ERR_SHAPE;
  L->nq = cdiv(m->q_len, m->block);
  L->nk = cdiv(m->kv_len, m->block);
  if (L->nq + L->nk > 65535 || m->rows > 65535) return FA_ERR_SHAPE;
  auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
  L->flags_bytes = up((size_t)m->rows * L->nq * L->nk);
  L->qdoc_off = L->flags_bytes;
  L->kdoc_off = L->qdoc_off + up((size_t)m->rows * L->nq * 4);
  L->total = L->kdoc_off + up((size_t)m->rows * L->nk * 4);
  return FA_OK;
}

// compute units of the current device (cached per device)
int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

int fwd_launch(const fa_params* p, const fa_kv_cache* kv, const void* q, const void* k, const void* v, void* o,
               float* lse, bool split, int n_splits, void* workspace, size_t workspace_bytes, void* stream) {
  if (!p) return FA_ERR_NULL;
  (void)device_scratch();
  if (p->dtype == FA_DTYPE_FP8_E4M3) return FA_ERR_DTYPE;  // fa_fwd_fp8
  if (n_splits > 64) return FA_ERR_SHAPE;
  Tiles t;
  int rc = default_tiles(p, &t);
  if (rc) return rc;
  FwdArgs a;
  rc = build_problem(p, t, &a.p);
  if (rc) return rc;
  if (!q || !k || !v || !o || !lse) return FA_ERR_NULL;
  if (!aligned16({q, k, v, o})) return FA_ERR_SHAPE;
  if (a.p.has_tables && (a.p.mblk_q % t.bm || a.p.mblk_kv % t.bn)) return FA_ERR_TABLES;
  if (a.p.has_tables && !a.p.kv_num && !a.p.full_kv_num) return FA_ERR_TABLES;
  if (kv) {  // paged / per-batch-length keys: the bf16 interval kernel, 128-row tiles
    if (p->dtype != FA_DTYPE_BF16 || !interval_masks(a.p) || t.bm != 128 || t.bn != 64) return FA_ERR_UNSUPPORTED;
    if (kv->page_table) {
      if (kv->page_size < t.bn || kv->page_size % t.bn || kv->num_pages < 1) return FA_ERR_SHAPE;
      if ((long long)kv->max_pages * kv->page_size < p->Skv) return FA_ERR_SHAPE;
      a.page_table = kv->page_table;
      a.page_size = kv->page_size;
      a.max_pages = kv->max_pages;
      a.num_pages = kv->num_pages;
    }
    a.kv_lens = kv->kv_lens;
  }
  a.pack = choose_pack(p, t, a.p);
  a.n_splits = split ? choose_splits(p, t, a.p, n_splits, device_cus()) : 1;
  if (a.n_splits > 1) {
    if (!workspace || workspace_bytes < split_bytes(p, a.n_splits) || !aligned16({workspace}))
      return FA_ERR_WORKSPACE;
    a.part = static_cast<float*>(workspace);
  }
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = o;
  a.lse = lse;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool m = has_mods(a.p);
  if (p->dtype == FA_DTYPE_BF16)
    return m ? fwd_d<uint16_t, true>(a, p->D, t, s) : fwd_d<uint16_t, false>(a, p->D, t, s);
  return m ? fwd_d<float, true>(a, p->D, t, s) : fwd_d<float, false>(a, p->D, t, s);
}

#include "user_mods.h"

}  // namespace

extern "C" {

int fa_abi_version(void) { return FA_ABI_VERSION; }

uint64_t fa_mods_source_hash(void) { return kRtcHash; }

const char* fa_strerror(int status) {
  switch (status) {
    case FA_OK: return "success";
    case FA_ERR_NULL: return "a required pointer is null";
    case FA_ERR_SHAPE: return "invalid or inconsistent sizes";
    case FA_ERR_DTYPE: return "unknown dtype";
    case FA_ERR_UNSUPPORTED: return "no kernel for this head dim / tile configuration";
    case FA_ERR_TABLES: return "block tables inconsistent with the problem sizes";
    case FA_ERR_WORKSPACE: return "workspace missing or too small";
    case FA_ERR_LAUNCH: return "HIP kernel launch failed";
    case FA_ERR_VERSION:
      return "ABI version mismatch: fa_params.abi_version, or a mods code blob built from other kernel headers";
    case FA_ERR_TOO_LARGE: return "B * Hq * Sq exceeds fa_bwd_noalloc_max_rows()";
    case FA_ERR_COMPILE: return "the run-time compile of the user mods failed (see the compile log)";
    default: return "unknown status";
  }
}

size_t fa_fwd_splitkv_workspace_bytes(const fa_params* p, int n_splits) {
  Tiles t;
  Problem pr;
  if (!p || default_tiles(p, &t) || build_problem(p, t, &pr)) return 0;
  if (n_splits > 64) return 0;
  return split_bytes(p, choose_splits(p, t, pr, n_splits, device_cus()));
}

int fa_fwd_splitkv(const fa_params* p, const void* q, const void* k, const void* v, void* o, float* lse,
                   int n_splits, void* workspace, size_t workspace_bytes, void* stream) {
  return fwd_launch(p, nullptr, q, k, v, o, lse, true, n_splits, workspace, workspace_bytes, stream);
}

int fa_fwd(const fa_params* p, const void* q, const void* k, const void* v, void* o, float* lse,
           void* stream) {
  return fwd_launch(p, nullptr, q, k, v, o, lse, false, 1, nullptr, 0, stream);
}

int fa_fwd_fp8(const fa_params* p, const fa_fp8_inputs* in, void* o, float* lse, void* stream) {
  if (!p || !in) return FA_ERR_NULL;
  (void)device_scratch();
  if (p->dtype != FA_DTYPE_FP8_E4M3) return FA_ERR_DTYPE;
  Tiles t;
  int rc = default_tiles(p, &t);
  if (rc) return rc;
  fa::Fp8FwdArgs a;
  rc = build_problem(p, t, &a.p);
  if (rc) return rc;
  if (p->D != 64 && p->D != 128) return FA_ERR_UNSUPPORTED;
  if (!interval_masks(a.p)) return FA_ERR_UNSUPPORTED;  // document labels: contiguous runs only
  if (!in->q || !in->k || !in->vt || !in->q_scale || !in->k_scale || !in->v_scale || !o || !lse) return FA_ERR_NULL;
  if (!aligned16({in->q, in->k, in->vt, o})) return FA_ERR_SHAPE;
  if (in->v_ld < p->Skv || in->v_ld % 128) return FA_ERR_SHAPE;
  if ((long long)p->D * in->v_ld > 0xffffffffll || (long long)p->Skv * p->D > 0xffffffffll ||
      (long long)p->Sq * p->D > 0xffffffffll)
    return FA_ERR_SHAPE;  // one head's rows within a 32-bit buffer range
  if (a.p.has_tables && (a.p.mblk_q % t.bm || a.p.mblk_kv % t.bn)) return FA_ERR_TABLES;
  if (a.p.has_tables && !a.p.kv_num && !a.p.full_kv_num) return FA_ERR_TABLES;
  a.q = static_cast<const uint8_t*>(in->q);
  a.k = static_cast<const uint8_t*>(in->k);
  a.vt = static_cast<const uint8_t*>(in->vt);
  a.ldv = in->v_ld;
  a.q_scale = in->q_scale;
  a.k_scale = in->k_scale;
  a.v_scale = in->v_scale;
  a.o = o;
  a.lse = lse;
  return fa::launch_fwd_fp8(a, p->D, has_mods(a.p), static_cast<hipStream_t>(stream));
}

int fa_quantize_fp8(const void* x, int32_t heads, int32_t S, int32_t D, int32_t transpose, void* out, float* scale,
                    void* stream) {
  if (!x || !out || !scale) return FA_ERR_NULL;
  if (heads < 1 || S < 1 || (transpose != 0 && transpose != 1)) return FA_ERR_SHAPE;
  if (D != 32 && D != 64 && D != 128) return FA_ERR_UNSUPPORTED;
  if (!aligned16({x, out})) return FA_ERR_SHAPE;
  if ((long long)heads * cdiv(S, fa::kFp8ScaleRows) > 0x7fffffffll) return FA_ERR_SHAPE;
  fa::QuantArgs a;
  a.x = static_cast<const uint16_t*>(x);
  a.out = static_cast<uint8_t*>(out);
  a.scale = scale;
  a.heads = heads;
  a.S = S;
  a.D = D;
  a.ld = cdiv(S, fa::kFp8ScaleRows) * fa::kFp8ScaleRows;
  a.transpose = transpose;
  return fa::launch_quant_fp8(a, static_cast<hipStream_t>(stream));
}

size_t fa_fwd_kvcache_workspace_bytes(const fa_params* p, const fa_kv_cache* kv, int n_splits) {
  (void)kv;
  return fa_fwd_splitkv_workspace_bytes(p, n_splits);
}

int fa_fwd_kvcache(const fa_params* p, const fa_kv_cache* kv, const void* q, const void* k_cache,
                   const void* v_cache, void* o, float* lse, int n_splits, void* workspace, size_t workspace_bytes,
                   void* stream) {
  if (!kv) return FA_ERR_NULL;
  return fwd_launch(p, kv, q, k_cache, v_cache, o, lse, true, n_splits, workspace, workspace_bytes, stream);
}

size_t fa_bwd_workspace_bytes(const fa_params* p) {
  if (!p) return 0;
  return delta_bytes(p);
}

int fa_bwd(const fa_params* p, const void* q, const void* k, const void* v, const void* o,
           const float* lse, const void* dout, void* dq, void* dk, void* dv, void* workspace,
           size_t workspace_bytes, void* stream) {
  if (!p) return FA_ERR_NULL;
  if (!q || !k || !v || !o || !lse || !dout || !dq || !dk || !dv) return FA_ERR_NULL;
  if (!aligned16({q, k, v, o, dout, dq, dk, dv})) return FA_ERR_SHAPE;
  if (!workspace || workspace_bytes < delta_bytes(p)) return FA_ERR_WORKSPACE;
  BwdArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = o;
  a.lse = lse;
  a.dout = dout;
  a.dq = dq;
  a.dk = dk;
  a.dv = dv;
  a.delta = static_cast<float*>(workspace);
  return bwd_stages(p, a, kStageAll, static_cast<hipStream_t>(stream));
}

size_t fa_bwd_noalloc_max_rows(void) { return kScratchFloats; }

int fa_bwd_noalloc(const fa_params* p, const void* q, const void* k, const void* v, const void* o,
                   const float* lse, const void* dout, void* dq, void* dk, void* dv, void* stream) {
  if (!p) return FA_ERR_NULL;
  if (p->dtype == FA_DTYPE_FP8_E4M3) return FA_ERR_DTYPE;  // the fp8 path is forward-only
  if (!q || !k || !v || !o || !lse || !dout || !dq || !dk || !dv) return FA_ERR_NULL;
  if (!aligned16({q, k, v, o, dout, dq, dk, dv})) return FA_ERR_SHAPE;
  if (p->B < 1 || p->Hq < 1 || p->Sq < 1) return FA_ERR_SHAPE;
  if ((size_t)p->B * p->Hq * p->Sq > kScratchFloats) return FA_ERR_TOO_LARGE;
  float* delta = device_scratch();
  if (!delta) return FA_ERR_LAUNCH;
  BwdArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = o;
  a.lse = lse;
  a.dout = dout;
  a.dq = dq;
  a.dk = dk;
  a.dv = dv;
  a.delta = delta;  // every row is written (by the Delta pass or the dQ kernel) before it is read
  return bwd_stages(p, a, kStageAll, static_cast<hipStream_t>(stream));
}

int fa_bwd_preprocess(const fa_params* p, const void* o, const void* dout, float* delta, void* stream) {
  if (!p) return FA_ERR_NULL;
  if (!o || !dout || !delta) return FA_ERR_NULL;
  if (!aligned16({o, dout})) return FA_ERR_SHAPE;
  BwdArgs a{};
  a.o = o;
  a.dout = dout;
  a.delta = delta;
  return bwd_stages(p, a, kStageDelta, static_cast<hipStream_t>(stream));
}

int fa_bwd_dkdv(const fa_params* p, const void* q, const void* k, const void* v, const void* dout,
                const float* lse, const float* delta, void* dk, void* dv, void* stream) {
  if (!p) return FA_ERR_NULL;
  if (!q || !k || !v || !dout || !lse || !delta || !dk || !dv) return FA_ERR_NULL;
  if (!aligned16({q, k, v, dout, dk, dv})) return FA_ERR_SHAPE;
  BwdArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.dout = dout;
  a.lse = lse;
  a.delta = const_cast<float*>(delta);
  a.dk = dk;
  a.dv = dv;
  return bwd_stages(p, a, kStageDkdv, static_cast<hipStream_t>(stream));
}

int fa_bwd_dq(const fa_params* p, const void* q, const void* k, const void* v, const void* dout,
              const float* lse, const float* delta, void* dq, void* stream) {
  if (!p) return FA_ERR_NULL;
  if (!q || !k || !v || !dout || !lse || !delta || !dq) return FA_ERR_NULL;
  if (!aligned16({q, k, v, dout, dq})) return FA_ERR_SHAPE;
  BwdArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.dout = dout;
  a.lse = lse;
  a.delta = const_cast<float*>(delta);
  a.dq = dq;
  return bwd_stages(p, a, kStageDq, static_cast<hipStream_t>(stream));
}

int fa_mods_compile(const char* policy_source, int dtype, int D, int flags, void** blob, size_t* blob_bytes,
                    char* log, size_t log_bytes) {
  if (!blob || !blob_bytes) return FA_ERR_NULL;
  std::vector<char> b;
  const int rc = compile_mods(policy_source, dtype, D, flags, &b, log, log_bytes);
  if (rc) return rc;
  void* mem = malloc(b.size());
  if (!mem) return FA_ERR_NULL;
  memcpy(mem, b.data(), b.size());
  *blob = mem;
  *blob_bytes = b.size();
  return FA_OK;
}

void fa_mods_free_blob(void* blob) { free(blob); }

int fa_mods_load(const void* blob, size_t blob_bytes, fa_mods** out) { return load_mods(blob, blob_bytes, out); }

int fa_mods_unload(fa_mods* m) {
  if (!m) return FA_ERR_NULL;
  const int rc = hipModuleUnload(m->module) == hipSuccess ? FA_OK : FA_ERR_LAUNCH;
  delete m;
  return rc;
}

int fa_mods_fwd(const fa_mods* m, const fa_params* p, const void* const* bufs, int nbufs, const void* q,
                const void* k, const void* v, void* o, float* lse, void* stream) {
  FwdArgs a;
  Tiles t;
  int rc = mods_problem(m, p, bufs, nbufs, &a.p, &t);
  if (rc) return rc;
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev != m->device) return FA_ERR_LAUNCH;
  if (!q || !k || !v || !o || !lse) return FA_ERR_NULL;
  if (!aligned16({q, k, v, o})) return FA_ERR_SHAPE;
  if (a.p.has_tables && (a.p.mblk_q % t.bm || a.p.mblk_kv % t.bn)) return FA_ERR_TABLES;
  if (a.p.has_tables && !a.p.kv_num && !a.p.full_kv_num) return FA_ERR_TABLES;
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = o;
  a.lse = lse;
  const unsigned grid = (unsigned)(a.p.B * a.p.Hq * cdiv(a.p.Sq, t.bm));
  return launch_module(m->fwd, grid, 256, a, static_cast<hipStream_t>(stream));
}

}  // extern "C"

namespace {

// The backward stages with user mods: Delta (the library's own kernel), dK/dV
// and dQ (the run-time compiled ones).
int mods_bwd_stages(const fa_mods* m, const fa_params* p, const void* const* bufs, int nbufs, BwdArgs& a,
                    int stages, hipStream_t s) {
  Tiles t;
  int rc = mods_problem(m, p, bufs, nbufs, &a.p, &t);
  if (rc) return rc;
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev != m->device) return FA_ERR_LAUNCH;
  if (a.p.has_tables && (stages & (kStageDkdv | kStageDq))) {
    if (a.p.mblk_q % t.bm || a.p.mblk_kv % t.bn || a.p.mblk_kv % t.bkv || a.p.mblk_q % t.bq) return FA_ERR_TABLES;
    if ((stages & kStageDq) && !a.p.kv_num && !a.p.full_kv_num) return FA_ERR_TABLES;
    if ((stages & kStageDkdv) && !a.p.q_num && !a.p.full_q_num) return FA_ERR_TABLES;
  }
  if (stages & kStageDelta) {
    if (p->dtype == FA_DTYPE_BF16)
      rc = p->D == 32 ? fa::launch_delta<uint16_t, 32>(a, s) : p->D == 64 ? fa::launch_delta<uint16_t, 64>(a, s)
                                                                    : fa::launch_delta<uint16_t, 128>(a, s);
    else
      rc = p->D == 32 ? fa::launch_delta<float, 32>(a, s) : p->D == 64 ? fa::launch_delta<float, 64>(a, s)
                                                                 : fa::launch_delta<float, 128>(a, s);
    if (rc) return rc;
  }
  if (stages & kStageDkdv) {
    rc = launch_module(m->dkdv, (unsigned)(a.p.B * a.p.Hkv * cdiv(a.p.Skv, t.bkv)), 256, a, s);
    if (rc) return rc;
  }
  if (stages & kStageDq) rc = launch_module(m->dq, (unsigned)(a.p.B * a.p.Hq * cdiv(a.p.Sq, t.bm)), 256, a, s);
  return rc;
}

}  // namespace

extern "C" {

int fa_mods_bwd(const fa_mods* m, const fa_params* p, const void* const* bufs, int nbufs, const void* q,
                const void* k, const void* v, const void* o, const float* lse, const void* dout, void* dq,
                void* dk, void* dv, void* workspace, size_t workspace_bytes, void* stream) {
  if (!m || !p) return FA_ERR_NULL;
  if (!q || !k || !v || !o || !lse || !dout || !dq || !dk || !dv) return FA_ERR_NULL;
  if (!aligned16({q, k, v, o, dout, dq, dk, dv})) return FA_ERR_SHAPE;
  if (!workspace || workspace_bytes < delta_bytes(p)) return FA_ERR_WORKSPACE;
  BwdArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = o;
  a.lse = lse;
  a.dout = dout;
  a.dq = dq;
  a.dk = dk;
  a.dv = dv;
  a.delta = static_cast<float*>(workspace);
  return mods_bwd_stages(m, p, bufs, nbufs, a, kStageDelta | kStageDkdv | kStageDq,
                         static_cast<hipStream_t>(stream));
}

int fa_mods_bwd_dkdv(const fa_mods* m, const fa_params* p, const void* const* bufs, int nbufs, const void* q,
                     const void* k, const void* v, const void* dout, const float* lse, const float* delta, void* dk,
                     void* dv, void* stream) {
  if (!m || !p) return FA_ERR_NULL;
  if (!q || !k || !v || !dout || !lse || !delta || !dk || !dv) return FA_ERR_NULL;
  if (!aligned16({q, k, v, dout, dk, dv})) return FA_ERR_SHAPE;
  BwdArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.dout = dout;
  a.lse = lse;
  a.delta = const_cast<float*>(delta);
  a.dk = dk;
  a.dv = dv;
  return mods_bwd_stages(m, p, bufs, nbufs, a, kStageDkdv, static_cast<hipStream_t>(stream));
}

int fa_mods_bwd_dq(const fa_mods* m, const fa_params* p, const void* const* bufs, int nbufs, const void* q,
                   const void* k, const void* v, const void* dout, const float* lse, const float* delta, void* dq,
                   void* stream) {
  if (!m || !p) return FA_ERR_NULL;
  if (!q || !k || !v || !dout || !lse || !delta || !dq) return FA_ERR_NULL;
  if (!aligned16({q, k, v, dout, dq})) return FA_ERR_SHAPE;
  BwdArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.dout = dout;
  a.lse = lse;
  a.delta = const_cast<float*>(delta);
  a.dq = dq;
  return mods_bwd_stages(m, p, bufs, nbufs, a, kStageDq, static_cast<hipStream_t>(stream));
}

size_t fa_mask_build_workspace_bytes(const fa_mask_build* m) {
  MaskLayout L;
  return mask_layout(m, &L) == FA_OK ? L.total : 0;
}

int fa_build_block_mask(const fa_mask_build* m, void* workspace, size_t workspace_bytes, void* stream) {
  MaskLayout L;
  const int rc = mask_layout(m, &L);
  if (rc != FA_OK) return rc;
  int32_t* outs[] = {m->sampled_num, m->sampled_indices, m->kv_num_blocks, m->kv_indices, m->full_kv_num_blocks,
                     m->full_kv_indices, m->q_num_blocks, m->q_indices, m->full_q_num_blocks, m->full_q_indices,
                     m->max_counts};
  for (int32_t* o : outs)
    if (!o) return FA_ERR_NULL;
  if (!workspace || workspace_bytes < L.total) return FA_ERR_WORKSPACE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  fa::MaskBuild b;
  b.rows = m->rows;
  b.q_len = m->q_len;
  b.kv_len = m->kv_len;
  b.block = m->block;
  b.nq = L.nq;
  b.nk = L.nk;
  b.left = m->window_left < 0 ? -1 : m->window_left;
  b.right = m->window_right < 0 ? -1 : m->window_right;
  b.doc = m->doc_ids;
  b.doc_len = m->doc_len;
  b.flags = reinterpret_cast<uint8_t*>(ws);
  b.qdoc = reinterpret_cast<int32_t*>(ws + L.qdoc_off);
  b.kdoc = reinterpret_cast<int32_t*>(ws + L.kdoc_off);
  hipLaunchKernelGGL(fa::mb_zero, dim3(1), dim3(64), 0, s, m->max_counts, 5);
  if (b.doc)
    hipLaunchKernelGGL(fa::mb_block_docs, dim3(b.rows, L.nq > L.nk ? L.nq : L.nk), dim3(64), 0, s, b);
  hipLaunchKernelGGL(fa::mb_classify, dim3(b.rows, L.nq), dim3(256), 0, s, b);
  fa::CompactArgs c;
  c.m = b;
  // sampled (bit 2), kv partial (live, not full), kv full; q partial, q full
  c.lists[0] = {m->sampled_num, m->sampled_indices, m->max_counts + 0, 4, 4};
  c.lists[1] = {m->kv_num_blocks, m->kv_indices, m->max_counts + 1, 3, 1};
  c.lists[2] = {m->full_kv_num_blocks, m->full_kv_indices, m->max_counts + 2, 2, 2};
  c.lists[3] = {m->q_num_blocks, m->q_indices, m->max_counts + 3, 3, 1};
  c.lists[4] = {m->full_q_num_blocks, m->full_q_indices, m->max_counts + 4, 2, 2};
  hipLaunchKernelGGL(fa::mb_compact, dim3(b.rows, L.nq > L.nk ? L.nq : L.nk, 5), dim3(256), 0, s, c);
  return launch_status();
}

}  // extern "C"
