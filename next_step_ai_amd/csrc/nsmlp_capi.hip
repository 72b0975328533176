// C ABI of the nsmlp library: argument validation, workspace carving and
// kernel launches.  Declarations and the reference interfaces each entry
// point replaces are in include/nsmlp.h.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <mutex>

#include "nsmlp_internal.h"

namespace nsmlp {

namespace {

thread_local char g_err[512] = "";

constexpr size_t kAlign = 256;
// Fixed counter region at the start of every workspace (zeroed once by
// nsmlp_workspace_init, restored to zero by the kernels that use it).
constexpr size_t kStatusOff = 0;
constexpr size_t kServedOff = 16;  // [2] u32 block counts: HBM slots, host copies
constexpr size_t kBlkCountOff = 256;
constexpr int kMaxK = 32768;
constexpr size_t kRowCountOff = kBlkCountOff + (size_t)kMaxK * sizeof(int);
constexpr int kMaxRowChunks = 1024;
constexpr size_t kCounterBytes = kRowCountOff + (size_t)kMaxRowChunks * sizeof(int) + 256;

constexpr int kRowsPerChunk = 256;
constexpr int kMaxGroups = 64;

size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int env_int(const char* name, int dflt) {
  const char* v = getenv(name);
  if (v == nullptr || *v == 0) return dflt;
  return atoi(v);
}

// Fault injection, for tests of a caller's failure handling: the reference
// runtime counts failures of its single-kernel decode and turns it off after
// three (RT:5626-5637), drops to the dequant fallback on any exception of the
// v1 path (RT:5681-5685) and tells an out-of-memory error by its message
// (runtime/_helpers.py:301-308).  A spec "name=kind[:count],..." makes the
// named compute entry points (name without the nsmlp_ prefix, or * for all)
// fail before they touch the device.  kind: oom (NSMLP_EHIP, the message says
// "out of memory"), hip (NSMLP_EHIP), inval (NSMLP_EINVAL), nospc
// (NSMLP_ENOSPC), nodev (NSMLP_ENODEV); count: the number of calls that fail
// (default: every call).  The first matching rule with calls left applies.
struct FaultRule {
  char name[64];
  int code;
  bool oom;
  int left;  // < 0: every call
};
constexpr int kMaxFaultRules = 16;
std::mutex g_fault_mu;
std::atomic<int> g_fault_armed{0};
FaultRule g_fault_rules[kMaxFaultRules];
int g_fault_n = 0;

// Parses spec into rules; returns the rule count, or -1 for a bad spec.
int fault_parse(const char* spec, FaultRule (&rules)[kMaxFaultRules]) {
  int n = 0;
  const char* p = spec;
  while (*p) {
    const char* end = strchr(p, ',');
    const size_t len = end ? (size_t)(end - p) : strlen(p);
    if (len > 0) {
      if (n == kMaxFaultRules || len >= 128) return -1;
      char item[128];
      memcpy(item, p, len);
      item[len] = 0;
      char* eq = strchr(item, '=');
      if (eq == nullptr || eq == item || (size_t)(eq - item) >= sizeof(rules[n].name)) return -1;
      *eq = 0;
      char* kind = eq + 1;
      char* colon = strchr(kind, ':');
      int count = -1;
      if (colon != nullptr) {
        *colon = 0;
        char* tail = nullptr;
        const long c = strtol(colon + 1, &tail, 10);
        if (tail == colon + 1 || *tail != 0 || c < 1 || c > (1L << 30)) return -1;
        count = (int)c;
      }
      FaultRule& r = rules[n];
      snprintf(r.name, sizeof(r.name), "%s", item);
      r.oom = false;
      r.left = count;
      if (strcmp(kind, "oom") == 0) {
        r.code = NSMLP_EHIP;
        r.oom = true;
      } else if (strcmp(kind, "hip") == 0) {
        r.code = NSMLP_EHIP;
      } else if (strcmp(kind, "inval") == 0) {
        r.code = NSMLP_EINVAL;
      } else if (strcmp(kind, "nospc") == 0) {
        r.code = NSMLP_ENOSPC;
      } else if (strcmp(kind, "nodev") == 0) {
        r.code = NSMLP_ENODEV;
      } else {
        return -1;
      }
      ++n;
    }
    if (end == nullptr) break;
    p = end + 1;
  }
  return n;
}

int fault_set(const char* spec) {
  FaultRule rules[kMaxFaultRules];
  const int n = spec ? fault_parse(spec, rules) : 0;
  if (n < 0) return set_error(NSMLP_EINVAL, "bad fault-injection spec \"%s\" (name=kind[:count],...)", spec);
  std::lock_guard<std::mutex> lk(g_fault_mu);
  for (int i = 0; i < n; ++i) g_fault_rules[i] = rules[i];
  g_fault_n = n;
  g_fault_armed.store(n > 0 ? 1 : 0, std::memory_order_release);
  return NSMLP_OK;
}

// NSMLP_FAULT_INJECT is read when the library loads; a bad spec there makes
// every compute entry point fail with NSMLP_EINVAL.
bool g_fault_env_bad = false;
const int g_fault_env_init = [] {
  const char* s = getenv("NSMLP_FAULT_INJECT");
  if (s != nullptr && *s != 0 && fault_set(s) != NSMLP_OK) {
    g_fault_env_bad = true;
    g_fault_armed.store(1, std::memory_order_release);
  }
  return 0;
}();

const char* fault_kind_name(int code) {
  switch (code) {
    case NSMLP_EINVAL: return "NSMLP_EINVAL";
    case NSMLP_ENOSPC: return "NSMLP_ENOSPC";
    case NSMLP_ENODEV: return "NSMLP_ENODEV";
    default: return "NSMLP_EHIP";
  }
}

// Called first by every compute entry point: NSMLP_OK unless a rule fires.
int fault_point(const char* name) {
  if (g_fault_armed.load(std::memory_order_acquire) == 0) return NSMLP_OK;
  std::lock_guard<std::mutex> lk(g_fault_mu);
  if (g_fault_env_bad) return set_error(NSMLP_EINVAL, "nsmlp_%s: NSMLP_FAULT_INJECT is not a valid spec", name);
  for (int i = 0; i < g_fault_n; ++i) {
    FaultRule& r = g_fault_rules[i];
    if (r.left == 0 || (strcmp(r.name, "*") != 0 && strcmp(r.name, name) != 0)) continue;
    if (r.left > 0) --r.left;
    if (r.oom) return set_error(r.code, "nsmlp_%s: HIP error out of memory (injected fault)", name);
    return set_error(r.code, "nsmlp_%s: injected fault (%s)", name, fault_kind_name(r.code));
  }
  return NSMLP_OK;
}

#define NSMLP_FAULT_POINT(name)             \
  do {                                      \
    const int fault_rc_ = fault_point(name); \
    if (fault_rc_) return fault_rc_;        \
  } while (0)

// NF4 code values (QLoRA normal-float 4-bit table).
const float kNF4[16] = {
    -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f, -0.28444138169288635f,
    -0.18477343022823334f, -0.09105003625154495f, 0.0f, 0.07958029955625534f, 0.16093020141124725f,
    0.24611230194568634f, 0.33791524171829224f, 0.44070982933044434f, 0.5626170039176941f, 0.7229568362236023f,
    1.0f};

std::mutex g_mid_mu;
bool g_mid_ready[256] = {false};

int ensure_midpoints() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 256) return set_error(NSMLP_ENODEV, "no HIP device");
  std::lock_guard<std::mutex> lk(g_mid_mu);
  if (g_mid_ready[dev]) return NSMLP_OK;
  float mid[15];
  for (int i = 0; i < 15; ++i) mid[i] = (float)(((double)kNF4[i] + (double)kNF4[i + 1]) * 0.5);
  set_nf4_midpoints(mid);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(NSMLP_EHIP, "NF4 midpoint upload: %s", hipGetErrorString(e));
  g_mid_ready[dev] = true;
  return NSMLP_OK;
}

// Columns per gate/up split: the largest of {2048, 1024, 512, 256} dividing
// H that still gives >= 1024 workgroups (k * H / cs), else 256.
int choose_cs(int H, int k) {
  static const int forced = env_int("NSMLP_GU_COLS", 0);  // measurement switch, read once
  if (forced == 256 || forced == 512 || forced == 1024 || forced == 2048)
    if (H % forced == 0) return forced;
  const int cands[4] = {2048, 1024, 512, 256};
  for (int c : cands)
    if (H % c == 0 && (long long)k * (H / c) >= 1024) return c;
  for (int c = 256; c <= 2048; c *= 2)
    if (H % c == 0 && (long long)k * (H / c) >= 1024) return c;
  return 256;
}

int choose_groups(int H, int k) {
  int chunks = (H + kRowsPerChunk - 1) / kRowsPerChunk;
  int g = (1024 + chunks - 1) / chunks;
  static const int forced = env_int("NSMLP_DOWN_GROUPS", 0);  // measurement switch, read once
  if (forced > 0) g = forced;
  int cap = k < kMaxGroups ? k : kMaxGroups;
  if (g < 1) g = 1;
  if (g > cap) g = cap;
  return g;
}

struct DecodeWs {
  size_t part, act, act_scale, outpart, total;
};

DecodeWs decode_ws_layout(int H, int k) {
  DecodeWs w;
  size_t off = align_up(kCounterBytes);
  w.part = off;
  off += align_up((size_t)k * (size_t)(H / 256) * 64 * sizeof(float));
  w.act = off;
  off += align_up((size_t)k * 16 * sizeof(uint32_t));
  w.act_scale = off;
  off += align_up((size_t)k * sizeof(float));
  w.outpart = off;
  off += align_up((size_t)kMaxGroups * (size_t)H * sizeof(float));
  w.total = off;
  return w;
}

struct RouteWs {
  size_t lat16, scores, lat_part, lat_p64, lat_p32, lat_und, lat_und_n, lat_m, sc_und, sc_und_n, total;
};

RouteWs route_ws_layout(size_t base, int rows, int H, int R, int NB) {
  RouteWs w;
  size_t off = align_up(base);
  w.lat16 = off;
  off += align_up((size_t)rows * R * sizeof(uint16_t));
  w.scores = off;
  off += align_up((size_t)rows * NB * sizeof(uint16_t));
  w.lat_part = off;
  if (rows < kLatSplitRows) off += align_up((size_t)rows * R * kLatParts * 3 * sizeof(double));
  w.lat_p64 = w.lat_p32 = w.lat_und = w.lat_und_n = w.lat_m = w.sc_und = w.sc_und_n = off;
  if (rows >= kLatSplitRows) {
    const size_t n = (size_t)rows * R, P = (size_t)latent_mf_parts(rows, R, H);
    w.lat_p64 = off;
    off += align_up(P * n * sizeof(double));
    w.lat_p32 = off;
    off += align_up(P * n * sizeof(float));
    w.lat_und = off;
    off += align_up(n * sizeof(int));
    w.lat_und_n = off;
    off += align_up(sizeof(int));
    w.lat_m = off;
    off += align_up(n * sizeof(uint16_t));
    w.sc_und = off;
    off += align_up((size_t)rows * NB * sizeof(int));
    w.sc_und_n = off;
    off += align_up(sizeof(int));
  }
  w.total = off;
  return w;
}

ProjView row_block_view(const uint8_t* packed, const float* absmax, int H, int qbs) {
  ProjView v;
  v.packed = packed;
  v.absmax = absmax;
  v.row_stride = H / 2;
  v.blk_stride = 32LL * (H / 2);
  v.abs_row_stride = H / qbs;
  v.abs_blk_stride = 32LL * (H / qbs);
  return v;
}

ProjView down_block_major_view(const uint8_t* packed, const float* absmax, int H) {
  ProjView v;
  v.packed = packed;
  v.absmax = absmax;
  v.row_stride = 16;
  v.blk_stride = 16LL * H;
  v.abs_row_stride = 1;
  v.abs_blk_stride = H;
  return v;
}

int validate_decode_shape(int H, int qbs, int k) {
  if (H <= 0 || H % 256 != 0 || H > (1 << 18))
    return set_error(NSMLP_EINVAL, "hidden size %d must be a positive multiple of 256", H);
  if (qbs < 32 || (qbs & (qbs - 1)) != 0 || H % qbs != 0)
    return set_error(NSMLP_EINVAL, "quant block size %d must be a power of two >= 32 dividing hidden size %d", qbs, H);
  if (k <= 0 || k > kMaxK) return set_error(NSMLP_EINVAL, "k=%d out of range [1, %d]", k, kMaxK);
  if (H / kRowsPerChunk > kMaxRowChunks) return set_error(NSMLP_EINVAL, "hidden size %d too large", H);
  return NSMLP_OK;
}

int fill_decode_ws(DecodeArgs& a, void* ws, size_t ws_bytes) {
  DecodeWs L = decode_ws_layout(a.H, a.k);
  if (ws == nullptr || ws_bytes < L.total)
    return set_error(NSMLP_ENOSPC, "decode workspace needs %zu bytes, got %zu", L.total, ws_bytes);
  if (((uintptr_t)ws & (kAlign - 1)) != 0) return set_error(NSMLP_EINVAL, "workspace must be 256-byte aligned");
  char* base = (char*)ws;
  a.status = (int*)(base + kStatusOff);
  a.served = (uint32_t*)(base + kServedOff);
  a.blk_count = (int*)(base + kBlkCountOff);
  a.row_count = (int*)(base + kRowCountOff);
  a.part = (float*)(base + L.part);
  // streaming path: [k][32] activations and [k] block references fit in the
  // [k][H/256][64] split partials of the generic path
  a.st_act = a.part;
  a.st_enc = (uint32_t*)(a.part + (size_t)a.k * 32);
  a.st_bid = (int32_t*)(a.st_enc + a.k);
  a.act = (uint32_t*)(base + L.act);
  a.act_scale = (float*)(base + L.act_scale);
  a.outpart = (float*)(base + L.outpart);
  return NSMLP_OK;
}

void fill_decode_tiling(DecodeArgs& a) {
  a.qbs_shift = __builtin_ctz((unsigned)a.qbs);
  a.cs = choose_cs(a.H, a.k);
  a.splits = a.H / a.cs;
  a.groups = choose_groups(a.H, a.k);
  a.rows_per_chunk = kRowsPerChunk;
  a.chunks = (a.H + kRowsPerChunk - 1) / kRowsPerChunk;
  a.st_gu_wgs = 0;
  static const int generic_only = env_int("NSMLP_DECODE_SPLIT", 0);  // measurement switch, read once
  if (generic_only == 0) plan_streaming(a, device_cus());
}

int run_decode(const DecodeArgs& a, hipStream_t s) {
  if (a.st_gu_wgs > 0) {
    launch_decode_streaming(a, s);
    return check_launch("decode");
  }
  launch_decode_gate_up(a, s);
  int rc = check_launch("decode gate/up");
  if (rc) return rc;
  launch_decode_down(a, s);
  return check_launch("decode down");
}

int validate_route(int rows, int H, int R, int NB, int k, int flags) {
  if (rows <= 0) return set_error(NSMLP_EINVAL, "rows=%d must be positive", rows);
  if (H <= 0 || H > 65535) return set_error(NSMLP_EINVAL, "hidden size %d out of range [1, 65535]", H);
  if (R <= 0 || R > 1024) return set_error(NSMLP_EINVAL, "basis rank %d out of range [1, 1024]", R);
  if (NB <= 0 || NB > kMaxSelect) return set_error(NSMLP_EINVAL, "num_blocks %d out of range [1, 65535]", NB);
  if (k <= 0 || k > NB) return set_error(NSMLP_EINVAL, "k=%d out of range [1, %d]", k, NB);
  if ((flags & NSMLP_ROUTE_SORTED) && k > 16384) return set_error(NSMLP_EINVAL, "sorted routing limited to k <= 16384");
  return NSMLP_OK;
}

int fill_route(RouteArgs& r, const void* x, int rows, int H, const void* enc_w, const void* enc_b, int R,
               int basis_top_k, const void* score_w, const void* score_b, const void* dbn, int NB, int flags, int k,
               int32_t* sel, void* latent_out, void* scores_out, char* base, size_t route_base) {
  RouteWs L = route_ws_layout(route_base, rows, H, R, NB);
  r.x = (const uint16_t*)x;
  r.rows = rows;
  r.H = H;
  r.enc_w = (const uint16_t*)enc_w;
  r.enc_b = (const uint16_t*)enc_b;
  r.R = R;
  r.basis_top_k = basis_top_k;
  r.score_w = (const uint16_t*)score_w;
  r.score_b = (const uint16_t*)score_b;
  r.dbn = (const uint16_t*)dbn;
  r.NB = NB;
  r.legacy_abs = (flags & NSMLP_ROUTE_LEGACY_ABS) ? 1 : 0;
  r.sorted = (flags & NSMLP_ROUTE_SORTED) ? 1 : 0;
  r.k = k;
  r.vec = (H % 8 == 0) && aligned16(x) && aligned16(enc_w);
  r.svec = (R % 8 == 0) && aligned16(score_w);
  r.sel = sel;
  r.latent_out = (uint16_t*)latent_out;
  r.scores_out = (uint16_t*)scores_out;
  r.lat16 = (uint16_t*)(base + L.lat16);
  r.scores = (uint16_t*)(base + L.scores);
  r.status = (int*)(base + kStatusOff);
  r.lat_part = rows < kLatSplitRows ? (double*)(base + L.lat_part) : nullptr;
  const bool mf = rows >= kLatSplitRows;
  r.lat_p64 = mf ? (double*)(base + L.lat_p64) : nullptr;
  r.lat_p32 = mf ? (float*)(base + L.lat_p32) : nullptr;
  r.lat_und = mf ? (int*)(base + L.lat_und) : nullptr;
  r.lat_und_n = mf ? (int*)(base + L.lat_und_n) : nullptr;
  r.lat_nparts = mf ? latent_mf_parts(rows, R, H) : 0;
  r.lat_m = mf ? (uint16_t*)(base + L.lat_m) : nullptr;
  r.sc_und = mf ? (int*)(base + L.sc_und) : nullptr;
  r.sc_und_n = mf ? (int*)(base + L.sc_und_n) : nullptr;
  r.clear_words = nullptr;
  return NSMLP_OK;
}

int table_to_args(const nsmlp_slot_table* t, DecodeArgs& a) {
  if (t == nullptr) return set_error(NSMLP_EINVAL, "slot table is NULL");
  if (t->I <= 0 || t->I % 32 != 0) return set_error(NSMLP_EINVAL, "intermediate size %d must be a multiple of 32", t->I);
  const bool dq = t->dq_block > 0;
  if (t->dq_block < 0 || (dq && (t->dq_block & (t->dq_block - 1)) != 0))
    return set_error(NSMLP_EINVAL, "dq_block %d must be 0 or a power of two", t->dq_block);
  if (t->code == nullptr) return set_error(NSMLP_EINVAL, "code must be non-NULL");
  if (t->n_slots > 0) {
    const bool abs_ok = dq ? (t->gate_qabsmax && t->up_qabsmax && t->down_qabsmax)
                           : (t->gate_absmax && t->up_absmax && t->down_absmax);
    if (!t->gate_packed || !t->up_packed || !t->down_packed || !abs_ok)
      return set_error(NSMLP_EINVAL, "slot storage pointers must be non-NULL");
  }
  if (t->host_gate_packed != nullptr) {
    const bool abs_ok = dq ? (t->host_gate_qabsmax && t->host_up_qabsmax && t->host_down_qabsmax)
                           : (t->host_gate_absmax && t->host_up_absmax && t->host_down_absmax);
    if (!t->host_up_packed || !t->host_down_packed || !abs_ok)
      return set_error(NSMLP_EINVAL, "host copy pointers must all be non-NULL (or host_gate_packed NULL)");
  }
  if (dq && (!t->gate_absmax2 || !t->up_absmax2 || !t->down_absmax2 || !t->gate_code2 || !t->up_code2 ||
             !t->down_code2))
    return set_error(NSMLP_EINVAL, "double-quantised absmax needs absmax2 and code2 of every projection");
  if (t->n_slots < 0) return set_error(NSMLP_EINVAL, "n_slots must be >= 0");
  if (t->lookup == nullptr && t->n_slots < t->I / 32)
    return set_error(NSMLP_EINVAL, "identity lookup needs n_slots >= num_blocks");
  const void* ptrs[] = {t->gate_packed, t->up_packed, t->down_packed, t->host_gate_packed, t->host_up_packed,
                        t->host_down_packed};
  for (const void* p : ptrs)
    if (p && !aligned16(p)) return set_error(NSMLP_EINVAL, "packed NF4 storage must be 16-byte aligned");
  memset(&a, 0, sizeof(a));
  a.H = t->H;
  a.qbs = t->qbs;
  a.NB = t->I / 32;
  a.n_slots = t->n_slots;
  a.lookup = t->lookup;
  a.gate = row_block_view(t->gate_packed, t->gate_absmax, t->H, t->qbs);
  a.up = row_block_view(t->up_packed, t->up_absmax, t->H, t->qbs);
  a.down = down_block_major_view(t->down_packed, t->down_absmax, t->H);
  a.host_gate = row_block_view(t->host_gate_packed, t->host_gate_absmax, t->H, t->qbs);
  a.host_up = row_block_view(t->host_up_packed, t->host_up_absmax, t->H, t->qbs);
  a.host_down = down_block_major_view(t->host_down_packed, t->host_down_absmax, t->H);
  a.code = a.code_up = a.code_down = t->code;
  a.down_bias = (const uint16_t*)t->down_bias;
  if (dq) {
    a.dq = 1;
    a.dq_shift = __builtin_ctz((unsigned)t->dq_block);
    a.gate.absmax = a.up.absmax = a.down.absmax = nullptr;
    a.host_gate.absmax = a.host_up.absmax = a.host_down.absmax = nullptr;
    a.gate.qabsmax = t->gate_qabsmax;
    a.up.qabsmax = t->up_qabsmax;
    a.down.qabsmax = t->down_qabsmax;
    a.host_gate.qabsmax = t->host_gate_qabsmax;
    a.host_up.qabsmax = t->host_up_qabsmax;
    a.host_down.qabsmax = t->host_down_qabsmax;
    a.gate.absmax2 = a.host_gate.absmax2 = t->gate_absmax2;
    a.up.absmax2 = a.host_up.absmax2 = t->up_absmax2;
    a.down.absmax2 = a.host_down.absmax2 = t->down_absmax2;
    a.gate.code2 = a.host_gate.code2 = t->gate_code2;
    a.up.code2 = a.host_up.code2 = t->up_code2;
    a.down.code2 = a.host_down.code2 = t->down_code2;
    a.gate.offset = a.host_gate.offset = t->gate_offset;
    a.up.offset = a.host_up.offset = t->up_offset;
    a.down.offset = a.host_down.offset = t->down_offset;
  }
  return NSMLP_OK;
}

}  // namespace

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(NSMLP_EHIP, "%s launch failed: %s", what, hipGetErrorString(e));
  return NSMLP_OK;
}

}  // namespace nsmlp

using namespace nsmlp;

namespace nsmlp {
namespace {

template <typename AbsT>
int gather_rows_impl(const uint8_t* src_packed, const AbsT* src_absmax, int src_blocks, const int32_t* blocks, int n,
                     int in_features, int qbs, uint8_t* dst_packed, AbsT* dst_absmax, void* stream) {
  if (n < 0 || src_blocks < 0 || in_features <= 0 || in_features % 32 != 0 || qbs <= 0 ||
      (32LL * in_features) % qbs != 0)
    return set_error(NSMLP_EINVAL, "bad row-block gather geometry");
  if (n == 0) return NSMLP_OK;
  if (!src_packed || !src_absmax || !blocks || !dst_packed || !dst_absmax)
    return set_error(NSMLP_EINVAL, "NULL tensor argument");
  if (!aligned16(src_packed) || !aligned16(dst_packed)) return set_error(NSMLP_EINVAL, "packed must be 16-byte aligned");
  launch_gather_rows<AbsT>(src_packed, src_absmax, blocks, src_blocks, n, 16LL * in_features,
                           32LL * in_features / qbs, dst_packed, dst_absmax, (hipStream_t)stream);
  return check_launch("gather rows");
}

template <typename AbsT>
int gather_down_impl(const uint8_t* src_packed, const AbsT* src_absmax, const int32_t* blocks, int n,
                     int out_features, int in_features, int qbs, int dst_layout, uint8_t* dst_packed,
                     AbsT* dst_absmax, void* stream) {
  if (n < 0 || out_features <= 0 || in_features <= 0 || in_features % 32 != 0 || qbs <= 0 || qbs % 32 != 0 ||
      in_features % qbs != 0)
    return set_error(NSMLP_EINVAL, "bad down-column gather geometry");
  if (dst_layout != NSMLP_DOWN_BLOCK_MAJOR && dst_layout != NSMLP_DOWN_GATHERED)
    return set_error(NSMLP_EINVAL, "unknown down layout %d", dst_layout);
  if (n == 0) return NSMLP_OK;
  if (!src_packed || !src_absmax || !blocks || !dst_packed || !dst_absmax)
    return set_error(NSMLP_EINVAL, "NULL tensor argument");
  if (!aligned16(src_packed) || !aligned16(dst_packed)) return set_error(NSMLP_EINVAL, "packed must be 16-byte aligned");
  launch_gather_down<AbsT>(src_packed, src_absmax, blocks, n, out_features, in_features, qbs, dst_layout, dst_packed,
                           dst_absmax, (hipStream_t)stream);
  return check_launch("gather down");
}

}  // namespace
}  // namespace nsmlp

// ------------------------------------------------ no-allocation decode layer
// The scratch of nsmlp_decode_layer_noalloc_f16: one array per device (each
// GPU holds its own copy), used through the address hipGetSymbolAddress
// gives for it on that device, never through its name in host code.
constexpr size_t kScratchBytes = (size_t)256 << 10;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace nsmlp {
namespace {

std::mutex g_scratch_mu;
char* g_scratch_ptr[256] = {nullptr};

// The calling thread's current device's scratch; on the first call for a
// device its address is looked up (with that device current) and its status
// word cleared by a fill kernel on `s` (no memset).
int device_scratch(hipStream_t s, char** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 256) return set_error(NSMLP_ENODEV, "no HIP device");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return set_error(NSMLP_EHIP, "scratch address on device %d: %s", dev, hipGetErrorString(e));
    launch_zero_u32((uint32_t*)p, (long long)(kAlign / 4), s);
    const int rc = check_launch("scratch status clear");
    if (rc) return rc;
    g_scratch_ptr[dev] = (char*)p;
  }
  *out = g_scratch_ptr[dev];
  return NSMLP_OK;
}

}  // namespace
}  // namespace nsmlp

extern "C" {

const char* nsmlp_last_error(void) { return g_err; }

int nsmlp_version(void) { return 105; }

int nsmlp_fault_inject(const char* spec) { return fault_set(spec); }

int nsmlp_device_supported(int device) {
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) return 0;
  return strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}

int nsmlp_workspace_init(void* ws, size_t ws_bytes, void* stream) {
  if (ws == nullptr || ws_bytes < kCounterBytes)
    return set_error(NSMLP_ENOSPC, "workspace needs at least %zu bytes", kCounterBytes);
  launch_zero_u32((uint32_t*)ws, (long long)(kCounterBytes / 4), (hipStream_t)stream);
  return check_launch("workspace init");
}

int nsmlp_workspace_take_status(void* ws, int32_t* dst, void* stream) {
  if (ws == nullptr) return set_error(NSMLP_EINVAL, "ws must be non-NULL");
  if (((uintptr_t)ws & (kAlign - 1)) != 0) return set_error(NSMLP_EINVAL, "workspace must be 256-byte aligned");
  launch_take_status((int*)((char*)ws + kStatusOff), (int*)dst, (hipStream_t)stream);
  return check_launch("take status");
}

int nsmlp_workspace_take_block_counts(void* ws, int64_t* dst, void* stream) {
  if (ws == nullptr || dst == nullptr) return set_error(NSMLP_EINVAL, "ws and dst must be non-NULL");
  if (((uintptr_t)ws & (kAlign - 1)) != 0) return set_error(NSMLP_EINVAL, "workspace must be 256-byte aligned");
  if (((uintptr_t)dst & 7) != 0) return set_error(NSMLP_EINVAL, "dst must be 8-byte aligned");
  launch_take_counts((uint32_t*)((char*)ws + kServedOff), (long long*)dst, (hipStream_t)stream);
  return check_launch("take block counts");
}

size_t nsmlp_route_workspace_bytes(int rows, int H, int R, int NB, int k) {
  (void)k;
  return route_ws_layout(kCounterBytes, rows, H, R, NB).total;
}

int nsmlp_route_f16(const void* x, int rows, int H, const void* enc_w, const void* enc_b, int R, int basis_top_k,
                    const void* score_w, const void* score_b, const void* down_block_norm, int NB, int flags, int k,
                    int32_t* sel, void* latent_out, void* scores_out, void* ws, size_t ws_bytes, void* stream) {
  NSMLP_FAULT_POINT("route_f16");
  int rc = validate_route(rows, H, R, NB, k, flags);
  if (rc) return rc;
  if (!x || !enc_w || !score_w || !sel) return set_error(NSMLP_EINVAL, "x, enc_w, score_w and sel must be non-NULL");
  size_t need = nsmlp_route_workspace_bytes(rows, H, R, NB, k);
  if (ws == nullptr || ws_bytes < need)
    return set_error(NSMLP_ENOSPC, "route workspace needs %zu bytes, got %zu", need, ws_bytes);
  RouteArgs r;
  fill_route(r, x, rows, H, enc_w, enc_b, R, basis_top_k, score_w, score_b, down_block_norm, NB, flags, k, sel,
             latent_out, scores_out, (char*)ws, kCounterBytes);
  launch_route(r, (hipStream_t)stream);
  return check_launch("route");
}

size_t nsmlp_decode_workspace_bytes(int H, int k) { return decode_ws_layout(H, k).total; }

static int decode_slots(const nsmlp_slot_table* table, const void* x, const void* residual, const int32_t* sel,
                        int k, void* out, void* ws, size_t ws_bytes, void* stream) {
  DecodeArgs a;
  int rc = table_to_args(table, a);
  if (rc) return rc;
  rc = validate_decode_shape(a.H, a.qbs, k);
  if (rc) return rc;
  if (!x || !sel || !out) return set_error(NSMLP_EINVAL, "x, sel and out must be non-NULL");
  if (!aligned16(x)) return set_error(NSMLP_EINVAL, "x must be 16-byte aligned");
  if (k > a.NB) return set_error(NSMLP_EINVAL, "k=%d exceeds num_blocks=%d", k, a.NB);
  a.x = (const uint16_t*)x;
  a.k = k;
  a.sel = sel;
  a.out = (uint16_t*)out;
  a.residual = (const uint16_t*)residual;
  rc = fill_decode_ws(a, ws, ws_bytes);
  if (rc) return rc;
  fill_decode_tiling(a);
  return run_decode(a, (hipStream_t)stream);
}

int nsmlp_decode_slots_f16(const nsmlp_slot_table* table, const void* x, const int32_t* sel, int k, void* out,
                           void* ws, size_t ws_bytes, void* stream) {
  NSMLP_FAULT_POINT("decode_slots_f16");
  return decode_slots(table, x, nullptr, sel, k, out, ws, ws_bytes, stream);
}

int nsmlp_decode_slots_add_f16(const nsmlp_slot_table* table, const void* x, const void* residual,
                               const int32_t* sel, int k, void* out, void* ws, size_t ws_bytes, void* stream) {
  NSMLP_FAULT_POINT("decode_slots_add_f16");
  if (residual == nullptr) return set_error(NSMLP_EINVAL, "residual must be non-NULL");
  return decode_slots(table, x, residual, sel, k, out, ws, ws_bytes, stream);
}

size_t nsmlp_layer_workspace_bytes(int H, int R, int NB, int k) {
  size_t d = decode_ws_layout(H, k).total;
  size_t r = route_ws_layout(d, 1, H, R, NB).total;
  return r + align_up((size_t)k * sizeof(int32_t));
}

static int decode_layer(const nsmlp_router* router, const nsmlp_slot_table* table, const void* x,
                        const void* residual, int k, int32_t* sel_out, void* out, void* ws, size_t ws_bytes,
                        void* stream) {
  if (router == nullptr) return set_error(NSMLP_EINVAL, "router is NULL");
  DecodeArgs a;
  int rc = table_to_args(table, a);
  if (rc) return rc;
  rc = validate_decode_shape(a.H, a.qbs, k);
  if (rc) return rc;
  rc = validate_route(1, a.H, router->R, router->NB, k, router->flags);
  if (rc) return rc;
  if (router->NB != a.NB)
    return set_error(NSMLP_EINVAL, "router num_blocks %d != intermediate blocks %d", router->NB, a.NB);
  if (!x || !out || !router->enc_w || !router->score_w)
    return set_error(NSMLP_EINVAL, "x, out, enc_w and score_w must be non-NULL");
  if (!aligned16(x)) return set_error(NSMLP_EINVAL, "x must be 16-byte aligned");
  size_t need = nsmlp_layer_workspace_bytes(a.H, router->R, router->NB, k);
  if (ws == nullptr || ws_bytes < need)
    return set_error(NSMLP_ENOSPC, "layer workspace needs %zu bytes, got %zu", need, ws_bytes);
  a.x = (const uint16_t*)x;
  a.k = k;
  a.out = (uint16_t*)out;
  a.residual = (const uint16_t*)residual;
  rc = fill_decode_ws(a, ws, ws_bytes);
  if (rc) return rc;
  fill_decode_tiling(a);
  size_t dtotal = decode_ws_layout(a.H, k).total;
  RouteWs RL = route_ws_layout(dtotal, 1, a.H, router->R, router->NB);
  int32_t* sel = sel_out ? sel_out : (int32_t*)((char*)ws + RL.total);
  RouteArgs r;
  fill_route(r, x, 1, a.H, router->enc_w, router->enc_b, router->R, router->basis_top_k, router->score_w,
             router->score_b, router->down_block_norm, router->NB, router->flags & NSMLP_ROUTE_LEGACY_ABS, k, sel,
             nullptr, nullptr, (char*)ws, dtotal);
  hipStream_t s = (hipStream_t)stream;
  if (a.st_gu_wgs > 0 && streaming_can_select(a.NB, k)) {
    // the streaming gate/up kernel selects the blocks itself from the scores
    launch_route_scores(r, s);
    rc = check_launch("route");
    if (rc) return rc;
    a.sel = nullptr;
    a.sel_scores = r.scores;
    a.sel_out = sel_out;
    return run_decode(a, s);
  }
  launch_route(r, s);
  rc = check_launch("route");
  if (rc) return rc;
  a.sel = sel;
  return run_decode(a, s);
}

int nsmlp_decode_layer_f16(const nsmlp_router* router, const nsmlp_slot_table* table, const void* x, int k,
                           int32_t* sel_out, void* out, void* ws, size_t ws_bytes, void* stream) {
  NSMLP_FAULT_POINT("decode_layer_f16");
  return decode_layer(router, table, x, nullptr, k, sel_out, out, ws, ws_bytes, stream);
}

int nsmlp_decode_layer_add_f16(const nsmlp_router* router, const nsmlp_slot_table* table, const void* x,
                               const void* residual, int k, int32_t* sel_out, void* out, void* ws, size_t ws_bytes,
                               void* stream) {
  NSMLP_FAULT_POINT("decode_layer_add_f16");
  if (residual == nullptr) return set_error(NSMLP_EINVAL, "residual must be non-NULL");
  return decode_layer(router, table, x, residual, k, sel_out, out, ws, ws_bytes, stream);
}

int nsmlp_decode_layer_noalloc_f16(const nsmlp_router* router, const nsmlp_slot_table* table, const void* x,
                                   const void* residual, int k, int32_t* sel_out, void* out, int32_t* status_out,
                                   void* stream) {
  NSMLP_FAULT_POINT("decode_layer_noalloc_f16");
  if (router == nullptr) return set_error(NSMLP_EINVAL, "router is NULL");
  DecodeArgs a;
  int rc = table_to_args(table, a);
  if (rc) return rc;
  rc = validate_decode_shape(a.H, a.qbs, k);
  if (rc) return rc;
  rc = validate_route(1, a.H, router->R, router->NB, k, router->flags);
  if (rc) return rc;
  if (router->NB != a.NB)
    return set_error(NSMLP_EINVAL, "router num_blocks %d != intermediate blocks %d", router->NB, a.NB);
  if (!x || !out || !router->enc_w || !router->score_w)
    return set_error(NSMLP_EINVAL, "x, out, enc_w and score_w must be non-NULL");
  if (!aligned16(x)) return set_error(NSMLP_EINVAL, "x must be 16-byte aligned");
  a.x = (const uint16_t*)x;
  a.k = k;
  a.out = (uint16_t*)out;
  a.residual = (const uint16_t*)residual;
  fill_decode_tiling(a);
  if (a.st_gu_wgs <= 0 || !streaming_can_select(a.NB, k))
    return set_error(NSMLP_EINVAL,
                     "no-allocation decode covers the streaming kernels only: hidden size a multiple of 2048 up to "
                     "16384, num_blocks <= 4096, k <= 2048 (got H=%d, num_blocks=%d, k=%d)",
                     a.H, a.NB, k);
  // scratch layout: status word, the gate/up kernel's activations and block
  // references, the down partials (more than one block group), latent, scores
  size_t off = kAlign;
  const size_t o_act = off;
  off += align_up((size_t)k * 32 * sizeof(float));
  const size_t o_enc = off;
  off += align_up((size_t)k * sizeof(uint32_t));
  const size_t o_bid = off;
  off += align_up((size_t)k * sizeof(int32_t));
  const size_t o_part = off;
  if (a.st_dn_gx > 1) off += align_up((size_t)a.st_dn_gx * a.H * sizeof(float));
  const size_t o_route = off;
  off = route_ws_layout(o_route, 1, a.H, router->R, router->NB).total;
  if (off > kScratchBytes)
    return set_error(NSMLP_EINVAL, "no-allocation decode needs %zu bytes of scratch for H=%d, k=%d, num_blocks=%d; "
                     "the per-device scratch holds %zu (use nsmlp_decode_layer_f16 with a workspace)",
                     off, a.H, k, a.NB, kScratchBytes);
  hipStream_t s = (hipStream_t)stream;
  char* base = nullptr;
  rc = device_scratch(s, &base);
  if (rc) return rc;
  a.status = (int*)base;
  a.served = (uint32_t*)(base + kServedOff);
  a.st_act = (float*)(base + o_act);
  a.st_enc = (uint32_t*)(base + o_enc);
  a.st_bid = (int32_t*)(base + o_bid);
  a.outpart = (float*)(base + o_part);
  RouteArgs r;
  fill_route(r, x, 1, a.H, router->enc_w, router->enc_b, router->R, router->basis_top_k, router->score_w,
             router->score_b, router->down_block_norm, router->NB, router->flags & NSMLP_ROUTE_LEGACY_ABS, k, nullptr,
             nullptr, nullptr, base, o_route);
  // the call's status word and block counts start at zero: the first router
  // kernel clears them before anything of the call is written
  r.clear_words = (int*)base;
  launch_route_scores(r, s);
  rc = check_launch("route");
  if (rc) return rc;
  a.sel = nullptr;
  a.sel_scores = r.scores;
  a.sel_out = sel_out;
  rc = run_decode(a, s);
  if (rc) return rc;
  if (status_out != nullptr) {
    launch_take_status(a.status, status_out, s);
    rc = check_launch("take status");
  }
  return rc;
}

static int dense_guard_splits(int H, int NB, int M) {
  // block ranges of the down GEMM: enough workgroups for the CUs with one
  // 256-token tile.  S depends on the layer shape only, not on M: the fp32
  // partials are added per range, so a token's output bits then do not
  // depend on how many tokens share the call.
  (void)M;
  const int tiles = H / 256;
  int S = 1;
  while (S < 8 && tiles * S < 256 && S * 2 <= NB / 2) S *= 2;
  return S;
}

// The prefill's down runs as the dense GEMM over a scattered act matrix when
// the tokens' blocks cover most of the layer (M k >= 2 NB) and the shapes fit
// it; otherwise as the grouped per-block down.
static bool prefill_dense_down(int H, int NB, int M, int k) {
  return H % 256 == 0 && NB % 4 == 0 && (long long)M * k >= 2LL * NB && (long long)M * NB * 64 < (1LL << 31) &&
         (long long)M * H * 2 < (1LL << 31);
}

size_t nsmlp_prefill_workspace_bytes(int H, int NB, int M, int k) {
  if (H <= 0 || NB <= 0 || M <= 0 || k <= 0) return 0;
  const size_t words = (size_t)(M + 31) / 32, TG = (size_t)(M + 127) / 128, nk = (size_t)M * (size_t)k;
  size_t off = align_up(kCounterBytes);
  off += align_up((size_t)NB * words * 4);        // bitmap
  off += align_up(((size_t)NB + 1) * 4);          // offsets
  off += align_up((size_t)NB * (TG + 1) * 4);     // group starts
  off += align_up(nk * 4);                         // tokens
  if (prefill_dense_down(H, NB, M, k)) {
    off += align_up((size_t)M * NB * 64);          // dense act [M][NB 32] fp16
    off += align_up((size_t)dense_guard_splits(H, NB, M) * M * H * 4);  // partial sums
  } else {
    off += align_up(nk * 32 * 2);                  // act per (block, token) entry
  }
  return off;
}

int nsmlp_prefill_slots_f16(const nsmlp_slot_table* table, const void* x, int M, const int32_t* sel, int k, void* out,
                            void* ws, size_t ws_bytes, void* stream) {
  NSMLP_FAULT_POINT("prefill_slots_f16");
  PrefillArgs p;
  memset(&p, 0, sizeof(p));
  int rc = table_to_args(table, p.d);
  if (rc) return rc;
  rc = validate_decode_shape(p.d.H, p.d.qbs, k);
  if (rc) return rc;
  if (M <= 0 || M > 65536) return set_error(NSMLP_EINVAL, "M=%d out of range [1, 65536]", M);
  if ((long long)M * p.d.H * 2 >= (1LL << 31) || (long long)M * k * 64 >= (1LL << 31))
    return set_error(NSMLP_EINVAL, "M=%d too large for one prefill call at H=%d, k=%d (split the tokens)", M, p.d.H, k);
  if (k > p.d.NB) return set_error(NSMLP_EINVAL, "k=%d exceeds num_blocks=%d", k, p.d.NB);
  if (!x || !sel || !out) return set_error(NSMLP_EINVAL, "x, sel and out must be non-NULL");
  if (!aligned16(x)) return set_error(NSMLP_EINVAL, "x must be 16-byte aligned");
  const size_t need = nsmlp_prefill_workspace_bytes(p.d.H, p.d.NB, M, k);
  if (ws == nullptr || ws_bytes < need)
    return set_error(NSMLP_ENOSPC, "prefill workspace needs %zu bytes, got %zu", need, ws_bytes);
  if (((uintptr_t)ws & (kAlign - 1)) != 0) return set_error(NSMLP_EINVAL, "workspace must be 256-byte aligned");
  char* base = (char*)ws;
  p.d.status = (int*)(base + kStatusOff);
  p.d.qbs_shift = __builtin_ctz((unsigned)p.d.qbs);
  p.x = (const uint16_t*)x;
  p.M = M;
  p.sel = sel;
  p.k = k;
  p.out = (uint16_t*)out;
  p.words = (M + 31) / 32;
  p.TG = (M + 127) / 128;
  const size_t nk = (size_t)M * (size_t)k;
  size_t off = align_up(kCounterBytes);
  p.bitmap = (uint32_t*)(base + off);
  off += align_up((size_t)p.d.NB * p.words * 4);
  p.offsets = (int32_t*)(base + off);
  off += align_up(((size_t)p.d.NB + 1) * 4);
  p.grp = (int32_t*)(base + off);
  off += align_up((size_t)p.d.NB * (p.TG + 1) * 4);
  p.tokens = (int32_t*)(base + off);
  off += align_up(nk * 4);
  // the grouped down fits in the dense path's workspace (M k <= M NB)
  if (prefill_dense_down(p.d.H, p.d.NB, M, k) && dense_down_fits(p.d, dense_guard_splits(p.d.H, p.d.NB, M))) {
    rc = dense_down_check();
    if (rc) return rc;
    p.act_dense = (uint16_t*)(base + off);
    off += align_up((size_t)M * p.d.NB * 64);
    p.part = (float*)(base + off);
    p.S = dense_guard_splits(p.d.H, p.d.NB, M);
  } else {
    p.act = (uint16_t*)(base + off);
  }
  launch_prefill(p, (hipStream_t)stream);
  return check_launch("prefill");
}

// The dense MLP runs the tokens in chunks of at most kDenseChunk (a multiple
// of the 256-token tile, so each token's tile and sums are those of one
// call over all tokens): the workspace, act [chunk][I] fp16 and S partials
// [chunk][H] fp32, stays bounded however long the prompt (at the 405B shape
// about 0.37 GB instead of 2.9 GB at 8192 tokens).  Each chunk reads the
// weights once more, a few percent of its MFMA time.
constexpr int kDenseChunk = 1024;

size_t nsmlp_dense_mlp_workspace_bytes(int H, int I, int M) {
  if (H <= 0 || I <= 0 || M <= 0) return 0;
  const size_t S = (size_t)dense_guard_splits(H, I / 32, M);
  const size_t Mc = (size_t)(M < kDenseChunk ? M : kDenseChunk);
  // the down partials; the gate/up tail's partials use the same space first
  const size_t part = S * Mc * H * 4, tail = dense_gu_tail_bytes((int)Mc);
  return align_up(kCounterBytes) + align_up(Mc * I * 2) + align_up(part > tail ? part : tail);
}

int nsmlp_dense_mlp_slots_f16(const nsmlp_slot_table* table, const void* x, int M, const void* residual, void* out,
                              void* ws, size_t ws_bytes, void* stream) {
  NSMLP_FAULT_POINT("dense_mlp_slots_f16");
  DenseGuardArgs g;
  memset(&g, 0, sizeof(g));
  int rc = table_to_args(table, g.d);
  if (rc) return rc;
  const int H = g.d.H, I = g.d.NB * 32;
  if (H % 256 != 0 || I % 128 != 0)
    return set_error(NSMLP_EINVAL, "dense MLP needs hidden %% 256 == 0 and intermediate %% 128 == 0 (got %d, %d)", H, I);
  if (g.d.qbs < 32 || (g.d.qbs & (g.d.qbs - 1)) != 0 || H % g.d.qbs != 0)
    return set_error(NSMLP_EINVAL, "quant block size %d must be a power of two >= 32 dividing %d", g.d.qbs, H);
  if (M <= 0) return set_error(NSMLP_EINVAL, "M=%d must be positive", M);
  if ((long long)kDenseChunk * I * 2 >= (1LL << 31) || (long long)kDenseChunk * H * 2 >= (1LL << 31))
    return set_error(NSMLP_EINVAL, "dense MLP shape H=%d, I=%d too large", H, I);
  if (!x || !out) return set_error(NSMLP_EINVAL, "x and out must be non-NULL");
  if (!aligned16(x)) return set_error(NSMLP_EINVAL, "x must be 16-byte aligned");
  const size_t need = nsmlp_dense_mlp_workspace_bytes(H, I, M);
  if (ws == nullptr || ws_bytes < need)
    return set_error(NSMLP_ENOSPC, "dense MLP workspace needs %zu bytes, got %zu", need, ws_bytes);
  if (((uintptr_t)ws & (kAlign - 1)) != 0) return set_error(NSMLP_EINVAL, "workspace must be 256-byte aligned");
  char* base = (char*)ws;
  g.d.status = (int*)(base + kStatusOff);
  g.d.qbs_shift = __builtin_ctz((unsigned)g.d.qbs);
  g.x = (const uint16_t*)x;
  g.M = M;
  g.S = dense_guard_splits(H, g.d.NB, M);
  if (!dense_down_fits(g.d, g.S))
    return set_error(NSMLP_EINVAL, "dense MLP: the down weights of %d slots at H=%d exceed 31-bit offsets", g.d.n_slots, H);
  rc = dense_down_check();
  if (rc) return rc;
  const int Mc = M < kDenseChunk ? M : kDenseChunk;
  size_t off = align_up(kCounterBytes);
  g.act = (uint16_t*)(base + off);
  off += align_up((size_t)Mc * I * 2);
  g.part = (float*)(base + off);
  for (int t0 = 0; t0 < M; t0 += kDenseChunk) {
    DenseGuardArgs c = g;
    c.M = M - t0 < kDenseChunk ? M - t0 : kDenseChunk;
    c.x = (const uint16_t*)x + (size_t)t0 * H;
    c.out = (uint16_t*)out + (size_t)t0 * H;
    c.residual = residual ? (const uint16_t*)residual + (size_t)t0 * H : nullptr;
    launch_dense_guard(c, (hipStream_t)stream);
    rc = check_launch("dense MLP");
    if (rc) return rc;
  }
  return NSMLP_OK;
}

size_t nsmlp_single_kernel_workspace_bytes(int H, int top_k) { return decode_ws_layout(H, top_k).total; }

int nsmlp_single_kernel_decode_f16(const void* x, const uint8_t* gate_packed, const float* gate_absmax,
                                   const float* gate_code, const uint8_t* up_packed, const float* up_absmax,
                                   const float* up_code, const uint8_t* down_packed, const float* down_absmax,
                                   const float* down_code, void* out, float* out_accum, int H, int block_size,
                                   int qbs, int top_k, void* ws, size_t ws_bytes, void* stream) {
  NSMLP_FAULT_POINT("single_kernel_decode_f16");
  if (block_size != 32) return set_error(NSMLP_EINVAL, "block_size must be 32 (got %d)", block_size);
  int rc = validate_decode_shape(H, qbs, top_k);
  if (rc) return rc;
  if (!x || !gate_packed || !gate_absmax || !gate_code || !up_packed || !up_absmax || !up_code || !down_packed ||
      !down_absmax || !down_code || !out)
    return set_error(NSMLP_EINVAL, "NULL tensor argument");
  if (!aligned16(x) || !aligned16(gate_packed) || !aligned16(up_packed) || !aligned16(down_packed))
    return set_error(NSMLP_EINVAL, "x and packed weights must be 16-byte aligned");
  DecodeArgs a;
  memset(&a, 0, sizeof(a));
  a.H = H;
  a.qbs = qbs;
  a.k = top_k;
  a.NB = top_k;
  a.n_slots = top_k;
  a.x = (const uint16_t*)x;
  a.gate = row_block_view(gate_packed, gate_absmax, H, qbs);
  a.up = row_block_view(up_packed, up_absmax, H, qbs);
  a.down.packed = down_packed;
  a.down.absmax = down_absmax;
  a.down.row_stride = 16LL * top_k;
  a.down.blk_stride = 16;
  a.down.abs_row_stride = top_k;
  a.down.abs_blk_stride = 1;
  a.code = gate_code;
  a.code_up = up_code;
  a.code_down = down_code;
  a.out = (uint16_t*)out;
  a.out_f32 = out_accum;
  rc = fill_decode_ws(a, ws, ws_bytes);
  if (rc) return rc;
  fill_decode_tiling(a);
  return run_decode(a, (hipStream_t)stream);
}

size_t nsmlp_fused_decode_workspace_bytes(int H, int kk) { return decode_ws_layout(H, kk).total; }

int nsmlp_fused_decode_gathered_f16(const void* x, int H, const int32_t* active_idx, int kk, int A,
                                    const void* flat_mask, const uint8_t* gate_packed, const float* gate_absmax,
                                    const float* gate_code, const void* gate_bias, const uint8_t* up_packed,
                                    const float* up_absmax, const float* up_code, const void* up_bias,
                                    const uint8_t* down_packed, const float* down_absmax, const float* down_code,
                                    const void* down_bias, int qbs, void* out, void* ws, size_t ws_bytes,
                                    void* stream) {
  NSMLP_FAULT_POINT("fused_decode_gathered_f16");
  int rc = validate_decode_shape(H, qbs, kk);
  if (rc) return rc;
  if (A <= 0 || A > kMaxSelect) return set_error(NSMLP_EINVAL, "A=%d out of range", A);
  if (!x || !active_idx || !gate_packed || !gate_absmax || !gate_code || !up_packed || !up_absmax || !up_code ||
      !down_packed || !down_absmax || !down_code || !out)
    return set_error(NSMLP_EINVAL, "NULL tensor argument");
  if (!aligned16(x) || !aligned16(gate_packed) || !aligned16(up_packed) || !aligned16(down_packed))
    return set_error(NSMLP_EINVAL, "x and packed weights must be 16-byte aligned");
  DecodeArgs a;
  memset(&a, 0, sizeof(a));
  a.H = H;
  a.qbs = qbs;
  a.k = kk;
  a.NB = A;
  a.n_slots = A;
  a.sel = active_idx;
  a.skip_negative = 1;
  a.x = (const uint16_t*)x;
  a.gate = row_block_view(gate_packed, gate_absmax, H, qbs);
  a.up = row_block_view(up_packed, up_absmax, H, qbs);
  a.down.packed = down_packed;
  a.down.absmax = down_absmax;
  a.down.row_stride = 16LL * A;
  a.down.blk_stride = 16;
  a.down.abs_row_stride = A;
  a.down.abs_blk_stride = 1;
  a.code = gate_code;
  a.code_up = up_code;
  a.code_down = down_code;
  a.mask = (const uint16_t*)flat_mask;
  a.gate_bias = (const uint16_t*)gate_bias;
  a.up_bias = (const uint16_t*)up_bias;
  a.down_bias = (const uint16_t*)down_bias;
  a.out = (uint16_t*)out;
  rc = fill_decode_ws(a, ws, ws_bytes);
  if (rc) return rc;
  fill_decode_tiling(a);
  return run_decode(a, (hipStream_t)stream);
}

size_t nsmlp_output_linear_workspace_bytes(int rows, int kk, int in_dim) {
  return align_up(kCounterBytes) + align_up((size_t)rows * kk * (size_t)(in_dim / 256 > 0 ? in_dim / 256 : 1) * 32 *
                                            sizeof(float));
}

int nsmlp_output_linear_nf4_f16(const void* x, int rows, int in_dim, const int32_t* active_idx, int kk, int A,
                                const void* flat_mask, const uint8_t* packed, const float* absmax, const float* code,
                                int qbs, const void* bias, int block_size, void* out, void* ws, size_t ws_bytes,
                                void* stream) {
  NSMLP_FAULT_POINT("output_linear_nf4_f16");
  if (block_size != 32) return set_error(NSMLP_EINVAL, "block_size must be 32 (got %d)", block_size);
  if (rows <= 0 || kk <= 0 || A <= 0) return set_error(NSMLP_EINVAL, "rows, kk and A must be positive");
  if (in_dim <= 0 || in_dim % 256 != 0) return set_error(NSMLP_EINVAL, "input_dim %d must be a multiple of 256", in_dim);
  if (qbs <= 0 || qbs % 32 != 0 || in_dim % qbs != 0)
    return set_error(NSMLP_EINVAL, "quant block size %d must be a multiple of 32 dividing %d", qbs, in_dim);
  if (!x || !active_idx || !packed || !absmax || !code || !out) return set_error(NSMLP_EINVAL, "NULL tensor argument");
  if (!aligned16(packed)) return set_error(NSMLP_EINVAL, "packed weight must be 16-byte aligned");
  size_t need = nsmlp_output_linear_workspace_bytes(rows, kk, in_dim);
  if (ws == nullptr || ws_bytes < need)
    return set_error(NSMLP_ENOSPC, "output-linear workspace needs %zu bytes, got %zu", need, ws_bytes);
  LinearArgs l;
  memset(&l, 0, sizeof(l));
  l.x = (const uint16_t*)x;
  l.rows = rows;
  l.in_dim = in_dim;
  l.active_idx = active_idx;
  l.kk = kk;
  l.A = A;
  l.packed = packed;
  l.absmax = absmax;
  l.code = code;
  l.qbs = qbs;
  l.mask = (const uint16_t*)flat_mask;
  l.bias = (const uint16_t*)bias;
  l.out = (uint16_t*)out;
  l.cs = choose_cs(in_dim, rows * kk);
  l.splits = in_dim / l.cs;
  l.part = (float*)((char*)ws + align_up(kCounterBytes));
  launch_output_linear(l, (hipStream_t)stream);
  return check_launch("output linear");
}

int nsmlp_input_linear_nf4_f16(const void* x, int rows, int in_features, const int32_t* active_idx, int kk,
                               const uint8_t* packed, const float* absmax, const float* code, int qbs,
                               int out_features, const void* bias, int block_size, void* out, void* stream) {
  NSMLP_FAULT_POINT("input_linear_nf4_f16");
  if (block_size <= 0 || block_size % 32 != 0)
    return set_error(NSMLP_EINVAL, "block_size must be a multiple of 32 (got %d)", block_size);
  if (rows <= 0 || kk <= 0 || out_features <= 0) return set_error(NSMLP_EINVAL, "rows, kk, out_features must be > 0");
  if (in_features <= 0 || in_features % block_size != 0)
    return set_error(NSMLP_EINVAL, "in_features %d must be a multiple of block_size %d", in_features, block_size);
  if ((long long)kk * (block_size / 32) > INT32_MAX / 2) return set_error(NSMLP_EINVAL, "kk * block_size too large");
  if (qbs <= 0 || qbs % 32 != 0 || in_features % qbs != 0)
    return set_error(NSMLP_EINVAL, "quant block size %d must be a multiple of 32 dividing %d", qbs, in_features);
  if (!x || !active_idx || !packed || !absmax || !code || !out) return set_error(NSMLP_EINVAL, "NULL tensor argument");
  if (!aligned16(packed)) return set_error(NSMLP_EINVAL, "packed weight must be 16-byte aligned");
  LinearArgs l;
  memset(&l, 0, sizeof(l));
  l.x = (const uint16_t*)x;
  l.rows = rows;
  l.in_dim = in_features;
  l.out_dim = out_features;
  l.active_idx = active_idx;
  l.kk = kk;
  l.packed = packed;
  l.absmax = absmax;
  l.code = code;
  l.qbs = qbs;
  l.bias = (const uint16_t*)bias;
  l.out = (uint16_t*)out;
  l.bm = block_size / 32;
  launch_input_linear(l, (hipStream_t)stream);
  return check_launch("input linear");
}

int nsmlp_dense_linear_nf4_f16(const nsmlp_nf4_matrix* w, const void* x, int rows, void* out, float* out_f32,
                               void* stream) {
  NSMLP_FAULT_POINT("dense_linear_nf4_f16");
  if (!w) return set_error(NSMLP_EINVAL, "NULL matrix");
  const int in = w->in_features, O = w->out_features, qbs = w->qbs;
  if (rows < 0 || O <= 0) return set_error(NSMLP_EINVAL, "rows must be >= 0 and out_features > 0");
  if (in <= 0 || in % 32 != 0 || in > 16384)
    return set_error(NSMLP_EINVAL,
                     "in_features %d must be a multiple of 32 up to 16384 (nsmlp_input_linear_nf4_f16 takes any)", in);
  if (qbs < 32 || (qbs & (qbs - 1)) != 0 || in % qbs != 0)
    return set_error(NSMLP_EINVAL, "quant block size %d must be a power of two >= 32 dividing %d", qbs, in);
  const bool dq = w->dq_block > 0;
  if (w->dq_block < 0 || (dq && (w->dq_block & (w->dq_block - 1)) != 0))
    return set_error(NSMLP_EINVAL, "dq_block %d must be 0 or a power of two", w->dq_block);
  const long long pbytes = (long long)O * (in / 2);
  const long long nabs = (long long)O * (in / qbs);
  if (pbytes >= (1LL << 31) || nabs * 4 >= (1LL << 31))
    return set_error(NSMLP_EINVAL, "matrix of %d x %d exceeds 2 GiB of packed weight", O, in);
  if (rows == 0) return NSMLP_OK;
  if (!x || !out || !w->packed || !w->code) return set_error(NSMLP_EINVAL, "NULL tensor argument");
  if (dq ? (!w->qabsmax || !w->absmax2 || !w->code2) : !w->absmax)
    return set_error(NSMLP_EINVAL, "NULL absmax argument");
  if (!aligned16(w->packed) || !aligned16(x)) return set_error(NSMLP_EINVAL, "packed weight and x must be 16-byte aligned");
  RowsArgs a;
  memset(&a, 0, sizeof(a));
  a.in = in;
  a.out = O;
  a.qbs_shift = __builtin_ctz((unsigned)qbs);
  a.packed = w->packed;
  a.rs = in / 2;
  a.p_bytes = (int)pbytes;
  a.ars = in / qbs;
  a.dq = dq ? 1 : 0;
  if (dq) {
    a.qabsmax = w->qabsmax;
    a.a_bytes = (int)nabs;
    a.absmax2 = w->absmax2;
    a.dq_shift = __builtin_ctz((unsigned)w->dq_block);
    a.a2_bytes = (int)(((nabs + w->dq_block - 1) >> a.dq_shift) * 4);
    a.code2 = w->code2;
    a.offset = w->offset;
  } else {
    a.absmax = w->absmax;
    a.a_bytes = (int)(nabs * 4);
  }
  a.code = w->code;
  const int cus = device_cus();
  for (int t = 0; t < rows; t += 2) {
    const int nt = rows - t >= 2 ? 2 : 1;
    if (!plan_rows(a, nt, cus)) return set_error(NSMLP_EINVAL, "dense linear geometry not supported");
    a.x = (const uint16_t*)x + (long long)t * in;
    a.y = (uint16_t*)out + (long long)t * O;
    a.out_f32 = out_f32 ? out_f32 + (long long)t * O : nullptr;
    launch_rows(a, nt, (hipStream_t)stream);
  }
  return check_launch("dense linear");
}

int nsmlp_silu_mul_f16(const void* gate, const void* up, void* out, long long n, void* stream) {
  NSMLP_FAULT_POINT("silu_mul_f16");
  if (n < 0 || (n > 0 && (!gate || !up || !out))) return set_error(NSMLP_EINVAL, "bad silu_mul arguments");
  if (n == 0) return NSMLP_OK;
  launch_silu_mul((const uint16_t*)gate, (const uint16_t*)up, (uint16_t*)out, n, (hipStream_t)stream);
  return check_launch("silu_mul");
}

int nsmlp_gather_row_blocks(const uint8_t* src_packed, const float* src_absmax, int src_blocks,
                            const int32_t* blocks, int n, int in_features, int qbs, uint8_t* dst_packed,
                            float* dst_absmax, void* stream) {
  return gather_rows_impl<float>(src_packed, src_absmax, src_blocks, blocks, n, in_features, qbs, dst_packed,
                                 dst_absmax, stream);
}

int nsmlp_gather_row_blocks_q8(const uint8_t* src_packed, const uint8_t* src_qabsmax, int src_blocks,
                               const int32_t* blocks, int n, int in_features, int qbs, uint8_t* dst_packed,
                               uint8_t* dst_qabsmax, void* stream) {
  if (n < 0 || src_blocks < 0 || in_features <= 0 || in_features % 32 != 0 || qbs <= 0 || in_features % qbs != 0)
    return set_error(NSMLP_EINVAL, "bad row-block gather geometry");
  if (n == 0) return NSMLP_OK;
  if (!src_qabsmax || !blocks || !dst_qabsmax || (src_packed == nullptr) != (dst_packed == nullptr))
    return set_error(NSMLP_EINVAL, "NULL tensor argument");
  if ((src_packed && !aligned16(src_packed)) || (dst_packed && !aligned16(dst_packed)))
    return set_error(NSMLP_EINVAL, "packed must be 16-byte aligned");
  launch_gather_rows_q8(src_packed, src_qabsmax, blocks, src_blocks, n, 16LL * in_features, in_features / qbs,
                        dst_packed, dst_qabsmax, (hipStream_t)stream);
  return check_launch("gather rows (u8 absmax)");
}

int nsmlp_gather_down_columns(const uint8_t* src_packed, const float* src_absmax, const int32_t* blocks, int n,
                              int out_features, int in_features, int qbs, int dst_layout, uint8_t* dst_packed,
                              float* dst_absmax, void* stream) {
  return gather_down_impl<float>(src_packed, src_absmax, blocks, n, out_features, in_features, qbs, dst_layout,
                                 dst_packed, dst_absmax, stream);
}

int nsmlp_gather_down_columns_q8(const uint8_t* src_packed, const uint8_t* src_qabsmax, const int32_t* blocks, int n,
                                 int out_features, int in_features, int qbs, int dst_layout, uint8_t* dst_packed,
                                 uint8_t* dst_qabsmax, void* stream) {
  return gather_down_impl<uint8_t>(src_packed, src_qabsmax, blocks, n, out_features, in_features, qbs, dst_layout,
                                   dst_packed, dst_qabsmax, stream);
}

int nsmlp_absmax_dq_quantize(const float* absmax, long long n, int dq_block, const float* code2, float offset,
                             uint8_t* q, float* absmax2, void* stream) {
  if (n < 0 || dq_block <= 0 || dq_block > 4096 || (dq_block & (dq_block - 1)) != 0)
    return set_error(NSMLP_EINVAL, "dq_block %d must be a power of two in [1, 4096]", dq_block);
  if (n == 0) return NSMLP_OK;
  if (!absmax || !code2 || !q || !absmax2) return set_error(NSMLP_EINVAL, "NULL tensor argument");
  launch_absmax_dq(absmax, n, dq_block, code2, offset, q, absmax2, (hipStream_t)stream);
  return check_launch("absmax double quantisation");
}

int nsmlp_absmax_dq_dequantize(const uint8_t* q, long long n, int dq_block, const float* code2, const float* absmax2,
                               float offset, float* out, void* stream) {
  if (n < 0 || dq_block <= 0 || (dq_block & (dq_block - 1)) != 0)
    return set_error(NSMLP_EINVAL, "dq_block %d must be a power of two", dq_block);
  if (n == 0) return NSMLP_OK;
  if (!q || !code2 || !absmax2 || !out) return set_error(NSMLP_EINVAL, "NULL tensor argument");
  launch_absmax_undq(q, n, __builtin_ctz((unsigned)dq_block), code2, absmax2, offset, out, (hipStream_t)stream);
  return check_launch("absmax double dequantisation");
}

int nsmlp_host_device_pointer(const void* host, void** device_ptr) {
  if (!host || !device_ptr) return set_error(NSMLP_EINVAL, "NULL pointer");
  hipError_t e = hipHostGetDevicePointer(device_ptr, const_cast<void*>(host), 0);
  if (e != hipSuccess) return set_error(NSMLP_EHIP, "hipHostGetDevicePointer: %s", hipGetErrorString(e));
  return NSMLP_OK;
}

int nsmlp_synth_normal_f16(uint64_t seed, long long n, float std, void* out, void* stream) {
  if (n < 0 || (n > 0 && !out)) return set_error(NSMLP_EINVAL, "bad synth arguments");
  if (n == 0) return NSMLP_OK;
  launch_synth_normal_f16(seed, n, std, (uint16_t*)out, (hipStream_t)stream);
  return check_launch("synth normal f16");
}

int nsmlp_synth_normal_f32(uint64_t seed, long long n, float std, float* out, void* stream) {
  if (n < 0 || (n > 0 && !out)) return set_error(NSMLP_EINVAL, "bad synth arguments");
  if (n == 0) return NSMLP_OK;
  launch_synth_normal_f32(seed, n, std, out, (hipStream_t)stream);
  return check_launch("synth normal f32");
}

int nsmlp_synth_nf4(uint64_t seed, long long n, int qbs, float std, uint8_t* packed, float* absmax, void* stream) {
  if (qbs <= 0 || qbs % 8 != 0 || n < 0 || n % qbs != 0)
    return set_error(NSMLP_EINVAL, "n=%lld must be a multiple of the quant block size %d (multiple of 8)", n, qbs);
  if (n == 0) return NSMLP_OK;
  if (!packed || !absmax) return set_error(NSMLP_EINVAL, "NULL output");
  if (((uintptr_t)packed & 3u) != 0) return set_error(NSMLP_EINVAL, "packed must be 4-byte aligned");
  int rc = ensure_midpoints();
  if (rc) return rc;
  launch_nf4_quant(nullptr, seed, std, n, qbs, true, packed, absmax, (hipStream_t)stream);
  return check_launch("synth nf4");
}

int nsmlp_nf4_quantize_f32(const float* w, long long n, int qbs, uint8_t* packed, float* absmax, void* stream) {
  if (qbs <= 0 || qbs % 8 != 0 || n < 0 || n % qbs != 0)
    return set_error(NSMLP_EINVAL, "n=%lld must be a multiple of the quant block size %d (multiple of 8)", n, qbs);
  if (n == 0) return NSMLP_OK;
  if (!w || !packed || !absmax) return set_error(NSMLP_EINVAL, "NULL tensor argument");
  if (((uintptr_t)packed & 3u) != 0) return set_error(NSMLP_EINVAL, "packed must be 4-byte aligned");
  int rc = ensure_midpoints();
  if (rc) return rc;
  launch_nf4_quant(w, 0, 0.0f, n, qbs, false, packed, absmax, (hipStream_t)stream);
  return check_launch("nf4 quantize");
}

size_t nsmlp_cache_workspace_bytes(int n) {
  if (n < 0) n = 0;
  // the counter region first (left untouched: the workspace may be shared
  // with the decode entry points), then the novel and copy lists
  return align_up(kCounterBytes) + align_up((size_t)n * 4) * 3 + align_up(4);
}

int nsmlp_cache_promote(const nsmlp_slot_table* table, const nsmlp_cache_state* cache, const int32_t* blocks, int n,
                        int flags, int32_t* slot_out, void* ws, size_t ws_bytes, void* stream) {
  NSMLP_FAULT_POINT("cache_promote");
  if (table == nullptr || cache == nullptr) return set_error(NSMLP_EINVAL, "table and cache must be non-NULL");
  DecodeArgs a;
  int rc = table_to_args(table, a);
  if (rc != NSMLP_OK) return rc;
  if (n < 0 || n > 65535) return set_error(NSMLP_EINVAL, "n = %d out of range [0, 65535]", n);
  if (n > 0 && blocks == nullptr) return set_error(NSMLP_EINVAL, "blocks must be non-NULL");
  if ((flags & ~NSMLP_CACHE_GROW_ONLY) != 0) return set_error(NSMLP_EINVAL, "unknown flags 0x%x", flags);
  const int cap = cache->capacity;
  if (cap < 1 || cap > kMaxCacheSlots)
    return set_error(NSMLP_EINVAL, "cache capacity %d out of range [1, %d]", cap, kMaxCacheSlots);
  if (cap != table->n_slots)
    return set_error(NSMLP_EINVAL, "cache capacity %d differs from the table's n_slots %d", cap, table->n_slots);
  if (cache->lookup == nullptr || (const int32_t*)cache->lookup != table->lookup)
    return set_error(NSMLP_EINVAL, "the cache's lookup must be the table's (non-NULL) lookup");
  if (cache->slot_block == nullptr || cache->slot_score == nullptr || cache->active_count == nullptr)
    return set_error(NSMLP_EINVAL, "slot_block, slot_score and active_count must be non-NULL");
  if (table->host_gate_packed == nullptr)
    return set_error(NSMLP_EINVAL, "promotion copies blocks from the table's host copies, which are absent");
  if (n > 0 && (ws == nullptr || ws_bytes < nsmlp_cache_workspace_bytes(n)))
    return set_error(NSMLP_ENOSPC, "workspace of %zu bytes < %zu", ws_bytes, nsmlp_cache_workspace_bytes(n));
  if (n == 0) return NSMLP_OK;
  CacheArgs c;
  memset(&c, 0, sizeof(c));
  c.NB = a.NB;
  c.capacity = cap;
  c.n = n;
  c.grow_only = (flags & NSMLP_CACHE_GROW_ONLY) ? 1 : 0;
  c.lookup = cache->lookup;
  c.slot_block = cache->slot_block;
  c.slot_score = cache->slot_score;
  c.active = cache->active_count;
  c.blocks = blocks;
  c.plan_out = slot_out;
  if (((uintptr_t)ws & (kAlign - 1)) != 0) return set_error(NSMLP_EINVAL, "workspace must be 256-byte aligned");
  uint8_t* w = (uint8_t*)ws + align_up(kCounterBytes);
  const size_t ln = align_up((size_t)n * 4);
  c.novel = (int32_t*)w;
  c.copy_block = (int32_t*)(w + ln);
  c.copy_slot = (int32_t*)(w + 2 * ln);
  c.n_copy = (int32_t*)(w + 3 * ln);
  const bool dq = table->dq_block > 0;
  const long long H = table->H, A = H / table->qbs;
  const void* src[6] = {table->host_gate_packed,
                        dq ? (const void*)table->host_gate_qabsmax : (const void*)table->host_gate_absmax,
                        table->host_up_packed,
                        dq ? (const void*)table->host_up_qabsmax : (const void*)table->host_up_absmax,
                        table->host_down_packed,
                        dq ? (const void*)table->host_down_qabsmax : (const void*)table->host_down_absmax};
  const void* dst[6] = {table->gate_packed, dq ? (const void*)table->gate_qabsmax : (const void*)table->gate_absmax,
                        table->up_packed, dq ? (const void*)table->up_qabsmax : (const void*)table->up_absmax,
                        table->down_packed,
                        dq ? (const void*)table->down_qabsmax : (const void*)table->down_absmax};
  const long long bytes[6] = {16 * H, dq ? 32 * A : 128 * A, 16 * H, dq ? 32 * A : 128 * A, 16 * H, dq ? H : 4 * H};
  for (int i = 0; i < 6; ++i) {
    if (src[i] == nullptr || dst[i] == nullptr)
      return set_error(NSMLP_EINVAL, "slot and host-copy arrays must all be non-NULL");
    if (!aligned16(src[i]) || !aligned16(dst[i]) || bytes[i] % 16 != 0)
      return set_error(NSMLP_EINVAL, "slot and host-copy arrays must be 16-byte aligned");
    c.src[i] = (const uint8_t*)src[i];
    c.dst[i] = (uint8_t*)const_cast<void*>(dst[i]);  // the table's slots are written in place
    c.bytes[i] = bytes[i];
  }
  launch_cache_promote(c, (hipStream_t)stream);
  return check_launch("nsmlp_cache_promote");
}

int nsmlp_cache_record_f32(float* counts, int NB, const int32_t* blocks, int rows, int k, const float* row_weights,
                           void* stream) {
  NSMLP_FAULT_POINT("cache_record_f32");
  if (counts == nullptr || NB <= 0) return set_error(NSMLP_EINVAL, "counts must be non-NULL and NB >= 1");
  if (rows < 0 || k < 0 || (long long)rows * k >= (1LL << 31))
    return set_error(NSMLP_EINVAL, "rows %d x k %d out of range", rows, k);
  if ((long long)rows * k == 0) return NSMLP_OK;
  if (blocks == nullptr) return set_error(NSMLP_EINVAL, "blocks must be non-NULL");
  launch_cache_record(counts, NB, blocks, rows, k, row_weights, (hipStream_t)stream);
  return check_launch("nsmlp_cache_record_f32");
}

}  // extern "C"
