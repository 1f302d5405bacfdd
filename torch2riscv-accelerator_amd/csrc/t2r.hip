// libt2r.so: the C-ABI of include/t2r.h over the gfx950 kernels (one translation unit).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstddef>
#include <cstring>
#include <type_traits>
#include <mutex>
#include <new>
#include <vector>

#include "../../include/t2r.h"
#include "t2r_attn.h"
#include "t2r_device.h"
#include "t2r_gemm.h"
#include "t2r_gemv.h"
#include "t2r_misc.h"

namespace t2r {
__constant__ float c_sfu[kSfuWords];
}

// The workspace of every model made by t2r_model_create_static on a device: one array per device,
// held until the process ends. Its first T2R_STATIC_STATE_BYTES hold each pool slot's carried state
// (kStateSlotBytes a slot: the status word, the split attention's counters and SPLIT 1's sums), the
// rest is the scratch of one call, shared by all such models there (their calls must not overlap).
// Host code uses its per-device address from hipGetSymbolAddress (g_scratch_addr), never the name.
static __device__ __align__(256) char scratch[T2R_STATIC_WORKSPACE_BYTES];

using namespace t2r;

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_init_mu;
bool g_inited[kMaxDevices];
const float* g_sfu_addr[kMaxDevices];
char* g_scratch_addr[kMaxDevices];

// The SFU tables (llm/sfu.py:42-56): segment start T and slope S of each function, computed in
// double and rounded once to float.
void sfu_host_tables(float* t) {
  for (int k = 0; k < 64; ++k) {
    const double te = std::pow(2.0, k / 64.0), te1 = std::pow(2.0, (k + 1) / 64.0);
    t[kSfuExpT + k] = (float)te;
    t[kSfuExpS + k] = (float)(te1 - te);
    const double m = 1.0 + k / 64.0;
    const double tr = 1.0 / m;
    t[kSfuRecT + k] = (float)tr;
    t[kSfuRecS + k] = (float)(1.0 / (m + 1.0 / 64.0) - tr);
  }
  for (int j = 0; j < 128; ++j) {
    const int k = j & 63;
    const double m2 = j < 64 ? 1.0 + k / 64.0 : 2.0 * (1.0 + k / 64.0);
    const double step = j < 64 ? 1.0 / 64.0 : 2.0 / 64.0;
    const double tq = 1.0 / std::sqrt(m2);
    t[kSfuRsqT + j] = (float)tq;
    t[kSfuRsqS + j] = (float)(1.0 / std::sqrt(m2 + step) - tq);
  }
}

int ensure_init() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return T2R_EHIP;
  std::lock_guard<std::mutex> lk(g_init_mu);
  if (g_inited[dev]) return T2R_OK;
  float t[kSfuWords];
  sfu_host_tables(t);
  // sfu_exp_sm's table identities: F(T[63] + S[63]) = 2 and T[0] = 1
  if (t[kSfuExpT + 63] + t[kSfuExpS + 63] != 2.0f || t[kSfuExpT] != 1.0f) return T2R_EHIP;
  if (hipMemcpyToSymbol(HIP_SYMBOL(c_sfu), t, sizeof(t), 0, hipMemcpyHostToDevice) != hipSuccess) return T2R_EHIP;
  void* addr = nullptr;
  if (hipGetSymbolAddress(&addr, HIP_SYMBOL(c_sfu)) != hipSuccess || addr == nullptr) return T2R_EHIP;
  // the prefill attention keeps up to kPreMaxLds of score rows in LDS (160 KB per CU on gfx950)
  const void* pre[] = {(const void*)k_attn_pre<32>, (const void*)k_attn_pre<64>, (const void*)k_attn_pre<128>,
                       (const void*)k_attn_pre<32, true>, (const void*)k_attn_pre<64, true>,
                       (const void*)k_attn_pre<128, true>};
  for (const void* f : pre)
    if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kPreMaxLds) != hipSuccess)
      return T2R_EHIP;
  if (hipFuncSetAttribute((const void*)k_attn_pw<128, false>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)ap_lds<128>()) != hipSuccess ||
      hipFuncSetAttribute((const void*)k_attn_pw<64, false>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)ap_lds<64>()) != hipSuccess ||
      hipFuncSetAttribute((const void*)k_attn_pw<128, true>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)ap_lds<128>()) != hipSuccess ||
      hipFuncSetAttribute((const void*)k_attn_pw<64, true>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)ap_lds<64>()) != hipSuccess)
    return T2R_EHIP;
  // the GEMM's deep-ring configuration: 128 KB of LDS, one workgroup per CU
  const void* deep[] = {(const void*)k_gemm_d<EPI_STORE, false, 128, 4>, (const void*)k_gemm_d<EPI_STORE, true, 128, 4>,
                        (const void*)k_gemm_d<EPI_RESID, false, 128, 4>, (const void*)k_gemm_d<EPI_RESID, true, 128, 4>,
                        (const void*)k_gemm_d<EPI_SWIGLU, false, 128, 4>};
  for (const void* f : deep)
    if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kGemmDDeepLds) != hipSuccess)
      return T2R_EHIP;
  // the wave-split-K linears: four wave rings of 2 x (64 + TN) x 128 bytes (128 / 160 KB)
  if (hipFuncSetAttribute((const void*)k_gemm_w<EPI_STORE, 64, 64>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)gemm_w_lds<64, 64>()) != hipSuccess ||
      hipFuncSetAttribute((const void*)k_gemm_w<EPI_RESID, 64, 64>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)gemm_w_lds<64, 64>()) != hipSuccess ||
      hipFuncSetAttribute((const void*)k_gemm_w<EPI_STORE, 64, 96>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)gemm_w_lds<64, 96>()) != hipSuccess ||
      hipFuncSetAttribute((const void*)k_gemm_w<EPI_RESID, 64, 96>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)gemm_w_lds<64, 96>()) != hipSuccess)
    return T2R_EHIP;
  // the grouped decode attention: score rows of caches up to kMaxS positions
  const void* gqa[] = {(const void*)k_attn_gqa<4, false, 1>, (const void*)k_attn_gqa<4, true, 1>,
                       (const void*)k_attn_gqa<4, false, 2>, (const void*)k_attn_gqa<4, true, 2>,
                       (const void*)k_attn_gqa<8, false, 1>, (const void*)k_attn_gqa<8, true, 1>,
                       (const void*)k_attn_gqa<8, false, 2>, (const void*)k_attn_gqa<8, true, 2>};
  for (const void* f : gqa)
    if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kGqaMaxLds) != hipSuccess)
      return T2R_EHIP;
  // the two-row-group batched GEMV at eight waves: 8 x 8448 bytes of LDS (the int32 tile of 64 rows)
  const void* bg2[] = {(const void*)k_bgemv<EPI_STORE, 8, false, 2>, (const void*)k_bgemv<EPI_STORE, 8, true, 2>,
                       (const void*)k_bgemv<EPI_RESID, 8, false, 2>, (const void*)k_bgemv<EPI_RESID, 8, true, 2>,
                       (const void*)k_bgemv<EPI_SWIGLU, 8, false, 2>};
  for (const void* f : bg2)
    if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, 8 * bg_wave_lds(2)) != hipSuccess)
      return T2R_EHIP;
  if (hipFuncSetAttribute((const void*)k_gemm_d<EPI_SWIGLU, false, 128, 3, 2 * kGT>,
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)kGemmDTallLds) != hipSuccess)
    return T2R_EHIP;
  void* ws = nullptr;
  if (hipGetSymbolAddress(&ws, HIP_SYMBOL(scratch)) != hipSuccess || ws == nullptr) return T2R_EHIP;
  g_sfu_addr[dev] = (const float*)addr;
  g_scratch_addr[dev] = (char*)ws;
  g_inited[dev] = true;
  return T2R_OK;
}

#define T2R_INIT()                 \
  do {                             \
    int rc_ = ensure_init();       \
    if (rc_ != T2R_OK) return rc_; \
  } while (0)

inline int launched() { return hipGetLastError() == hipSuccess ? T2R_OK : T2R_EHIP; }
inline hipStream_t S(void* s) { return (hipStream_t)s; }
inline int cdiv(long long a, long long b) { return (int)((a + b - 1) / b); }

// The device address of this device's SFU tables: kernels that stage them into LDS read them
// through this plain pointer (a load from the __constant__ symbol itself may be moved by the
// compiler to its first use, behind the weight loads).
const float* sfu_table_ptr() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  return g_sfu_addr[dev];
}

GemvArgs gemv_args() {
  GemvArgs a;
  std::memset(&a, 0, sizeof(a));
  a.D = 16;
  a.tab = sfu_table_ptr();
  return a;
}

// positions a prefill row may attend to: the caller's bound (t2r_prefill_at), else the cache length
int pre_cap(const AttnArgs& a) { return a.t_cap > 0 && a.t_cap < a.S ? a.t_cap : a.S; }

// the multi-row prefill attention: head dims 16..128 (multiples of 16), cache rows whose
// score rows fit the LDS the kernels are set up for (kPreMaxLds)
bool pre_ok(const AttnArgs& a) {
  return a.hd % 16 == 0 && a.hd <= 128 && attn_pre_lds_bytes(pre_cap(a), (a.hd + 31) & ~31) <= kPreMaxLds;
}
// ... and its 32-row form (k_attn_pw): head dims 128 and 64 without the HF options, rows attending to at
// most ap_keys positions
bool pw_ok(const AttnArgs& a) {
  if (attn_opt(a) || !(a.D == 8 || a.D == 16)) return false;
  return (a.hd == 128 && pre_cap(a) <= ap_keys<128>()) || (a.hd == 64 && pre_cap(a) <= ap_keys<64>());
}
// the multi-row ATTN_ONLY launch runs k_attn_pw (only then may q come as int8 rows: AttnArgs::q8)
inline bool pw_takes(const AttnArgs& a) { return a.tab != nullptr && a.kv_row_stride == 0 && pw_ok(a); }

// batch-1 decode attention split over workgroups per head (k_attn_dec's SPLIT forms): the heads of a
// model whose shape takes it (head dim 128, caches over 512 rows, 4 splits a head in at most 256
// workgroups), else 0
constexpr int kSplits = 4;
inline int split_heads(const t2r_model_desc& d) {
  return d.head_dim == 128 && d.seq_len > 512 && d.heads * kSplits <= 256 ? d.heads : 0;
}
inline bool attn_split(const AttnArgs& a, int rows) {
  return a.nsplit > 1 && rows == 1 && a.hd == 128 && a.sp_s && a.sp_o && a.sp_acc && a.sp_sync;
}
// ... and whether it leaves its int32 P.V sums per split for the next linear (SPLIT 2) instead of att
inline bool attn_split_to_linear(const AttnArgs& a, int rows) { return attn_split(a, rows) && !attn_opt(a); }

int attn_launch(int mode, const AttnArgs& a, int rows, hipStream_t st) {
  if (a.H <= 0 || a.Hk <= 0 || a.H % a.Hk || a.hd <= 0 || a.hd > kMaxHd || a.hd % 8 || a.S <= 0 || a.S > kMaxS ||
      (a.D != 8 && a.D != 16))
    return T2R_ESHAPE;
  // int8 q rows (AttnArgs::q8) pass from the prep kernels at head dims 64 / 128 to k_attn_pw only
  if (a.q8 != nullptr && (mode == ATTN_FUSED || (mode == ATTN_PREP && a.hd != 64 && a.hd != 128) ||
                          (mode == ATTN_ONLY && !pw_takes(a))))
    return T2R_ESHAPE;
  const size_t lds = mode == ATTN_PREP ? 0 : attn_lds_bytes(a.S, a.D);
  dim3 grid(a.H, rows), block(kAttnThreads);
  const bool c16 = a.hd % 16 == 0;
  // batched decode: per (row, KV head) its group of 2..4 query heads, over G / gw workgroups
  const int G = a.H / a.Hk;
  const bool opt = attn_opt(a);                 // the HF options: the kernels' OPT instantiations
  // the group split over workgroups: two query heads each for four-head groups, else one
  // (G / gw workgroups per KV head), each with its gw heads' score rows in LDS
  const int gw = G == 4 ? 2 : 1;
  if (mode == ATTN_FUSED && rows > 1 && a.tab != nullptr && G >= 2 && G <= kGqaMaxG &&
      (a.hd == 64 || a.hd == 128) && attn_gqa_lds_bytes(a.S, a.D, gw) <= kGqaMaxLds) {
    const dim3 gs(a.Hk * (G / gw), rows);
    const size_t gl = attn_gqa_lds_bytes(a.S, a.D, gw);
    if (gw == 2) {
      if (a.hd == 64) {
        if (opt) launch((k_attn_gqa<4, true, 2>), gs, dim3(kGqaThreads), gl, st, a);
        else launch((k_attn_gqa<4, false, 2>), gs, dim3(kGqaThreads), gl, st, a);
      } else {
        if (opt) launch((k_attn_gqa<8, true, 2>), gs, dim3(kGqaThreads), gl, st, a);
        else launch((k_attn_gqa<8, false, 2>), gs, dim3(kGqaThreads), gl, st, a);
      }
    } else {
      if (a.hd == 64) {
        if (opt) launch((k_attn_gqa<4, true, 1>), gs, dim3(kGqaThreads), gl, st, a);
        else launch((k_attn_gqa<4, false, 1>), gs, dim3(kGqaThreads), gl, st, a);
      } else {
        if (opt) launch((k_attn_gqa<8, true, 1>), gs, dim3(kGqaThreads), gl, st, a);
        else launch((k_attn_gqa<8, false, 1>), gs, dim3(kGqaThreads), gl, st, a);
      }
    }
    return launched();
  }
  if (mode == ATTN_FUSED && a.tab != nullptr && a.hd % 16 == 0 &&
      (a.hd == 16 || a.hd == 32 || a.hd == 48 || a.hd == 64 || a.hd == 128)) {
    const size_t dl = attn_dec_lds_bytes(a.S, a.D);
    if (attn_split(a, rows)) {
      // (without the HF options the next linear adds the splits' sums: attn_split_to_linear)
      const dim3 gs(a.H, a.nsplit);
      if (opt) launch((k_attn_dec<8, true, 1>), gs, block, dl, st, a);
      else launch((k_attn_dec<8, false, 2>), gs, block, dl, st, a);
    } else if (opt) {
      switch (a.hd / 16) {
        case 1: launch((k_attn_dec<1, true>), grid, block, dl, st, a); break;
        case 2: launch((k_attn_dec<2, true>), grid, block, dl, st, a); break;
        case 3: launch((k_attn_dec<3, true>), grid, block, dl, st, a); break;
        case 4: launch((k_attn_dec<4, true>), grid, block, dl, st, a); break;
        default: launch((k_attn_dec<8, true>), grid, block, dl, st, a); break;
      }
    } else {
      switch (a.hd / 16) {
        case 1: launch((k_attn_dec<1>), grid, block, dl, st, a); break;
        case 2: launch((k_attn_dec<2>), grid, block, dl, st, a); break;
        case 3: launch((k_attn_dec<3>), grid, block, dl, st, a); break;
        case 4: launch((k_attn_dec<4>), grid, block, dl, st, a); break;
        default: launch((k_attn_dec<8>), grid, block, dl, st, a); break;
      }
    }
  } else if (mode == ATTN_FUSED) {
    if (c16) launch((k_attn<ATTN_FUSED, 16>), grid, block, lds, st, a);
    else launch((k_attn<ATTN_FUSED, 8>), grid, block, lds, st, a);
  } else if (mode == ATTN_PREP) {
    const dim3 pg(cdiv(a.H + a.Hk, kPrepWaves), rows), pb(64 * kPrepWaves);
    // two vectors a wave over many rows (C3 prefill 5.86 -> 5.77 ms, C4 1.85 -> 1.83 ms); a short
    // prompt keeps a wave per vector, for the parallelism (C2's 40 rows: 1.53 against 1.57 ms)
    // at head dim 64 two rows a wave, all their loads issued first (C4's prep 5.7 -> 5.4 us; at head
    // dim 128 two rows took 14.6 against 13.0 us)
    const dim3 pg2(cdiv(a.H + a.Hk, 2 * kPrepWaves), rows), pg2r(cdiv(a.H + a.Hk, 2 * kPrepWaves), cdiv(rows, 2));
    if (a.hd == 128 && rows >= 256) launch((k_attn_prep_h2<128, 1>), pg2, pb, 0, st, a, rows);
    else if (a.hd == 64 && rows >= 256) launch((k_attn_prep_h2<64, 2>), pg2r, pb, 0, st, a, rows);
    else if (a.hd == 128) launch(k_attn_prep_h<128>, pg, pb, 0, st, a);
    else if (a.hd == 64) launch(k_attn_prep_h<64>, pg, pb, 0, st, a);
    else launch(k_attn_prep, pg, pb, 0, st, a);
  } else if (pw_takes(a)) {
    const dim3 grid_pw(a.H, cdiv(rows, kApRows));
    // (q quantized by the prep kernel when the caller set q8: the Q8I form)
    if (a.q8 != nullptr) {
      if (a.hd == 128) launch((k_attn_pw<128, true>), grid_pw, dim3(kApThreads), ap_lds<128>(), st, a, rows);
      else launch((k_attn_pw<64, true>), grid_pw, dim3(kApThreads), ap_lds<64>(), st, a, rows);
    } else if (a.hd == 128) {
      launch((k_attn_pw<128, false>), grid_pw, dim3(kApThreads), ap_lds<128>(), st, a, rows);
    } else {
      launch((k_attn_pw<64, false>), grid_pw, dim3(kApThreads), ap_lds<64>(), st, a, rows);
    }
  } else if (a.tab != nullptr && a.kv_row_stride == 0 && pre_ok(a)) {
    const int hdp = (a.hd + 31) & ~31;
    dim3 pg(a.H, cdiv(rows, kPreRows));
    const size_t pl = attn_pre_lds_bytes(pre_cap(a), hdp);
    if (opt) {
      if (hdp == 32) launch((k_attn_pre<32, true>), pg, dim3(pre_threads(hdp)), pl, st, a, rows);
      else if (hdp == 64) launch((k_attn_pre<64, true>), pg, dim3(pre_threads(hdp)), pl, st, a, rows);
      else launch((k_attn_pre<128, true>), pg, dim3(pre_threads(hdp)), pl, st, a, rows);
    } else {
      if (hdp == 32) launch((k_attn_pre<32>), pg, dim3(pre_threads(hdp)), pl, st, a, rows);
      else if (hdp == 64) launch((k_attn_pre<64>), pg, dim3(pre_threads(hdp)), pl, st, a, rows);
      else launch((k_attn_pre<128>), pg, dim3(pre_threads(hdp)), pl, st, a, rows);
    }
  } else {
    if (c16) launch((k_attn<ATTN_ONLY, 16>), grid, block, lds, st, a);
    else launch((k_attn<ATTN_ONLY, 8>), grid, block, lds, st, a);
  }
  return launched();
}

// ---------------------------------------------------------------- the resident model
constexpr int kMaxLayers = 256;

struct Model {
  t2r_model_desc d;
  float kvc[kMaxLayers * 4];        // [L, 4]
  int32_t kv_flags[kMaxLayers];     // [L]: bit 0 K per channel, bit 1 V per channel
  int pool_slot = -1;               // t2r_model_create_static: its slot in the static pool
  int q_dim, kv_dim, qkv_dim, ffn_rows, max_in;
  int32_t* part;                    // split-K partial sums of the prefill linears
  int part_rows;
  // a residual linear (Wo, W2) whose split-K partials in `part` are not yet added into x: the
  // next row norm/quant of x finishes them in the same pass (k_rows_fin_quant), any other reader
  // of x first runs the plain finish (fin_flush)
  int pend_z = 0, pend_rows = 0;
  const float* pend_sw = nullptr;
  float* x;
  float* qkv;
  float* att;
  float* u;
  int8_t* xq;
  float* sx;
  float* logits;
  unsigned long long* keys;
  int32_t* ids;
  float* wts;
  int8_t* mxq;
  float* msx;
  int32_t* status;
  // batch-1 decode attention split over workgroups per head (nsplit > 1; 0 when the shape does not take
  // it or the device cannot hold a launch's workgroups at once): published scores [H, S] and SPLIT 2's
  // per-split P.V sums [4, H, kMaxHd] (both within one step); SPLIT 1's met sums [H, kMaxHd] and the
  // arrival counters [H, 2], carried from launch to launch (zeroed at creation)
  int nsplit = 0;
  float* sp_s;
  int32_t* sp_o;
  int32_t* sp_acc;
  uint32_t* sp_sync;
  // MoE over many rows, grouped by expert: route lists, the routes' int8 expert outputs and scales,
  // and their weighted down projections (MoE models only)
  int32_t* moe_off = nullptr;
  int32_t* moe_list = nullptr;
  int8_t* moe_hq = nullptr;
  float* moe_sh = nullptr;
  float* moe_t = nullptr;
  // batched decode (t2r_decode_batch): the caches of the step's sequences, kv_rs bytes apart
  int8_t* kcb = nullptr;
  int8_t* vcb = nullptr;
  long long kv_rs = 0;
  // t2r_prefill_at: positions start .. start + M - 1 (device), and their bound for the attention
  int32_t* pos_rows = nullptr;
  int t_cap = 0;
  // kernel timing (t2r_model_profile)
  int prof_mask = 0;
  std::vector<hipEvent_t> ev;
  std::vector<int32_t> ev_kind;
  int ev_used = 0;
};

// the launches of one kernel class between a start and a stop event (kernel start / kernel end)
struct ProfScope {
  Model* m;
  bool on;
  ProfScope(Model* m_, int kind, hipStream_t) : m(m_), on(false) {
    if ((m->prof_mask >> kind) & 1 && m->ev_used + 2 <= (int)m->ev.size()) {
      on = true;
      m->ev_kind[m->ev_used / 2] = kind;
      g_launch_events.start = m->ev[m->ev_used];
      g_launch_events.stop = m->ev[m->ev_used + 1];
    }
  }
  ~ProfScope() {
    if (on) {
      m->ev_used += 2;
      g_launch_events = LaunchEvents();
    }
  }
};

void free_events(Model* m) {
  for (hipEvent_t e : m->ev) (void)hipEventDestroy(e);
  m->ev.clear();
  m->ev_kind.clear();
  m->ev_used = 0;
  m->prof_mask = 0;
}

struct Carve {
  char* base;
  long long off;
  template <class T>
  T* take(long long n) {
    off = (off + 255) / 256 * 256;
    T* p = base ? (T*)(base + off) : nullptr;
    off += n * (long long)sizeof(T);
    return p;
  }
};

// The state a model carries from one call to the next (the status word, the split attention's counters
// and SPLIT 1's sums) comes first, from `state` when ext_state (a static model's own pool slot), else
// from the workspace; the rest is the scratch of one call. Returns the workspace bytes; *state_bytes
// (when given) the state's.
long long carve(Model* m, char* base, int M, char* state = nullptr, bool ext_state = false,
                long long* state_bytes = nullptr) {
  const t2r_model_desc& d = m->d;
  Carve c{base, 0}, cs{state, 0};
  Carve& st = ext_state ? cs : c;
  const int hs = split_heads(d);
  m->status = st.take<int32_t>(1);
  m->sp_sync = st.take<uint32_t>(2LL * hs);
  m->sp_acc = st.take<int32_t>((long long)hs * kMaxHd);
  if (state_bytes) *state_bytes = st.off;
  m->x = c.take<float>((long long)M * d.dim);
  m->qkv = c.take<float>((long long)M * m->qkv_dim);
  m->att = c.take<float>((long long)M * m->q_dim);
  m->u = c.take<float>((long long)M * m->ffn_rows);
  m->xq = c.take<int8_t>((long long)M * m->max_in);
  m->sx = c.take<float>(M);
  m->logits = c.take<float>(d.vocab);
  m->keys = c.take<unsigned long long>(M);
  const int k = d.top_k > 0 ? d.top_k : 1;
  m->ids = c.take<int32_t>((long long)M * k);
  m->wts = c.take<float>((long long)M * k);
  m->mxq = c.take<int8_t>((long long)M * d.dim);
  m->msx = c.take<float>(M);
  m->pos_rows = c.take<int32_t>(M);
  m->sp_s = c.take<float>((long long)hs * d.seq_len);
  m->sp_o = c.take<int32_t>((long long)kSplits * hs * kMaxHd);
  if (d.n_experts > 0) {
    const long long routes = (long long)M * k;
    m->moe_off = c.take<int32_t>(d.n_experts + 1);
    m->moe_list = c.take<int32_t>(routes);
    m->moe_hq = c.take<int8_t>(routes * d.hidden);
    m->moe_sh = c.take<float>(routes);
    m->moe_t = c.take<float>(routes * d.dim);
  }
  // split-K partial sums of the prefill linears: 4 splits of up to 2048 rows of the widest
  // STORE / RESID output (C3's 2032-row prompt: 133 MB)
  m->part_rows = M < 2048 ? M : 2048;
  m->part = c.take<int32_t>(4LL * m->part_rows * (m->qkv_dim > d.dim ? m->qkv_dim : d.dim));
  return c.off;
}

void model_dims(Model* m) {
  const t2r_model_desc& d = m->d;
  m->q_dim = d.heads * d.head_dim;
  m->kv_dim = d.kv_heads * d.head_dim;
  m->qkv_dim = m->q_dim + 2 * m->kv_dim;
  m->ffn_rows = d.n_experts > 0 ? d.top_k * d.hidden : d.hidden;
  int mi = d.dim;
  if (m->q_dim > mi) mi = m->q_dim;
  if (d.hidden > mi) mi = d.hidden;
  m->max_in = mi;
}

// the caller's descriptor as the current version: an ABI-1 descriptor ends before the HF options,
// which are then off
bool desc_read(const t2r_model_desc* in, t2r_model_desc* out) {
  if (!in || (in->abi_version != 1 && in->abi_version != T2R_ABI_VERSION)) return false;
  std::memset(out, 0, sizeof(*out));
  std::memcpy(out, in, in->abi_version == 1 ? offsetof(t2r_model_desc, attn_qsum) : sizeof(*out));
  out->abi_version = T2R_ABI_VERSION;
  return true;
}

int validate(const t2r_model_desc* d) {
  if (!d || d->abi_version != T2R_ABI_VERSION) return T2R_EINVAL;
  if ((d->attn_qsum != 0 && d->attn_qsum != 1) || (d->ffn_act != 0 && d->ffn_act != 1)) return T2R_EINVAL;
  if (d->kv_channel_flags) {
    for (int l = 0; l < d->layers; ++l) {
      if (d->kv_channel_flags[l] & ~3) return T2R_EINVAL;
      if (d->kv_channel_flags[l] && !d->kv_channel) return T2R_EINVAL;
    }
  }
  if (d->dim <= 0 || d->hidden <= 0 || d->layers <= 0 || d->layers > kMaxLayers || d->heads <= 0 ||
      d->kv_heads <= 0 || d->head_dim <= 0 || d->vocab <= 0 || d->seq_len <= 0)
    return T2R_ESHAPE;
  if (d->heads % d->kv_heads || d->heads / d->kv_heads > kMaxG || d->head_dim > kMaxHd || d->head_dim % 8)
    return T2R_ESHAPE;
  const int q = d->heads * d->head_dim, kv = d->kv_heads * d->head_dim;
  if (d->dim % 16 || d->hidden % 16 || q % 16 || kv % 16 || d->dim > kMaxK || d->hidden > kMaxK || q > kMaxK)
    return T2R_ESHAPE;
  if (d->seq_len > kMaxS) return T2R_ESHAPE;
  if (d->D != 8 && d->D != 16) return T2R_ESHAPE;
  if (d->n_experts < 0 || (d->n_experts > 0 && (d->top_k < 1 || d->top_k > 8 || d->top_k > d->n_experts ||
                                                d->n_experts > 64 || d->hidden > 1024)))
    return T2R_ESHAPE;
  if (!d->emb_q || !d->emb_s || !d->cls_q || !d->cls_s || !d->rms_att || !d->rms_ffn || !d->rms_final ||
      !d->wqkv || !d->s_wqkv || !d->wo || !d->s_wo || !d->rope_cos || !d->rope_sin || !d->kv_consts ||
      !d->k_cache || !d->v_cache || !d->workspace)
    return T2R_EINVAL;
  if (d->qk_norm && (!d->q_norm || !d->k_norm)) return T2R_EINVAL;
  if (d->n_experts > 0) {
    if (!d->router || !d->s_router || !d->wg || !d->s_wg || !d->wu || !d->s_wu || !d->wd || !d->s_wd) return T2R_EINVAL;
  } else if (!d->w1 || !d->s_w1 || !d->w3 || !d->s_w3 || !d->w2 || !d->s_w2) {
    return T2R_EINVAL;
  }
  if (d->max_rows < 1) return T2R_ERANGE;
  return T2R_OK;
}

// the pending residual linear's finish on its own: x += dequant(sum of the partials)
int fin_flush(Model* m, hipStream_t st) {
  if (m->pend_z <= 1) return T2R_OK;
  GemmArgs a;
  std::memset(&a, 0, sizeof(a));
  a.s_x = m->sx; a.s_w = m->pend_sw; a.M = m->pend_rows; a.N = m->d.dim; a.K = m->d.dim;
  a.y = m->x; a.y_stride = m->d.dim; a.res = m->x; a.part = m->part;
  const int nz = m->pend_z;
  m->pend_z = 0;
  const long long total = (long long)a.M * a.N;
  launch((k_gemm_fin<EPI_RESID>), dim3((unsigned)(total < 4096LL * 256 ? (total + 255) / 256 : 4096)), dim3(256), 0, st, a,
         nz);
  return launched();
}

int rows_quant_staged(Model* m, const float* x, long long x_stride, const float* g, int K, int rows, hipStream_t st);

// RMSNorm (g != nullptr) and quant_act of `rows` rows x[rows, K] into the workspace's int8 rows. On
// the residual rows with a pending residual-linear finish, the finish runs in the same pass.
int rows_quant(Model* m, const float* x, long long x_stride, const float* g, int K, int rows, hipStream_t st) {
  if (m->pend_z > 1 && x == m->x) {
    const bool fused = g != nullptr && rows == m->pend_rows && K == m->d.dim && x_stride == K && K % 16 == 0 &&
                       K <= 8 * 1024 && ((uintptr_t)g & 15) == 0;
    if (!fused) {
      int rc = fin_flush(m, st);
      if (rc) return rc;
    } else {
      GemvArgs a = gemv_args();
      a.x = x; a.x_stride = x_stride; a.g = g; a.K = K; a.D = m->d.D; a.eps = m->d.eps; a.inv_n = (float)(1.0 / K);
      a.xq_out = m->xq; a.xq_stride = K; a.sx_out = m->sx;
      FinArgs f;
      f.part = m->part; f.zstride = (long long)rows * K; f.nz = m->pend_z; f.s_w = m->pend_sw; f.s_x = m->sx;
      f.x = m->x;
      m->pend_z = 0;
      const int nc = cdiv(K, 1024);
      const dim3 grid(rows), block(kGemvThreads);
      if (nc <= 1) launch(k_rows_fin_quant<1>, grid, block, 0, st, a, f);
      else if (nc <= 2) launch(k_rows_fin_quant<2>, grid, block, 0, st, a, f);
      else if (nc <= 4) launch(k_rows_fin_quant<4>, grid, block, 0, st, a, f);
      else launch(k_rows_fin_quant<8>, grid, block, 0, st, a, f);
      return launched();
    }
  }
  return rows_quant_staged(m, x, x_stride, g, K, rows, st);
}

int rows_quant_staged(Model* m, const float* x, long long x_stride, const float* g, int K, int rows, hipStream_t st) {
  GemvArgs a = gemv_args();
  a.x = x; a.x_stride = x_stride; a.g = g; a.K = K; a.D = m->d.D; a.eps = m->d.eps; a.inv_n = (float)(1.0 / K);
  a.xq_out = m->xq; a.xq_stride = K; a.sx_out = m->sx;
  const bool staged = K % 16 == 0 && K <= kMaxK && a.tab != nullptr && ((uintptr_t)x & 15) == 0 && x_stride % 4 == 0 &&
                      (g == nullptr || ((uintptr_t)g & 15) == 0);
  if (!staged) {
    launch(k_rows_norm_quant, dim3(rows), dim3(kGemvThreads), 0, st, a, g != nullptr ? 1 : 0, (float*)nullptr, 0LL);
    return launched();
  }
  const int nc = cdiv(K, 1024);
  const dim3 grid(rows), block(kGemvThreads);
  if (g != nullptr) {
    if (nc <= 1) launch((k_rows_quant<PRO_NORM_QUANT, 1>), grid, block, 0, st, a);
    else if (nc <= 2) launch((k_rows_quant<PRO_NORM_QUANT, 2>), grid, block, 0, st, a);
    else if (nc <= 4) launch((k_rows_quant<PRO_NORM_QUANT, 4>), grid, block, 0, st, a);
    else launch((k_rows_quant<PRO_NORM_QUANT, 8>), grid, block, 0, st, a);
  } else {
    if (nc <= 1) launch((k_rows_quant<PRO_QUANT, 1>), grid, block, 0, st, a);
    else if (nc <= 2) launch((k_rows_quant<PRO_QUANT, 2>), grid, block, 0, st, a);
    else if (nc <= 4) launch((k_rows_quant<PRO_QUANT, 4>), grid, block, 0, st, a);
    else launch((k_rows_quant<PRO_QUANT, 8>), grid, block, 0, st, a);
  }
  return launched();
}

// a prefill linear layer on the workspace's int8 rows (int8 MFMA)
// defer_z (STORE): the caller finishes a split itself (its split count back in *defer_z, partials in
// m->part). A residual linear into x leaves a split's finish pending for the next norm/quant of x.
// argmax (STORE): per row the greedy key into argmax[row] (zeroed before) when the batched-decode
// kernel runs the linear; *argmax_done says whether it did
template <int EPI>
int rows_linear(Model* m, const int8_t* w, const float* s_w, const int8_t* w3, const float* s_w3, int N, int K, int rows,
                float* y, long long y_stride, hipStream_t st, int* defer_z = nullptr,
                unsigned long long* argmax = nullptr, bool* argmax_done = nullptr) {
  GemmArgs a;
  std::memset(&a, 0, sizeof(a));
  a.xq = m->xq; a.s_x = m->sx; a.w = w; a.s_w = s_w; a.w3 = w3; a.s_w3 = s_w3;
  a.M = rows; a.N = N; a.K = K; a.y = y; a.y_stride = y_stride; a.res = EPI == EPI_RESID ? y : nullptr;
  a.part = m->part;
  a.part_cap = 4LL * m->part_rows * (m->qkv_dim > m->d.dim ? m->qkv_dim : m->d.dim);
  a.tab = sfu_table_ptr();
  a.act = m->d.ffn_act;
  if (m->pend_z > 1) return T2R_ESTATE;          // the partials buffer still holds an unfinished linear
  if (argmax_done) *argmax_done = false;
  if (argmax && EPI == EPI_STORE && rows <= kBgMaxRows * kBgMaxGroups) {
    a.argmax_key = argmax;
    const int r = bgemv_launch<EPI>(a, st, nullptr);
    if (r == 0) {
      if (argmax_done) *argmax_done = true;
      return T2R_OK;
    }
    if (r != -1) return T2R_EHIP;
    a.argmax_key = nullptr;                      // not taken: the GEMM below, the caller's argmax after it
  }
  const bool resid_x = EPI == EPI_RESID && y == m->x && y_stride == m->d.dim && N == m->d.dim;
  int z = 1;
  if (gemm_launch<EPI>(a, st, m->part_rows, resid_x || defer_z ? &z : nullptr)) return T2R_EHIP;
  if (defer_z) {
    *defer_z = z;
  } else if (z > 1) {
    m->pend_z = z;
    m->pend_rows = rows;
    m->pend_sw = s_w;
  }
  return T2R_OK;
}

// one decoder layer on `rows` rows of the workspace at device positions pos[rows]
// RUN_DECODE: one row per decode GEMV (rows on grid y), fused attention; RUN_PREFILL: rows of one
// sequence through the MFMA GEMMs and the prefill attention; RUN_BATCH: one sequence per row (its
// own position and cache, m->kcb / m->vcb), the MFMA GEMMs and the fused per-row attention.
enum { RUN_DECODE = 0, RUN_PREFILL = 1, RUN_BATCH = 2 };

// the attention launch arguments of layer l (its cache, constants and options)
AttnArgs layer_attn_args(Model* m, int l, const int32_t* pos, int mode) {
  const t2r_model_desc& d = m->d;
  const bool batch = mode == RUN_BATCH;
  AttnArgs at;
  std::memset(&at, 0, sizeof(at));
  at.qkv = m->qkv; at.qkv_stride = m->qkv_dim;
  at.kc = (batch ? m->kcb : d.k_cache) + (long long)l * d.seq_len * m->kv_dim;
  at.vc = (batch ? m->vcb : d.v_cache) + (long long)l * d.seq_len * m->kv_dim;
  at.kv_row_stride = batch ? m->kv_rs : 0;
  at.t_cap = mode == RUN_PREFILL ? m->t_cap : 0;
  at.pos = pos;
  at.qn = d.qk_norm ? d.q_norm + (long long)l * d.head_dim : nullptr;
  at.kn = d.qk_norm ? d.k_norm + (long long)l * d.head_dim : nullptr;
  at.cos_t = d.rope_cos; at.sin_t = d.rope_sin;
  const float* kc4 = m->kvc + (size_t)l * 4;
  at.inv_sk = kc4[0]; at.inv_sv = kc4[1]; at.a_k = kc4[2]; at.a_v = kc4[3];
  at.eps = d.eps; at.inv_hd = (float)(1.0 / d.head_dim);
  at.H = d.heads; at.Hk = d.kv_heads; at.hd = d.head_dim; at.D = d.D; at.S = d.seq_len;
  at.att = m->att; at.att_stride = m->q_dim;
  at.tab = sfu_table_ptr();
  at.qsum = d.attn_qsum;
  at.status = m->status;
  // batch-1 decode at head dim 128 over caches of more than 512 rows: each head's keys over 4
  // workgroups (k_attn_dec's SPLIT form), all of them resident at once (checked at creation)
  if (mode == RUN_DECODE && m->nsplit > 1) {
    at.nsplit = m->nsplit;
    at.sp_s = m->sp_s; at.sp_o = m->sp_o; at.sp_acc = m->sp_acc; at.sp_sync = m->sp_sync;
  }
  if (m->kv_flags[l]) {
    const float* ch = d.kv_channel + (long long)l * 4 * m->kv_dim;   // s_k, 1/s_k, 1/s_v, a_v
    if (m->kv_flags[l] & 1) { at.ch_sk = ch; at.ch_isk = ch + m->kv_dim; }
    if (m->kv_flags[l] & 2) { at.ch_isv = ch + 2 * m->kv_dim; at.ch_av = ch + 3 * m->kv_dim; }
  }
  return at;
}

// the decode Wqkv GEMV of layer l: RMSNorm + quant_act of x, the q | k | v rows
GemvArgs layer_qkv_args(Model* m, int l) {
  const t2r_model_desc& d = m->d;
  GemvArgs a = gemv_args();
  a.w = d.wqkv + (long long)l * m->qkv_dim * d.dim;
  a.s_w = d.s_wqkv + (long long)l * m->qkv_dim;
  a.x = m->x; a.x_stride = d.dim; a.g = d.rms_att + (long long)l * d.dim; a.inv_n = (float)(1.0 / d.dim);
  a.eps = d.eps; a.D = d.D;
  a.N = m->qkv_dim; a.K = d.dim; a.y = m->qkv; a.y_stride = m->qkv_dim;
  return a;
}

int run_layer(Model* m, int l, int rows, const int32_t* pos, int mode, hipStream_t st) {
  const t2r_model_desc& d = m->d;
  const bool decode = mode == RUN_DECODE, batch = mode == RUN_BATCH;
  const long long L_dim = (long long)l * d.dim;
  const float inv_d = (float)(1.0 / d.dim);
  int rc;
  // Wqkv: RMSNorm + quant_act + linear
  GemvArgs a = layer_qkv_args(m, l);
  int qz = 1;                                       // prefill: Wqkv's split finished by the prep kernel
  // (the timed class of a multi-row linear is the GEMM alone: its row norm/quant runs before the scope)
  if (decode) {
    ProfScope p(m, T2R_PROF_QKV, st);
    if ((rc = gemv_launch<PRO_NORM_QUANT, EPI_STORE>(a, rows, st))) return rc;
  } else {
    if ((rc = rows_quant(m, m->x, d.dim, d.rms_att + L_dim, d.dim, rows, st))) return rc;
    ProfScope p(m, T2R_PROF_QKV, st);
    if ((rc = rows_linear<EPI_STORE>(m, a.w, a.s_w, nullptr, nullptr, m->qkv_dim, d.dim, rows, m->qkv, m->qkv_dim, st,
                                     mode == RUN_PREFILL ? &qz : nullptr)))
      return rc;
  }
  // attention (QK-norm, RoPE, KV append fused for decode)
  AttnArgs at = layer_attn_args(m, l, pos, mode);
  if (qz > 1) {
    at.part = m->part; at.part_nz = qz; at.part_zstride = (long long)rows * m->qkv_dim;
    at.part_sw = a.s_w; at.part_sx = m->sx;
  }
  {
    ProfScope p(m, T2R_PROF_ATTN, st);
    if (decode || batch) {
      if ((rc = attn_launch(ATTN_FUSED, at, rows, st))) return rc;
    } else {
      // k_attn_pw at head dim 128 takes q as the prep kernel's int8 rows: in xq (free from the Wqkv
      // linear to the Wo row quant) with their scales in u (free until the FFN): C3's attention 62.5
      // against 65.6 us from fp32 q. (At head dim 64 the prep kernel's quant_act costs
      // what the attention saves: C4's prep 6.3 against 5.3 us, its attention 10.3 against 11.3.)
      if (pw_takes(at) && d.head_dim == 128 && m->ffn_rows >= d.heads) {
        at.q8 = m->xq; at.q8_stride = m->q_dim; at.q8s = m->u;
      }
      if ((rc = attn_launch(ATTN_PREP, at, rows, st))) return rc;
      if ((rc = attn_launch(ATTN_ONLY, at, rows, st))) return rc;
    }
  }
  // Wo: quant_act(att) + linear + residual
  a = gemv_args();
  a.w = d.wo + (long long)l * d.dim * m->q_dim;
  a.s_w = d.s_wo + L_dim;
  a.x = m->att; a.x_stride = m->q_dim;
  a.N = d.dim; a.K = m->q_dim; a.y = m->x; a.y_stride = d.dim; a.res = m->x; a.res_stride = d.dim;
  if (decode && attn_split_to_linear(at, rows)) {
    // the split attention left its four per-split int32 P.V sums: x = F(f32(sum) a_v), then quant_act
    a.xs = m->sp_o; a.xs_stride = m->q_dim; a.xs_scale = at.a_v;
    ProfScope p(m, T2R_PROF_WO, st);
    if ((rc = gemv_launch<PRO_SPLITQ, EPI_RESID>(a, rows, st))) return rc;
  } else if (decode) {
    ProfScope p(m, T2R_PROF_WO, st);
    if ((rc = gemv_launch<PRO_QUANT, EPI_RESID>(a, rows, st))) return rc;
  } else {
    if ((rc = rows_quant(m, m->att, m->q_dim, nullptr, m->q_dim, rows, st))) return rc;
    ProfScope p(m, T2R_PROF_WO, st);
    if ((rc = rows_linear<EPI_RESID>(m, a.w, a.s_w, nullptr, nullptr, d.dim, m->q_dim, rows, m->x, d.dim, st))) return rc;
  }
  if (d.n_experts == 0) {
    // SwiGLU: RMSNorm + quant_act + W1 / W3 + gate
    a = gemv_args();
    a.w = d.w1 + (long long)l * d.hidden * d.dim; a.s_w = d.s_w1 + (long long)l * d.hidden;
    a.w3 = d.w3 + (long long)l * d.hidden * d.dim; a.s_w3 = d.s_w3 + (long long)l * d.hidden;
    a.x = m->x; a.x_stride = d.dim; a.g = d.rms_ffn + L_dim; a.inv_n = inv_d; a.eps = d.eps; a.D = d.D;
    a.N = d.hidden; a.K = d.dim; a.y = m->u; a.y_stride = m->ffn_rows; a.act = d.ffn_act;
    if (decode) {
      ProfScope p(m, T2R_PROF_FFN_UP, st);
      if ((rc = gemv_launch<PRO_NORM_QUANT, EPI_SWIGLU>(a, rows, st))) return rc;
    } else {
      if ((rc = rows_quant(m, m->x, d.dim, d.rms_ffn + L_dim, d.dim, rows, st))) return rc;
      ProfScope p(m, T2R_PROF_FFN_UP, st);
      if ((rc = rows_linear<EPI_SWIGLU>(m, a.w, a.s_w, a.w3, a.s_w3, d.hidden, d.dim, rows, m->u, m->ffn_rows, st)))
        return rc;
    }
    // W2: quant_act(u) + linear + residual
    a = gemv_args();
    a.w = d.w2 + (long long)l * d.dim * d.hidden; a.s_w = d.s_w2 + L_dim;
    a.x = m->u; a.x_stride = m->ffn_rows;
    a.N = d.dim; a.K = d.hidden; a.y = m->x; a.y_stride = d.dim; a.res = m->x; a.res_stride = d.dim;
    if (decode) {
      ProfScope p(m, T2R_PROF_FFN_DOWN, st);
      if ((rc = gemv_launch<PRO_QUANT, EPI_RESID>(a, rows, st))) return rc;
    } else {
      if ((rc = rows_quant(m, m->u, m->ffn_rows, nullptr, d.hidden, rows, st))) return rc;
      ProfScope p(m, T2R_PROF_FFN_DOWN, st);
      if ((rc = rows_linear<EPI_RESID>(m, a.w, a.s_w, nullptr, nullptr, d.dim, d.hidden, rows, m->x, d.dim, st)))
        return rc;
    }
  } else {
    if ((rc = fin_flush(m, st))) return rc;         // the router reads x
    const int E = d.n_experts, k = d.top_k, Fe = d.hidden;
    RouteArgs ra;
    std::memset(&ra, 0, sizeof(ra));
    ra.a = gemv_args();
    ra.a.w = d.router + (long long)l * E * d.dim; ra.a.s_w = d.s_router + (long long)l * E;
    ra.a.x = m->x; ra.a.x_stride = d.dim; ra.a.g = d.rms_ffn + L_dim; ra.a.inv_n = inv_d; ra.a.eps = d.eps;
    ra.a.D = d.D; ra.a.N = E; ra.a.K = d.dim; ra.a.xq_out = m->mxq; ra.a.xq_stride = d.dim; ra.a.sx_out = m->msx;
    ra.k = k; ra.ids = m->ids; ra.wts = m->wts;
    if (!gemv_operands_ok<PRO_NORM_QUANT, EPI_STORE>(ra.a) || d.dim % d.D) return T2R_ESHAPE;
    // expert gate / up of the k selected experts (rows j * Fe + n of the selected tables)
    a = gemv_args();
    a.w = d.wg + (long long)l * E * Fe * d.dim; a.s_w = d.s_wg + (long long)l * E * Fe;
    a.w3 = d.wu + (long long)l * E * Fe * d.dim; a.s_w3 = d.s_wu + (long long)l * E * Fe;
    a.xq = m->mxq; a.xq_stride = d.dim; a.s_x = m->msx;
    a.ids = m->ids; a.rows_per_id = Fe; a.ids_stride = k;
    a.N = k * Fe; a.K = d.dim; a.y = m->u; a.y_stride = m->ffn_rows; a.act = d.ffn_act;
    auto route_rows = [&]() {
      const int nc = cdiv(d.dim, 1024);
      if (nc <= 2) launch(k_moe_route<2>, dim3(rows), dim3(kGemvThreads), 0, st, ra);
      else if (nc <= 4) launch(k_moe_route<4>, dim3(rows), dim3(kGemvThreads), 0, st, ra);
      else launch(k_moe_route<8>, dim3(rows), dim3(kGemvThreads), 0, st, ra);
    };
    const bool grouped = rows >= 8 && m->moe_t != nullptr && E <= 64 && k <= 8 && Fe % 32 == 0 && Fe <= 1024 &&
                         d.dim % 32 == 0 && ((uintptr_t)a.w & 15) == 0 && ((uintptr_t)a.w3 & 15) == 0 &&
                         ((uintptr_t)d.wd & 15) == 0;
    if (grouped) {
      // many rows: every row routed, the routes listed per expert, then each expert's linears over
      // its routes (its weights read once per 32 routes), the routes' quant_act, and the ordered combine
      {
        ProfScope p(m, T2R_PROF_ROUTE, st);
        route_rows();
        launch(k_moe_lists, dim3(1), dim3(256), 0, st, (const int32_t*)m->ids, rows * k, E, m->moe_off, m->moe_list);
        if ((rc = launched())) return rc;
      }
      MoeGemmArgs g;
      std::memset(&g, 0, sizeof(g));
      g.off = m->moe_off; g.list = m->moe_list; g.k = k; g.tab = sfu_table_ptr(); g.act = d.ffn_act;
      g.ngrp = cdiv(rows, 32);                      // an expert takes at most one route of each row
      auto go = [&](auto mode, int K) {
        constexpr int MODE = decltype(mode)::value;
        const int nw = cdiv(K, kBgWin);
        const dim3 grid((unsigned)((long long)E * g.ntile * g.ngrp));
        if (nw >= 8) launch((k_moe_gemm<MODE, 8>), grid, dim3(512), 8 * kBgWaveLds, st, g);
        else if (nw >= 4) launch((k_moe_gemm<MODE, 4>), grid, dim3(256), 4 * kBgWaveLds, st, g);
        else if (nw >= 2) launch((k_moe_gemm<MODE, 2>), grid, dim3(128), 2 * kBgWaveLds, st, g);
        else launch((k_moe_gemm<MODE, 1>), grid, dim3(64), kBgWaveLds, st, g);
      };
      {
        ProfScope p(m, T2R_PROF_FFN_UP, st);
        g.xq = m->mxq; g.s_x = m->msx; g.w = a.w; g.s_w = a.s_w; g.w3 = a.w3; g.s_w3 = a.s_w3; g.y = m->u;
        g.N = Fe; g.K = d.dim; g.ntile = cdiv(Fe, 16);
        go(std::integral_constant<int, MOE_GU>(), g.K);
        if ((rc = launched())) return rc;
      }
      {
        ProfScope p(m, T2R_PROF_FFN_DOWN, st);
        launch(k_moe_hq, dim3(cdiv(rows * k, 4)), dim3(256), 0, st, (const float*)m->u, rows * k, Fe, m->moe_hq, m->moe_sh);
        g.xq = m->moe_hq; g.s_x = m->moe_sh; g.w = d.wd + (long long)l * E * d.dim * Fe; g.s_w = d.s_wd + (long long)l * E * d.dim;
        g.w3 = nullptr; g.s_w3 = nullptr; g.wts = m->wts; g.y = m->moe_t; g.N = d.dim; g.K = Fe; g.ntile = cdiv(d.dim, 32);
        go(std::integral_constant<int, MOE_DN>(), g.K);
        launch(k_moe_combine, dim3(cdiv(d.dim, 256), rows), dim3(256), 0, st, (const float*)m->moe_t, k, d.dim, m->x,
               (long long)d.dim);
        if ((rc = launched())) return rc;
      }
      return T2R_OK;
    }
    if (d.dim <= 1024 && k <= 8) {
      // the router fused into the gate / up GEMV: every block routes its row, then its tiles
      MoeUpArgs mu;
      mu.r = ra;
      mu.up = a;
      const GemvShape g = gemv_shape<1>(a.N);
      ProfScope p(m, T2R_PROF_FFN_UP, st);
      if (g.ru >= 4) launch((k_moe_up<1, 4>), dim3(g.blocks, rows), dim3(kGemvThreads), 0, st, mu);
      else if (g.ru == 2) launch((k_moe_up<1, 2>), dim3(g.blocks, rows), dim3(kGemvThreads), 0, st, mu);
      else launch((k_moe_up<1, 1>), dim3(g.blocks, rows), dim3(kGemvThreads), 0, st, mu);
      if ((rc = launched())) return rc;
    } else {
      {
        ProfScope p(m, T2R_PROF_ROUTE, st);
        route_rows();
        if ((rc = launched())) return rc;
      }
      ProfScope p(m, T2R_PROF_FFN_UP, st);
      if ((rc = gemv_launch<PRO_XQ, EPI_SWIGLU>(a, rows, st))) return rc;
    }
    MoeDownArgs md;
    md.u = m->u; md.wd = d.wd + (long long)l * E * d.dim * Fe; md.s_wd = d.s_wd + (long long)l * E * d.dim;
    md.ids = m->ids; md.wts = m->wts; md.x = m->x; md.k = k; md.F = Fe; md.dim = d.dim; md.x_stride = d.dim;
    const int blocks = cdiv(d.dim, 4);
    {
      ProfScope p(m, T2R_PROF_FFN_DOWN, st);
      launch(k_moe_down, dim3(blocks, rows), dim3(256), 0, st, md);
      if ((rc = launched())) return rc;
    }
  }
  return T2R_OK;
}

// final RMSNorm + quant_act + classifier of workspace row `row`, with the greedy argmax
int run_final(Model* m, int row, float* logits, int32_t* next_token, int32_t* pos, int advance, hipStream_t st) {
  const t2r_model_desc& d = m->d;
  int rc = fin_flush(m, st);
  if (rc) return rc;
  GemvArgs a = gemv_args();
  a.w = d.cls_q; a.s_w = d.cls_s;
  a.x = m->x + (long long)row * d.dim; a.g = d.rms_final; a.inv_n = (float)(1.0 / d.dim); a.eps = d.eps; a.D = d.D;
  a.N = d.vocab; a.K = d.dim; a.y = logits ? logits : m->logits; a.argmax_key = m->keys;
  {
    ProfScope p(m, T2R_PROF_CLS, st);
    rc = gemv_launch<PRO_NORM_QUANT, EPI_STORE>(a, 1, st);
  }
  if (rc) return rc;
  if (next_token || advance) {
    launch(k_finish, dim3(1), dim3(64), 0, st, m->keys, next_token, pos, advance);
    return launched();
  }
  return T2R_OK;
}

// whether every workgroup of one split decode attention launch (kSplits per head) can be resident at
// once on this device: the splits of a head wait for each other
bool split_fits(const t2r_model_desc& d, int heads) {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return false;
  const void* ks[] = {(const void*)k_attn_dec<8, false, 2>, (const void*)k_attn_dec<8, true, 1>};
  for (const void* k : ks) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, kAttnThreads, attn_dec_lds_bytes(d.seq_len, d.D)) !=
        hipSuccess)
      return false;
    if ((long long)per_cu * cus < (long long)heads * kSplits) return false;
  }
  return true;
}

// The model's state from a validated descriptor whose workspace is in dv (the caller's or the static
// one's scratch part); state: a static model's slot for its carried state (else in the workspace).
// Synchronises the device: creation is set-up, not a capturable call.
int model_init(Model* m, const t2r_model_desc& dv, char* state = nullptr, long long state_cap = 0) {
  m->d = dv;
  const t2r_model_desc* desc = &m->d;
  model_dims(m);
  long long sb = 0;
  if (carve(m, nullptr, desc->max_rows, nullptr, state != nullptr, &sb) > desc->workspace_bytes || sb > (state ? state_cap : sb))
    return T2R_ENOMEM;
  carve(m, (char*)desc->workspace, desc->max_rows, state, state != nullptr);
  const int hs = split_heads(m->d);
  m->nsplit = hs > 0 && split_fits(m->d, hs) ? kSplits : 0;
  // the carried state starts clear: the status word, the split counters and SPLIT 1's sums
  if (hipMemset(m->status, 0, sizeof(int32_t)) != hipSuccess ||
      (hs > 0 && hipMemset(m->sp_acc, 0, sizeof(int32_t) * (size_t)hs * kMaxHd) != hipSuccess) ||
      (hs > 0 && hipMemset(m->sp_sync, 0, sizeof(uint32_t) * 2 * (size_t)hs) != hipSuccess) ||
      hipDeviceSynchronize() != hipSuccess)
    return T2R_EHIP;
  std::memcpy(m->kvc, desc->kv_consts, sizeof(float) * 4 * desc->layers);
  for (int l = 0; l < desc->layers; ++l) m->kv_flags[l] = desc->kv_channel_flags ? desc->kv_channel_flags[l] : 0;
  m->d.kv_consts = nullptr;
  m->d.kv_channel_flags = nullptr;
  return T2R_OK;
}

// the handles of t2r_model_create_static: a fixed pool, so that creating one allocates nothing; slot i's
// carried state at i * kStateSlotBytes of the static array
constexpr int kStaticModels = 8;
constexpr long long kStateSlotBytes = T2R_STATIC_STATE_BYTES / kStaticModels;
static_assert(kStateSlotBytes >= 256 + 2 * 4 * 64 + 256 + 64 * kMaxHd * 4, "a slot holds the state of 64 split heads");
std::mutex g_pool_mu;
Model g_pool[kStaticModels];
bool g_pool_used[kStaticModels];

}  // namespace

// ================================================================== C-ABI
extern "C" {

int t2r_abi_version(void) { return T2R_ABI_VERSION; }

const char* t2r_strerror(int code) {
  switch (code) {
    case T2R_OK: return "ok";
    case T2R_EINVAL: return "invalid argument";
    case T2R_ESHAPE: return "shape not supported (XERR_SHAPE)";
    case T2R_ERANGE: return "index or size out of range (XERR_RANGE)";
    case T2R_EHIP: return "HIP runtime error";
    case T2R_ENOMEM: return "workspace too small";
    case T2R_ESTATE: return "bad model state";
    default: return "unknown error";
  }
}

int t2r_init(void) { return ensure_init(); }

int t2r_sfu_tables(uint32_t* out) {
  if (!out) return T2R_EINVAL;
  T2R_INIT();
  if (hipMemcpyFromSymbol(out, HIP_SYMBOL(c_sfu), kSfuWords * 4, 0, hipMemcpyDeviceToHost) != hipSuccess)
    return T2R_EHIP;
  return T2R_OK;
}

int t2r_sfu(int fn, const uint32_t* x, uint32_t* y, int64_t n, void* stream) {
  if (fn < 0 || fn > 3 || n < 0 || (n > 0 && (!x || !y))) return T2R_EINVAL;
  T2R_INIT();
  if (n == 0) return T2R_OK;
  long long blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  launch(k_sfu, dim3((unsigned)blocks), dim3(256), 0, S(stream), fn, x, y, (long long)n);
  return launched();
}

int t2r_sfu_check(int fn, uint64_t first, uint64_t count, uint32_t* out, void* stream) {
  if (fn < 0 || fn > 7 || !out || first > 0xFFFFFFFFull || count > 0x100000000ull - first) return T2R_EINVAL;
  T2R_INIT();
  launch(k_sfu_check_init, dim3(1), dim3(64), 0, S(stream), out);
  if (count > 0) launch(k_sfu_check, dim3(8192), dim3(256), 0, S(stream), fn, (unsigned long long)first,
                        (unsigned long long)count, out);
  return launched();
}

int t2r_fp32_op(int op, const uint32_t* a, const uint32_t* b, uint32_t* y, int64_t n, void* stream) {
  if (op < 0 || op > 8 || n < 0 || (n > 0 && (!a || !b || !y))) return T2R_EINVAL;
  T2R_INIT();
  if (n == 0) return T2R_OK;
  long long blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  launch(k_fp32op, dim3((unsigned)blocks), dim3(256), 0, S(stream), op, a, b, y, (long long)n);
  return launched();
}

int t2r_requant(const int32_t* r, int64_t n, int scale, int shift, int zp, int lo, int hi, int8_t* out,
                void* stream) {
  if (n < 0 || (n > 0 && (!r || !out))) return T2R_EINVAL;
  if (shift < 0 || shift > 31 || scale < -32768 || scale > 32767 || lo > hi) return T2R_ERANGE;
  T2R_INIT();
  if (n == 0) return T2R_OK;
  long long blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  launch(k_requant, dim3((unsigned)blocks), dim3(256), 0, S(stream), r, (long long)n, scale, shift, zp,
                     lo, hi, out);
  return launched();
}

int t2r_embed(const int8_t* emb_q, const float* emb_s, const int32_t* tokens, int rows, int dim, int vocab, float* x,
              int32_t* status, void* stream) {
  if (!emb_q || !emb_s || !tokens || !x) return T2R_EINVAL;
  if (rows <= 0 || dim <= 0 || vocab <= 0) return T2R_ESHAPE;
  T2R_INIT();
  launch(k_embed, dim3(rows), dim3(256), 0, S(stream), emb_q, emb_s, tokens, dim, vocab, x,
                     (long long)dim, (unsigned long long*)nullptr, 0, status);
  return launched();
}

int t2r_rmsnorm(const float* x, const float* g, int rows, int n, float eps, int D, float* out, void* stream) {
  if (!x || !g || !out) return T2R_EINVAL;
  if (rows <= 0 || n <= 0 || n > kMaxK || (D != 8 && D != 16)) return T2R_ESHAPE;
  T2R_INIT();
  launch(k_rmsnorm, dim3(rows), dim3(256), 0, S(stream), x, g, n, (float)(1.0 / n), eps, D, out);
  return launched();
}

int t2r_quant_act(const float* x, int rows, int n, int8_t* xq, float* s_x, void* stream) {
  if (!x || !xq || !s_x) return T2R_EINVAL;
  if (rows <= 0 || n <= 0 || n > kMaxK || n % 16) return T2R_ESHAPE;
  T2R_INIT();
  GemvArgs a = gemv_args();
  a.x = x; a.x_stride = n; a.K = n; a.xq_out = xq; a.xq_stride = n; a.sx_out = s_x;
  launch(k_rows_norm_quant, dim3(rows), dim3(kGemvThreads), 0, S(stream), a, 0, (float*)nullptr, 0LL);
  return launched();
}

int t2r_gemv_w8a8(const int8_t* w, const float* s_w, const int8_t* xq, const float* s_x, int N, int K, float* y,
                  int32_t* acc_out, const float* residual, void* stream) {
  if (!w || !s_w || !xq || !s_x || !y) return T2R_EINVAL;
  if (N <= 0 || K <= 0 || K % 16 || K > kMaxK) return T2R_ESHAPE;
  T2R_INIT();
  GemvArgs a = gemv_args();
  a.w = w; a.s_w = s_w; a.xq = xq; a.xq_stride = K; a.s_x = s_x; a.N = N; a.K = K;
  a.acc_out = acc_out; a.y = y; a.y_stride = N;
  if (residual) {
    a.res = residual; a.res_stride = N;
    return gemv_launch<PRO_XQ, EPI_RESID>(a, 1, S(stream)) ? T2R_EHIP : T2R_OK;
  }
  return gemv_launch<PRO_XQ, EPI_STORE>(a, 1, S(stream)) ? T2R_EHIP : T2R_OK;
}

int t2r_gemm_w8a8(const int8_t* w, const float* s_w, const int8_t* xq, const float* s_x, int M, int N, int K,
                  float* y, int32_t* acc_out, const float* residual, void* stream) {
  if (!w || !s_w || !xq || !s_x || !y) return T2R_EINVAL;
  if (M <= 0 || N <= 0 || K <= 0 || K % 16 || K > kMaxK) return T2R_ESHAPE;
  T2R_INIT();
  GemmArgs a;
  std::memset(&a, 0, sizeof(a));
  a.xq = xq; a.s_x = s_x; a.w = w; a.s_w = s_w; a.M = M; a.N = N; a.K = K; a.y = y; a.y_stride = N;
  a.acc_out = acc_out;
  if (residual) {
    a.res = residual;
    return gemm_launch<EPI_RESID>(a, S(stream)) ? T2R_EHIP : T2R_OK;
  }
  return gemm_launch<EPI_STORE>(a, S(stream)) ? T2R_EHIP : T2R_OK;
}

int t2r_rope(float* v, const float* cos_t, const float* sin_t, const int32_t* pos, int rows, int n, int half, int S_,
             void* stream) {
  if (!v || !cos_t || !sin_t || !pos) return T2R_EINVAL;
  if (rows <= 0 || n <= 0 || half <= 0 || n % (2 * half) || S_ <= 0) return T2R_ESHAPE;
  T2R_INIT();
  launch(k_rope, dim3(rows), dim3(256), 0, S(stream), v, cos_t, sin_t, pos, n, half, S_);
  return launched();
}

int t2r_kv_append_ch(const float* k, const float* v, float inv_sk, float inv_sv, const float* inv_sk_ch,
                     const float* inv_sv_ch, int8_t* kc, int8_t* vc, const int32_t* pos, int rows, int kv_dim, int S_,
                     void* stream) {
  if (!k || !v || !kc || !vc || !pos) return T2R_EINVAL;
  if (rows <= 0 || kv_dim <= 0 || S_ <= 0) return T2R_ESHAPE;
  T2R_INIT();
  launch(k_kv_append, dim3(rows), dim3(256), 0, S(stream), k, v, inv_sk, inv_sv, inv_sk_ch, inv_sv_ch, kc, vc, pos,
         kv_dim, S_);
  return launched();
}

int t2r_kv_append(const float* k, const float* v, float inv_sk, float inv_sv, int8_t* kc, int8_t* vc,
                  const int32_t* pos, int rows, int kv_dim, int S_, void* stream) {
  return t2r_kv_append_ch(k, v, inv_sk, inv_sv, nullptr, nullptr, kc, vc, pos, rows, kv_dim, S_, stream);
}

int t2r_attn_decode_opt(const float* q, const int8_t* kc, const int8_t* vc, const int32_t* pos, int rows, int H,
                        int Hk, int hd, int S_, float a_k, float a_v, int D, int flags, const float* ch_sk,
                        const float* ch_av, float* att, void* stream) {
  if (!q || !kc || !vc || !pos || !att) return T2R_EINVAL;
  if (flags & ~T2R_ATTN_QSUM) return T2R_EINVAL;
  if (rows <= 0) return T2R_ESHAPE;
  T2R_INIT();
  AttnArgs a;
  std::memset(&a, 0, sizeof(a));
  a.qkv = (float*)q; a.qkv_stride = (long long)H * hd;
  a.kc = (int8_t*)kc; a.vc = (int8_t*)vc; a.pos = pos;
  a.a_k = a_k; a.a_v = a_v; a.H = H; a.Hk = Hk; a.hd = hd; a.D = D; a.S = S_;
  a.att = att; a.att_stride = (long long)H * hd;
  a.qsum = flags & T2R_ATTN_QSUM;
  a.ch_sk = ch_sk; a.ch_av = ch_av;
  return attn_launch(ATTN_ONLY, a, rows, S(stream));
}

int t2r_attn_prefill(const float* q, const int8_t* kc, const int8_t* vc, const int32_t* pos, int M, int H, int Hk,
                     int hd, int S_, float a_k, float a_v, int D, int flags, const float* ch_sk, const float* ch_av,
                     float* att, void* stream) {
  if (!q || !kc || !vc || !pos || !att) return T2R_EINVAL;
  if (flags & ~T2R_ATTN_QSUM) return T2R_EINVAL;
  if (M <= 0) return T2R_ESHAPE;
  T2R_INIT();
  AttnArgs a;
  std::memset(&a, 0, sizeof(a));
  a.qkv = (float*)q; a.qkv_stride = (long long)H * hd;
  a.kc = (int8_t*)kc; a.vc = (int8_t*)vc; a.pos = pos;
  a.a_k = a_k; a.a_v = a_v; a.H = H; a.Hk = Hk; a.hd = hd; a.D = D; a.S = S_;
  a.att = att; a.att_stride = (long long)H * hd;
  a.qsum = flags & T2R_ATTN_QSUM;
  a.ch_sk = ch_sk; a.ch_av = ch_av;
  a.tab = sfu_table_ptr();                       // the multi-row kernel (k_attn_pre) where it takes the shape
  return attn_launch(ATTN_ONLY, a, M, S(stream));
}

int t2r_attn_decode(const float* q, const int8_t* kc, const int8_t* vc, const int32_t* pos, int rows, int H, int Hk,
                    int hd, int S_, float a_k, float a_v, int D, float* att, void* stream) {
  return t2r_attn_decode_opt(q, kc, vc, pos, rows, H, Hk, hd, S_, a_k, a_v, D, 0, nullptr, nullptr, att, stream);
}

int t2r_gated_ffn_w8a8(int act, const int8_t* w1, const float* s_w1, const int8_t* w3, const float* s_w3,
                       const int8_t* xq, const float* s_x, int F, int K, float* u_out, int8_t* hq, float* s_h,
                       void* stream) {
  if (!w1 || !s_w1 || !w3 || !s_w3 || !xq || !s_x || !u_out || !hq || !s_h) return T2R_EINVAL;
  if (act != 0 && act != 1) return T2R_EINVAL;
  if (F <= 0 || F % 16 || F > kMaxK) return T2R_ESHAPE;
  T2R_INIT();
  GemvArgs a = gemv_args();
  a.w = w1; a.s_w = s_w1; a.w3 = w3; a.s_w3 = s_w3; a.xq = xq; a.xq_stride = K; a.s_x = s_x;
  a.N = F; a.K = K; a.y = u_out; a.y_stride = F; a.act = act;
  int rc = gemv_launch<PRO_XQ, EPI_SWIGLU>(a, 1, S(stream));
  if (rc) return rc;
  return t2r_quant_act(u_out, 1, F, hq, s_h, stream);
}

int t2r_swiglu_w8a8(const int8_t* w1, const float* s_w1, const int8_t* w3, const float* s_w3, const int8_t* xq,
                    const float* s_x, int F, int K, float* u_out, int8_t* hq, float* s_h, void* stream) {
  return t2r_gated_ffn_w8a8(0, w1, s_w1, w3, s_w3, xq, s_x, F, K, u_out, hq, s_h, stream);
}

int t2r_moe_route(const float* scores, int rows, int E, int k, int D, int32_t* ids, float* weights, void* stream) {
  if (!scores || !ids || !weights) return T2R_EINVAL;
  if (rows <= 0 || E <= 0 || E > 64 || k < 1 || k > 8 || k > E || (D != 8 && D != 16)) return T2R_ESHAPE;
  T2R_INIT();
  launch(k_route_scores, dim3(rows), dim3(64), 0, S(stream), scores, E, k, D, ids, weights);
  return launched();
}

int t2r_argmax(const float* x, int rows, int n, int32_t* idx, void* stream) {
  if (!x || !idx) return T2R_EINVAL;
  if (rows <= 0 || n <= 0) return T2R_ESHAPE;
  T2R_INIT();
  launch(k_argmax, dim3(rows), dim3(256), 0, S(stream), x, n, idx);
  return launched();
}

// ---------------------------------------------------------------- model level
int64_t t2r_model_workspace_bytes(const t2r_model_desc* desc, int max_rows) {
  Model m;
  if (!desc_read(desc, &m.d) || max_rows < 1) return -1;
  model_dims(&m);
  return carve(&m, nullptr, max_rows);
}

int t2r_model_create(const t2r_model_desc* desc, void** model) {
  if (!model) return T2R_EINVAL;
  *model = nullptr;
  t2r_model_desc dv;
  if (!desc_read(desc, &dv)) return T2R_EINVAL;
  int rc = validate(&dv);
  if (rc) return rc;
  T2R_INIT();
  Model* m = new (std::nothrow) Model();
  if (!m) return T2R_ENOMEM;
  if ((rc = model_init(m, dv))) {
    delete m;
    return rc;
  }
  *model = m;
  return T2R_OK;
}

int t2r_model_create_static(const t2r_model_desc* desc, void** model) {
  if (!model) return T2R_EINVAL;
  *model = nullptr;
  t2r_model_desc dv;
  if (!desc_read(desc, &dv)) return T2R_EINVAL;
  if (dv.workspace != nullptr || dv.workspace_bytes != 0) return T2R_EINVAL;   // the library's array is the workspace
  T2R_INIT();
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices || !g_scratch_addr[dev]) return T2R_EHIP;
  dv.workspace = g_scratch_addr[dev] + T2R_STATIC_STATE_BYTES;
  dv.workspace_bytes = T2R_STATIC_WORKSPACE_BYTES - T2R_STATIC_STATE_BYTES;
  int rc = validate(&dv);
  if (rc) return rc;
  Model* m = nullptr;
  {
    std::lock_guard<std::mutex> lk(g_pool_mu);
    for (int i = 0; i < kStaticModels && !m; ++i)
      if (!g_pool_used[i]) {
        g_pool_used[i] = true;
        m = &g_pool[i];
        *m = Model();
        m->pool_slot = i;
      }
  }
  if (!m) return T2R_ESTATE;                     // every static model slot is taken
  if ((rc = model_init(m, dv, g_scratch_addr[dev] + (long long)m->pool_slot * kStateSlotBytes, kStateSlotBytes))) {
    t2r_model_destroy(m);
    return rc;                                   // T2R_ENOMEM: max_rows needs more than the static array
  }
  *model = m;
  return T2R_OK;
}

void t2r_model_destroy(void* model) {
  Model* m = (Model*)model;
  if (!m) return;
  free_events(m);
  if (m->pool_slot >= 0) {
    std::lock_guard<std::mutex> lk(g_pool_mu);
    g_pool_used[m->pool_slot] = false;
    m->pool_slot = -1;
    return;
  }
  delete m;
}

int t2r_model_status(void* model, int32_t* out, int clear) {
  Model* m = (Model*)model;
  if (!m || !out) return T2R_EINVAL;
  // every stream's work first (a non-blocking stream is not ordered with the copy's default stream)
  if (hipDeviceSynchronize() != hipSuccess) return T2R_EHIP;
  if (hipMemcpy(out, m->status, sizeof(int32_t), hipMemcpyDeviceToHost) != hipSuccess) return T2R_EHIP;
  if (clear && hipMemset(m->status, 0, sizeof(int32_t)) != hipSuccess) return T2R_EHIP;
  return T2R_OK;
}

int t2r_model_profile(void* model, int mask, int max_launches) {
  Model* m = (Model*)model;
  if (!m || mask < 0 || max_launches < 0 || (mask && max_launches == 0)) return T2R_EINVAL;
  free_events(m);
  if (!mask) return T2R_OK;
  m->ev.resize((size_t)2 * max_launches);
  m->ev_kind.assign((size_t)max_launches, -1);
  for (auto& e : m->ev)
    if (hipEventCreate(&e) != hipSuccess) {
      e = nullptr;
      free_events(m);
      return T2R_EHIP;
    }
  m->prof_mask = mask;
  return T2R_OK;
}

int t2r_model_profile_read(void* model, int32_t* kinds, float* ms, int max) {
  Model* m = (Model*)model;
  if (!m || max < 0 || (max > 0 && (!kinds || !ms))) return T2R_EINVAL;
  const int n = m->ev_used / 2;
  if (n > 0 && hipEventSynchronize(m->ev[m->ev_used - 1]) != hipSuccess) return T2R_EHIP;
  for (int i = 0; i < n && i < max; ++i) {
    kinds[i] = m->ev_kind[i];
    if (hipEventElapsedTime(&ms[i], m->ev[2 * i], m->ev[2 * i + 1]) != hipSuccess) return T2R_EHIP;
  }
  m->ev_used = 0;
  return n;
}

int t2r_decode_step(void* model, const int32_t* token, int32_t* pos, float* logits, int32_t* next_token, int flags,
                    void* stream) {
  Model* m = (Model*)model;
  if (!m || !token || !pos) return T2R_EINVAL;
  if (flags & ~T2R_ADVANCE_POS) return T2R_EINVAL;
  T2R_INIT();
  m->pend_z = 0;
  hipStream_t st = S(stream);
  const t2r_model_desc& d = m->d;
  int rc;
  {
    ProfScope p(m, T2R_PROF_OTHER, st);
    launch(k_embed, dim3(1), dim3(256), 0, st, d.emb_q, d.emb_s, token, d.dim, d.vocab, m->x,
                       (long long)d.dim, m->keys, 1, m->status);
    rc = launched();
  }
  if (rc) return rc;
  for (int l = 0; l < d.layers; ++l)
    if ((rc = run_layer(m, l, 1, pos, RUN_DECODE, st))) return rc;
  return run_final(m, 0, logits, next_token, pos, flags & T2R_ADVANCE_POS, st);
}

int t2r_prefill(void* model, const int32_t* tokens, const int32_t* positions, int M, float* last_logits,
                int32_t* next_token, void* stream) {
  Model* m = (Model*)model;
  if (!m || !tokens || !positions) return T2R_EINVAL;
  if (M < 1 || M > m->d.max_rows) return T2R_ERANGE;
  T2R_INIT();
  m->pend_z = 0;
  hipStream_t st = S(stream);
  const t2r_model_desc& d = m->d;
  launch(k_embed, dim3(M), dim3(256), 0, st, d.emb_q, d.emb_s, tokens, d.dim, d.vocab, m->x,
                     (long long)d.dim, m->keys, 1, m->status);
  int rc = launched();
  if (rc) return rc;
  for (int l = 0; l < d.layers; ++l)
    if ((rc = run_layer(m, l, M, positions, RUN_PREFILL, st))) return rc;
  return run_final(m, M - 1, last_logits, next_token, nullptr, 0, st);
}

int t2r_prefill_at(void* model, const int32_t* tokens, int start, int M, float* last_logits, int32_t* next_token,
                   void* stream) {
  Model* m = (Model*)model;
  if (!m || !tokens) return T2R_EINVAL;
  if (M < 1 || M > m->d.max_rows || start < 0 || start + M > m->d.seq_len) return T2R_ERANGE;
  T2R_INIT();
  hipStream_t st = S(stream);
  launch(k_iota, dim3(cdiv(M, 256)), dim3(256), 0, st, m->pos_rows, start, M);
  int rc = launched();
  if (rc) return rc;
  m->t_cap = start + M;
  rc = t2r_prefill(model, tokens, m->pos_rows, M, last_logits, next_token, stream);
  m->t_cap = 0;
  return rc;
}

int t2r_decode_batch(void* model, const int32_t* tokens, const int32_t* positions, int B, int8_t* k_caches,
                     int8_t* v_caches, int64_t cache_stride, float* logits, int32_t* next_tokens, void* stream) {
  Model* m = (Model*)model;
  if (!m || !tokens || !positions || !k_caches || !v_caches || !logits) return T2R_EINVAL;
  if (B < 1 || B > m->d.max_rows) return T2R_ERANGE;
  const t2r_model_desc& d = m->d;
  const long long cache_bytes = (long long)d.layers * d.seq_len * m->kv_dim;
  if (B > 1 && cache_stride < cache_bytes) return T2R_ESHAPE;
  T2R_INIT();
  m->pend_z = 0;
  hipStream_t st = S(stream);
  launch(k_embed, dim3(B), dim3(256), 0, st, d.emb_q, d.emb_s, tokens, d.dim, d.vocab, m->x, (long long)d.dim,
         m->keys, B, m->status);
  int rc = launched();
  if (rc) return rc;
  m->kcb = k_caches;
  m->vcb = v_caches;
  m->kv_rs = B > 1 ? cache_stride : 0;
  for (int l = 0; l < d.layers && rc == 0; ++l) rc = run_layer(m, l, B, positions, RUN_BATCH, st);
  m->kcb = m->vcb = nullptr;
  m->kv_rs = 0;
  if (rc) return rc;
  // every row's final RMSNorm + quant_act, the classifier over the rows, a first-maximum per row
  if ((rc = rows_quant(m, m->x, d.dim, d.rms_final, d.dim, B, st))) return rc;
  bool fused = false;                              // greedy keys in the classifier's epilogue
  {
    ProfScope p(m, T2R_PROF_CLS, st);
    if ((rc = rows_linear<EPI_STORE>(m, d.cls_q, d.cls_s, nullptr, nullptr, d.vocab, d.dim, B, logits, d.vocab, st,
                                     nullptr, next_tokens ? m->keys : nullptr, &fused)))
      return rc;
  }
  if (next_tokens) {
    if (fused) launch(k_keys_tokens, dim3(cdiv(B, 64)), dim3(64), 0, st, (const unsigned long long*)m->keys, next_tokens, B);
    else launch(k_argmax, dim3(B), dim3(256), 0, st, (const float*)logits, d.vocab, next_tokens);
    return launched();
  }
  return T2R_OK;
}

}  // extern "C"
