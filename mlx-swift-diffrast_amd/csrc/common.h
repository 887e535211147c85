// Shared device helpers for the gfx950 kernels (wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <vector>
#include <stdint.h>

#include <string>

#include "diffrast_mi355x.h"

namespace dr {

// ---------------------------------------------------------------------------
// errors
// ---------------------------------------------------------------------------

void set_error(const std::string& msg);

#define DR_CHECK_ARG(cond, msg)              \
  do {                                       \
    if (!(cond)) {                           \
      ::dr::set_error(std::string(msg));     \
      return DR_ERR_ARGUMENT;                \
    }                                        \
  } while (0)

#define DR_CHECK_HIP(expr)                                                         \
  do {                                                                             \
    hipError_t e_ = (expr);                                                        \
    if (e_ != hipSuccess) {                                                        \
      ::dr::set_error(std::string(#expr) + ": " + hipGetErrorString(e_));          \
      return DR_ERR_HIP;                                                           \
    }                                                                              \
  } while (0)

#define DR_CHECK_LAUNCH() DR_CHECK_HIP(hipGetLastError())

// ---------------------------------------------------------------------------
// scratch memory, kept per (device, stream), grow-only
// ---------------------------------------------------------------------------

enum Slot {
  SLOT_RAST_REC = 0,  // per-triangle screen records
  SLOT_RAST_RECT,     // per-triangle tile rectangles
  SLOT_RAST_CNT,      // per-tile counters / offsets
  SLOT_RAST_LIST,     // tile -> triangle lists
  SLOT_RAST_ITEMS,    // range-mode item prefix
  SLOT_TOPO,          // edge hash table
  SLOT_DPYR,          // mip pyramid gradient
  SLOT_SMALL,         // small device-side counters
  SLOT_LOSS,          // partial sums of the loss
  SLOT_AA_REC,        // per (image, triangle) silhouette records (antialias)
  SLOT_DPOS64,        // fp64 accumulator of d_pos (rasterize and antialias backward)
  SLOT_RBWD_REC,      // per (image, triangle) records of the rasterize backward
  SLOT_DATTR_COPY,    // copies of a small d_attr (interpolate backward)
  SLOT_COUNT
};

struct Scratch {
  void* ptr[SLOT_COUNT] = {};
  size_t cap[SLOT_COUNT] = {};
  // Tile-list capacity protocol (rasterize): the largest per-tile count of
  // a call is written into pinned host memory by a kernel after the call; a
  // later call reads it (once that kernel has run) and raises the capacity
  // if needed.
  // pinned_total[1] receives the sum of the counts (the list entries) of
  // the same call, whose (image, triangle) items were stat_items: their
  // ratio, tiles_per_item, picks the forward kernel of later calls.
  int64_t* pinned_total = nullptr;      // 2 values
  int64_t* pinned_total_dev = nullptr;  // the same memory as a kernel writes it
  hipEvent_t total_event = nullptr;
  bool total_pending = false;
  int bin_cap = 0;  // slots per tile list, 0 = not known yet
  int64_t stat_items = 0;
  double tiles_per_item = 0.0;
  // The LDS binning's fill pass writes the same two figures per wave
  // instead (its largest final tile count, its list entries), here, for up
  // to kWaveStatsMax waves; the host reduces the stat_waves pairs into
  // pinned_total once total_event has passed.  No kernel then reduces them.
  static constexpr int64_t kWaveStatsMax = 16384;
  int64_t* wave_stats = nullptr;      // 2 * kWaveStatsMax values
  int64_t* wave_stats_dev = nullptr;  // the same memory as a kernel writes it
  int64_t stat_waves = 0;
  // Range-mode item prefix, staged through a ring of pinned host buffers:
  // a buffer is reused once the copy that read it has run (its event), so
  // a call waits only when it is kStageRing calls ahead of the device.
  static constexpr int kStageRing = 4;
  int64_t* stage[kStageRing] = {};
  size_t stage_cap[kStageRing] = {};
  hipEvent_t stage_event[kStageRing] = {};
  bool stage_pending[kStageRing] = {};
  int stage_next = 0;
  // fp64 d_pos accumulator (SLOT_DPOS64): k_acc_to_f32 leaves the elements
  // it converts zero, so the next call need not clear them; acc64_zero
  // counts the leading elements of buffer acc64_buf known to be zero.
  const void* acc64_buf = nullptr;
  int64_t acc64_zero = 0;
  // d_attr copies (SLOT_DATTR_COPY), left zero by k_sum_copies the same way.
  const void* copy_buf = nullptr;
  int64_t copy_zero = 0;
  // The previous dr_rasterize_fwd* call on this stream, whose triangle
  // setup and tile lists (SLOT_RAST_*) dr_rasterize_fwd_again may reuse.
  struct {
    bool valid = false;
    const float* pos = nullptr;
    const int32_t* tri = nullptr;
    int64_t pos_stride = 0;
    int N = 0, V = 0, T = 0, H = 0, W = 0, max_per_tile = 0, C = 0;
    bool range = false;
    std::vector<int32_t> ranges;
    int64_t n_items = 0, max_items = 0;
    bool px = false;  // the forward kernel it ran (k_raster_px)
    bool brec = false;  // it also wrote the backward's records (SLOT_RBWD_REC)
    uint64_t capture_id = 0;  // the capture it was made in (0: none)
  } last_raster;
  // Whether last_raster may be reused by the current call (same capture,
  // or both uncaptured on a stream that never saw a capture).
  bool last_raster_reusable() const {
    return last_raster.valid && last_raster.capture_id == cur_capture &&
           (cur_capture != 0 || !captured);
  }
  // A dr_rasterize_bwd has run on this stream, so forwards write the
  // backward's per-triangle records with their setup.
  bool rbwd_want = false;
  // HIP graph capture.  cur_capture: the capture sequence of the current
  // call (0 when the stream is not being captured), set by scratch_for.
  // Once a call has been captured on this stream (`captured`), a replay of
  // that graph may run between any two later calls: buffers a graph may
  // point at are never freed (a grown slot retires the old buffer until
  // dr_release_scratch), and one call reuses another's results only within
  // one capture (last_raster.capture_id), never between uncaptured calls.
  uint64_t cur_capture = 0;
  bool captured = false;
  std::vector<void*> retired;
};

// A pinned host buffer of the range-mode staging ring holding at least
// `n` int64 values, free to overwrite (waits for the copy that last read
// it, if it has not run yet); nullptr on error.
int64_t* stage_acquire(Scratch* sc, size_t n, int& slot);
// Records that the copy just enqueued on `stream` reads ring buffer `slot`.
int stage_release(Scratch* sc, int slot, hipStream_t stream);

// Compute units of the current device (cached per device).
int device_cu_count();

// The capture sequence `stream` is being captured into (a HIP graph), or
// 0 when it is not.  Under capture the library neither allocates nor
// waits: scratch that would have to grow, a first rasterize call that would
// count its tiles, and the range-mode staging are refused with
// DR_ERR_CAPTURE.
uint64_t stream_capture_id(hipStream_t stream);

// Returns the scratch record of (current device, stream), with its
// cur_capture set for this call; nullptr on error.
Scratch* scratch_for(hipStream_t stream);
// Ensures slot `s` holds at least `bytes`; returns its pointer or nullptr.
void* scratch_get(Scratch* sc, hipStream_t stream, int s, size_t bytes);
// The status to return after scratch_for / scratch_get / stage_acquire
// gave nullptr on this thread: DR_ERR_CAPTURE, DR_ERR_MEMORY or DR_ERR_HIP.
int scratch_fail();

// ---------------------------------------------------------------------------
// kernel timing (dr_profile_*): when enabled, each launch made inside a
// ProfScope is bracketed by HIP events on its stream.
// ---------------------------------------------------------------------------

extern bool g_prof_enabled;

struct ProfScope {
  const char* name;
  hipStream_t stream;
  hipEvent_t start = nullptr;
  ProfScope(const char* n, hipStream_t s);
  ~ProfScope();
};

#define DR_TIMED(NAME, STREAM) ::dr::ProfScope dr_prof_scope_(NAME, STREAM)

// ---------------------------------------------------------------------------
// device helpers
// ---------------------------------------------------------------------------

constexpr int kWave = 64;

// Float -> int32 as the hardware converts (v_cvt_i32_f32: truncation,
// out-of-range values saturate, NaN -> 0), one instruction; C's cast leaves
// those cases undefined, and spelling them out costs branches.  The oracle
// uses the same definition.
__device__ __forceinline__ int f2i(float x) {
  int r;
  asm("v_cvt_i32_f32 %0, %1" : "=v"(r) : "v"(x));
  return r;
}

// q = i / d, r = i % d for 0 <= i and 0 < d: a 32-bit division while i fits
// in 31 bits (several times cheaper than the 64-bit one).
__device__ __forceinline__ void divmod64(int64_t i, int d, int64_t& q, int& r) {
  if (i <= 0x7fffffff) {
    const int ii = (int)i, qq = ii / d;
    q = qq;
    r = ii - qq * d;
  } else {
    q = i / d;
    r = (int)(i - q * d);
  }
}

// Whether a triangle's three vertex ids index rows [0, V) of its vertex
// buffer.  Triangles that fail are not drawn and get no gradient, so no
// input can send a vertex read out of range.
__device__ __forceinline__ bool verts_ok(int i0, int i1, int i2, int V) {
  return (unsigned)i0 < (unsigned)V && (unsigned)i1 < (unsigned)V && (unsigned)i2 < (unsigned)V;
}

__device__ __forceinline__ int xcd_remap(int b, int B) {
  // Blocks are dealt round-robin to the 8 XCDs; give each XCD a contiguous
  // run of tiles so neighbouring tiles share that XCD's L2.
  if ((B & 7) != 0) return b;
  return (b & 7) * (B >> 3) + (b >> 3);
}

__device__ __forceinline__ int lane_id() { return (int)__lane_id(); }

// Streaming accesses with the non-temporal hint: per-pixel inputs read
// once and outputs the next kernel streams in again leave L2's reused lines
// (texels, vertex rows, triangle records) in place.  Measured on the
// 8 x 1024^2 chain: texture forward 0.080 -> 0.071 ms, interpolate forward
// 0.084 -> 0.081 ms, the step 1.153 -> 1.130 ms.  Not used where the next
// kernel reads the output while it may still be cached and would then
// have to fetch it again (antialias out before the loss, the interpolate
// backward's d_rast before the rasterize backward: both measured slower).
typedef float dr_f4v __attribute__((ext_vector_type(4)));
typedef float dr_f2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float4 ld_nt4(const float* p) {
  const dr_f4v v = __builtin_nontemporal_load(reinterpret_cast<const dr_f4v*>(p));
  return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float2 ld_nt2(const float* p) {
  const dr_f2v v = __builtin_nontemporal_load(reinterpret_cast<const dr_f2v*>(p));
  return make_float2(v.x, v.y);
}
__device__ __forceinline__ void st_nt4(float* p, float4 v) {
  dr_f4v x = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(x, reinterpret_cast<dr_f4v*>(p));
}
__device__ __forceinline__ void st_nt2(float* p, float2 v) {
  dr_f2v x = {v.x, v.y};
  __builtin_nontemporal_store(x, reinterpret_cast<dr_f2v*>(p));
}


// Wave-uniform values: keep them in scalar registers.
__device__ __forceinline__ float uni(float x) {
  return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(x)));
}
__device__ __forceinline__ uint64_t uni(uint64_t x) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)x);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(x >> 32));
  return ((uint64_t)hi << 32) | lo;
}
// x of lane l (l wave-uniform): two scalar reads instead of an LDS permute
__device__ __forceinline__ uint64_t lane_value(uint64_t x, int l) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)x, l);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(x >> 32), l);
  return ((uint64_t)hi << 32) | lo;
}

// Wave reductions with DPP row operations (VALU only) and four readlanes:
// quad xor 1, quad xor 2, row half-mirror and row mirror leave every lane
// holding its 16-lane row's result; the rows are then combined in scalars.
template <int CTRL>
__device__ __forceinline__ int dpp_mov(int v) {
  return __builtin_amdgcn_update_dpp(v, v, CTRL, 0xF, 0xF, false);
}

template <typename Op>
__device__ __forceinline__ int wave_reduce_i(int v, Op op) {
  v = op(v, dpp_mov<0xB1>(v));   // quad_perm [1,0,3,2]
  v = op(v, dpp_mov<0x4E>(v));   // quad_perm [2,3,0,1]
  v = op(v, dpp_mov<0x141>(v));  // row_half_mirror
  v = op(v, dpp_mov<0x140>(v));  // row_mirror
  const int r0 = __builtin_amdgcn_readlane(v, 0), r1 = __builtin_amdgcn_readlane(v, 16);
  const int r2 = __builtin_amdgcn_readlane(v, 32), r3 = __builtin_amdgcn_readlane(v, 48);
  return op(op(r0, r1), op(r2, r3));
}

// Shift within 16-lane rows (row_shr:n = 0x110 + n, row_shl:n = 0x100 + n);
// lanes whose source is outside the row read 0.
template <int CTRL>
__device__ __forceinline__ int dpp_shift(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, true);
}

// Step D of the scan, masked on the sending side: lane l's value reaches
// lane l + D when both lie in one run (run start of l + D <= l); any other
// lane sends +0.  The receiver then adds unconditionally, so the shift
// fuses into the add (one DPP instruction per value) and the sums equal a
// conditional add's.
template <int D, int M>
__device__ __forceinline__ void run_scan_step(int li, int s, float (&v)[M]) {
  const int s_to = dpp_shift<0x100 + D>(s);  // run start of lane l + D
  const bool send = li + D <= 15 && s_to <= li;
  float w[M];  // all masks first: a DPP read right after the VALU write of its
               // source waits two cycles
#pragma unroll
  for (int i = 0; i < M; ++i) w[i] = send ? v[i] : 0.0f;
#pragma unroll
  for (int i = 0; i < M; ++i) v[i] += __int_as_float(dpp_shift<0x110 + D>(__float_as_int(w[i])));
}

__device__ __forceinline__ int wave_max(int v) {
  return wave_reduce_i(v, [](int a, int b) { return a > b ? a : b; });
}

__device__ __forceinline__ int wave_or(int v) {
  return wave_reduce_i(v, [](int a, int b) { return a | b; });
}

// Runs of equal keys along each 16-lane row (the row of pixels a wave row
// holds): every lane's v[] becomes the sum of its run's values up to
// itself (a segmented Hillis-Steele scan over DPP row shifts), and the
// run's last lane, which then holds the run total, gets true.  Summing a
// run before it meets an LDS atomic matters: lanes of one instruction that
// hit one address are serialised (~11 cycles each for fp64 adds).  All 64
// lanes must execute this; give each inactive lane a key of its own.
struct RowRun {
  int li, s;  // lane within its 16-lane row, start of its run
  bool tail;  // last lane of its run
};

__device__ __forceinline__ RowRun row_run(uint64_t key) {
  RowRun r;
  r.li = lane_id() & 15;
  const int li = r.li;
  const int klo = (int)(uint32_t)key, khi = (int)(uint32_t)(key >> 32);
  // every lane must execute the shifts (a DPP read of a lane that is
  // switched off returns 0), so no short-circuit evaluation here
  const int plo = dpp_shift<0x111>(klo), phi = dpp_shift<0x111>(khi);
  const int nlo = dpp_shift<0x101>(klo), nhi = dpp_shift<0x101>(khi);
  const bool head = (li == 0) | (plo != klo) | (phi != khi);
  r.tail = (li == 15) | (nlo != klo) | (nhi != khi);
  int s = head ? li : 0;  // run start: max-scan of head positions
  int a = dpp_shift<0x111>(s);
  if (li >= 1) s = max(s, a);
  a = dpp_shift<0x112>(s);
  if (li >= 2) s = max(s, a);
  a = dpp_shift<0x114>(s);
  if (li >= 4) s = max(s, a);
  a = dpp_shift<0x118>(s);
  if (li >= 8) s = max(s, a);
  r.s = s;
  return r;
}

template <int M>
__device__ __forceinline__ void row_run_scan(const RowRun& r, float (&v)[M]) {
  run_scan_step<1>(r.li, r.s, v);
  run_scan_step<2>(r.li, r.s, v);
  run_scan_step<4>(r.li, r.s, v);
  run_scan_step<8>(r.li, r.s, v);
}

// The same scan with only as many steps as the longest run in the wave
// needs (`maxlen`, wave-uniform): a run of length r is summed after
// ceil(log2 r) steps.
template <int M>
__device__ __forceinline__ void row_run_scan_n(const RowRun& r, float (&v)[M], int maxlen) {
  if (maxlen > 1) run_scan_step<1>(r.li, r.s, v);
  if (maxlen > 2) run_scan_step<2>(r.li, r.s, v);
  if (maxlen > 4) run_scan_step<4>(r.li, r.s, v);
  if (maxlen > 8) run_scan_step<8>(r.li, r.s, v);
}

template <int M>
__device__ __forceinline__ bool row_run_sum(uint64_t key, float (&v)[M]) {
  const RowRun r = row_run(key);
  row_run_scan_n(r, v, wave_max(r.li - r.s + 1));
  return r.tail;
}

__device__ __forceinline__ float wave_sum(float v) {
  auto add = [](int a, int b) { return __float_as_int(__int_as_float(a) + __int_as_float(b)); };
  return __int_as_float(wave_reduce_i(__float_as_int(v), add));
}

template <int CTRL>
__device__ __forceinline__ float dpp_movf(float v) {
  return __int_as_float(dpp_mov<CTRL>(__float_as_int(v)));
}

// v + (v of lane l ^ 32) and v + (v of lane l ^ 16), with the gfx950 lane
// swaps (one VALU instruction each, no LDS round trip).  permlane32_swap
// exchanges lanes 32..63 of its first operand with lanes 0..31 of its
// second; permlane16_swap exchanges the odd 16-lane rows of the first with
// the even rows of the second.  Given v twice, the two results hold v and
// its partner's value in every lane.
__device__ __forceinline__ float add_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float add_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Sixteen wave sums at once.  A transposing butterfly (row mirror, half-row
// mirror, then the two quad swaps; each step keeps half of the values and
// adds the partner's half) leaves lane l with value (l & 15) summed over
// its 16-lane row, and two exchanges across rows finish it: every lane
// returns the total of value (lane & 15).  About 70 instructions instead of
// 16 separate reductions.  All 64 lanes must execute this.
__device__ __forceinline__ float wave_sum16(const float (&a)[16]) {
  const int l = lane_id();
  float v8[8], v4[4], v2[2];
  const bool b3 = (l >> 3) & 1, b2 = (l >> 2) & 1, b1 = (l >> 1) & 1, b0 = l & 1;
#pragma unroll
  for (int i = 0; i < 8; ++i)  // row_mirror: partner 15 - (l & 15)
    v8[i] = (b3 ? a[i + 8] : a[i]) + dpp_movf<0x140>(b3 ? a[i] : a[i + 8]);
#pragma unroll
  for (int i = 0; i < 4; ++i)  // row_half_mirror: partner 7 - (l & 7)
    v4[i] = (b2 ? v8[i + 4] : v8[i]) + dpp_movf<0x141>(b2 ? v8[i] : v8[i + 4]);
#pragma unroll
  for (int i = 0; i < 2; ++i)  // quad_perm [2,3,0,1]
    v2[i] = (b1 ? v4[i + 2] : v4[i]) + dpp_movf<0x4E>(b1 ? v4[i] : v4[i + 2]);
  float v = (b0 ? v2[1] : v2[0]) + dpp_movf<0xB1>(b0 ? v2[0] : v2[1]);  // quad_perm [1,0,3,2]
  return add_xor32(add_xor16(v));
}

// Four wave sums at once, the same way: the two quad swaps leave lane l
// with value (l & 3) summed over its quad, row rotations by 4 and 8 add the
// row's four quads, and the lane swaps the four rows.  Every lane returns
// the total of value (lane & 3).  All 64 lanes must execute this.
__device__ __forceinline__ float wave_sum4(const float (&a)[4]) {
  const int l = lane_id();
  const bool b1 = (l >> 1) & 1, b0 = l & 1;
  float v2[2];
#pragma unroll
  for (int i = 0; i < 2; ++i)  // quad_perm [2,3,0,1]
    v2[i] = (b1 ? a[i + 2] : a[i]) + dpp_movf<0x4E>(b1 ? a[i] : a[i + 2]);
  float v = (b0 ? v2[1] : v2[0]) + dpp_movf<0xB1>(b0 ? v2[0] : v2[1]);  // quad_perm [1,0,3,2]
  v += dpp_movf<0x124>(v);  // row_ror:4
  v += dpp_movf<0x128>(v);  // row_ror:8
  return add_xor32(add_xor16(v));
}

__device__ __forceinline__ int wave_min(int v) {
  return wave_reduce_i(v, [](int a, int b) { return a < b ? a : b; });
}

// Per-half minimum of two signed 16-bit values packed in an int.
__device__ __forceinline__ int pk16_min(int a, int b) {
  typedef short short2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(int, __builtin_elementwise_min(__builtin_bit_cast(short2_t, a),
                                                           __builtin_bit_cast(short2_t, b)));
}

__device__ __forceinline__ int wave_min_pk16(int v) { return wave_reduce_i(v, pk16_min); }

__device__ __forceinline__ int pack16(int lo, int hi) {
  return (int)(((uint32_t)(uint16_t)(int16_t)lo) | ((uint32_t)(uint16_t)(int16_t)hi << 16));
}
__device__ __forceinline__ int unpack16_lo(int v) { return (int)(int16_t)(v & 0xffff); }
__device__ __forceinline__ int unpack16_hi(int v) { return (int)(int16_t)((uint32_t)v >> 16); }


// Scatter-add of M values per lane into addresses that are equal for all
// lanes with the same (`key`, `key2`).  Up to kProbes candidate groups are
// probed (alternating the lowest and highest pending lane as leader); a
// group of at least kGroupMin lanes is summed across the wave and written by
// its leader.  Every other lane then issues its own atomics, all lanes in
// one pass (no per-lane serialisation).  Inactive lanes pass valid = false;
// every lane of the wave must call this.
constexpr int kGroupMin = 6;
constexpr int kProbes = 4;

__device__ __forceinline__ int probe_leader(uint64_t pending, int probe) {
  return (probe & 1) ? 63 - __clzll((long long)pending) : __ffsll((long long)pending) - 1;
}

template <int M>
__device__ __forceinline__ void group_atomic_add(bool valid, uint64_t key, float* const (&addr)[M],
                                                 const float (&val)[M], uint32_t key2 = 0) {
  uint64_t pending = __ballot(valid);
  bool mine = valid;
  const int lane = lane_id();
#pragma unroll 1
  for (int probe = 0; probe < kProbes && pending; ++probe) {
    const int leader = probe_leader(pending, probe);
    const uint64_t lkey = lane_value(key, leader);
    const uint32_t lkey2 = (uint32_t)__builtin_amdgcn_readlane((int)key2, leader);
    const bool member = mine && key == lkey && key2 == lkey2;
    const uint64_t members = __ballot(member);
    pending &= ~members;
    if (__popcll(members) >= kGroupMin) {
#pragma unroll
      for (int i = 0; i < M; ++i) {
        const float s = wave_sum(member ? val[i] : 0.0f);
        if (lane == leader && s != 0.0f) unsafeAtomicAdd(addr[i], s);
      }
      if (member) mine = false;
    }
  }
  if (mine) {
#pragma unroll
    for (int i = 0; i < M; ++i)
      if (val[i] != 0.0f) unsafeAtomicAdd(addr[i], val[i]);
  }
}

// ---------------------------------------------------------------------------
// Workgroup scatter aggregation in LDS.  Contributions are keyed by their
// destination address; an open-addressing table sums them with LDS
// atomics, and the flush issues one global atomic per distinct destination
// and value.  A lane whose probe sequence finds no room adds to global
// memory directly.
//
// Sums are kept in fp64: on gfx950 an LDS fp32 atomic add is issued one lane
// at a time (about 3 cycles per active lane, ~190 cycles per full wave),
// while the fp64 add takes ~8 cycles per wave, like the integer atomics.
// The fp64 partial sums are also exact for the few hundred fp32 terms a
// workgroup adds; each is rounded once to fp32 when flushed.
// ---------------------------------------------------------------------------

constexpr unsigned long long kEmptyKey = ~0ull;
constexpr int kLdsProbes = 8;

// Values are stored component-major (val[j][entry]): an entry's NV values
// 8 * NV bytes apart would put the entries of a wave's atomics on a few
// banks only (entry * 2 * NV mod 32); 8 bytes apart they spread over 16.
template <int NV, int CAP>
struct LdsTable {
  unsigned long long key[CAP];
  double val[NV][CAP];
};

__device__ __forceinline__ uint32_t addr_hash(uint64_t k) {
  return (uint32_t)(((k >> 2) * 0x9E3779B97F4A7C15ull) >> 32);
}

template <int NV, int CAP>
__device__ __forceinline__ void lds_table_clear(LdsTable<NV, CAP>& t) {
  for (int i = threadIdx.x; i < CAP; i += blockDim.x) {
    t.key[i] = kEmptyKey;
#pragma unroll
    for (int j = 0; j < NV; ++j) t.val[j][i] = 0.0;
  }
}

// Adds v[0..NV) to dst[0..NV) (D: float, or double for an fp64
// accumulator in global memory).
template <int NV, int CAP, typename D>
__device__ __forceinline__ void lds_table_add(LdsTable<NV, CAP>& t, D* dst, const float* v) {
  bool any = false;
#pragma unroll
  for (int j = 0; j < NV; ++j) any = any || v[j] != 0.0f;
  if (!any) return;
  const uint64_t key = (uint64_t)dst;
  uint32_t h = addr_hash(key) & (CAP - 1);
#pragma unroll 1
  for (int probe = 0; probe < kLdsProbes; ++probe) {
    unsigned long long cur = t.key[h];
    if (cur == kEmptyKey) cur = atomicCAS(&t.key[h], kEmptyKey, (unsigned long long)key);
    if (cur == kEmptyKey || cur == key) {
#pragma unroll
      for (int j = 0; j < NV; ++j)
        if (v[j] != 0.0f) atomicAdd(&t.val[j][h], (double)v[j]);
      return;
    }
    h = (h + 1) & (CAP - 1);
  }
#pragma unroll
  for (int j = 0; j < NV; ++j)
    if (v[j] != 0.0f) unsafeAtomicAdd(dst + j, (D)v[j]);
}

// Writes the table out (call after a barrier) and leaves it cleared; the
// keys are addresses of D values (what lds_table_add was given).
// Consecutive lanes take consecutive values of one entry, so the atomics of
// an entry share a cache line request.
template <int NV, int CAP, typename D = float>
__device__ __forceinline__ void lds_table_flush(LdsTable<NV, CAP>& t) {
  for (int i = threadIdx.x; i < CAP * NV; i += blockDim.x) {
    const int e = i / NV, j = i - e * NV;
    const unsigned long long k = t.key[e];
    if (k != kEmptyKey) {
      const double v = t.val[j][e];
      if (v != 0.0) unsafeAtomicAdd((D*)k + j, (D)v);
      t.val[j][e] = 0.0;
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < CAP; i += blockDim.x) t.key[i] = kEmptyKey;
}

// The same table keeping a list of the entries taken since the last flush,
// so a flush visits those instead of all CAP entries (for large tables that
// a tile fills only in part).
template <int NV, int CAP>
struct LdsTableU {
  LdsTable<NV, CAP> t;
  int n;
  uint16_t slot[CAP];
};

template <int NV, int CAP>
__device__ __forceinline__ void lds_table_clear(LdsTableU<NV, CAP>& u) {
  lds_table_clear(u.t);
  if (threadIdx.x == 0) u.n = 0;
}

template <int NV, int CAP, typename D>
__device__ __forceinline__ void lds_table_add(LdsTableU<NV, CAP>& u, D* dst, const float* v) {
  static_assert(CAP <= 65536, "slots are 16-bit");
  auto& t = u.t;
  bool any = false;
#pragma unroll
  for (int j = 0; j < NV; ++j) any = any || v[j] != 0.0f;
  if (!any) return;
  const uint64_t key = (uint64_t)dst;
  uint32_t h = addr_hash(key) & (CAP - 1);
#pragma unroll 1
  for (int probe = 0; probe < kLdsProbes; ++probe) {
    unsigned long long cur = t.key[h];
    if (cur == kEmptyKey) {
      cur = atomicCAS(&t.key[h], kEmptyKey, (unsigned long long)key);
      if (cur == kEmptyKey) u.slot[atomicAdd(&u.n, 1)] = (uint16_t)h;  // taken here
    }
    if (cur == kEmptyKey || cur == key) {
#pragma unroll
      for (int j = 0; j < NV; ++j)
        if (v[j] != 0.0f) atomicAdd(&t.val[j][h], (double)v[j]);
      return;
    }
    h = (h + 1) & (CAP - 1);
  }
#pragma unroll
  for (int j = 0; j < NV; ++j)
    if (v[j] != 0.0f) unsafeAtomicAdd(dst + j, (D)v[j]);
}

// Writes the taken entries out (call after a barrier) and leaves the table
// cleared; the caller's next barrier orders the reset count before new adds.
template <int NV, int CAP, typename D = float>
__device__ __forceinline__ void lds_table_flush(LdsTableU<NV, CAP>& u) {
  auto& t = u.t;
  const int m = u.n;
  for (int i = threadIdx.x; i < m * NV; i += blockDim.x) {
    const int e = u.slot[i / NV], j = i - (i / NV) * NV;
    const double v = t.val[j][e];
    if (v != 0.0) unsafeAtomicAdd((D*)t.key[e] + j, (D)v);
    t.val[j][e] = 0.0;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < m; i += blockDim.x) t.key[u.slot[i]] = kEmptyKey;
  if (threadIdx.x == 0) u.n = 0;
}

// The same for the last use of a table in a workgroup that ends after it:
// no barrier and no reset.
template <int NV, int CAP, typename D = float>
__device__ __forceinline__ void lds_table_flush_last(LdsTableU<NV, CAP>& u) {
  auto& t = u.t;
  const int m = u.n;
  for (int i = threadIdx.x; i < m * NV; i += blockDim.x) {
    const int e = u.slot[i / NV], j = i - (i / NV) * NV;
    const double v = t.val[j][e];
    if (v != 0.0) unsafeAtomicAdd((D*)t.key[e] + j, (D)v);
  }
}

// dst = (float)acc, or dst += (float)acc: the one rounding of a gradient
// summed in fp64 across workgroups (so the result does not depend on the
// order in which the workgroups' atomics land).
__global__ void k_acc_to_f32(double* __restrict__ acc, float* __restrict__ dst, int64_t n,
                             int accumulate);

template <typename T>
__global__ void fill_kernel(T* __restrict__ p, T v, int64_t n) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) p[i] = v;
}

// 16-byte stores for a 16-byte aligned run of 4-byte values; the n % 4 tail
// is written by the first threads.
template <typename T>
__global__ void fill4_kernel(T* __restrict__ p, T v, int64_t n) {
  static_assert(sizeof(T) == 4, "4-byte values");
  const int64_t n4 = n >> 2;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const uint32_t b = __builtin_bit_cast(uint32_t, v);
  uint4* q = reinterpret_cast<uint4*>(p);
  for (int64_t j = i; j < n4; j += stride) q[j] = make_uint4(b, b, b, b);
  if (i < (n & 3)) p[n4 * 4 + i] = v;
}

// Fill with a kernel (not hipMemsetAsync) so the call stays graph-capturable.
template <typename T>
inline hipError_t fill_async(T* p, T v, int64_t n, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  DR_TIMED("fill", s);
  if constexpr (sizeof(T) == 4) {
    if (((uintptr_t)p & 15) == 0 && n >= 1024) {
      int64_t blocks = (n / 4 + 255) / 256;
      if (blocks > 8192) blocks = 8192;
      hipLaunchKernelGGL(fill4_kernel<T>, dim3((unsigned)blocks), dim3(256), 0, s, p, v, n);
      return hipGetLastError();
    }
  }
  int64_t blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(fill_kernel<T>, dim3((unsigned)blocks), dim3(256), 0, s, p, v, n);
  return hipGetLastError();
}

// Two 16-byte aligned runs of 4-byte values in one launch.
template <typename T>
__global__ void fill4x2_kernel(T* __restrict__ p0, int64_t n0, T* __restrict__ p1, int64_t n1,
                               T v) {
  static_assert(sizeof(T) == 4, "4-byte values");
  const int64_t a = n0 >> 2, n4 = a + (n1 >> 2);
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const uint32_t b = __builtin_bit_cast(uint32_t, v);
  uint4* q0 = reinterpret_cast<uint4*>(p0);
  uint4* q1 = reinterpret_cast<uint4*>(p1);
  for (int64_t j = i; j < n4; j += stride) {
    if (j < a) q0[j] = make_uint4(b, b, b, b);
    else q1[j - a] = make_uint4(b, b, b, b);
  }
  if (i < (n0 & 3)) p0[a * 4 + i] = v;
  if (i < (n1 & 3)) p1[(n1 >> 2) * 4 + i] = v;
}

// Fills two buffers with v: one launch when both are 16-byte aligned.
template <typename T>
inline hipError_t fill2_async(T* p0, int64_t n0, T* p1, int64_t n1, T v, hipStream_t s) {
  if constexpr (sizeof(T) == 4) {
    if (n0 > 0 && n1 > 0 && ((uintptr_t)p0 & 15) == 0 && ((uintptr_t)p1 & 15) == 0) {
      DR_TIMED("fill", s);
      int64_t blocks = (n0 / 4 + n1 / 4 + 255) / 256;
      if (blocks < 1) blocks = 1;
      if (blocks > 8192) blocks = 8192;
      hipLaunchKernelGGL(fill4x2_kernel<T>, dim3((unsigned)blocks), dim3(256), 0, s, p0, n0, p1,
                         n1, v);
      return hipGetLastError();
    }
  }
  hipError_t e = fill_async(p0, v, n0, s);
  if (e != hipSuccess) return e;
  return fill_async(p1, v, n1, s);
}

inline unsigned grid_for(int64_t n, int block) {
  return (unsigned)((n + block - 1) / block);
}

// An fp64 accumulator of n values (library scratch, zero on the stream:
// cleared here unless the last acc64_end on this stream left it zero).
double* acc64_begin(hipStream_t stream, int64_t n);
// Rounds the accumulator into dst (overwrite, or add when accumulate) and
// zeroes it for the next acc64_begin.
int acc64_end(double* acc, float* dst, int64_t n, bool accumulate, hipStream_t stream);

}  // namespace dr
