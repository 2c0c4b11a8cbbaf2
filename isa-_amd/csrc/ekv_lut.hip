// Flash-EKV LUT CIMLinear for gfx950 (MI355X): LUT build, forward, backward.
//
// The operator (reference: src/isa/kernels/transformer_ffn/ekv_lut_triton.py:25-62
// and cuda/ekv_cuda.cu:193-341) evaluates, for every (token m, output o, input k),
//   dV+ = x[m,k] - vth_pos[o,k],  dV- = x[m,k] - vth_neg[o,k]
//   L(dV) = T[i0] + a * (T[i0+1] - T[i0]),  c = clamp((dV - dmin) * s, 0, N-1),
//           i0 = trunc(c), a = c - i0,  s = (N-1) / (dmax - dmin)
//   out[m,o] = clamp(sum_k (L_I(dV+) - L_I(dV-)) * r[m,k], out_min, out_max),
//           r = 1 / (1 + x / V_sat)
// and the backward from the derivative table D = dI/ddV:
//   dX[m,k]   = sum_o G[m,o] * ((L_D(dV+) - L_D(dV-)) * r - (L_I(dV+) - L_I(dV-)) * r^2 / V_sat)
//   dVth+[o,k] = -sum_m G[m,o] * L_D(dV+) * r
//   dVth-[o,k] = +sum_m G[m,o] * L_D(dV-) * r
//
// MI355X design (one process, one device, caller-owned memory):
//  * The table lives in LDS as padded records in intercept form: record i holds
//    {T[i] - i*dT[i], dT[i]} with dT[i] = T[i+1] - T[i], so L(c) = fma(c, dT, A) on the raw
//    coordinate c. Forward records {A_I, dI} (8 B, one ds_read_b64 per branch); backward
//    records as an I half {A_I, dI} and a D half {A_D, dD} kSplitRecords records apart (two
//    ds_read_b64 per branch from one address), or interleaved 16-byte records read with
//    one ds_read_b128 when the split table does not fit. The random gathers of a wave
//    collide in the LDS banks once its thresholds span more than 32 records; those bank
//    conflicts, not VALU work, set the kernels' speed.
//    kPad replicated end records on each side reproduce the reference's coordinate clamp
//    exactly for coordinates within kPad-1 entries of the table range, so a kernel whose
//    operand ranges fit (checked on device from the prep kernel's range partials) runs a
//    clamp-free inner loop: sub, cvt_u32, lshl_add, ds_read, fma per branch (the forward:
//    sub, add, and, ds_read, fma, its record address formed from the bits of a float sum).
//  * A prep kernel writes the token-side operands pre-scaled into LUT-index units
//    (xs = (x - dmin) * s + kPad, r, and -r/V_sat for the backward) and the threshold
//    operands transposed to [K][O] as {vth_pos * s, vth_neg * s}, padded so the hot loops
//    carry no bounds tests.
//  * Lanes run along outputs o: the 64 gathers of one instruction share (m, k), so they
//    fall inside the narrow window spanned by the thresholds. Token-side operands are
//    wave-uniform and reach the VALU as SGPR operands (s_load), costing no VGPRs.
//  * Forward: each wave owns MR tokens x 64*ORR outputs and reduces over K (or, when the
//    plan splits K to keep MR high on layers with few output blocks, over one K range, the
//    ranges then summed in order by split_reduce_kernel) in registers.
//  * Backward: each wave owns 64*ORR outputs x KR inputs and streams a range of tokens,
//    keeping dVth accumulators in registers; the per-token dX partial sums over its
//    outputs are reduced across the wave with lane exchanges (the exact-formula kernels:
//    through an LDS transpose buffer), then written as one partial per output block. Two
//    small deterministic reduction kernels combine the output-block partials (dX) and
//    token-range partials (dVth). No atomics in any sum (the only atomic, the optional
//    output-statistics max, is order-free): every result is bitwise reproducible.

#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>
#include <type_traits>

#include <algorithm>
#include <cmath>
#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "isa_ekv.h"

namespace {

// Token-side records are read-only for the whole launch and their addresses are
// wave-uniform: reading them through the constant address space lets the compiler use
// scalar loads (SGPR operands) instead of vector loads with per-use latency stalls.
using const_f32 = const __attribute__((address_space(4))) float;

__device__ inline float2 load_uniform2(const float2* p) {
    const_f32* q = (const_f32*)(p);
    return make_float2(q[0], q[1]);
}

__device__ inline float load_uniform1(const float* p) { return *(const_f32*)(p); }

__device__ inline float4 load_uniform4(const float4* p) {
    const_f32* q = (const_f32*)(p);
    return make_float4(q[0], q[1], q[2], q[3]);
}

constexpr int kPad = 16;          // replicated end records on each side of the LDS table
constexpr int kFwdORR = 4;        // outputs per lane, forward
#ifndef ISA_EKV_BWD_ORR
#define ISA_EKV_BWD_ORR 4
#endif
#ifndef ISA_EKV_BWD_KR
#define ISA_EKV_BWD_KR 2
#endif
#ifndef ISA_EKV_BWD_SCHED
#define ISA_EKV_BWD_SCHED 0
#endif
constexpr int kBwdORR = ISA_EKV_BWD_ORR;  // outputs per lane, backward (2 or 4)
constexpr int kBwdKR = ISA_EKV_BWD_KR;    // inputs per wave, table backward (2 or 4)
constexpr int kBwdKRExact = 4;            // inputs per wave, exact and measured backward
constexpr int kRedSlots = 16;             // dX transpose buffer: tokens x inputs slots per batch
static_assert((kBwdORR == 2 || kBwdORR == 4) && (kBwdKR == 2 || kBwdKR == 4), "backward tile");
constexpr int kRedStride = 68;    // floats per slot row in the transpose buffer (64 + pad)
constexpr int kPrepBlocksX = 1024; // prep blocks for the token side
constexpr int kPrepBlocksW = 256; // prep blocks for the threshold side
constexpr int kMaxEntriesFwd = 16384;   // LDS-resident forward table
constexpr int kMaxEntriesBwd = 8192;    // LDS-resident backward table
// Larger tables are read from global memory (L2-resident) by the fwd/bwd_global kernels;
// coordinates stay exact integers in fp32 up to this size.
constexpr int kMaxEntriesGlobal = 1 << 22;
#ifndef ISA_EKV_BWD_MIN_BLOCKS
#define ISA_EKV_BWD_MIN_BLOCKS 2  // table-backward blocks per CU the VGPR budget is held to (64 VGPRs at 2)
#endif
// The waves per SIMD that budget means for 16-wave blocks (the second __launch_bounds__
// argument is waves per SIMD, which caps the VGPRs at 512 / that many)
constexpr int kBwdWavesPerEU = ISA_EKV_BWD_MIN_BLOCKS * 16 / 4;
#ifndef ISA_EKV_BWD_LANE_RED
#define ISA_EKV_BWD_LANE_RED 1  // dX reduction: 0 LDS buffers, 1 lane exchanges, 2 lane exchanges when the table crowds LDS
#endif
#ifndef ISA_EKV_BWD_SPLIT
#define ISA_EKV_BWD_SPLIT 1
#endif
// Backward tables of up to this many padded records use the split LDS layout (the D
// halves sit kSplitRecords * 8 bytes after the I halves: within the 16-bit ds offset).
constexpr int kSplitRecords = 4096 + 2 * kPad;

// Thresholds spread over more table records than ISA_EKV_RANK_MAX_SPREAD leave a half-wave's
// ranks hundreds of records apart; there the two-copy launch's windowed copies do better
// (GPT-L fc1 backward, 16-class rank deal: 11.93 ms ranked against 12.12 ms with two copies at
// 400 records, 12.27 against 12.18 at 450). The greedy deal (ISA_EKV_RANK_GREEDY_MIN) halves
// the conflicts past ~100 records but costs ~0.5 ms per GPT-L call, as much as it saves: off
// (4128 records, past any spread) unless set.
#ifndef ISA_EKV_RANK_MAX_SPREAD
#define ISA_EKV_RANK_MAX_SPREAD 420
#endif
#ifndef ISA_EKV_RANK_GREEDY_MIN
#define ISA_EKV_RANK_GREEDY_MIN 4128
#endif

__host__ __device__ inline int lut_records(int n) { return n + 2 * kPad; }
constexpr int kLdsBytes = 160 * 1024;
constexpr int64_t kCUs = 256;  // MI355X compute units (a fixed plan input: workspace sizes must not depend on the device)

// Planning option ISA_EKV_OPT_COPY_MIN_CELLS: LUT calls of fewer cells never consider the
// second table copy, whose assignment pass (and, in the backward, second main launch) costs
// a small call more than the copy can save.
std::atomic<int64_t> g_copy_min_cells{(int64_t)1 << 28};

// Planning option ISA_EKV_OPT_RANKED: whether table backwards may run the ranked kernel.
std::atomic<int64_t> g_ranked{1};

// Planning option ISA_EKV_OPT_WINDOW_COPIES: the most bank-rotated copies of the coordinate
// window a LUT forward, or a table backward's two-copy launch, may hold (3 to 32; below 3
// neither holds them). With record addresses from float bits the forward waits on its LDS
// reads (index unit 88-92% busy), and at the headline's narrow fc2 window 32 copies run the
// forward ~2% faster than 16, the assignment pass included: 32.
std::atomic<int64_t> g_window_copies{32};

// Planning options ISA_EKV_OPT_RANK_MAX_SPREAD / ISA_EKV_OPT_RANK_GREEDY_MIN: the widest threshold
// spread (table records) the ranked backward takes, and the spread past which its branches are
// dealt by the greedy bank-aware deal (bwd_deal_kernel) instead of by rank (bwd_rank_kernel).
std::atomic<int64_t> g_rank_max_spread{ISA_EKV_RANK_MAX_SPREAD};
std::atomic<int64_t> g_rank_greedy_min{ISA_EKV_RANK_GREEDY_MIN};

// Planning option ISA_EKV_OPT_RANK_XCD_ORDER: 1 gives each XCD a contiguous range of the ranked
// launch's blocks (consecutive inputs of one output block and token split), 0 keeps the
// hardware's round-robin order.
std::atomic<int64_t> g_rank_xcd_order{0};

bool copies_pay(int64_t M, int64_t K, int64_t O) {
    return (double)M * (double)K * (double)O >= (double)g_copy_min_cells.load(std::memory_order_relaxed);
}

thread_local char g_last_error[512] = "";

// Optional per-launch timing of the two main kernels (isa_ekv_profile_begin/_end): HIP
// events recorded on the launch stream around each forward / backward main kernel.
struct ProfiledLaunch {
    hipEvent_t start, stop;
    int kind;  // 0 forward main kernel, 1 backward main kernel, 2 whole forward call, 3 whole backward call
};
constexpr int kProfKinds = 4;
constexpr int kMaxProfiled = 4096;
bool g_profiling = false;
ProfiledLaunch g_prof[kMaxProfiled];
int g_prof_count = 0;

void prof_start(hipStream_t s, int kind, ProfiledLaunch** slot) {
    *slot = nullptr;
    if (!g_profiling || g_prof_count >= kMaxProfiled) return;
    ProfiledLaunch* p = &g_prof[g_prof_count];
    if (hipEventCreate(&p->start) != hipSuccess) return;
    if (hipEventCreate(&p->stop) != hipSuccess) {
        (void)hipEventDestroy(p->start);
        return;
    }
    p->kind = kind;
    (void)hipEventRecord(p->start, s);
    ++g_prof_count;
    *slot = p;
}

void prof_stop(hipStream_t s, ProfiledLaunch* slot) {
    if (slot) (void)hipEventRecord(slot->stop, s);
}

// Shader-clock sampling of the main kernels while profiling (isa_ekv_profile_begin/_clock): a
// per-device buffer of kClockKinds x {shader cycles, wall-clock ticks, blocks} (the backward's
// three kinds adjacent: a backward launch set gets the first, the two-copy kernel adds 3 and the
// ranked kernel 6), to which wave 0
// of every block of an instrumented main kernel adds its own clock64 / wall_clock64 spans
// (BlockClock). The cycle sum over the tick sum is the mean shader clock the CUs ran that
// kernel at, under its own load (the board lowers the clock under heavy VALU + LDS work).
constexpr int kClockKinds = 4;   // 0 LUT forward, 1 one-copy, 2 two-copy and 3 ranked table backward
constexpr int kClockMaxDevices = 64;
unsigned long long* g_clock_buf[kClockMaxDevices] = {};

unsigned long long* clock_acc(int kind) {
    if (!g_profiling) return nullptr;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kClockMaxDevices || !g_clock_buf[dev]) return nullptr;
    return g_clock_buf[dev] + 3 * kind;
}

// Times a whole library call (every kernel it enqueues), closing on every return path.
struct CallTimer {
    hipStream_t stream;
    ProfiledLaunch* slot = nullptr;
    CallTimer(hipStream_t s, int kind, bool on = true) : stream(s) {
        if (on) prof_start(s, kind, &slot);
    }
    ~CallTimer() { prof_stop(stream, slot); }
};

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

int hip_fail(hipError_t err, const char* what) {
    return fail(static_cast<int>(err), "%s: %s", what, hipGetErrorString(err));
}

inline int64_t round_up(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

// ----------------------------------------------------------------------------------
// LUT build (reference: src/isa/approximations/delta_lut.py:12-35). Each entry is
// evaluated in fp64 and rounded once to fp32; slopes are fp32 differences of the
// rounded entries, so fma(a, T[i+1]-T[i], T[i]) matches ekv_cuda.cu:35 for the fp32 table.
// ----------------------------------------------------------------------------------

struct DeviceParams {
    double n, u_t, i_s, v_d;
    double delta_min, delta_max;
    int n_entries;
};

__device__ inline double softplus_ref(double u) {
    // torch.nn.functional.softplus(beta=1, threshold=20)
    return u > 20.0 ? u : log1p(exp(u));
}

__device__ inline double sig_from_sp(double sp) {
    // flash_transistor.py:27-29: 1 - exp(-sp), or 1 above the softplus threshold
    return sp > 20.0 ? 1.0 : -expm1(-sp);
}

__device__ inline void lut_entry(const DeviceParams& p, int j, float* ti, float* td) {
    const int n = p.n_entries;
    const double delta =
        n > 1 ? p.delta_min + (double)j * ((p.delta_max - p.delta_min) / (double)(n - 1))
              : p.delta_min;
    const double inv_2nut = 1.0 / (2.0 * p.n * p.u_t);
    const double sp1 = softplus_ref(delta * inv_2nut);
    const double sp2 = softplus_ref((delta - p.v_d) * inv_2nut);
    *ti = (float)(p.i_s * (sp1 * sp1 - sp2 * sp2));
    *td = (float)(p.i_s * 2.0 * inv_2nut * (sp1 * sig_from_sp(sp1) - sp2 * sig_from_sp(sp2)));
}

__device__ inline unsigned short f32_to_bf16_rne(float f) {
    unsigned int u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (unsigned short)((u >> 16) | 0x40u);  // quiet NaN
    u += 0x7fffu + ((u >> 16) & 1u);
    return (unsigned short)(u >> 16);
}

// Intercept form of padded record idx: L(c) = T[i] + (c - idx) * dT = (T[i] - idx * dT) + c * dT,
// so the kernels evaluate fma(c, dT, A) on the raw coordinate c (no fractional part).
// A is formed in fp64 from the fp32 entry and slope and rounded once.
__device__ inline float intercept(float t, float dt, int idx) {
    return (float)((double)t - (double)idx * (double)dt);
}

// Records are stored whole (forward 8 B, backward 16 B) so one ds_read_b64/b128 fetches
// a record: the words of a record sit in adjacent banks.
__device__ inline void store_record(void* dst, int layout, int idx, float t, float dt, float d, float dd) {
    if (layout == ISA_EKV_LUT_FWD)
        static_cast<float2*>(dst)[idx] = make_float2(intercept(t, dt, idx), dt);
    else
        static_cast<float4*>(dst)[idx] = make_float4(intercept(t, dt, idx), dt, intercept(d, dd, idx), dd);
}

__global__ void lut_build_kernel(DeviceParams p, int layout, void* dst) {
    const int n = p.n_entries;
    const int total = (layout == ISA_EKV_LUT_PLAIN_F32 || layout == ISA_EKV_LUT_PLAIN_BF16)
                          ? n
                          : lut_records(n);
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    if (layout == ISA_EKV_LUT_PLAIN_F32) {
        float ti, td;
        lut_entry(p, idx, &ti, &td);
        static_cast<float*>(dst)[idx] = ti;
        static_cast<float*>(dst)[n + idx] = td;
        return;
    }
    if (layout == ISA_EKV_LUT_PLAIN_BF16) {
        float ti, td;
        lut_entry(p, idx, &ti, &td);
        static_cast<unsigned short*>(dst)[idx] = f32_to_bf16_rne(ti);
        static_cast<unsigned short*>(dst)[n + idx] = f32_to_bf16_rne(td);
        return;
    }
    // padded record idx holds table entry j = idx - kPad, clamped to [0, n-1]; records
    // outside the interior carry zero slopes so they reproduce the clamped end values
    const int j = idx - kPad;
    const int jc = j < 0 ? 0 : (j > n - 1 ? n - 1 : j);
    float i0, d0;
    lut_entry(p, jc, &i0, &d0);
    float si = 0.0f, sd = 0.0f;
    if (j >= 0 && j < n - 1) {
        float i1, d1;
        lut_entry(p, j + 1, &i1, &d1);
        si = i1 - i0;
        sd = d1 - d0;
    }
    store_record(dst, layout, idx, i0, si, d0, sd);
}

// Pack plain tables into the padded records. bf16 sources are widened exactly as the
// reference's .float() before its CUDA backward (cuda_backend.py:68-69).
__device__ inline float load_table(const void* t, int i, int bf16) {
    if (bf16) return __uint_as_float((unsigned int)static_cast<const unsigned short*>(t)[i] << 16);
    return static_cast<const float*>(t)[i];
}

__global__ void lut_pack_kernel(const void* ti, const void* td, int n, int src_bf16, int layout, void* dst) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= lut_records(n)) return;
    const int j = idx - kPad;
    const int jc = j < 0 ? 0 : (j > n - 1 ? n - 1 : j);
    const float i0 = load_table(ti, jc, src_bf16);
    const float d0 = layout == ISA_EKV_LUT_BWD ? load_table(td, jc, src_bf16) : 0.0f;
    float si = 0.0f, sd = 0.0f;
    if (j >= 0 && j < n - 1) {
        si = load_table(ti, j + 1, src_bf16) - i0;
        if (layout == ISA_EKV_LUT_BWD) sd = load_table(td, j + 1, src_bf16) - d0;
    }
    store_record(dst, layout, idx, i0, si, d0, sd);
}

// ----------------------------------------------------------------------------------
// Prep: token side [M][Kp] records and threshold side [Kp][Op] pairs, plus per-block
// (min, max) partials of the scaled coordinates. NaN maps to an infinite partial so the
// kernels' range tests fail and their general (clamping / selecting) loops run.
//   LUT mode:   token coordinate xs = (x - dmin) * s + kPad, threshold coordinate w * s.
//   exact mode: coordinates in log2 units, tx = x * a, tw = w * a with a = log2(e)/(2 n U_T);
//               the records for the range-checked loop hold 2^tx and 2^-tw (formed in fp64),
//               so 2^(tx - tw) is one multiply; the general loop reads tx and tw.
// Token records: {c, r} (forward) or {c, r, -r / z_div, 0} (backward), r = 1/(1 + x/V_sat).
// ----------------------------------------------------------------------------------

struct PrepArgs {
    const float* x;
    const float* wp;
    const float* wn;
    int64_t M, K, O, Kp, Op;
    float xoff, scale, xadd;  // token coordinate fma(x - xoff, scale, xadd); threshold w * scale
    double scale_d;           // exact mode: the same scale in fp64 for the exponentials
    float v_sat, z_div;        // backward token z = -r / z_div
    float pad_coord;          // coordinate of padded inputs k >= K (r = 0 there)
    int rec_floats;           // 2 or 4
    int exact;
    float* xrec;              // [M][Kp][rec_floats]: LUT coordinates, or 2^tx in exact mode
    float2* wsT;              // [Kp][Op]: LUT coordinates, or 2^-tw in exact mode
    float* xrec_slow;         // exact mode: [M][Kp][rec_floats] with tx
    float2* wsT_slow;         // exact mode: [Kp][Op] with tw
    float2* partials;         // [kPrepBlocksX + kPrepBlocksW]
    const float* in_affine;   // optional device {scale, shift}: the layer input is clamp(x*scale + shift)
    float in_lo, in_hi;
    unsigned* stat_bits;      // optional: the forward's output-statistics word, cleared here
};

// Input voltage mapping clamp(x * scale + shift, lo, hi) (cim.py:37-39): product and sum
// rounded separately as the two tensor ops do (no fma contraction); NaN stays NaN as
// torch.clamp keeps it.
__device__ inline float mapped_pre(float x, float scale, float shift) {
#pragma clang fp contract(off)
    const float prod = x * scale;
    return prod + shift;
}

__device__ inline float input_map(float x, float scale, float shift, float lo, float hi) {
    const float pre = mapped_pre(x, scale, shift);
    return pre != pre ? pre : fminf(fmaxf(pre, lo), hi);
}

__device__ inline void block_minmax(float lo, float hi, float2* out) {
    __shared__ float s_lo[32], s_hi[32];
    for (int off = 32; off > 0; off >>= 1) {
        lo = fminf(lo, __shfl_xor(lo, off));
        hi = fmaxf(hi, __shfl_xor(hi, off));
    }
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) {
        s_lo[wave] = lo;
        s_hi[wave] = hi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        const int nw = blockDim.x >> 6;
        for (int i = 1; i < nw; ++i) {
            lo = fminf(lo, s_lo[i]);
            hi = fmaxf(hi, s_hi[i]);
        }
        *out = make_float2(lo, hi);
    }
}

// Token side of the prep: the flattened [M][Kp] record space is walked in chunks of four
// block widths; each thread builds four records a block width apart, so every load and
// store instruction of a wave covers consecutive records (4-byte loads of x, 8- or
// 16-byte record stores).
template <int REC>
__device__ inline void store_token(float* dst, int64_t e, float c, float r, float z) {
    if constexpr (REC == 2)
        reinterpret_cast<float2*>(dst)[e] = make_float2(c, r);
    else
        reinterpret_cast<float4*>(dst)[e] = make_float4(c, r, z, 0.0f);
}

template <int REC, bool EXACT>
__device__ inline void prep_tokens(const PrepArgs& a, int b, float& lo, float& hi) {
    const float aff_s = a.in_affine ? a.in_affine[0] : 1.0f;
    const float aff_b = a.in_affine ? a.in_affine[1] : 0.0f;
    const int64_t total = a.M * a.Kp;
    const int64_t chunk = 4 * (int64_t)blockDim.x;
    for (int64_t base = (int64_t)b * chunk; base < total; base += (int64_t)kPrepBlocksX * chunk) {
        int64_t q = base + threadIdx.x;
        int64_t m, k;
        if (total <= 0xffffffffll) {
            m = (uint32_t)q / (uint32_t)a.Kp;
        } else {
            m = q / a.Kp;
        }
        k = q - m * a.Kp;
        float xv[4];  // loads first: four independent requests in flight
        int64_t mj[4], kj[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            mj[j] = m;
            kj[j] = k;
            // padded inputs k >= K read input K - 1 (their records repeat its coordinate)
            xv[j] = (q < total && a.K > 0) ? a.x[m * a.K + (k < a.K ? k : a.K - 1)] : 0.0f;
            q += blockDim.x;
            k += blockDim.x;
            while (k >= a.Kp) {
                k -= a.Kp;
                ++m;
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t e = mj[j] * a.Kp + kj[j];
            if (e >= total) break;
            float c, r, f = 1.0f;
            const bool real = kj[j] < a.K;
            if (a.K > 0) {
                // a padded input k >= K is input K - 1 again (coordinate, and thresholds on the
                // threshold side) with r = 0: its cells read records the real cells read, so
                // they stay inside any table window the range partials select, and add 0
                float x = xv[j];
                if (a.in_affine) x = input_map(x, aff_s, aff_b, a.in_lo, a.in_hi);
                c = fmaf(x - a.xoff, a.scale, a.xadd);
                r = real ? 1.0f / (1.0f + x / a.v_sat) : 0.0f;
                if (EXACT) f = (float)exp2((double)x * a.scale_d);
                if (real) {
                    const bool bad = c != c;
                    lo = fminf(lo, bad ? -INFINITY : c);
                    hi = fmaxf(hi, bad ? INFINITY : c);
                }
            } else {
                c = a.pad_coord;  // K == 0: every input is padding, paired with zero thresholds
                r = 0.0f;
            }
            const float z = -r / a.z_div;
            if (EXACT) {
                store_token<REC>(a.xrec, e, f, r, z);
                store_token<REC>(a.xrec_slow, e, c, r, z);
            } else {
                store_token<REC>(a.xrec, e, c, r, z);
            }
        }
    }
}

// Prep block b of kPrepBlocksX + kPrepBlocksW (token side, then threshold side).
__device__ inline void prep_block(const PrepArgs& a, int b) {
    if (a.stat_bits && b == 0 && threadIdx.x == 0) *a.stat_bits = 0u;
    float lo = INFINITY, hi = -INFINITY;
    if (b < kPrepBlocksX) {
        if (a.exact) {
            if (a.rec_floats == 2)
                prep_tokens<2, true>(a, b, lo, hi);
            else
                prep_tokens<4, true>(a, b, lo, hi);
        } else {
            if (a.rec_floats == 2)
                prep_tokens<2, false>(a, b, lo, hi);
            else
                prep_tokens<4, false>(a, b, lo, hi);
        }
        block_minmax(lo, hi, &a.partials[b]);
        return;
    }
    // threshold side: 64(o) x 32(k) tiles of raw thresholds transposed through LDS
    __shared__ float2 tile[32][65];
    const int64_t n_ot = a.Op / 64, n_kt = (a.Kp + 31) / 32;  // Op: multiple of 256; Kp: of 8
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
    for (int64_t t = b - kPrepBlocksX; t < n_ot * n_kt; t += kPrepBlocksW) {
        const int64_t ot = t % n_ot, kt = t / n_ot;
        // load: rows o (64), cols k (32), coalesced along k
        for (int rr = ty; rr < 64; rr += 8) {
            int64_t o = ot * 64 + rr;
            const int64_t k = kt * 32 + tx;
            float2 v = make_float2(0.0f, 0.0f);
            if (a.K > 0 && a.O > 0) {
                const bool real = o < a.O && k < a.K;
                if (o >= a.O) o = a.O - 1;  // padded outputs copy a real row; results are dropped
                const int64_t kc = k < a.K ? k : a.K - 1;  // padded inputs copy input K - 1 (r = 0)
                v = make_float2(a.wp[o * a.K + kc], a.wn[o * a.K + kc]);
                if (real) {
                    const float p = v.x * a.scale, q = v.y * a.scale;
                    const bool bad = (p != p) || (q != q);
                    lo = fminf(lo, bad ? -INFINITY : fminf(p, q));
                    hi = fmaxf(hi, bad ? INFINITY : fmaxf(p, q));
                }
            }
            tile[tx][rr] = v;
        }
        __syncthreads();
        // store: rows k (32), cols o (64), coalesced along o
        for (int rr = ty; rr < 32; rr += 8) {
            const int64_t k = kt * 32 + rr;
            if (k < a.Kp) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const float2 v = tile[rr][h * 32 + tx];
                    const int64_t e = k * a.Op + ot * 64 + h * 32 + tx;
                    const float2 c = make_float2(v.x * a.scale, v.y * a.scale);
                    if (a.exact) {
                        a.wsT[e] = make_float2((float)exp2(-(double)v.x * a.scale_d),
                                               (float)exp2(-(double)v.y * a.scale_d));
                        a.wsT_slow[e] = c;
                    } else {
                        a.wsT[e] = c;
                    }
                }
            }
        }
        __syncthreads();
    }
    block_minmax(lo, hi, &a.partials[b]);
}

__global__ __launch_bounds__(256) void prep_kernel(PrepArgs a) { prep_block(a, blockIdx.x); }

// Copies elements [0, n) of src into LDS through store(i, value), the block's threads taking
// every blockDim.x-th element and issuing BATCH loads before their stores (a strided loop that
// stores each load before issuing the next waits out one memory latency per element).
template <int BATCH, typename T, typename Store>
__device__ inline void stage_to_lds(const T* __restrict__ src, int n, Store store) {
    for (int base = threadIdx.x; base < n; base += BATCH * (int)blockDim.x) {
        T v[BATCH];
#pragma unroll
        for (int j = 0; j < BATCH; ++j) {
            const int i = base + j * (int)blockDim.x;
            if (i < n) v[j] = src[i];
        }
#pragma unroll
        for (int j = 0; j < BATCH; ++j) {
            const int i = base + j * (int)blockDim.x;
            if (i < n) store(i, v[j]);
        }
    }
}

// Range of the prep kernel's coordinates: token side (xlo, xhi), threshold side (wlo, whi),
// wave-uniform.
struct CoordRange {
    float xlo, xhi, wlo, whi;
};

// Every lane issues its loads (16-byte pairs of partials) in two rounds of five, each round's
// before its first use: two memory latencies per call, where a loop that consumes each load
// before the next waits out twenty, at 20 VGPRs.
__device__ inline CoordRange read_coord_range(const float2* __restrict__ partials) {
    static_assert(kPrepBlocksX % 256 == 0 && kPrepBlocksW % 256 == 0, "two rounds of 16-byte pairs per lane");
    constexpr int NX = kPrepBlocksX / 256, NW = kPrepBlocksW / 256;  // loads per lane and round
    const int lane = threadIdx.x & 63;
    const float4* p4 = reinterpret_cast<const float4*>(partials);  // 256-byte aligned workspace slot
    float xlo = INFINITY, xhi = -INFINITY, wlo = INFINITY, whi = -INFINITY;
#pragma unroll
    for (int round = 0; round < 2; ++round) {
        float4 px[NX], pw[NW];
#pragma unroll
        for (int j = 0; j < NX; ++j) px[j] = p4[lane + 64 * (round * NX + j)];
#pragma unroll
        for (int j = 0; j < NW; ++j) pw[j] = p4[kPrepBlocksX / 2 + lane + 64 * (round * NW + j)];
#pragma unroll
        for (int j = 0; j < NX; ++j) {
            xlo = fminf(xlo, fminf(px[j].x, px[j].z));
            xhi = fmaxf(xhi, fmaxf(px[j].y, px[j].w));
        }
#pragma unroll
        for (int j = 0; j < NW; ++j) {
            wlo = fminf(wlo, fminf(pw[j].x, pw[j].z));
            whi = fmaxf(whi, fmaxf(pw[j].y, pw[j].w));
        }
    }
    for (int off = 32; off > 0; off >>= 1) {
        xlo = fminf(xlo, __shfl_xor(xlo, off));
        xhi = fmaxf(xhi, __shfl_xor(xhi, off));
        wlo = fminf(wlo, __shfl_xor(wlo, off));
        whi = fmaxf(whi, __shfl_xor(whi, off));
    }
    return CoordRange{xlo, xhi, wlo, whi};
}

// LUT kernels: every coordinate difference lies within the padded table, so the loop needs
// no clamp (the kPad replicated end records reproduce the reference's clamp there).
__device__ inline bool coords_in_padded_range(const float2* __restrict__ partials, int n_pad_entries) {
    const CoordRange c = read_coord_range(partials);
    const bool ok = (c.xlo - c.whi >= 1.0f) && (c.xhi - c.wlo <= (float)(n_pad_entries - 2));
    return __builtin_amdgcn_readfirstlane((int)ok) != 0;
}

// LUT forward with a second table copy: a gather's 64 lanes read the records of their own
// thresholds, and once the thresholds spread over more than ~100 records, lanes of a
// half-wave often hit one LDS bank pair with different records. A second copy of the table
// 16 bank pairs away (the copy starts T1 records after the first, T1 % 32 == 16) lets each
// (input, output) threshold pick the copy whose bank is less loaded (fwd_copy_assign_kernel;
// the choice folds into the threshold coordinate, c' = c + T1, and copy 1 stores
// A' = A - T1 dT so that fma(c', dT, A') = fma(c, dT, A)). With narrow thresholds (the
// initial ones span ~69 records) the lanes share records often enough that splitting them
// over two copies costs more than it saves, so the mode needs a wide spread and the
// clamp-free loop (the fold assumes unclamped coordinates).
constexpr float kFwdCopyMinWindow = 100.0f;  // threshold spread, in table records
constexpr size_t kFwdCopyLdsBytes = 80 * 1024;  // both copies, with two forward blocks per CU
constexpr int kFwdCopyMinInputs16 = 256;         // padded inputs per wave for the 16-wave copy blocks
constexpr int kFwdWinOffset = kSplitRecords + 16;  // second copy of a coordinate window (16 mod 32)

// second-copy offset (records, = 16 mod 32, past the first copy) and both copies' LDS bytes
inline int fwd_copy_offset(int n_entries) { return (int)((n_entries + 2 * kPad - 16 + 31) / 32 * 32) + 16; }
inline size_t fwd_copy_lds(int n_entries) { return (size_t)(fwd_copy_offset(n_entries) + n_entries + 2 * kPad) * 8; }

__device__ inline bool fwd_copies_mode(const float2* __restrict__ partials, int n_pad_entries) {
    const CoordRange c = read_coord_range(partials);
    const bool ok = (c.xlo - c.whi >= 1.0f) && (c.xhi - c.wlo <= (float)(n_pad_entries - 2)) &&
                    (c.whi - c.wlo >= kFwdCopyMinWindow);
    return __builtin_amdgcn_readfirstlane((int)ok) != 0;
}

template <bool CLAMP>
__device__ inline float coord(float xs, float ws, float cmin, float cmax) {
    float c = xs - ws;
    if (CLAMP) c = fminf(fmaxf(c, cmin), cmax);  // NaN -> cmin, as fmaxf(NaN, 0) in ekv_cuda.cu:20
    return c;
}

// ----------------------------------------------------------------------------------
// Cell evaluators. The forward and backward loops are written once over a cell policy
// that turns a token operand t (from the token record) and a threshold operand w (from
// the threshold record) into the per-threshold current term l (forward) or the pair
// (l, d) of current and derivative terms (backward), in the policy's units:
//   LUT:   l = L_I(dV), d = L_D(dV) from the LDS table (physical units).
//   exact: l = l1^2 - l2^2 and d = l1 s1 - l2 s2 with l_i = log2(1 + 2^t_i) and
//          s_i = sigmoid, t1 = tx - tw, t2 = t1 - V_D a; the caller's constants
//          I_S ln2^2 (current) and 2 a I_S ln2 (derivative, a in natural units) restore
//          the reference's I_S [sp1^2 - sp2^2] and I_S 2/(2nU_T) [sp1 s1 - sp2 s2]
//          (ekv_triton.py:33-66).
// ----------------------------------------------------------------------------------

// LDS record address from the bits of a float sum, for coordinates c with 1/16 <= c - lo <
// 2^20 and lo <= 2^19: t = fl(c + (2^20 - lo - 1/16)) lies in [2^20, 2^21), where the float
// grid is 1/8, and rounding c - lo - 1/16 to nearest (ties to even) on that grid keeps the
// integer part floor(c) - lo (an integer c is a tie that goes to the even neighbour, the
// integer itself; a c just below the next integer rounds to at most 7/8 past it). Below
// lo + 1/16 the sum stays under 2^20 and the bits are no address: the kernels' coordinates
// lie at least one record past lo (their windows keep two records of margin; with lo = 0 the
// clamp-free condition holds c >= 1 and the clamp c >= kPad). The
// mantissa bits of t above its three fraction bits are then (floor(c) - lo) * 8: the LDS
// byte address of the record when the table's record lo sits at LDS address 0, which is
// where the kernels that use this put their dynamic LDS (they declare no static LDS; the
// launch code checks that). The add and the mask issue at the VALU's full rate, where the
// v_cvt_u32_f32 and v_lshl_add_u32 of table[(unsigned)c] each take two issue cycles on
// gfx950, and an address formed from the table's pointer would cost one more add per gather
// (the dynamic LDS base is not known when the loads are formed).
typedef float f32x2 __attribute__((ext_vector_type(2)));
using lds_f32x2 = __attribute__((address_space(3))) const f32x2;
constexpr unsigned kRecAddrMask = 0x7FFFF8u;
__device__ inline float rec_addr_bias(int lo) { return (float)((1 << 20) - lo) - 0.0625f; }
__device__ inline float2 lds_record(float c, float bias) {
    const f32x2 v = *(lds_f32x2*)(size_t)(__float_as_uint(c + bias) & kRecAddrMask);
    return make_float2(v.x, v.y);
}

// Cells take both thresholds of a (token, output, input) cell at once: forward cells return
// l(+) - l(-); the LUT cells issue both gathers before using either. FLOAT_ADDR cells read
// an LDS table at LDS address 0 whose first record is record lo of the padded table, with
// lds_record and bias = rec_addr_bias(lo) (lut, that table, is then unused); the others read
// lut[c].
template <bool CLAMP, bool FLOAT_ADDR = false>
struct LutFwdCell {
    const float2* lut;
    float cmin, cmax;
    float bias;
    __device__ float2 record(float c) const { return FLOAT_ADDR ? lds_record(c, bias) : lut[(unsigned)c]; }
    __device__ float operator()(float xs, float wsp, float wsn) const {
        const float cp = coord<CLAMP>(xs, wsp, cmin, cmax);
        const float cn = coord<CLAMP>(xs, wsn, cmin, cmax);
        const float2 ep = record(cp);
        const float2 en = record(cn);
        return fmaf(cp, ep.y, ep.x) - fmaf(cn, en.y, en.x);
    }
    // token record {coordinate, r}; threshold record {+, -}
    __device__ float accumulate(float acc, float2 xv, float2 w) const {
        return fmaf((*this)(xv.x, w.x, w.y), xv.y, acc);
    }
    // two-phase form of accumulate (same arithmetic): fetch issues the gathers of one cell,
    // finish consumes them, so a loop can keep several cells' gathers in flight
    struct Pending {
        float cp, cn;
        float2 ep, en;
    };
    __device__ Pending fetch(float xs, float2 w) const {
        Pending q;
        q.cp = coord<CLAMP>(xs, w.x, cmin, cmax);
        q.cn = coord<CLAMP>(xs, w.y, cmin, cmax);
        q.ep = record(q.cp);
        q.en = record(q.cn);
        return q;
    }
    __device__ float finish(float acc, const Pending& q, float r) const {
        return fmaf(fmaf(q.cp, q.ep.y, q.ep.x) - fmaf(q.cn, q.en.y, q.en.x), r, acc);
    }
};

#ifndef ISA_EKV_FWD_TOKOPS
#define ISA_EKV_FWD_TOKOPS 16  // forward: token records (MR tokens x KU inputs) loaded per step
#endif
#ifndef ISA_EKV_FWD_WT
#define ISA_EKV_FWD_WT 3  // forward plan: target waves = WT x 256 CUs x 16
#endif
#ifndef ISA_EKV_FWD_FB
#define ISA_EKV_FWD_FB 4  // LUT forward: cells whose gathers are issued together
#endif

template <class Cell>
struct TwoPhaseCell : std::false_type {};
template <bool CLAMP, bool FLOAT_ADDR>
struct TwoPhaseCell<LutFwdCell<CLAMP, FLOAT_ADDR>> : std::true_type {};

// Backward cells return a pair view whose dp()/dn() (derivative terms) and lp()/ln()
// (current terms) the loop reads where it uses them; the LUT view holds the two gathered
// records and evaluates each term on demand.
struct LutBwdPair {
    float cp, cn;
    float4 ep, en;
    __device__ float dp() const { return fmaf(cp, ep.w, ep.z); }
    __device__ float dn() const { return fmaf(cn, en.w, en.z); }
    __device__ float lp() const { return fmaf(cp, ep.y, ep.x); }
    __device__ float ln() const { return fmaf(cn, en.y, en.x); }
};

template <bool CLAMP, class Table>
struct LutBwdCell {
    Table lut;
    float cmin, cmax;
    __device__ LutBwdPair operator()(float xs, float wsp, float wsn) const {
        LutBwdPair q;
        q.cp = coord<CLAMP>(xs, wsp, cmin, cmax);
        q.cn = coord<CLAMP>(xs, wsn, cmin, cmax);
        q.ep = lut[(unsigned)q.cp];
        q.en = lut[(unsigned)q.cn];
        return q;
    }
};

struct ValueBwdPair {
    float l_p, d_p, l_n, d_n;
    __device__ float dp() const { return d_p; }
    __device__ float dn() const { return d_n; }
    __device__ float lp() const { return l_p; }
    __device__ float ln() const { return l_n; }
};

// log2(1 + 2^t) as torch's softplus (threshold 20 in natural units: t = 20 log2 e), in
// log2 units; NaN propagates.
constexpr float kSoftplusLog2Threshold = 28.853900817779268f;

// log2(1 + e) for e >= 0, accurate to a few ulp also where 1 + e rounds (e << 1, the
// subthreshold cells). With w = fl(1 + e), d = e - (w - 1) is w's rounding error, exactly,
// and log2(w + d) = log2(w) + d / (w ln2) to second order. For e < 1, |d| <= 2^-25 and the
// 1/w factor in (1/2, 1] is dropped at a relative cost below |d|; for e >= 1 the clamp keeps
// the term below the rounding of log2(w) >= 1. v_log_f32 is accurate relative to its result.
constexpr float kInvLn2 = 1.4426950408889634f;

__device__ inline float log2_1p(float e) {
    const float w = 1.0f + e;
    const float d = e - (w - 1.0f);
    return fmaf(__builtin_amdgcn_fmed3f(d, -0x1p-24f, 0x1p-24f), kInvLn2, __builtin_amdgcn_logf(w));
}

// Range-checked exact cells: operands 2^tx and 2^-tw with |tx|, |tw| <= kExactFastBound
// and tx - tw <= kExactFastBound, so e = 2^(tx - tw) is a normal float below 2^60 and
// log2(1 + e) equals the thresholded softplus to rounding.
constexpr float kExactFastBound = 60.0f;

struct ExactFastFwdCell {
    float k2;  // 2^(-V_D a)
    __device__ float one(float ex, float ew) const {
        const float e1 = ex * ew, e2 = e1 * k2;
        const float l1 = log2_1p(e1), l2 = log2_1p(e2);
        return fmaf(l1, l1, -(l2 * l2));
    }
    __device__ float operator()(float ex, float ewp, float ewn) const { return one(ex, ewp) - one(ex, ewn); }
    __device__ float accumulate(float acc, float2 xv, float2 w) const {
        return fmaf((*this)(xv.x, w.x, w.y), xv.y, acc);
    }
};

struct ExactFastBwdCell {
    float k2;
    __device__ void one(float ex, float ew, float& l, float& d) const {
        const float e1 = ex * ew, e2 = e1 * k2;
        const float w1 = 1.0f + e1, w2 = 1.0f + e2;
        const float l1 = log2_1p(e1), l2 = log2_1p(e2);
        const float s1 = e1 * __builtin_amdgcn_rcpf(w1), s2 = e2 * __builtin_amdgcn_rcpf(w2);
        l = fmaf(l1, l1, -(l2 * l2));
        d = fmaf(l1, s1, -(l2 * s2));
    }
    __device__ ValueBwdPair operator()(float ex, float ewp, float ewn) const {
        ValueBwdPair q;
        one(ex, ewp, q.l_p, q.d_p);
        one(ex, ewn, q.l_n, q.d_n);
        return q;
    }
};

// General exact cells: any operands, including NaN and infinities.
__device__ inline void softplus_log2(float t, float& l, float& s) {
    const float e = __builtin_amdgcn_exp2f(t);
    const bool lin = t > kSoftplusLog2Threshold;
    l = lin ? t : log2_1p(e);
    s = lin ? 1.0f : e * __builtin_amdgcn_rcpf(1.0f + e);
}

struct ExactGeneralFwdCell {
    float c2;  // V_D a
    __device__ float one(float tx, float tw) const {
        const float t1 = tx - tw;
        float l1, l2, s1, s2;
        softplus_log2(t1, l1, s1);
        softplus_log2(t1 - c2, l2, s2);
        return fmaf(l1, l1, -(l2 * l2));
    }
    __device__ float operator()(float tx, float twp, float twn) const { return one(tx, twp) - one(tx, twn); }
    __device__ float accumulate(float acc, float2 xv, float2 w) const {
        return fmaf((*this)(xv.x, w.x, w.y), xv.y, acc);
    }
};

struct ExactGeneralBwdCell {
    float c2;
    __device__ void one(float tx, float tw, float& l, float& d) const {
        const float t1 = tx - tw;
        float l1, l2, s1, s2;
        softplus_log2(t1, l1, s1);
        softplus_log2(t1 - c2, l2, s2);
        l = fmaf(l1, l1, -(l2 * l2));
        d = fmaf(l1, s1, -(l2 * s2));
    }
    __device__ ValueBwdPair operator()(float tx, float twp, float twn) const {
        ValueBwdPair q;
        one(tx, twp, q.l_p, q.d_p);
        one(tx, twn, q.l_n, q.d_n);
        return q;
    }
};

__device__ inline bool exact_operands_in_fast_range(const float2* __restrict__ partials) {
    const CoordRange c = read_coord_range(partials);
    const float b = kExactFastBound;
    const bool ok = c.xlo >= -b && c.xhi <= b && c.wlo >= -b && c.whi <= b && c.xhi - c.wlo <= b;
    return __builtin_amdgcn_readfirstlane((int)ok) != 0;
}

// ----------------------------------------------------------------------------------
// Forward. Block = FWD_WAVES waves sharing one LDS table and one output block of
// 64*ORR outputs; wave w owns tokens [ (tile_m * FWD_WAVES + w) * MR, +MR ).
// ----------------------------------------------------------------------------------

// A block's shader-clock span (profiling only, acc non-null): every wave reads clock64 (shader
// cycles, s_memtime) and wall_clock64 (constant-rate ticks, s_memrealtime) into scalar
// registers at the start; wave 0 adds its spans and a block count to acc with vector atomics at
// the end. acc is a kernel argument, so the branch is uniform and costs no VGPRs.
struct BlockClock {
    unsigned long long* acc;
    long long c0, w0;
    __device__ explicit BlockClock(unsigned long long* a) : acc(a), c0(0), w0(0) {
        if (acc) {
            c0 = clock64();
            w0 = wall_clock64();
        }
    }
    __device__ void stop() const {
        if (acc && threadIdx.x == 0) {
            const long long c1 = clock64(), w1 = wall_clock64();
            atomicAdd(acc, (unsigned long long)(c1 - c0));
            atomicAdd(acc + 1, (unsigned long long)(w1 - w0));
            atomicAdd(acc + 2, 1ull);
        }
    }
};

struct FwdArgs {
    const float2* xrec;     // [M][Kp] token records {t, r}
    const float2* wsT;      // [Kp][Op] threshold records
    const float2* xrec_alt; // exact: general-loop token records {tx, r}
    const float2* wsT_alt;  // exact: general-loop threshold records
    const float2* lut;      // LUT: [NP] {A_I, dI}
    const float2* partials;
    float* out;             // [M][O]
    int M, O, Kp, Op, NP;
    int n_mt, n_ot;         // tiles along M (per block) and O
    float cmin, cmax, out_min, out_max;
    float out_scale;        // exact: I_S ln2^2
    float k2, c2;           // exact: 2^(-V_D a), V_D a
    // optional epilogue (layer glue): idiff is stored when given; out = glue(idiff)
    float* idiff;           // [M][O]
    const float* r_tia;     // device scalar: y = clamp(idiff * r, y_lo, y_hi), r = tia_gain(...)
    const float* r_log_scale;
    float r_log_lo, r_log_hi;
    float y_lo, y_hi;
    const float* adc_scale; // device [O]: out = y * adc_scale[o] + adc_shift[o]
    const float* adc_shift;
    unsigned* stat_bits;    // optional: atomic max of the |y| bit patterns (see layer_stat_bits)
    int glue;
    // K split (see plan_forward): n_split > 1 ranges of k_chunk padded inputs; each writes its
    // raw partial sums to split_part[s][M][O] and split_reduce_kernel finishes the outputs
    int n_split, k_chunk;
    float* split_part;
    int copy_offset;        // LUT: T1 > 0 when the launch may use the second table copy
    int copy_window;        // LUT: > 0: the copies hold only the coordinate window, of at most this many records
    int mc_budget, mc_max;  // LUT: mc_budget > 0: the launch may hold up to mc_max windowed copies in this many LDS records
    unsigned long long* clock_acc;  // profiling: {cycles, wall ticks, blocks} of this kernel (BlockClock), or null
};

// The work of one forward wave.
struct FwdTile {
    int m0, o_lane;    // first token of the wave, first output of the lane
    int k_lo, k_hi;    // padded-input range summed by this wave
    float* split_out;  // K split: this split's [M][O] partial sums (null: full sums, epilogue here)
};

// The TIA gain: r_tia[0], or CIMLinear's learnable gain r_tia_base * exp(clamp(log_scale,
// lo, hi)) (cim.py:74-77) with the same ops in the same order (clamp keeping NaN, the
// library expf, one rounded product). Wave-uniform.
__device__ inline float tia_gain(const float* r_tia, const float* log_scale, float lo, float hi) {
#pragma clang fp contract(off)
    const float base = load_uniform1(r_tia);
    if (!log_scale) return base;
    const float ls = load_uniform1(log_scale);
    const float c = ls != ls ? ls : fminf(fmaxf(ls, lo), hi);
    return base * expf(c);
}

// TIA gain and output clamp (cim.py:190-193) and the ADC affine (cim.py:243), applied to one
// output value: each tensor op's rounding kept (no contraction), NaN kept as torch.clamp does.
__device__ inline float layer_tia(float v, float r, bool has_r, float lo, float hi) {
#pragma clang fp contract(off)
    if (has_r) {
        v = v * r;
        v = v != v ? v : fminf(fmaxf(v, lo), hi);
    }
    return v;
}

__device__ inline float layer_adc(float v, const float* a_scale, const float* a_shift, int o) {
#pragma clang fp contract(off)
    if (a_scale) {
        const float prod = v * a_scale[o];
        v = prod + a_shift[o];
    }
    return v;
}

// |y| as an unsigned bit pattern: non-negative floats order as their bits, and every NaN
// pattern lies above +inf, so an unsigned max over them is the NaN-propagating max of
// torch.maximum / Tensor.max (cim.py:194-198).
__device__ inline unsigned layer_stat_bits(float y) { return __float_as_uint(y) & 0x7fffffffu; }

template <int MR, int ORR, bool CLAMP_OUT, class Cell>
__device__ inline void fwd_body(const FwdArgs& a, const Cell cell, const float2* xrec, const float2* wsT,
                                const FwdTile& tile) {
    const int m0 = tile.m0, o_lane = tile.o_lane;
    float acc[MR][ORR];
#pragma unroll
    for (int i = 0; i < MR; ++i)
#pragma unroll
        for (int j = 0; j < ORR; ++j) acc[i][j] = 0.0f;

    const float2* xrow[MR];
#pragma unroll
    for (int i = 0; i < MR; ++i) {
        const int m = min(m0 + i, a.M - 1);
        xrow[i] = xrec + (size_t)m * a.Kp;
    }
    const float4* wcol = reinterpret_cast<const float4*>(wsT + o_lane);
    const size_t wstride = (size_t)a.Op / 2;  // float4 per k row

    constexpr int KU = ISA_EKV_FWD_TOKOPS / MR >= 1 ? ISA_EKV_FWD_TOKOPS / MR : 1;  // token records per step
    static_assert(KU >= 1 && 8 % KU == 0, "Kp and the K-split ranges are multiples of 8");
    for (int k0 = tile.k_lo; k0 < tile.k_hi; k0 += KU) {
        float2 w[KU][ORR];
#pragma unroll
        for (int kk = 0; kk < KU; ++kk)
#pragma unroll
            for (int j = 0; j < ORR / 2; ++j) {
                const float4 v = wcol[(size_t)(k0 + kk) * wstride + j];
                w[kk][2 * j] = make_float2(v.x, v.y);
                w[kk][2 * j + 1] = make_float2(v.z, v.w);
            }
#pragma unroll
        for (int kk = 0; kk < KU; ++kk) {
#pragma unroll
            for (int i = 0; i < MR; ++i) {
                const float2 xv = load_uniform2(xrow[i] + k0 + kk);
                if constexpr (TwoPhaseCell<Cell>::value && ISA_EKV_FWD_FB > 0) {
                    constexpr int FB = ISA_EKV_FWD_FB < ORR ? ISA_EKV_FWD_FB : ORR;
#pragma unroll
                    for (int j0 = 0; j0 < ORR; j0 += FB) {
                        typename Cell::Pending q[FB];
#pragma unroll
                        for (int jj = 0; jj < FB; ++jj) q[jj] = cell.fetch(xv.x, w[kk][j0 + jj]);
#pragma unroll
                        for (int jj = 0; jj < FB; ++jj) acc[i][j0 + jj] = cell.finish(acc[i][j0 + jj], q[jj], xv.y);
                    }
                } else {
#pragma unroll
                    for (int j = 0; j < ORR; ++j) acc[i][j] = cell.accumulate(acc[i][j], xv, w[kk][j]);
                }
            }
        }
    }
    if (tile.split_out) {  // partial sums over this K range; split_reduce_kernel does the rest
#pragma unroll
        for (int i = 0; i < MR; ++i) {
            const int m = m0 + i;
            if (m >= a.M) break;
            float* prow = tile.split_out + (size_t)m * a.O;
#pragma unroll
            for (int j = 0; j < ORR; ++j)
                if (o_lane + j < a.O) prow[o_lane + j] = acc[i][j];
        }
        return;
    }
    if (a.glue) {
        const bool has_r = a.r_tia != nullptr;
        const float r = has_r ? tia_gain(a.r_tia, a.r_log_scale, a.r_log_lo, a.r_log_hi) : 1.0f;
        unsigned ymax = 0;
#pragma unroll
        for (int i = 0; i < MR; ++i) {
            const int m = m0 + i;
            if (m >= a.M) break;
            float* orow = a.out + (size_t)m * a.O;
            float* irow = a.idiff ? a.idiff + (size_t)m * a.O : nullptr;
#pragma unroll
            for (int j = 0; j < ORR; ++j) {
                const int o = o_lane + j;
                if (o >= a.O) continue;
                const float id = CLAMP_OUT ? fminf(fmaxf(acc[i][j], a.out_min), a.out_max) : acc[i][j] * a.out_scale;
                if (irow) irow[o] = id;
                const float y = layer_tia(id, r, has_r, a.y_lo, a.y_hi);
                ymax = max(ymax, layer_stat_bits(y));
                orow[o] = layer_adc(y, a.adc_scale, a.adc_shift, o);
            }
        }
        if (a.stat_bits) {  // wave-uniform; every lane of the wave is here (m0 is wave-uniform)
#pragma unroll
            for (int d = 32; d >= 1; d >>= 1) ymax = max(ymax, (unsigned)__shfl_xor((int)ymax, d, 64));
            if ((threadIdx.x & 63) == 0) atomicMax(a.stat_bits, ymax);
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < MR; ++i) {
        const int m = m0 + i;
        if (m >= a.M) break;
        float* orow = a.out + (size_t)m * a.O;
#pragma unroll
        for (int j = 0; j < ORR; ++j) {
            const int o = o_lane + j;
            if (o >= a.O) continue;
            if (CLAMP_OUT)
                orow[o] = fminf(fmaxf(acc[i][j], a.out_min), a.out_max);
            else
                orow[o] = acc[i][j] * a.out_scale;
        }
    }
}

constexpr int kFwdWaves = 8;

// Block index -> work index so that consecutive work indices run on one XCD: the hardware
// hands workgroups to the 8 XCDs round-robin by block index, so XCD x gets blocks x, x + 8,
// ...; they are given the contiguous work range [x * per_xcd, (x + 1) * per_xcd) (the blocks
// past 8 * per_xcd keep their index). Work that shares operands then shares that XCD's L2.
__device__ inline int xcd_work_index() {
    const int nb = gridDim.x;
    const int bid = blockIdx.x;
    const int per_xcd = nb / 8;
    return (per_xcd > 0 && bid < per_xcd * 8) ? (bid % 8) * per_xcd + bid / 8 : bid;
}

// Forward tile of this wave, in XCD-aware order: the blocks of one XCD walk consecutive token
// tiles of the same output block (and K split) and share that output block's threshold
// columns in their L2. Returns false for waves past M. Launches planned without a K split
// use SPLITS = false, which compiles them as if the split did not exist.
template <bool SPLITS>
__device__ inline bool fwd_tile(const FwdArgs& a, int MR, FwdTile& t) {
    int w = xcd_work_index();
    const int tiles = a.n_mt * a.n_ot;
    const int split = SPLITS && a.n_split > 1 ? w / tiles : 0;
    w -= split * tiles;
    const int tile_m = w % a.n_mt;
    const int tile_o = w / a.n_mt;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int wpb = blockDim.x >> 6;  // waves per block (8, or 16 for two 8192-entry tables)
    t.m0 = (tile_m * wpb + wave) * MR;
    t.o_lane = tile_o * 64 * kFwdORR + lane * kFwdORR;
    if (SPLITS && a.n_split > 1) {
        t.k_lo = split * a.k_chunk;
        t.k_hi = min(a.Kp, t.k_lo + a.k_chunk);
        t.split_out = a.split_part + (size_t)split * a.M * a.O;
    } else {
        t.k_lo = 0;
        t.k_hi = a.Kp;
        t.split_out = nullptr;
    }
    return t.m0 < a.M;
}

// Copy choice for the LUT forward's second table copy (see fwd_copies_mode). One thread per
// 32-lane problem: the thresholds one gather instruction's half-wave reads, i.e. input k,
// sign (+/-), output slot j of the lanes' kFwdORR outputs and half h of an output block:
// lanes l = 0..31 read output block * 256 + (32 h + l) * kFwdORR + j. Lane by lane, a lane
// whose threshold has the integer coordinate part of an earlier lane's takes that lane's
// copy (they read the same record for most tokens: a broadcast), otherwise the copy whose
// bank pair (floor coordinate, and its neighbour for the tokens whose fraction crosses the
// threshold's) has the smaller expected load so far. Copy-1 thresholds are stored as
// ws - T1 (so c' = xs - ws' = c + T1). Changes no record unless the launch is in copy mode.
constexpr int kAssignThreads = 128;

// Records [lo, lo + n) of the padded table hold every record the clamp-free loop reads, with
// two records of margin each side (the second copy's coordinates c + T1 round separately).
__device__ inline void coord_window(const CoordRange& c, int NP, int& lo, int& n) {
    const int l = max(0, (int)floorf(c.xlo - c.whi) - 2);
    const int h = min(NP - 1, (int)floorf(c.xhi - c.wlo) + 3);
    lo = __builtin_amdgcn_readfirstlane(l);
    n = __builtin_amdgcn_readfirstlane(h - l + 1);
}

// The launch's table-copy mode (fwd_copies_mode), wave-uniform; tables longer than
// max_window records also need their coordinate window to fit it.
__device__ inline bool launch_copy_mode(const float2* __restrict__ partials, int NP, int max_window) {
    bool on = fwd_copies_mode(partials, NP);
    if (on && NP > max_window) {
        int lo, n;
        coord_window(read_coord_range(partials), NP, lo, n);
        on = n <= max_window;
    }
    return on;
}

// Mode word values: 0 one table copy, 1 the second copy, kModeRanked the ranked backward (whose
// branch-deal pass runs before the copy assignment and records its decision first), and
// C >= kModeMultiMin: C bank-rotated copies of the coordinate window (fwd_multi_assign_kernel,
// which also runs before the two-copy assignment), recorded as kModeWindowed2 for C = 2.
constexpr int kModeRanked = 2;
constexpr int kModeMultiMin = 3;
constexpr int kMultiMax = 32;
constexpr int kModeWindowed2 = kMultiMax + 1;

// LANES = 32: 8-byte records, gathered by half-waves over 32 bank pairs; LANES = 16: 16-byte
// records, gathered by quarter-waves over 16 bank quads. Copy 1 sits LANES / 2 bins away.
// Every wave decides the launch's copy mode from the range partials (launch_copy_mode);
// block 0 records it in the mode word for the launches that follow.
template <int LANES>
__global__ __launch_bounds__(kAssignThreads) void fwd_copy_assign_kernel(float2* __restrict__ wsT,
                                                              const float2* __restrict__ partials, int NP,
                                                              int max_window, int* __restrict__ mode_word,
                                                              int64_t Kp, int64_t Op, int copy_offset,
                                                              int skip_from) {
    static_assert(LANES == 32 || LANES == 16, "half-wave or quarter-wave gathers");
    constexpr int kGroups = 64 / LANES, kMask = LANES - 1;
    // skip_from > 0: a pass earlier in the call recorded a mode of its own (the ranked backward,
    // skip_from = kModeRanked; the forward's windowed copies, skip_from = kModeMultiMin), which
    // this call keeps (this pass writes only 0 or 1, so every block reads the same decision)
    if (skip_from > 0 && __builtin_amdgcn_readfirstlane(*mode_word) >= skip_from) return;
    const bool on = launch_copy_mode(partials, NP, max_window);
    if (blockIdx.x == 0 && threadIdx.x == 0) *mode_word = on ? 1 : 0;
    if (!on) return;
    __shared__ float s_cnt[LANES][kAssignThreads];  // per-thread bank loads; [bin][thread]: conflict-free
    const int tid = threadIdx.x;
    const int64_t n_ot = Op / (64 * kFwdORR);
    const int64_t p = (int64_t)blockIdx.x * blockDim.x + tid;
    if (p >= Kp * n_ot * kFwdORR * 2 * kGroups) return;
    const int sign = (int)(p & 1), group = (int)((p >> 1) % kGroups);
    const int64_t rest0 = (p >> 1) / kGroups;
    const int j = (int)(rest0 % kFwdORR);
    const int64_t rest = rest0 / kFwdORR;
    const int64_t tile = rest % n_ot, k = rest / n_ot;
    float* w0 = reinterpret_cast<float*>(wsT + k * Op + tile * 64 * kFwdORR + j) + sign;
    const int64_t lane_stride = 2 * kFwdORR;  // floats between consecutive lanes' records
    const float t1 = (float)copy_offset;
#pragma unroll
    for (int b = 0; b < LANES; ++b) s_cnt[b][tid] = 0.0f;
    unsigned chosen = 0;  // bit l: lane l took copy 1
    float fls[LANES];     // integer coordinate parts of the lanes (registers: the loops unroll)
#pragma unroll
    for (int l = 0; l < LANES; ++l) {
        float* wp = w0 + (int64_t)(LANES * group + l) * lane_stride;
        const float w = *wp;
        const float fl = floorf(w);
        const float fr = w - fl;
        int c = -1;
#pragma unroll
        for (int b = l - 1; b >= 0; --b)  // the earliest match wins
            if (fls[b] == fl) c = (chosen >> b) & 1;
        if (c < 0) {
            // bank bin of the record at floor(u) - fl (weight 1 - fr) and one below (fr);
            // floor(u) is common to the lane group, so bin = -fl mod LANES (+LANES/2 for copy 1)
            const int r0 = (-(int)fl) & kMask, r1 = (r0 + LANES / 2) & kMask;
            const int m0 = (r0 + kMask) & kMask, m1 = (r1 + kMask) & kMask;
            const float v0 = (1.0f - fr) * s_cnt[r0][tid] + fr * s_cnt[m0][tid];
            const float v1 = (1.0f - fr) * s_cnt[r1][tid] + fr * s_cnt[m1][tid];
            c = v1 < v0 ? 1 : 0;
            s_cnt[c ? r1 : r0][tid] += 1.0f - fr;
            s_cnt[c ? m1 : m0][tid] += fr;
        }
        fls[l] = fl;
        chosen |= (unsigned)c << l;
        if (c) *wp = w - t1;
    }
}

// LUT forward with C bank-rotated copies of the coordinate window (3 <= C <= 32, or 2 where
// three do not fit), the generalisation of the second copy that also pays at narrow spreads. Copy c holds the
// window's records from LDS record T_c = c * stride + floor(32 c / C) (stride = the window
// rounded up to 32 records), so its bank pairs sit floor(32 c / C) from copy 0's; a threshold
// that takes copy c is stored as ws - T_c and copy c's records as {A - T_c dT, dT}, as for the
// second copy. A launch takes the most copies (up to the host's maximum) whose layout fits
// its LDS allocation, when the clamp-free loop runs: the assignment pass and the forward
// kernel decide it from the same range partials.
struct MultiLayout {
    int copies, stride, lo, n;  // copies == 0: not in this mode
    int dhalf;                  // split tables: the D halves' distance from the I halves, in records
};

// Bank-pair rotation and first LDS record of copy c.
__host__ __device__ inline int multi_rot(int c, int copies) { return c * 32 / copies; }
__host__ __device__ inline int multi_offset(int c, int copies, int stride) {
    return c * stride + multi_rot(c, copies);
}

// The clamp-free loop's condition (coords_in_padded_range) on a range already read.
__device__ inline bool clamp_free(const CoordRange& c, int NP) {
    return __builtin_amdgcn_readfirstlane((int)((c.xlo - c.whi >= 1.0f) && (c.xhi - c.wlo <= (float)(NP - 2)))) != 0;
}

// Two copies where three do not fit (wide windows): copy 1 sixteen bank pairs from copy 0.
// dhalf > 0 (the backward's split tables): each copy also holds the D halves of its records,
// dhalf records after its I halves, for windows of at most max_window records (wider ones, up
// to wide_dhalf records, with the D halves wide_dhalf records on), and only when the
// thresholds spread over at least kFwdCopyMinWindow records (below that the backward's
// one-copy launch, two blocks per CU, beats the copies' one block: 9.37 against 9.54 ms at the
// headline's 69 records).
__device__ inline MultiLayout multi_layout(const CoordRange& cr, int NP, int budget, int max_copies, int dhalf,
                                           int max_window, int wide_dhalf = 0) {
    const MultiLayout none{0, 0, 0, NP, 0};
    MultiLayout m = none;
    if (max_copies < kModeMultiMin || !clamp_free(cr, NP)) return none;
    if (dhalf > 0 && __builtin_amdgcn_readfirstlane((int)(cr.whi - cr.wlo >= kFwdCopyMinWindow)) == 0) return none;
    coord_window(cr, NP, m.lo, m.n);
    if (m.n > max_window) {
        if (m.n > wide_dhalf) return none;
        dhalf = wide_dhalf;
    }
    const int stride = (dhalf + m.n + 31) & ~31;
    for (int c = min(max_copies, kMultiMax); c >= 2; --c) {
        if (multi_offset(c - 1, c, stride) + dhalf + m.n <= budget) {
            m.copies = c;
            m.stride = stride;
            m.dhalf = dhalf;
            return m;
        }
    }
    return none;
}

__host__ __device__ inline int multi_mode_word(int copies) { return copies == 2 ? kModeWindowed2 : copies; }

__device__ inline MultiLayout fwd_multi_layout(const CoordRange& cr, int NP, int budget, int max_copies) {
    return multi_layout(cr, NP, budget, max_copies, 0, NP);
}

__device__ inline bool ranked_mode(const float2* __restrict__ partials, int NP, float max_spread,
                                   float* spread);

// Copy choice for the windowed copies. A problem is the 32 thresholds one half-wave gather
// reads (as in fwd_copy_assign_kernel<32>: input k, sign, output slot j, half of an output
// block); kMcGroup threads share it, each pricing C / kMcGroup of the copies. The thresholds
// are taken in increasing order, so that lanes reading one record for a token follow each
// other. At kMultiSamples token-coordinate fractions f_q = (q + 1/2) / kMultiSamples, a
// threshold w = W + g reads record floor(u) - W - [f_q < g] for a token at u: bank pair
// -W - [f_q < g] plus the copy's rotation, up to the common floor(u). Each threshold takes the
// copy that least raises the sum over the samples of the squared number of distinct records
// per bank pair (nothing at a sample where the copy already holds the threshold's record), a
// surrogate of the half-wave's conflict degree, with the number of records per bank pair and
// sample kept as two bit planes (one record or more, two or more: the increase 2 n + 1 is
// priced with n capped at 2). On uniform thresholds over a 68-record window it lowers the
// expected conflict degree from 2.21 (one copy) to 1.97 (4 copies), 1.84 (8) and 1.51 (32).
constexpr int kMultiSamples = 8;  // one bit per sample in the bit planes
constexpr int kMcProblems = 64;   // problems per assignment block
constexpr int kMcGroup = 4;       // threads per problem
constexpr int kMcThreads = kMcProblems * kMcGroup;

// s_pe[i][problem], i in [0, 64): bank pair b = i % 32's planes (bits 0-7 one record or more
// per sample, bits 8-15 two or more) in the low half and bank pair b - 1's in the high half,
// stored twice so that copy c's pair for base bank b0 is entry b0 + floor(32 c / C), unwrapped.
// s_info[rank][problem]: the sorted threshold's base bank pair b0 = -W mod 32 (bits 0-4), its
// samples reading the record below (bits 5-12), the samples whose record differs from the
// previous threshold's (bits 13-20) and its lane (bits 21-25).
template <int kPer>  // copies priced by this thread: c = sub + kMcGroup * i < copies, i < kPer
__device__ inline void multi_greedy(const float* s_sw, const unsigned* s_info, unsigned* s_pe, int prob, int sub,
                                    bool active, float* w0, int64_t lane_stride, int copies, int stride) {
    static_assert(kPer >= 1 && kPer * kMcGroup <= kMultiMax && kMcGroup == 4 && kMultiSamples == 8,
                  "copies per thread; quads; a byte of samples");
    unsigned held[kPer];  // bit q: copy c holds the current run's record at sample q
    int rot[kPer];        // copy c's bank-pair rotation
    bool valid[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int c = sub + kMcGroup * i;
        valid[i] = c < copies;
        rot[i] = valid[i] ? multi_rot(c, copies) : 0;
        held[i] = 0u;
    }
    for (int it = 0; it < 32; ++it) {
        const unsigned info = s_info[it * kMcProblems + prob];
        const int b0 = (int)(info & 31u);
        const unsigned lo = (info >> 5) & 0xffu, chg = (info >> 13) & 0xffu, hi = lo ^ 0xffu;
        const unsigned m_all = (hi | lo << 16) * 0x101u;  // the samples' planes at b (hi) and b - 1 (lo)
        const unsigned* pe = s_pe + b0 * kMcProblems + prob;
        unsigned v[kPer];
        unsigned best = 0xffffffffu;
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            held[i] &= ~chg;
            v[i] = pe[rot[i] * kMcProblems];
            const unsigned x = v[i] & m_all & ~__builtin_amdgcn_perm(0u, held[i], 0u);  // unheld samples only
            const unsigned cost = (unsigned)__builtin_popcount(held[i] ^ 0xffu) + 2u * (unsigned)__builtin_popcount(x);
            if (valid[i]) best = min(best, cost << 5 | (unsigned)(sub + kMcGroup * i));
        }
        // the quad's minimum (ties: the lowest copy)
        best = min(best, (unsigned)__builtin_amdgcn_update_dpp(0, (int)best, 0xb1, 0xf, 0xf, false));  // quad_perm 1,0,3,2
        best = min(best, (unsigned)__builtin_amdgcn_update_dpp(0, (int)best, 0x4e, 0xf, 0xf, false));  // quad_perm 2,3,0,1
        const int bc = (int)(best & 31u), ib = bc / kMcGroup;
        const bool own = bc % kMcGroup == sub;
        unsigned vb = v[0], hb = held[0];
        int rb = rot[0];
#pragma unroll
        for (int i = 1; i < kPer; ++i)
            if (i == ib) vb = v[i], hb = held[i], rb = rot[i];
#pragma unroll
        for (int i = 0; i < kPer; ++i)
            if (own && i == ib) held[i] = 0xffu;  // copy bc now holds the threshold's records
        if (own) {
            const unsigned mh = hi & ~hb, ml = lo & ~hb;
            const unsigned add_b = mh | (mh & vb) << 8;          // bank pair b*
            const unsigned add_m = ml | (ml & (vb >> 16)) << 8;  // bank pair b* - 1
            const int bs = (b0 + rb) & 31;
            const int bp = (bs + 1) & 31, bm = (bs + 31) & 31;
            atomicOr(&s_pe[bs * kMcProblems + prob], add_b | add_m << 16);
            atomicOr(&s_pe[(bs + 32) * kMcProblems + prob], add_b | add_m << 16);
            atomicOr(&s_pe[bp * kMcProblems + prob], add_b << 16);
            atomicOr(&s_pe[(bp + 32) * kMcProblems + prob], add_b << 16);
            atomicOr(&s_pe[bm * kMcProblems + prob], add_m);
            atomicOr(&s_pe[(bm + 32) * kMcProblems + prob], add_m);
            if (active && bc != 0)
                w0[(int64_t)(info >> 21) * lane_stride] = s_sw[it * kMcProblems + prob] - (float)(bc * stride + rb);
        }
        // the next threshold's reads of s_pe come after these updates (one wave: in order)
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
}

// Samples f_q < g of a threshold w = W + g (they read the record below -W).
__device__ inline unsigned multi_lo_mask(float w, float fl) {
    const int nlo = min(kMultiSamples, max(0, (int)ceilf((w - fl) * (float)kMultiSamples - 0.5f)));
    return (1u << nlo) - 1u;
}

// Block 0 records the launch's mode in the mode word: the number of copies, or 0 (the two-copy
// pass that follows then decides between one and two copies).
// (The backward's two-copy launch takes the same pass with dhalf > 0; after_rank > 0: the
// ranked backward's spread limit, and when its mode applies it keeps the word its pass wrote.)
__global__ __launch_bounds__(kMcThreads) void fwd_multi_assign_kernel(float2* __restrict__ wsT,
                                                          const float2* __restrict__ partials, int NP, int budget,
                                                          int max_copies, int* __restrict__ mode_word, int64_t Kp,
                                                          int64_t Op, int dhalf, int max_window, int wide_dhalf,
                                                          float after_rank) {
    if (after_rank > 0.0f && ranked_mode(partials, NP, after_rank, nullptr)) return;
    const MultiLayout ml =
        multi_layout(read_coord_range(partials), NP, budget, max_copies, dhalf, max_window, wide_dhalf);
    if (blockIdx.x == 0 && threadIdx.x == 0) *mode_word = multi_mode_word(ml.copies);
    if (ml.copies == 0) return;
    __shared__ float s_sw[32 * kMcProblems];       // [rank][problem]: the thresholds in order
    __shared__ unsigned s_info[32 * kMcProblems];  // [rank][problem] (multi_greedy)
    __shared__ unsigned s_pe[64 * kMcProblems];    // bit planes (multi_greedy)
    const int tid = threadIdx.x;
    for (int i = tid; i < 64 * kMcProblems; i += kMcThreads) s_pe[i] = 0u;
    const int prob = tid / kMcGroup, sub = tid % kMcGroup;
    constexpr int kGroups = 2;
    const int64_t n_ot = Op / (64 * kFwdORR);
    const int64_t p = (int64_t)blockIdx.x * kMcProblems + prob;
    const bool active = p < Kp * n_ot * kFwdORR * 2 * kGroups;
    const int sign = (int)(p & 1), group = (int)((p >> 1) % kGroups);
    const int64_t rest0 = (p >> 1) / kGroups;
    const int j = (int)(rest0 % kFwdORR);
    const int64_t rest = rest0 / kFwdORR;
    const int64_t tile = rest % n_ot, k = rest / n_ot;
    const int64_t lane_stride = 2 * kFwdORR;  // floats between consecutive lanes' records
    float* w0 = reinterpret_cast<float*>(wsT + k * Op + tile * 64 * kFwdORR + j) + sign + 32 * group * lane_stride;
    // sort keys: order-preserving integer images of the thresholds (NaN included) with the lane
    // in the low 5 bits, so that they are distinct (the order is then exact to 32 ulps)
    auto sort_key = [](float w, int l) {
        const int b = __float_as_int(w);
        return ((b ^ ((b >> 31) & 0x7fffffff)) & ~31) | l;
    };
    int key[32];
#pragma unroll
    for (int l = 0; l < 32; ++l) key[l] = sort_key(active ? w0[l * lane_stride] : 0.0f, l);
#pragma unroll
    for (int i = 0; i < 32 / kMcGroup; ++i) {  // this thread's lanes l = sub + kMcGroup * i
        const int l = sub + kMcGroup * i;
        const float wl = active ? w0[l * lane_stride] : 0.0f;
        const int kl = sort_key(wl, l);
        int rank = 0;
#pragma unroll
        for (int q = 0; q < 32; ++q) rank += key[q] < kl ? 1 : 0;
        s_sw[rank * kMcProblems + prob] = wl;
        s_info[rank * kMcProblems + prob] = (unsigned)l;
    }
    __syncthreads();
    // per rank: base bank pair, low samples and the samples whose record changes from the
    // previous rank's (a new run of equal records starts there)
#pragma unroll
    for (int i = 0; i < 32 / kMcGroup; ++i) {
        const int r = sub + kMcGroup * i;
        const float w = s_sw[r * kMcProblems + prob];
        const float fl = floorf(w);
        const int wi = (int)fl;
        const unsigned lo = multi_lo_mask(w, fl);
        unsigned chg = 0xffu;
        if (r > 0) {
            const float wp = s_sw[(r - 1) * kMcProblems + prob];
            const float flp = floorf(wp);
            const int wpi = (int)flp;
            const unsigned lop = multi_lo_mask(wp, flp);
            // record -W - [f_q < g] equals the previous one's where W + lo_q = W' + lo'_q
            if (wi == wpi) chg = lo ^ lop;
            else if (wi == wpi + 1) chg = 0xffu & ~(lop & ~lo);
        }
        const unsigned lane = s_info[r * kMcProblems + prob];
        s_info[r * kMcProblems + prob] = (unsigned)((-wi) & 31) | lo << 5 | chg << 13 | lane << 21;
    }
    __syncthreads();
    if (ml.copies > 16)
        multi_greedy<8>(s_sw, s_info, s_pe, prob, sub, active, w0, lane_stride, ml.copies, ml.stride);
    else if (ml.copies > 8)
        multi_greedy<4>(s_sw, s_info, s_pe, prob, sub, active, w0, lane_stride, ml.copies, ml.stride);
    else if (ml.copies > 4)
        multi_greedy<2>(s_sw, s_info, s_pe, prob, sub, active, w0, lane_stride, ml.copies, ml.stride);
    else
        multi_greedy<1>(s_sw, s_info, s_pe, prob, sub, active, w0, lane_stride, ml.copies, ml.stride);
}

// The window's records [lo, lo + n) into LDS as the layout's copies (record i of copy c at
// LDS record T_c + i, holding {A - T_c dT, dT}).
__device__ inline void stage_window_copies(float2* dst, const float2* __restrict__ src, int n, int copies,
                                           int stride) {
    const int total = n * copies;
    for (int q = threadIdx.x; q < total; q += blockDim.x) {
        const int c = q / n, i = q - c * n;
        const float2 r = src[i];
        const int t = multi_offset(c, copies, stride);
        dst[t + i] = make_float2(fmaf(-(float)t, r.y, r.x), r.y);
    }
}

// The whole table (float2 records) into LDS, two records per 16-byte load when n is even.
__device__ inline void stage_table2(float2* dst, const float2* __restrict__ src, int n) {
    if ((n & 1) == 0) {
        float4* d4 = reinterpret_cast<float4*>(dst);
        stage_to_lds<8>(reinterpret_cast<const float4*>(src), n / 2, [&](int i, float4 v) { d4[i] = v; });
    } else {
        stage_to_lds<8>(src, n, [&](int i, float2 v) { dst[i] = v; });
    }
}

// WIN: the range is read before the table load, and the launch holds only the coordinate
// window its coordinates reach: as windowed copies, two copies of tables whose two full copies
// do not fit, or one copy. Launches that cannot hold copies (calls below the copy threshold)
// take the variant without WIN, which loads the whole table first, unless built with
// ISA_EKV_FWD_SMALL_WIN=1 (configs[0]'s forward: 35.6 against 35.2 us per launch, so reading
// the range before a third of the table costs as much as the smaller load saves).
#ifndef ISA_EKV_FWD_SMALL_WIN
#define ISA_EKV_FWD_SMALL_WIN 0
#endif
template <int MR, bool SPLITS, bool WIN = false>
__global__ __launch_bounds__(2 * kFwdWaves * 64) void fwd_kernel(FwdArgs a) {
    extern __shared__ float2 s_lut_fwd[];
    const BlockClock clk(a.clock_acc);
    if constexpr (!WIN) stage_table2(s_lut_fwd, a.lut, a.NP);
    // fast loop and copy mode from one read of the range partials (as coords_in_padded_range,
    // fwd_copies_mode, launch_copy_mode and fwd_multi_layout decide them; a second read costs
    // the main loop ~50 VGPRs)
    const CoordRange cr = read_coord_range(a.partials);
    const bool fast = clamp_free(cr, a.NP);
    bool copies = fast && a.copy_offset > 0 &&
                  __builtin_amdgcn_readfirstlane((int)(cr.whi - cr.wlo >= kFwdCopyMinWindow)) != 0;
    int lo = 0, n_rec = a.NP;  // records held per copy: [lo, lo + n_rec)
    if constexpr (WIN) {
        const MultiLayout ml = fwd_multi_layout(cr, a.NP, a.mc_budget, a.mc_max);
        if (ml.copies > 0) {
            copies = false;
            lo = ml.lo;
            n_rec = ml.n;
            stage_window_copies(s_lut_fwd, a.lut + lo, n_rec, ml.copies, ml.stride);
        } else {
            if (copies && a.copy_window > 0) {
                coord_window(cr, a.NP, lo, n_rec);
                copies = n_rec <= a.copy_window;
                if (!copies) lo = 0, n_rec = a.NP;
            }
            if (!copies) {
                // one copy: of the coordinate window the launch reaches when no coordinate
                // needs the clamp (a third of the table for mapped inputs at the initial
                // thresholds), else of the whole table
                if (fast) coord_window(cr, a.NP, lo, n_rec);
                else lo = 0, n_rec = a.NP;
                stage_table2(s_lut_fwd, a.lut + lo, n_rec);
            }
        }
    }
    if (copies) {  // record i of copy 1 holds {A - T1 dT, dT}: fma(c + T1, dT, A') = fma(c, dT, A)
        const float t1 = (float)a.copy_offset;
        const int t1i = a.copy_offset;
        stage_to_lds<8>(a.lut + lo, n_rec, [&](int i, float2 r) {
            if constexpr (WIN) s_lut_fwd[i] = r;
            s_lut_fwd[t1i + i] = make_float2(fmaf(-t1, r.y, r.x), r.y);
        });
    }
    __syncthreads();
    FwdTile t;
    if (fwd_tile<SPLITS>(a, MR, t)) {
        // record i of the table at LDS record i - lo (lo > 0 only for clamp-free launches, whose
        // coordinates, and those of every copy, lie two or more records past lo)
        const float bias = rec_addr_bias(lo);
        if (fast)
            fwd_body<MR, kFwdORR, true>(a, LutFwdCell<false, true>{s_lut_fwd, a.cmin, a.cmax, bias}, a.xrec, a.wsT, t);
        else
            fwd_body<MR, kFwdORR, true>(a, LutFwdCell<true, true>{s_lut_fwd, a.cmin, a.cmax, bias}, a.xrec, a.wsT, t);
    }
    clk.stop();
}

// LUT forward with the table in global memory (tables past kMaxEntriesFwd; the reference's
// Triton forward reads its table from global memory at any size, ekv_lut_triton.py:33-64):
// the same tiling and cells, the gathers served by the L1/L2 caches.
template <int MR, bool SPLITS>
__global__ __launch_bounds__(kFwdWaves * 64) void fwd_global_kernel(FwdArgs a) {
    const bool fast = coords_in_padded_range(a.partials, a.NP);
    FwdTile t;
    if (!fwd_tile<SPLITS>(a, MR, t)) return;
    if (fast)
        fwd_body<MR, kFwdORR, true>(a, LutFwdCell<false>{a.lut, a.cmin, a.cmax}, a.xrec, a.wsT, t);
    else
        fwd_body<MR, kFwdORR, true>(a, LutFwdCell<true>{a.lut, a.cmin, a.cmax}, a.xrec, a.wsT, t);
}

// Exact-formula forward (reference: ekv_triton.py:69-91): same tiling, no table.
template <int MR, bool SPLITS>
__global__ __launch_bounds__(kFwdWaves * 64) void fwd_exact_kernel(FwdArgs a) {
    const bool fast = exact_operands_in_fast_range(a.partials);
    FwdTile t;
    if (!fwd_tile<SPLITS>(a, MR, t)) return;
    if (fast)
        fwd_body<MR, kFwdORR, false>(a, ExactFastFwdCell{a.k2}, a.xrec, a.wsT, t);
    else
        fwd_body<MR, kFwdORR, false>(a, ExactGeneralFwdCell{a.c2}, a.xrec_alt, a.wsT_alt, t);
}

// ----------------------------------------------------------------------------------
// Backward. Wave item = (output block ob of 64*ORR outputs, input block kb of KR inputs,
// token split sp). Each lane keeps dVth accumulators for its ORR x KR (o, k) pairs over
// the split's tokens; per token, the lane's partial dX over its outputs is summed across the
// wave (lane exchanges, or the LDS transpose buffer in the exact kernel), giving one dX
// partial per (ob, m, k).
// ----------------------------------------------------------------------------------

struct BwdArgs {
    const float4* xrec;     // [M][Kp] token records {t, r, -r / z_div, 0}
    const float2* wsT;      // [Kp][Op] threshold records
    const float4* xrec_alt; // exact: general-loop token records {tx, r, -r / z_div, 0}
    const float2* wsT_alt;  // exact: general-loop threshold records
    const float* grad;      // [M][ldg]
    const float4* lut;      // LUT: [NP] {A_I, dI, A_D, dD}
    const float2* partials;
    const int* copy_mode;   // kBwdOneCopy / kBwdTwoCopies launches: 1 when the copies are in use
    float* dx_part;         // [n_ob][M][K]            (need_x)
    float* dv_part;         // [S][2][Kp][Op]          (need_w)
    int M, K, O, Kp, Op, ldg, NP;
    int n_ob, n_kb, n_split, m_chunk;
    int n_items;
    int dv_group;           // 1: each group of kDvGroup consecutive items (token splits) is summed
                            // in its block, one dVth partial plane per group (see bwd_item)
    float cmin, cmax;
    float k2, c2;           // exact: 2^(-V_D a), V_D a
    int mc_budget, mc_max;  // split tables: the two-copy launch may hold up to mc_max windowed copies
    unsigned long long* clock_acc;  // profiling: {cycles, wall ticks, blocks} of this kernel (BlockClock), or null
    int xcd_order;          // ranked launch: 1 runs each token split's blocks on one XCD (xcd_work_index)
};

// LDS table views for the backward. Interleaved: one 16-byte record {A_I, dI, A_D, dD} per
// coordinate (one ds_read_b128). Split: the I halves in one array and the D halves
// kSplitRecords records further on, reached through the instruction's immediate offset
// (two ds_read_b64 from one address). Random 8-byte gathers cost fewer bank-conflict
// cycles per byte than 16-byte ones, and a dVth-only backward never reads the I halves.
struct BwdTableInterleaved {
    const float4* t;
    __device__ float4 operator[](unsigned i) const { return t[i]; }
};
template <int DOFF>
struct BwdTableSplitAt {  // D halves DOFF records after the I halves
    const float2* t;
    __device__ float4 operator[](unsigned i) const {
        const float2 ri = t[i];
        const float2 rd = t[i + DOFF];
        return make_float4(ri.x, ri.y, rd.x, rd.y);
    }
};
using BwdTableSplit = BwdTableSplitAt<kSplitRecords>;

// Cross-lane dX reduction without LDS (gfx950 lane exchanges): the wave's four per-lane
// partials v0..v3 (one per input of the wave) are summed over all 64 lanes so that every
// lane of 16-lane row r ends with the total of one input. permlane32_swap exchanges a
// register's upper half with another register's lower half, so adding the two results
// pairs lanes l and l+32 of one input; permlane16_swap does the same across adjacent
// 16-lane rows; four row rotations finish each row. The order of the additions is fixed,
// so the result is reproducible. wave_rows_input() gives, per lane, which input its row
// holds: the same exchanges applied to the labels 0..3 (both outputs of an exchange carry
// one label at every lane).
template <int N>
__device__ inline float dpp_row_rotate(float v) {  // row_ror:N within each 16-lane row
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x120 + N, 0xf, 0xf, false));
}

__device__ inline float wave_sum_rows4(float v0, float v1, float v2, float v3) {
    const auto p01 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v0), __float_as_uint(v1), false, false);
    const auto p23 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v2), __float_as_uint(v3), false, false);
    const float t01 = __uint_as_float(p01[0]) + __uint_as_float(p01[1]);
    const float t23 = __uint_as_float(p23[0]) + __uint_as_float(p23[1]);
    const auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(t01), __float_as_uint(t23), false, false);
    float u = __uint_as_float(q[0]) + __uint_as_float(q[1]);
    u += dpp_row_rotate<8>(u);
    u += dpp_row_rotate<4>(u);
    u += dpp_row_rotate<2>(u);
    u += dpp_row_rotate<1>(u);
    return u;
}

__device__ inline int wave_rows_input() {
    const auto p01 = __builtin_amdgcn_permlane32_swap(0u, 1u, false, false);
    const auto p23 = __builtin_amdgcn_permlane32_swap(2u, 3u, false, false);
    const auto q = __builtin_amdgcn_permlane16_swap(p01[0], p23[0], false, false);
    return (int)q[0];
}

// Two inputs per wave: after the half exchange each 32-lane half holds one input's
// pair sums; the row exchange of that register with itself folds rows 0+1 and 2+3.
__device__ inline float wave_sum_rows2(float v0, float v1) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v0), __float_as_uint(v1), false, false);
    const float t = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    const auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(t), __float_as_uint(t), false, false);
    float u = __uint_as_float(q[0]) + __uint_as_float(q[1]);
    u += dpp_row_rotate<8>(u);
    u += dpp_row_rotate<4>(u);
    u += dpp_row_rotate<2>(u);
    u += dpp_row_rotate<1>(u);
    return u;
}

__device__ inline int wave_rows_input2() {
    const auto p = __builtin_amdgcn_permlane32_swap(0u, 1u, false, false);
    const auto q = __builtin_amdgcn_permlane16_swap(p[0], p[0], false, false);
    return (int)q[0];
}

// Token splits summed per block in the grouped order (small plans, where the dVth partial
// planes would otherwise cost more traffic than the cells' reads).
constexpr int kDvGroup = 4;

struct BwdItem {
    int kb, ob, sp;  // input pair, output block, token split
};

// The work item's coordinates. Default order: inputs vary fastest, so the waves of a block
// share (output block, token split) and the G row slices they stream are fetched once into
// the CU's L1 and reused (blocks keep the hardware's round-robin XCD order: grouping one
// (output block, token split) on one XCD halves fc1's HBM reads of G but slows fc2 as much as
// it speeds fc1). Grouped order (dv_group): kDvGroup consecutive token splits first, so each
// group of kDvGroup waves shares (output block, inputs) and its dVth partials are summed in
// the block.
__device__ inline BwdItem bwd_item(const BwdArgs& a, int item) {
    BwdItem it;
    int rest;
    if (a.dv_group) {
        const int sp_lo = item % kDvGroup;
        rest = item / kDvGroup;
        it.kb = rest % a.n_kb;
        rest /= a.n_kb;
        it.ob = rest % a.n_ob;
        it.sp = (rest / a.n_ob) * kDvGroup + sp_lo;
    } else {
        it.kb = item % a.n_kb;
        rest = item / a.n_kb;
        it.ob = rest % a.n_ob;
        it.sp = rest / a.n_ob;
    }
    return it;
}

// LANE_RED: reduce each token's dX partials across the wave with lane exchanges
// (wave_sum_rows4) instead of the LDS transpose buffer (red unused), freeing LDS for
// tables too large to leave room for the buffers of 16 waves.
// DVG: the launch may run the grouped order (a.dv_group): dv_lds is then LDS of at least
// 2 * KR * ORR * 64 floats per wave that the block no longer reads (the table), and every wave
// of the block calls this with a valid item (the sum takes block barriers).
template <int KR, bool NEED_X, bool NEED_W, class Cell, bool LANE_RED = false, bool DVG = false>
__device__ inline void bwd_body(const BwdArgs& a, const Cell cell, const float4* xrec, const float2* wsT,
                                float* red, int item, float* dv_lds = nullptr) {
    constexpr int ORR = kBwdORR, MB = kRedSlots / KR;
    static_assert(!LANE_RED || KR == 4 || KR == 2, "the lane-exchange reduction sums two or four inputs per wave");
    const int lane = threadIdx.x & 63;
    const BwdItem it = bwd_item(a, item);
    const int kb = it.kb, ob = it.ob, sp = it.sp;
    const int o_lane = ob * 64 * ORR + lane * ORR;
    const int k0 = kb * KR;
    const int m_begin = sp * a.m_chunk;
    const int m_end = min(a.M, m_begin + a.m_chunk);

    float2 w[KR][ORR];
#pragma unroll
    for (int kk = 0; kk < KR; ++kk) {
        const float4* src = reinterpret_cast<const float4*>(wsT + (size_t)(k0 + kk) * a.Op + o_lane);
#pragma unroll
        for (int j = 0; j < ORR / 2; ++j) {
            const float4 v = src[j];
            w[kk][2 * j] = make_float2(v.x, v.y);
            w[kk][2 * j + 1] = make_float2(v.z, v.w);
        }
    }
    float accp[KR][ORR], accn[KR][ORR];
#pragma unroll
    for (int kk = 0; kk < KR; ++kk)
#pragma unroll
        for (int j = 0; j < ORR; ++j) accp[kk][j] = accn[kk][j] = 0.0f;

    // transpose-buffer reduction role of this lane: slot = lane / 4, quarter = lane % 4
    const int my_slot = lane >> 2;
    const int my_quarter = lane & 3;
    const int row_kk = !LANE_RED ? 0 : (KR == 4 ? wave_rows_input() : wave_rows_input2());  // input of this row's dX total

    // token m's operands are prefetched one step ahead (scalar token records, vector grads)
    const float4* xbase = xrec + k0;
    const float* gbase = a.grad + o_lane;
    float4 xn[KR];
    float gn[ORR];
    auto fetch = [&](int m) {
#pragma unroll
        for (int kk = 0; kk < KR; ++kk) xn[kk] = load_uniform4(xbase + (size_t)m * a.Kp + kk);
        if constexpr (ORR == 4) {
            const float4 g4 = *reinterpret_cast<const float4*>(gbase + (size_t)m * a.ldg);
            gn[0] = g4.x; gn[1] = g4.y; gn[2] = g4.z; gn[3] = g4.w;
        } else {
            const float2 g2 = *reinterpret_cast<const float2*>(gbase + (size_t)m * a.ldg);
            gn[0] = g2.x; gn[1] = g2.y;
        }
    };
    fetch(m_begin);

    for (int mb = m_begin; mb < m_end; mb += MB) {
#pragma unroll 1
        for (int s = 0; s < MB; ++s) {
            const int m = mb + s;
            float tv[KR];
            if (m < m_end) {
                float4 xcur[KR];
                float g[ORR];
#pragma unroll
                for (int kk = 0; kk < KR; ++kk) xcur[kk] = xn[kk];
#pragma unroll
                for (int j = 0; j < ORR; ++j) g[j] = gn[j];
                fetch(min(m + 1, m_end - 1));
#pragma unroll
                for (int kk = 0; kk < KR; ++kk) {
                    const float4 xv = xcur[kk];
                    float x1 = 0.0f, x2 = 0.0f;
#pragma unroll
                    for (int j = 0; j < ORR; ++j) {
                        const auto q = cell(xv.x, w[kk][j].x, w[kk][j].y);
                        const float dp = q.dp();
                        const float dn = q.dn();
                        const float gr = g[j] * xv.y;
                        if (NEED_X) {
                            const float lp = q.lp();
                            const float ln = q.ln();
                            x1 = fmaf(gr, dp - dn, x1);
                            x2 = fmaf(gr, lp - ln, x2);
                        }
                        if (NEED_W) {
                            accp[kk][j] = fmaf(gr, dp, accp[kk][j]);
                            accn[kk][j] = fmaf(gr, dn, accn[kk][j]);
                        }
                    }
                    tv[kk] = fmaf(x2, xv.z, x1);  // r*sum(G L_D) - r^2/V_sat*sum(G L_I), in d units
                    // at four inputs per wave keep one input's gathers in flight at a time (a
                    // scheduling fence: the measured-codebook dX runs 5% faster with it); at
                    // two the compiler's own schedule is as fast
                    if (ISA_EKV_BWD_SCHED || KR >= 4) __builtin_amdgcn_sched_barrier(0);
                }
            } else {
#pragma unroll
                for (int kk = 0; kk < KR; ++kk) tv[kk] = 0.0f;
            }
            if (NEED_X) {
                if constexpr (LANE_RED) {
                    if (m < m_end) {  // wave-uniform: every lane takes part in the exchanges
                        float sum;
                        if constexpr (KR == 4)
                            sum = wave_sum_rows4(tv[0], tv[1], tv[2], tv[3]);
                        else
                            sum = wave_sum_rows2(tv[0], tv[1]);
                        const int k = k0 + row_kk;
                        const bool writer = (lane & (KR == 4 ? 15 : 31)) == 0;  // one lane per input
                        if (writer && k < a.K) a.dx_part[((size_t)ob * a.M + m) * a.K + k] = sum;
                    }
                } else {
#pragma unroll
                    for (int kk = 0; kk < KR; ++kk) red[(s * KR + kk) * kRedStride + lane] = tv[kk];
                }
            }
        }
        if (NEED_X && !LANE_RED) {
            // all 64 lanes of this wave wrote MB*KR slots; LDS ops of one wave complete in
            // order, so only a compiler barrier is needed before reading other lanes' values
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            const float4* row = reinterpret_cast<const float4*>(red + my_slot * kRedStride + my_quarter * 16);
            float sum = 0.0f;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float4 v = row[q];
                sum += (v.x + v.y) + (v.z + v.w);
            }
            sum += __shfl_xor(sum, 1);
            sum += __shfl_xor(sum, 2);
            const int m = mb + my_slot / KR;
            const int k = k0 + my_slot % KR;
            if (my_quarter == 0 && m < m_end && k < a.K)
                a.dx_part[((size_t)ob * a.M + m) * a.K + k] = sum;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
    }
    if (NEED_W) {
        if constexpr (DVG) {
            if (a.dv_group) {  // block-uniform
                static_assert(ORR == 4, "one 16-byte slot per lane, input and sign");
                constexpr int kSlice = 2 * KR * 64;  // float4 slots per wave: [sign][input][lane]
                // 16 waves' slices reuse the split table's allocation (kSplitRecords 16-byte
                // records, the smallest a grouped plan launches with)
                static_assert(16 * kSlice * 16 <= kSplitRecords * 16, "grouped dVth sums exceed the table's LDS");
                __syncthreads();                     // no wave of the block reads the table any more
                float4* slots = reinterpret_cast<float4*>(dv_lds);
                float4* mine = slots + (threadIdx.x >> 6) * kSlice;
#pragma unroll
                for (int kk = 0; kk < KR; ++kk) {
                    mine[kk * 64 + lane] = make_float4(accp[kk][0], accp[kk][1], accp[kk][2], accp[kk][3]);
                    mine[(KR + kk) * 64 + lane] = make_float4(accn[kk][0], accn[kk][1], accn[kk][2], accn[kk][3]);
                }
                __syncthreads();
                // each group's kDvGroup slices summed in split order, one thread per float4 slot
                const int waves = blockDim.x >> 6;
                const int slots_out = (waves / kDvGroup) * kSlice;
                for (int t = threadIdx.x; t < slots_out; t += blockDim.x) {
                    const int g = t / kSlice, q = t - g * kSlice;
                    const float4* src = slots + g * kDvGroup * kSlice + q;
                    float4 sum = src[0];
#pragma unroll
                    for (int s2 = 1; s2 < kDvGroup; ++s2) {
                        const float4 v = src[s2 * kSlice];
                        sum.x += v.x; sum.y += v.y; sum.z += v.z; sum.w += v.w;
                    }
                    const BwdItem gi = bwd_item(a, (item - (item % waves)) + g * kDvGroup);
                    const int sign = q / (KR * 64), kk = (q / 64) % KR, ql = q % 64;
                    float* dst = a.dv_part + ((size_t)(gi.sp / kDvGroup) * 2 + sign) * a.Kp * a.Op +
                                 (size_t)(gi.kb * KR + kk) * a.Op + gi.ob * 64 * ORR + ql * ORR;
                    *reinterpret_cast<float4*>(dst) = sum;
                }
                return;
            }
        }
        float* dst_p = a.dv_part + (size_t)sp * 2 * a.Kp * a.Op;
        float* dst_n = dst_p + (size_t)a.Kp * a.Op;
#pragma unroll
        for (int kk = 0; kk < KR; ++kk) {
            float* pp = dst_p + (size_t)(k0 + kk) * a.Op + o_lane;
            float* pn = dst_n + (size_t)(k0 + kk) * a.Op + o_lane;
#pragma unroll
            for (int j = 0; j < ORR; ++j) {
                pp[j] = accp[kk][j];
                pn[j] = accn[kk][j];
            }
        }
    }
}

// Table-backward launch modes. kBwdAlone: the only launch. With the second table copy
// (split layout, see fwd_copies_mode) the host enqueues two launches of which the device
// picks one from the range partials: kBwdOneCopy (two 16-wave blocks per CU, exits in copy
// mode) and kBwdTwoCopies (both copies, 132 KB of LDS: one block per CU; exits otherwise).
// Copy 1 starts kBwdCopyOffset records after copy 0 (I half; its D half kSplitRecords
// further, as copy 0's), 16 bank pairs away.
constexpr int kBwdAlone = 0, kBwdOneCopy = 1, kBwdTwoCopies = 2;
#ifndef ISA_EKV_BWD_KR_TWO_COPIES
#define ISA_EKV_BWD_KR_TWO_COPIES 4
#endif
// one block per CU leaves the two-copy kernel the VGPRs for four inputs per wave (half the
// G traffic and lane exchanges per cell); its launch gets its own item count for them
constexpr int kBwdKRTwoCopies = ISA_EKV_BWD_KR_TWO_COPIES;
constexpr int kBwdCopyOffset = 2 * kSplitRecords + 16;
// interleaved 16-byte records (tables past kSplitRecords, their coordinate window held): copy 1
// 8 bank quads past copy 0's kSplitRecords records
constexpr int kBwdCopyOffsetI = kSplitRecords + 8;
constexpr size_t kBwdTwoCopiesLds = (size_t)(kBwdCopyOffset + 2 * kSplitRecords) * 8;
constexpr size_t kBwdTwoCopiesLdsI = (size_t)(kBwdCopyOffsetI + kSplitRecords) * 16;
// Windowed copies in the two-copy launch (split tables; mode word C >= kModeMultiMin, chosen
// by fwd_multi_assign_kernel with dhalf = kBwdWinDOffset): copy c holds the coordinate
// window's I records from LDS record T_c and their D records kBwdWinDOffset further (a
// multiple of 32 that is not one of 64, so the two reads stay two ds_read_b64 through the
// immediate offset), for windows of at most kBwdWinWindow records, in the whole LDS of the
// launch's one block per CU; wider windows (any of a split table's) take two copies with the
// D records kBwdWinWideDOffset on.
constexpr int kBwdWinWindow = 3008;
constexpr int kBwdWinDOffset = kBwdWinWindow + 32;
constexpr int kBwdWinWideDOffset = kSplitRecords;
constexpr int kBwdWinBudget = kLdsBytes / 8;  // records
static_assert(kBwdWinDOffset % 64 == 32 && kBwdWinWideDOffset % 64 == 32, "two ds_read_b64, not one read2st64");
static_assert(kBwdWinWideDOffset * 4 + 32 <= kBwdWinBudget, "two copies of a split table's window fit");
using BwdTableWin = BwdTableSplitAt<kBwdWinDOffset>;
using BwdTableWinWide = BwdTableSplitAt<kBwdWinWideDOffset>;

template <bool NEED_X, bool NEED_W, bool LANE_RED, int MODE, class Table, bool FAST_ONLY>
__device__ inline void bwd_table_items(const BwdArgs& a, const Table t, bool fast, float* red);

// The windowed copies of the two-copy launch (mode word C >= kModeMultiMin): the layout from
// the range partials as the assignment pass computed it, copy c's records {A - T_c dT, dT}.
template <bool NEED_X, bool NEED_W, class Table>
__device__ inline void bwd_windowed_items(const BwdArgs& a, const MultiLayout& ml, int dhalf) {
    extern __shared__ float4 s_lut_bwd[];
    float2* s_split = reinterpret_cast<float2*>(s_lut_bwd);
    const int n = ml.n, total = n * ml.copies;
    for (int q = threadIdx.x; q < total; q += blockDim.x) {
        const int c = q / n, i = q - c * n;
        const float4 r = a.lut[ml.lo + i];
        const int tc = multi_offset(c, ml.copies, ml.stride);
        const float ft = (float)tc;
        s_split[tc + i] = make_float2(fmaf(-ft, r.y, r.x), r.y);
        s_split[tc + dhalf + i] = make_float2(fmaf(-ft, r.w, r.z), r.w);
    }
    __syncthreads();
    bwd_table_items<NEED_X, NEED_W, true, kBwdTwoCopies, Table, true>(a, Table{s_split - ml.lo}, true, nullptr);
}

template <bool NEED_X, bool NEED_W>
__device__ inline void bwd_windowed_copies(const BwdArgs& a) {
    const MultiLayout ml = multi_layout(read_coord_range(a.partials), a.NP, a.mc_budget, a.mc_max, kBwdWinDOffset,
                                        kBwdWinWindow, kBwdWinWideDOffset);
    if (ml.copies == 0) return;  // (not reached: the pass records a count only when it fits)
    if (ml.dhalf == kBwdWinDOffset)
        bwd_windowed_items<NEED_X, NEED_W, BwdTableWin>(a, ml, kBwdWinDOffset);
    else
        bwd_windowed_items<NEED_X, NEED_W, BwdTableWinWide>(a, ml, kBwdWinWideDOffset);
}

// Returns whether this launch is the working one of its set (false: it exited on the mode word).
template <bool NEED_X, bool NEED_W, bool SPLIT, bool LANE_RED, int MODE>
__device__ inline bool bwd_table_body(const BwdArgs& a) {
    static_assert(kSplitRecords % 16 == 0 && kBwdCopyOffsetI % 16 == 8, "copy 1 eight bank quads away");
    extern __shared__ float4 s_lut_bwd[];
    float2* s_split = reinterpret_cast<float2*>(s_lut_bwd);
    // which launch of the set works: the branch-deal and copy assignment passes wrote the mode
    // word; the others exit before loading their table (the scalar load of the word costs no
    // VGPRs: the one-copy kernels keep their 64-VGPR budget)
    int lo = 0, n_rec = a.NP;  // table records held: [lo, lo + n_rec)
    if constexpr (MODE == kBwdTwoCopies) {
        const int mode = __builtin_amdgcn_readfirstlane(*a.copy_mode);
        if constexpr (SPLIT && LANE_RED)
            if (mode >= kModeMultiMin) {
                bwd_windowed_copies<NEED_X, NEED_W>(a);
                return true;
            }
        if (mode != 1) return false;
        // tables past kSplitRecords hold the window the launch's coordinates reach (the mode
        // word is set only when it fits)
        if (a.NP > kSplitRecords) {
            coord_window(read_coord_range(a.partials), a.NP, lo, n_rec);
            n_rec = min(n_rec, kSplitRecords);  // as the mode word's test: the window fits
        }
    }
    if constexpr (MODE == kBwdOneCopy)
        if (__builtin_amdgcn_readfirstlane(*a.copy_mode) != 0) return false;
    stage_to_lds<8>(a.lut + lo, n_rec, [&](int i, float4 rec) {
        if constexpr (SPLIT) {
            s_split[i] = make_float2(rec.x, rec.y);
            s_split[i + kSplitRecords] = make_float2(rec.z, rec.w);
            if constexpr (MODE == kBwdTwoCopies) {  // {A - T1 dT, dT} for both halves
                const float t1 = (float)kBwdCopyOffset;
                s_split[kBwdCopyOffset + i] = make_float2(fmaf(-t1, rec.y, rec.x), rec.y);
                s_split[kBwdCopyOffset + i + kSplitRecords] = make_float2(fmaf(-t1, rec.w, rec.z), rec.w);
            }
        } else {
            s_lut_bwd[i] = rec;
            if constexpr (MODE == kBwdTwoCopies) {
                const float t1 = (float)kBwdCopyOffsetI;
                s_lut_bwd[kBwdCopyOffsetI + i] =
                    make_float4(fmaf(-t1, rec.y, rec.x), rec.y, fmaf(-t1, rec.w, rec.z), rec.w);
            }
        }
    });
    __builtin_amdgcn_sched_barrier(0);  // the range loads after the table loads (VGPRs: one set live)
    const bool fast = coords_in_padded_range(a.partials, a.NP);
    __syncthreads();
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int table_records = SPLIT ? kSplitRecords : a.NP;
    float* red = LANE_RED ? nullptr
                          : reinterpret_cast<float*>(s_lut_bwd + table_records) + wave * (kRedSlots * kRedStride);
    using Table = typename std::conditional<SPLIT, BwdTableSplit, BwdTableInterleaved>::type;
    Table t;
    if constexpr (SPLIT)
        t = BwdTableSplit{s_split - lo};  // record i of the table at LDS record i - lo
    else
        t = BwdTableInterleaved{s_lut_bwd - lo};
    bwd_table_items<NEED_X, NEED_W, LANE_RED, MODE, Table, false>(a, t, fast, red);
    return true;
}

// The work items of a table-backward launch (the two-copy launch: persistent, one block per CU,
// each wave taking the plan's items in turn, so the launch costs little when it is not the
// working one and loads its tables once per CU when it is). FAST_ONLY: the clamp-free loop only.
template <bool NEED_X, bool NEED_W, bool LANE_RED, int MODE, class Table, bool FAST_ONLY>
__device__ inline void bwd_table_items(const BwdArgs& a, const Table t, bool fast, float* red) {
    const int waves = blockDim.x >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int stride = MODE == kBwdTwoCopies ? (int)gridDim.x : 0;
    constexpr int KRM = MODE == kBwdTwoCopies ? kBwdKRTwoCopies : kBwdKR;  // inputs per wave
    extern __shared__ float4 s_lut_bwd[];
    for (int vb = blockIdx.x;; vb += stride) {
        const int item = vb * waves + wave;
        if (item >= a.n_items) return;
        // the one-shot launch may sum its blocks' dVth partials in the table's LDS (dv_group)
        constexpr bool DVG = MODE == kBwdAlone;
        float* dv_lds = reinterpret_cast<float*>(s_lut_bwd);
        if (FAST_ONLY || fast)
            bwd_body<KRM, NEED_X, NEED_W, LutBwdCell<false, Table>, LANE_RED, DVG>(
                a, LutBwdCell<false, Table>{t, a.cmin, a.cmax}, a.xrec, a.wsT, red, item, dv_lds);
        else if constexpr (!FAST_ONLY)
            bwd_body<KRM, NEED_X, NEED_W, LutBwdCell<true, Table>, LANE_RED, DVG>(
                a, LutBwdCell<true, Table>{t, a.cmin, a.cmax}, a.xrec, a.wsT, red, item, dv_lds);
        if (MODE != kBwdTwoCopies) return;
    }
}

// The one-copy launches hold kBwdWavesPerEU waves per SIMD (two blocks per CU, 64 VGPRs); the
// two-copy launch runs one block per CU and may use the VGPRs of four waves per SIMD.
template <bool NEED_X, bool NEED_W, bool SPLIT, bool LANE_RED = false, int MODE = kBwdAlone>
__global__ __launch_bounds__(1024, kBwdWavesPerEU) void bwd_kernel(BwdArgs a) {
    static_assert(MODE != kBwdTwoCopies, "bwd_two_copies_kernel");
    const BlockClock clk(a.clock_acc);
    if (bwd_table_body<NEED_X, NEED_W, SPLIT, LANE_RED, MODE>(a)) clk.stop();  // (idle launches add nothing)
}

template <bool NEED_X, bool NEED_W, bool SPLIT>
__global__ __launch_bounds__(1024) void bwd_two_copies_kernel(BwdArgs a) {
    const BlockClock clk(a.clock_acc ? a.clock_acc + 3 : nullptr);  // the two-copy kind
    if (bwd_table_body<NEED_X, NEED_W, SPLIT, true, kBwdTwoCopies>(a)) clk.stop();
}

// ----------------------------------------------------------------------------------
// Ranked backward. A gather instruction's 32-lane halves conflict in the LDS banks when their
// records spread over more than 32 records, and with lanes along outputs they spread over the
// whole threshold window (69 records at the initial thresholds). The backward's sums do not
// care which lane evaluates which (output, sign) branch of an input: dVth± accumulates per
// branch over tokens, and dX sums every branch of an input per token. So per (input, block of
// 256 outputs) the branches are re-dealt by residue class. With kRankClasses = 16, class c
// (outputs c + 16 t, t < 16, each with its + and - threshold: 32 branches) goes to lanes c,
// c + 16, c + 32 and c + 48, ranked by threshold coordinate: ranks 0-15 to the first half-wave
// (even ranks to lane c, odd ranks to lane c + 16, rank 2 s + 1 in slot s), ranks 16-31 to
// the second. A gather instruction (one slot) then reads, across a half-wave, two adjacent
// ranks of 16 classes: at the initial thresholds' 69-record window, records inside a window of
// ~20 (the 32-class deal, one rank of 32 classes of 16 branches, spans ~30: measured 1.13
// instead of 1.95 ns per random gather per CU, 0.28 conflict cycles per LDS instruction).
// The cost is G: a branch's G[m][o] is no longer in its lane's registers. Each block (16
// waves, 16 consecutive inputs sharing the output block and token range) stages G for 8
// tokens at a time in LDS, as {G, -G} quads of 4 tokens per output (the sign of a - branch
// folds into its G), and a lane reads one 16-byte quad per slot and token group: lane c's
// quads sit in bank quad c mod 16, and a quarter-wave holds 16 different classes, so the reads
// are conflict-free. The staged G is read once per block, not once per wave.
// Each branch accumulates sign * sum_m G r L_D: dVth+ partials as the one-copy kernel (the same
// products in the same token order, so bitwise the same sums), dVth- partials negated back.
// ----------------------------------------------------------------------------------
constexpr int kRankWindow = 3008;   // table records each half of a ranked launch holds
#ifndef ISA_EKV_RANK_D_GAP
#define ISA_EKV_RANK_D_GAP 32
#endif
// the D halves start kRankDOffset records after the I halves: a multiple of 32 (both halves of
// a record in one bank pair, as the split tables) that is not one of 64, so the two reads stay
// two ds_read_b64 with an immediate offset rather than one ds_read2st64_b64
constexpr int kRankDOffset = kRankWindow + ISA_EKV_RANK_D_GAP;
constexpr int kRankChunk = 8;       // tokens per G staging round (two groups of four)
#ifndef ISA_EKV_RANK_WAVES
#define ISA_EKV_RANK_WAVES 16
#endif
// waves (inputs) per ranked block: two blocks per CU at 12 waves leave a wave ~80 VGPRs, room
// for several tokens' gathers in flight (at 16 waves, 64 VGPRs, one token's at a time)
constexpr int kRankWaves = ISA_EKV_RANK_WAVES;
static_assert(kRankWaves >= 8 && kRankWaves <= 16, "eight staging waves per ranked block");
constexpr int kRankGroupBytes = 2 * 256 * 16;                      // one token group: [sign][256] float4
constexpr unsigned kRankRingBase = (unsigned)(kRankDOffset + kRankWindow) * 8;  // G ring after the I and D halves
constexpr size_t kRankLds = (size_t)kRankRingBase + 4 * kRankGroupBytes;  // [buffer][group] x 8 KB
static_assert(2 * kRankLds <= (size_t)kLdsBytes, "two ranked blocks per CU");
static_assert((size_t)kRankDOffset * 8 < 65536 && 3 * kRankGroupBytes < 65536, "ds immediate offsets");

#ifndef ISA_EKV_RANK_CLASSES
#define ISA_EKV_RANK_CLASSES 16
#endif
// residue classes of a ranked deal (lane c's outputs are c + kRankClasses t): 16 or 32
constexpr int kRankClasses = ISA_EKV_RANK_CLASSES;
static_assert(kRankClasses == 16 || kRankClasses == 32, "a quarter-wave of distinct classes");
constexpr int kRankOut = 256 / kRankClasses;   // outputs per class in a block
constexpr int kRankBranches = 2 * kRankOut;    // branches per class
constexpr int kRankLanesHalf = 32 / kRankClasses;  // lanes of a class in each half-wave

struct RankArgs {
    const float2* wsT;    // [Kp][Op] threshold records {+, -}
    float* ws_ranked;     // [Kp][n_ob][64 lanes][8 slots] threshold coordinate of each slot's branch
    uint2* branch;        // [Kp][n_ob][64 lanes]: slot s in byte s: t (output c + kRankClasses t) | sign << 4
    const float2* partials;
    int* mode_word;
    int Kp, Op, n_ob, NP;
    float max_spread;     // the widest threshold spread (records) the ranked launch takes
    float greedy_min;     // spreads past this are dealt by bwd_deal_kernel, the rest by rank
};

#ifndef ISA_EKV_RANK_MERGE_MAX
#define ISA_EKV_RANK_MERGE_MAX 2  // most token splits the ranked launch merges per block
#endif

// Whether the ranked launch works (wave-uniform): the clamp-free loop, thresholds spread over at
// most max_spread records, and a coordinate window that fits the launch's table halves. *spread
// (nullable) receives the thresholds' spread in records.
__device__ inline bool ranked_mode(const float2* __restrict__ partials, int NP, float max_spread,
                                   float* spread = nullptr) {
    if (!coords_in_padded_range(partials, NP)) return false;
    const CoordRange c = read_coord_range(partials);
    if (spread) *spread = c.whi - c.wlo;
    if (!(c.whi - c.wlo <= max_spread)) return false;
    int lo, n;
    coord_window(c, NP, lo, n);
    return n <= kRankWindow;
}

// The branch deal, one thread per (input, output block, residue class): ranks by (coordinate,
// branch index), so ties keep a fixed order, and rank r goes to half-wave h = r / (B / 2)
// (B branches per class), lane c + kRankClasses (r' mod L) + 32 h and slot r' / L, where
// r' = r mod (B / 2) and L = the class's lanes per half-wave. Block 0 records the mode word.
// A block deals kRankQ (input, output block) pairs and writes their dealt thresholds from LDS
// as one contiguous run (each thread's own stores would land 32 bytes apart across a wave).
constexpr int kRankQ = 256 / kRankClasses;
__global__ __launch_bounds__(256) void bwd_rank_kernel(RankArgs a) {
    float spread = 0.0f;
    const bool on = ranked_mode(a.partials, a.NP, a.max_spread, &spread);  // block-uniform
    if (blockIdx.x == 0 && threadIdx.x == 0) *a.mode_word = on ? kModeRanked : 0;
    if (!on || spread > a.greedy_min) return;  // (wide spreads: bwd_deal_kernel deals)
    __shared__ float4 s_dealt[kRankQ * 64 * 2];  // per pair: 64 lanes x 8 slots
    const int64_t n_q = (int64_t)a.Kp * a.n_ob;
    const int64_t q0 = (int64_t)blockIdx.x * kRankQ;
    const int tq = threadIdx.x / kRankClasses, c = threadIdx.x % kRankClasses;
    const int64_t q = q0 + tq;  // k * n_ob + ob
    if (q < n_q) {
        const int ob = (int)(q % a.n_ob);
        const int64_t k = q / a.n_ob;
        const float2* src = a.wsT + k * a.Op + (int64_t)ob * 256 + c;
        float key[kRankBranches];  // branch i: output c + kRankClasses (i / 2), sign i % 2
#pragma unroll
        for (int t = 0; t < kRankOut; ++t) {
            const float2 w = src[kRankClasses * t];
            key[2 * t] = w.x;
            key[2 * t + 1] = w.y;
        }
        float* dst = reinterpret_cast<float*>(s_dealt) + tq * 64 * 8;
        unsigned codes[2 * kRankLanesHalf][2] = {};  // per lane of the class: slots 0-3, 4-7
#pragma unroll
        for (int i = 0; i < kRankBranches; ++i) {
            int rank = 0;
#pragma unroll
            for (int j = 0; j < kRankBranches; ++j) rank += (key[j] < key[i] || (key[j] == key[i] && j < i)) ? 1 : 0;
            const int h = rank / (kRankBranches / 2), r1 = rank % (kRankBranches / 2);
            const int li = r1 % kRankLanesHalf, slot = r1 / kRankLanesHalf;
            dst[(c + kRankClasses * li + 32 * h) * 8 + slot] = key[i];
            const unsigned code = (unsigned)((i >> 1) | ((i & 1) << 4)) << (8 * (slot & 3));
#pragma unroll
            for (int l = 0; l < 2 * kRankLanesHalf; ++l)
                if (l == h * kRankLanesHalf + li) {
                    if (slot < 4)
                        codes[l][0] |= code;
                    else
                        codes[l][1] |= code;
                }
        }
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int li = 0; li < kRankLanesHalf; ++li) {
                const int l = h * kRankLanesHalf + li;
                a.branch[q * 64 + c + kRankClasses * li + 32 * h] = make_uint2(codes[l][0], codes[l][1]);
            }
    }
    __syncthreads();
    const int n = (int)min<int64_t>(kRankQ, n_q - q0) * 64 * 2;
    float4* out = reinterpret_cast<float4*>(a.ws_ranked + q0 * 64 * 8);
    for (int i = threadIdx.x; i < n; i += 256) out[i] = s_dealt[i];
}

// ----------------------------------------------------------------------------------
// Greedy bank-aware deal (spreads past RankArgs::greedy_min records). Dealt by rank, a
// half-wave's 32 lanes read two adjacent ranks of 16 classes, which spread over a window that
// grows with the thresholds' spread (~0.09 of it per rank), so past ~100 records they collide
// in the LDS bank pairs (modelled 1.2 conflict cycles per gather at 135 records, the 8192-entry
// table's initial spread, and 4.5 at 1576, thresholds over [0, 5] V). Any deal within a class
// keeps the G reads conflict-free, so this one chooses, for each class in turn and each of its
// 32 branches in threshold order, the instruction (slot s and half-wave h: 16 per wave, each
// taking two branches of every class, lanes c + 16 i + 32 h) where it adds the fewest bank
// conflicts: the record a threshold w reads for a token at coordinate X + f is X + floor(f - w),
// so at kDealSamples token fractions f each instruction keeps, per bank pair, the number of
// distinct records (saturating at 3) and the first one's id; a record already there costs 0
// (a broadcast), a new bank pair 1, a bank pair holding n others 2 n + 1 (the growth of the
// squared load). Ties go to the lowest instruction. Modelled: 0.59 conflict cycles per gather
// at 135 records, 2.1 at 1576 (with four fractions 0.53 and 2.1); measured 0.49-0.53 at 135.
// The 512 choices of a problem are sequential: ~0.42 ms per GPT-L call (9216 problems, two per
// wave, ~33 instructions per placement), the chain of dependent steps with two waves per SIMD.
// ----------------------------------------------------------------------------------
constexpr int kDealWaves = 4;     // waves per block
constexpr int kDealPerWave = 2;   // (input, output block) problems per wave, one per 32-lane half
constexpr int kDealProblems = kDealWaves * kDealPerWave;  // per block
constexpr int kDealSamples = 2;   // token fractions each instruction's bank state is kept at
// bank-state column of one (instruction, fraction), in 16-bit entries: 32 bank pairs and two of
// padding, so that the 32 lanes of a half, each reading its own column, start 17 LDS banks apart
// (all distinct), and a problem's 32 columns (1088 entries) put the wave's second problem 32
// banks on (64-byte columns put every lane of a half on one of four banks)
constexpr int kDealCol = 34;
static_assert(kRankClasses == 16 && kRankBranches == 32, "16 classes of 32 branches in 16 instructions");
static_assert(16 * kDealSamples == 32, "a half-wave: 16 instructions x the fractions");

__device__ inline void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Two problems per wave, one per 32-lane half (a half past the last problem runs on zeros and
// writes nothing). While ranking, lane = class c x half p of its branches; then lane =
// instruction j x token fraction qs, owning that instruction's bank state at that fraction in
// LDS (per bank pair 16 bits: the distinct records there, 2 bits saturating at 3, and the first
// one's id), so only the cross-lane minima leave a lane. 7 KB per problem: two blocks per CU.
__global__ __launch_bounds__(kDealWaves * 64, 2) void bwd_deal_kernel(RankArgs a) {
    float spread = 0.0f;
    if (!ranked_mode(a.partials, a.NP, a.max_spread, &spread) || !(spread > a.greedy_min)) return;
    __shared__ __align__(16) float s_key[kDealProblems][16 * 32];  // [class][branch]; then the dealt [lane][slot]
    __shared__ __align__(16) float s_sorted[kDealProblems][16 * 32];  // [class][rank]
    __shared__ unsigned char s_code[kDealProblems][16 * 32];
    __shared__ __align__(16) unsigned short s_state[kDealProblems][16 * kDealSamples * kDealCol];  // [instruction][fraction][bank pair]
    __shared__ __align__(16) unsigned char s_bcode[kDealProblems][64 * 8];  // [lane][slot] branch codes
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int half = lane >> 5, hl = lane & 31;
    const int pi = wave * kDealPerWave + half;  // the half's problem slot in the block
    const int64_t n_q = (int64_t)a.Kp * a.n_ob;
    const int64_t q0 = ((int64_t)blockIdx.x * kDealWaves + wave) * kDealPerWave;
    if (q0 >= n_q) return;  // wave-uniform: the rest of the kernel syncs within the wave only
    const int64_t q = q0 + half;
    const bool live = q < n_q;  // uniform within the half

    // the class's 32 thresholds in (coordinate, branch) order: lane = class c x half p,
    // holding branches 16 p .. 16 p + 15 (branch i: output c + 16 (i / 2), sign i % 2)
    {
        const int c = hl & 15, p = hl >> 4;
        float key[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) key[u] = 0.0f;
        if (live) {
            const int ob = (int)(q % a.n_ob);
            const int64_t k = q / a.n_ob;
            const float2* src = a.wsT + k * a.Op + (int64_t)ob * 256 + c;
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const float2 w = src[16 * (8 * p + u)];
                key[2 * u] = w.x;
                key[2 * u + 1] = w.y;
            }
        }
        float* kc = &s_key[pi][c * 32];
#pragma unroll
        for (int u = 0; u < 16; ++u) kc[16 * p + u] = key[u];
        wave_lds_sync();
        int rank[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) rank[u] = 0;
        for (int jj = 0; jj < 32; ++jj) {
            const float kj = kc[jj];
#pragma unroll
            for (int u = 0; u < 16; ++u) rank[u] += (kj < key[u] || (kj == key[u] && jj < 16 * p + u)) ? 1 : 0;
        }
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int i = 16 * p + u;
            s_sorted[pi][c * 32 + rank[u]] = key[u];
            s_code[pi][c * 32 + rank[u]] = (unsigned char)((i >> 1) | ((i & 1) << 4));
        }
        unsigned* st32 = reinterpret_cast<unsigned*>(s_state[pi]);
        for (int u = hl; u < 16 * kDealSamples * kDealCol / 2; u += 32) st32[u] = 0u;
        wave_lds_sync();
    }

    // the greedy, one branch per step (class t / 32, rank t % 32). Each step reads the next
    // step's threshold and bank entry before it writes its own update, and patches the entry
    // when both steps touch the same one.
    const int j = hl >> 1, qs = hl & 1;  // this lane's instruction and token fraction
    const float frac = ((float)qs + 0.5f) / (float)kDealSamples;
    unsigned short* st = s_state[pi] + (j * kDealSamples + qs) * kDealCol;
    const float* srt = s_sorted[pi];
    float* s_out = s_key[pi];  // the keys are dead once sorted
    float w = srt[0];
    int rec = (int)floorf(frac - w);
    int b = rec & 31;
    unsigned e = st[b];
    int cap = 0;  // branches of the current class this lane's instruction holds
    for (int t = 0; t < 16 * 32; ++t) {
        const float wn = srt[min(t + 1, 16 * 32 - 1)];
        const int recn = (int)floorf(frac - wn);
        const int bn = recn & 31;
        unsigned en = st[bn];
        const unsigned n = e >> 14, id = e & 0x3FFFu, rid = (unsigned)rec & 0x3FFFu;
        int cost = n == 0u ? 1 : (id == rid ? 0 : 2 * (int)n + 1);
        cost += __builtin_amdgcn_update_dpp(0, cost, 0xb1, 0xf, 0xf, false);  // quad_perm 1,0,3,2: the pair
        // the cheapest instruction with room, ties to the lowest: min of cost x 16 + j over the
        // half (2 fractions x (2 x 3 + 1) bound a cost by 14; one instruction always has room):
        // a row's eight instructions by three row rotations, then the half's two rows by a
        // lane swap (rows 0-1 and 2-3: each half separately)
        int key = cap < 2 ? (cost << 4) | j : 0xFFFF;
        key = min(key, __builtin_amdgcn_update_dpp(0xFFFF, key, 0x122, 0xf, 0xf, false));  // row_ror:2
        key = min(key, __builtin_amdgcn_update_dpp(0xFFFF, key, 0x124, 0xf, 0xf, false));  // row_ror:4
        key = min(key, __builtin_amdgcn_update_dpp(0xFFFF, key, 0x128, 0xf, 0xf, false));  // row_ror:8
        const auto rw = __builtin_amdgcn_permlane16_swap((unsigned)key, (unsigned)key, false, false);
        const int jstar = min((int)rw[0], (int)rw[1]) & 15;
        if (j == jstar) {
            const unsigned eu = n == 0u ? ((1u << 14) | rid) : (id == rid ? e : ((min(n + 1u, 3u) << 14) | id));
            st[b] = (unsigned short)eu;
            if (bn == b) en = eu;  // the read above saw the entry before this write
            if (qs == 0) {
                const int c = t >> 5;
                const int L = c + 16 * cap + 32 * (jstar >> 3), slot = jstar & 7;
                s_out[L * 8 + slot] = w;
                s_bcode[pi][L * 8 + slot] = s_code[pi][t];
            }
            ++cap;
        }
        if ((t & 31) == 31) cap = 0;  // the next class
        w = wn;
        rec = recn;
        b = bn;
        e = en;
    }
    wave_lds_sync();
    if (live) {
        float4* out = reinterpret_cast<float4*>(a.ws_ranked + q * 64 * 8);
        const float4* so = reinterpret_cast<const float4*>(s_out);
        for (int i = hl; i < 64 * 8 / 4; i += 32) out[i] = so[i];
        for (int i = hl; i < 64; i += 32) a.branch[q * 64 + i] = *reinterpret_cast<const uint2*>(&s_bcode[pi][i * 8]);
    }
}

// Block = kRankWaves waves: inputs kg*W .. kg*W+W-1 (one per wave), one output block, one token split.
// Needs dX (the copies machinery's launches all do); NEED_W adds the dVth partials.
template <bool NEED_W>
__global__ __launch_bounds__(kRankWaves * 64, kRankWaves * 2 / 4) void bwd_ranked_kernel(BwdArgs a, const float* __restrict__ ws_ranked,
                                                                     const uint2* __restrict__ branch) {
    if (__builtin_amdgcn_readfirstlane(*a.copy_mode) != kModeRanked) return;
    const BlockClock clk(a.clock_acc ? a.clock_acc + 6 : nullptr);  // the ranked kind
    extern __shared__ float4 s_ranked[];
    char* smem = reinterpret_cast<char*>(s_ranked);
    float2* s_tab = reinterpret_cast<float2*>(smem);  // I halves [0, n), D halves [kRankDOffset, kRankDOffset + n)
    int lo, n;
    coord_window(read_coord_range(a.partials), a.NP, lo, n);
    stage_to_lds<8>(a.lut + lo, n, [&](int i, float4 rec) {
        s_tab[i] = make_float2(rec.x, rec.y);
        s_tab[kRankDOffset + i] = make_float2(rec.z, rec.w);
    });
    const float2* tab = s_tab - lo;  // record i of the table at LDS record i - lo
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n_kg = (a.Kp + kRankWaves - 1) / kRankWaves;
    int b = a.xcd_order ? xcd_work_index() : (int)blockIdx.x;
    const int kg = b % n_kg;
    b /= n_kg;
    const int ob = b % a.n_ob;
    const int sp = b / a.n_ob;
    const int k = kg * kRankWaves + wave;
    const bool active = k < a.Kp;  // wave-uniform; inactive waves still stage G and meet the barriers
    const int m_begin = sp * a.m_chunk;
    const int m_end = min(a.M, m_begin + a.m_chunk);
    const int c = lane % kRankClasses;  // the lane's residue class

    float ws[8];
    unsigned goff[8];  // byte address of each slot's G quad in ring buffer 0, group 0
    {
        uint2 pk = make_uint2(0u, 0u);
        float4 w0 = make_float4(0.f, 0.f, 0.f, 0.f), w1 = w0;
        if (active) {
            const size_t q = ((size_t)k * a.n_ob + ob) * 64 + lane;
            w0 = *reinterpret_cast<const float4*>(ws_ranked + q * 8);
            w1 = *reinterpret_cast<const float4*>(ws_ranked + q * 8 + 4);
            pk = branch[q];
        }
        ws[0] = w0.x; ws[1] = w0.y; ws[2] = w0.z; ws[3] = w0.w;
        ws[4] = w1.x; ws[5] = w1.y; ws[6] = w1.z; ws[7] = w1.w;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const unsigned code = ((s < 4 ? pk.x : pk.y) >> (8 * (s & 3))) & 0xffu;
            const unsigned t = code & 15u, sg = (code >> 4) & 1u;
            goff[s] = kRankRingBase + (sg * 256u + (unsigned)c + (unsigned)kRankClasses * t) * 16u;
        }
    }
    float acc[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) acc[s] = 0.0f;
    const int row_tok = wave_rows_input();  // which token of a group this lane's 16-lane row sums
    // this lane's dX partial for the first token of the split (written by one lane per row)
    float* const dxp = a.dx_part + ((size_t)ob * a.M + m_begin + row_tok) * a.K + k;

    // G staging by waves 0-7: each thread holds the quad (4 tokens) of one output and token
    // group; the wave decides the group, so each load's token row is wave-uniform and its buffer
    // descriptor (base at the row's output slice, 1 KB long, empty past the split's tokens,
    // whose loads then return 0) is formed in scalar registers
    const int so = tid & 255, stg = (wave >> 2) & 1;
    const bool stager = wave < 8;
    const unsigned gvoff = (unsigned)so * 4u;
    auto grow = [&](int m) {
        const float* base = a.grad + (size_t)m * a.ldg + (size_t)ob * 256;
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0, m < m_end ? 1024 : 0,
                                                 0x00027000);
    };
    auto gload = [&](int m0) {
        const int m = m0 + 4 * stg;
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)  // (the builtin returns the 32 loaded bits as an integer)
            v[j] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(grow(m + j), gvoff, 0, 0));
        return make_float4(v[0], v[1], v[2], v[3]);
    };
    auto gstore = [&](int buf, float4 v) {
        float4* d = reinterpret_cast<float4*>(smem + kRankRingBase + (size_t)(buf * 2 + stg) * kRankGroupBytes) + so;
        d[0] = v;
        d[256] = make_float4(-v.x, -v.y, -v.z, -v.w);  // the - half, 4 KB on
    };
    // one group of four tokens from ring buffer BUF, group TG
    auto group = [&](auto buf_c, auto tg_c, int mg) {
        constexpr int BUF = decltype(buf_c)::value, TG = decltype(tg_c)::value;
        float xs[4], rr[4], zz[4];
#pragma unroll
        for (int mm = 0; mm < 4; ++mm) {
            const int m = min(mg + mm, m_end - 1);
            const float4 xv = load_uniform4(a.xrec + (size_t)m * a.Kp + k);
            xs[mm] = xv.x;
            rr[mm] = xv.y;
            zz[mm] = xv.z;
        }
        // per token, r*sum(G L_D) - r^2/V_sat*sum(G L_I) as sum(G r (L_D + z L_I)), z = -r/V_sat
        float tv[4];
#pragma unroll
        for (int mm = 0; mm < 4; ++mm) tv[mm] = 0.0f;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            // the slot's reads: I and D records of four tokens, and their G quad
            float cc[4];
            float2 ei[4], ed[4];
#pragma unroll
            for (int mm = 0; mm < 4; ++mm) {
                cc[mm] = xs[mm] - ws[s];
                const unsigned i = (unsigned)cc[mm];
                ei[mm] = tab[i];
                ed[mm] = tab[i + kRankDOffset];
            }
            const float4 q = *reinterpret_cast<const float4*>(smem + goff[s] + (BUF * 2 + TG) * kRankGroupBytes);
            const float qv[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int mm = 0; mm < 4; ++mm) {
                const float li = fmaf(cc[mm], ei[mm].y, ei[mm].x);
                const float ld = fmaf(cc[mm], ed[mm].y, ed[mm].x);
                const float gr = qv[mm] * rr[mm];
                if (NEED_W) acc[s] = fmaf(gr, ld, acc[s]);
                tv[mm] = fmaf(gr, fmaf(zz[mm], li, ld), tv[mm]);
            }
            // the slot's dVth sum is formed here: left to itself the compiler sinks the chain
            // to the end of the group and keeps every (G r, L_D) pair live until then
            if (NEED_W) asm volatile("" : "+v"(acc[s]));
        }
        // summed over the wave (row r: token r)
        const float sum = wave_sum_rows4(tv[0], tv[1], tv[2], tv[3]);
        if ((lane & 15) == 0 && mg + row_tok < m_end && k < a.K) dxp[(size_t)(mg - m_begin) * a.K] = sum;
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;

    float4 gv = make_float4(0.f, 0.f, 0.f, 0.f);
    if (stager) gv = gload(m_begin);
    __syncthreads();  // the table halves are in place
    if (stager) gstore(0, gv);
    __syncthreads();
    // chunks alternate between the ring's two buffers; the next chunk's G loads are in flight
    // while this one is evaluated, and stored after it (one barrier per chunk)
    for (int m0 = m_begin; m0 < m_end; m0 += 2 * kRankChunk) {
        bool more = m0 + kRankChunk < m_end;
        if (more && stager) gv = gload(m0 + kRankChunk);
        if (active) {
            group(I0{}, I0{}, m0);
            group(I0{}, I1{}, m0 + 4);
        }
        if (more && stager) gstore(1, gv);
        __syncthreads();
        if (!more) break;
        const int m1 = m0 + kRankChunk;
        more = m1 + kRankChunk < m_end;
        if (more && stager) gv = gload(m1 + kRankChunk);
        if (active) {
            group(I1{}, I0{}, m1);
            group(I1{}, I1{}, m1 + 4);
        }
        if (more && stager) gstore(0, gv);
        __syncthreads();
        if (!more) break;
    }
    if (NEED_W && active) {
        const size_t q = ((size_t)k * a.n_ob + ob) * 64 + lane;
        const uint2 pk = branch[q];
        float* plane = a.dv_part + (size_t)sp * 2 * a.Kp * a.Op + (size_t)k * a.Op + (size_t)ob * 256 + c;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const unsigned code = ((s < 4 ? pk.x : pk.y) >> (8 * (s & 3))) & 0xffu;
            const unsigned t = code & 15u, sg = (code >> 4) & 1u;
            plane[(size_t)sg * a.Kp * a.Op + (unsigned)kRankClasses * t] = sg ? -acc[s] : acc[s];
        }
    }
    clk.stop();
}

// ----------------------------------------------------------------------------------
// Backward for tables past the one-table LDS limit, up to kMaxEntriesBwdHalf entries: two
// launches, each holding one 8-byte half of every record in LDS (131 KB at 16384 entries, one
// block per CU). The D pass gathers {A_D, dD} and forms dVth and dX's main term
// sum_o G r (L_D(d+) - L_D(d-)); the I pass gathers {A_I, dI} and forms dX's other term
// -r^2/V_sat sum_o G (L_I(d+) - L_I(d-)). Each writes its own plane of dX partials per output
// block, which dx_reduce_kernel sums with the others in plane order. The same tiling, prefetch
// and lane-exchange reduction as bwd_body with two inputs per wave.
// ----------------------------------------------------------------------------------

constexpr int kMaxEntriesBwdHalf = 16384;

template <int HALF, bool NEED_X, bool NEED_W, bool CLAMP>
__device__ inline void bwd_body_half(const BwdArgs& a, const float2* tab, int item) {
    constexpr int KR = kBwdKR, ORR = kBwdORR;
    static_assert(KR == 2, "the half-table passes reduce two inputs per wave");
    constexpr bool DVTH = HALF == 0 && NEED_W;
    const int lane = threadIdx.x & 63;
    const int kb = item % a.n_kb;
    const int rest = item / a.n_kb;
    const int ob = rest % a.n_ob;
    const int sp = rest / a.n_ob;
    const int o_lane = ob * 64 * ORR + lane * ORR;
    const int k0 = kb * KR;
    const int m_begin = sp * a.m_chunk;
    const int m_end = min(a.M, m_begin + a.m_chunk);

    float2 w[KR][ORR];
#pragma unroll
    for (int kk = 0; kk < KR; ++kk) {
        const float4* src = reinterpret_cast<const float4*>(a.wsT + (size_t)(k0 + kk) * a.Op + o_lane);
#pragma unroll
        for (int j = 0; j < ORR / 2; ++j) {
            const float4 v = src[j];
            w[kk][2 * j] = make_float2(v.x, v.y);
            w[kk][2 * j + 1] = make_float2(v.z, v.w);
        }
    }
    float accp[KR][ORR], accn[KR][ORR];
#pragma unroll
    for (int kk = 0; kk < KR; ++kk)
#pragma unroll
        for (int j = 0; j < ORR; ++j) accp[kk][j] = accn[kk][j] = 0.0f;
    const int row_kk = wave_rows_input2();  // input of this lane's row total
    const float4* xbase = a.xrec + k0;
    const float* gbase = a.grad + o_lane;
    float4 xn[KR];
    float gn[ORR];
    auto fetch = [&](int m) {
#pragma unroll
        for (int kk = 0; kk < KR; ++kk) xn[kk] = load_uniform4(xbase + (size_t)m * a.Kp + kk);
        const float4 g4 = *reinterpret_cast<const float4*>(gbase + (size_t)m * a.ldg);
        gn[0] = g4.x; gn[1] = g4.y; gn[2] = g4.z; gn[3] = g4.w;
    };
    fetch(m_begin);
    float* dx_plane = a.dx_part + (size_t)(HALF * a.n_ob + ob) * a.M * a.K;
#pragma unroll 1
    for (int m = m_begin; m < m_end; ++m) {
        float4 xcur[KR];
        float g[ORR];
#pragma unroll
        for (int kk = 0; kk < KR; ++kk) xcur[kk] = xn[kk];
#pragma unroll
        for (int j = 0; j < ORR; ++j) g[j] = gn[j];
        fetch(min(m + 1, m_end - 1));
        float tv[KR];
#pragma unroll
        for (int kk = 0; kk < KR; ++kk) {
            const float4 xv = xcur[kk];
            float x1 = 0.0f;
#pragma unroll
            for (int j = 0; j < ORR; ++j) {
                const float cp = coord<CLAMP>(xv.x, w[kk][j].x, a.cmin, a.cmax);
                const float cn = coord<CLAMP>(xv.x, w[kk][j].y, a.cmin, a.cmax);
                const float2 ep = tab[(unsigned)cp];
                const float2 en = tab[(unsigned)cn];
                const float vp = fmaf(cp, ep.y, ep.x), vn = fmaf(cn, en.y, en.x);
                const float gr = g[j] * xv.y;
                if (NEED_X) x1 = fmaf(gr, vp - vn, x1);
                if (DVTH) {
                    accp[kk][j] = fmaf(gr, vp, accp[kk][j]);
                    accn[kk][j] = fmaf(gr, vn, accn[kk][j]);
                }
            }
            tv[kk] = HALF == 0 ? x1 : x1 * xv.z;  // the I pass carries -r/V_sat
        }
        if (NEED_X) {
            const float sum = wave_sum_rows2(tv[0], tv[1]);
            const int k = k0 + row_kk;
            if ((lane & 31) == 0 && k < a.K) dx_plane[(size_t)m * a.K + k] = sum;
        }
    }
    if (DVTH) {
        float* dst_p = a.dv_part + (size_t)sp * 2 * a.Kp * a.Op;
        float* dst_n = dst_p + (size_t)a.Kp * a.Op;
#pragma unroll
        for (int kk = 0; kk < KR; ++kk) {
            float* pp = dst_p + (size_t)(k0 + kk) * a.Op + o_lane;
            float* pn = dst_n + (size_t)(k0 + kk) * a.Op + o_lane;
#pragma unroll
            for (int j = 0; j < ORR; ++j) {
                pp[j] = accp[kk][j];
                pn[j] = accn[kk][j];
            }
        }
    }
}

template <int HALF, bool NEED_X, bool NEED_W>
__global__ __launch_bounds__(1024) void bwd_half_kernel(BwdArgs a) {
    extern __shared__ float2 s_half[];
    stage_to_lds<8>(a.lut, a.NP, [&](int i, float4 rec) {
        s_half[i] = HALF == 0 ? make_float2(rec.z, rec.w) : make_float2(rec.x, rec.y);
    });
    __builtin_amdgcn_sched_barrier(0);
    const bool fast = coords_in_padded_range(a.partials, a.NP);
    __syncthreads();
    const int waves = blockDim.x >> 6;
    const int item = blockIdx.x * waves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (item >= a.n_items) return;
    if (fast)
        bwd_body_half<HALF, NEED_X, NEED_W, false>(a, s_half, item);
    else
        bwd_body_half<HALF, NEED_X, NEED_W, true>(a, s_half, item);
}

// LUT backward with the table in global memory (tables past kMaxEntriesBwdHalf: the reference's
// Triton backward, ekv_lut_triton.py:193-218, for CUDA_SHARED_BACKWARD off): interleaved
// records read through the caches, lane-exchange dX (no LDS: the dVth-only launch has no dX
// to reduce).
template <bool NEED_X, bool NEED_W>
__global__ __launch_bounds__(1024, ISA_EKV_BWD_MIN_BLOCKS) void bwd_global_kernel(BwdArgs a) {
    extern __shared__ float4 s_red_global[];
    constexpr bool LANE_RED = NEED_X;
    const bool fast = coords_in_padded_range(a.partials, a.NP);
    const int waves = blockDim.x >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    float* red = LANE_RED ? nullptr : reinterpret_cast<float*>(s_red_global) + wave * (kRedSlots * kRedStride);
    const int item = blockIdx.x * waves + wave;
    if (item >= a.n_items) return;
    const BwdTableInterleaved t{a.lut};
    if (fast)
        bwd_body<kBwdKR, NEED_X, NEED_W, LutBwdCell<false, BwdTableInterleaved>, LANE_RED>(
            a, LutBwdCell<false, BwdTableInterleaved>{t, a.cmin, a.cmax}, a.xrec, a.wsT, red, item);
    else
        bwd_body<kBwdKR, NEED_X, NEED_W, LutBwdCell<true, BwdTableInterleaved>, LANE_RED>(
            a, LutBwdCell<true, BwdTableInterleaved>{t, a.cmin, a.cmax}, a.xrec, a.wsT, red, item);
}

// Exact-formula backward (reference: ekv_triton.py:94-169): same work decomposition; LDS
// holds only the dX transpose buffers.
template <bool NEED_X, bool NEED_W>
__global__ __launch_bounds__(1024) void bwd_exact_kernel(BwdArgs a) {
    extern __shared__ float4 s_red_exact[];
    const bool fast = exact_operands_in_fast_range(a.partials);
    const int waves = blockDim.x >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    float* red = reinterpret_cast<float*>(s_red_exact) + wave * (kRedSlots * kRedStride);
    const int item = blockIdx.x * waves + wave;
    if (item >= a.n_items) return;
    if (fast)
        bwd_body<kBwdKRExact, NEED_X, NEED_W>(a, ExactFastBwdCell{a.k2}, a.xrec, a.wsT, red, item);
    else
        bwd_body<kBwdKRExact, NEED_X, NEED_W>(a, ExactGeneralBwdCell{a.c2}, a.xrec_alt, a.wsT_alt, red, item);
}

// ----------------------------------------------------------------------------------
// Measured-codebook projection (reference: measured_deployment/kernels/measured_lut_triton.py
// and the segmented path of measured_deployment/operator.py:164-224). Every physical cell
// (o, k) holds state ids a (positive) and b (negative) of a codebook of piecewise-linear
// measured I-V curves; for the clamped input v = clamp(x, lookup_min, lookup_max) in
// segment s,
//   out[m,o] = clamp(sum_k ((S[s][a] - S[s][b]) v + (C[s][a] - C[s][b])) * scale * r_tia, lo, hi)
// with S/C the segment slopes/intercepts; in pair mode the id names a precomputed
// difference curve and the b terms are absent. The table is laid out [segment][state]
// (float2 {S, C}) so the 64 lanes of one gather read one segment row; it is copied to LDS
// when it fits (the 24-state codebook: 60 x 24 x 8 B), else read from global memory. A
// zero record after the table serves padded inputs. The backward gives
//   dX[m,k] = [lookup_min <= x <= lookup_max] sum_o G'[m,o] (S[s][a] - S[s][b])
// with G' = G r_tia [lo <= out_pre <= hi] from glue_grad_kernel (no gradient for the
// fixed codebook, ids or r_tia, as the reference's detached buffers).
// ----------------------------------------------------------------------------------

constexpr size_t kMeasuredLdsBytes = 128 * 1024;

template <bool PAIR>
struct MeasuredFwdCell {
    const char* table;  // record byte offsets: segment row + state * 8
    // token record {segment row byte offset (bits), v}; id record {a * 8, b * 8} (bits)
    __device__ float accumulate(float acc, float2 xv, float2 w) const {
        const unsigned row = __float_as_uint(xv.x);
        const float2 ra = *reinterpret_cast<const float2*>(table + row + __float_as_uint(w.x));
        if (PAIR) return acc + fmaf(ra.x, xv.y, ra.y);
        const float2 rb = *reinterpret_cast<const float2*>(table + row + __float_as_uint(w.y));
        return acc + fmaf(ra.x - rb.x, xv.y, ra.y - rb.y);
    }
};

template <bool PAIR>
struct MeasuredBwdCell {
    const char* table;
    // dp - dn is the cell's slope difference; the current terms do not reach dX
    __device__ ValueBwdPair operator()(float row_bits, float wa, float wb) const {
        const unsigned row = __float_as_uint(row_bits);
        const float2 ra = *reinterpret_cast<const float2*>(table + row + __float_as_uint(wa));
        ValueBwdPair q{0.0f, ra.x, 0.0f, 0.0f};
        if (!PAIR) q.d_n = reinterpret_cast<const float2*>(table + row + __float_as_uint(wb))->x;
        return q;
    }
};

struct MeasuredPrepArgs {
    const float* x;          // [M][K]
    const short* ids_a;      // [O][K]
    const short* ids_b;      // [O][K] or null (pair mode)
    const float* slopes;     // [n_rows][n_seg]
    const float* intercepts; // [n_rows][n_seg]
    const float* vg;         // [n_seg + 1] (seg_mode 1)
    int64_t M, K, O, Kp, Op;
    int n_seg, n_rows;
    int seg_mode;            // 0 uniform floor, 1 searchsorted on vg, 2 rounded bins
    float voltage_min, inverse_step, lookup_min, lookup_max;
    int rec_floats;          // 2 (forward) or 4 (backward)
    float* xrec;             // [M][Kp][rec_floats]
    float2* idT;             // [Kp][Op]
    float2* table;           // [n_seg * n_rows + 1]
};

__device__ inline int measured_segment(const MeasuredPrepArgs& a, float v) {
    if (v != v) return a.seg_mode == 0 ? 0 : a.n_seg - 1;  // NaN: as float->int conversion / sorted last
    int s;
    if (a.seg_mode == 0) {
        s = (int)((v - a.voltage_min) * a.inverse_step);
    } else if (a.seg_mode == 1) {
        // searchsorted(vg, v, right=True) - 1: the number of grid points <= v, minus one
        int lo = 0, hi = a.n_seg + 1;
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (a.vg[mid] <= v)
                lo = mid + 1;
            else
                hi = mid;
        }
        s = lo - 1;
    } else {
        s = a.n_seg == 1 ? 0 : (int)rintf((v - a.lookup_min) * a.inverse_step);
    }
    return s < 0 ? 0 : (s > a.n_seg - 1 ? a.n_seg - 1 : s);
}

__global__ __launch_bounds__(256) void measured_prep_kernel(MeasuredPrepArgs a) {
    const int64_t zero_row = (int64_t)a.n_seg * a.n_rows * 8;  // byte offset of the zero record
    if (blockIdx.x < kPrepBlocksX) {
        for (int64_t m = blockIdx.x; m < a.M; m += kPrepBlocksX) {
            for (int k = threadIdx.x; k < (int)a.Kp; k += blockDim.x) {
                float v = 0.0f;
                unsigned row = (unsigned)zero_row;
                if (k < a.K) {
                    const float xv = a.x[m * a.K + k];
                    v = xv != xv ? xv : fminf(fmaxf(xv, a.lookup_min), a.lookup_max);
                    row = (unsigned)((int64_t)measured_segment(a, v) * a.n_rows * 8);
                }
                const int64_t e = m * a.Kp + k;
                if (a.rec_floats == 2)
                    reinterpret_cast<float2*>(a.xrec)[e] = make_float2(__uint_as_float(row), v);
                else
                    reinterpret_cast<float4*>(a.xrec)[e] = make_float4(__uint_as_float(row), 1.0f, 0.0f, v);
            }
        }
        return;
    }
    if (blockIdx.x < kPrepBlocksX + kPrepBlocksW) {
        // ids: 64(o) x 32(k) tiles transposed through LDS, ids clamped into the codebook
        __shared__ int2 tile[32][65];
        const int64_t n_ot = a.Op / 64, n_kt = (a.Kp + 31) / 32;
        const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
        for (int64_t t = blockIdx.x - kPrepBlocksX; t < n_ot * n_kt; t += kPrepBlocksW) {
            const int64_t ot = t % n_ot, kt = t / n_ot;
            for (int rr = ty; rr < 64; rr += 8) {
                int64_t o = ot * 64 + rr;
                const int64_t k = kt * 32 + tx;
                int2 v = make_int2(0, 0);  // padded inputs: state 0 on the zero record
                if (k < a.K && a.O > 0) {
                    if (o >= a.O) o = a.O - 1;  // padded outputs copy a real row; dropped
                    int ia = a.ids_a[o * a.K + k], ib = a.ids_b ? a.ids_b[o * a.K + k] : 0;
                    ia = ia < 0 ? 0 : (ia >= a.n_rows ? a.n_rows - 1 : ia);
                    ib = ib < 0 ? 0 : (ib >= a.n_rows ? a.n_rows - 1 : ib);
                    v = make_int2(ia * 8, ib * 8);
                }
                tile[tx][rr] = v;
            }
            __syncthreads();
            for (int rr = ty; rr < 32; rr += 8) {
                const int64_t k = kt * 32 + rr;
                if (k < a.Kp) {
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const int2 v = tile[rr][h * 32 + tx];
                        a.idT[k * a.Op + ot * 64 + h * 32 + tx] = make_float2(__int_as_float(v.x), __int_as_float(v.y));
                    }
                }
            }
            __syncthreads();
        }
        return;
    }
    // codebook records [segment][state] {slope, intercept} and the zero record
    const int64_t total = (int64_t)a.n_seg * a.n_rows;
    for (int64_t e = (int64_t)(blockIdx.x - kPrepBlocksX - kPrepBlocksW) * blockDim.x + threadIdx.x; e <= total;
         e += (int64_t)kPrepBlocksW * blockDim.x) {
        if (e == total) {
            a.table[e] = make_float2(0.0f, 0.0f);
        } else {
            const int64_t seg = e / a.n_rows, st = e - seg * a.n_rows;
            a.table[e] = make_float2(a.slopes[st * a.n_seg + seg], a.intercepts[st * a.n_seg + seg]);
        }
    }
}

template <int MR, bool PAIR, bool LDS>
__global__ __launch_bounds__(kFwdWaves * 64) void fwd_measured_kernel(FwdArgs a) {
    extern __shared__ float2 s_tab[];
    const float2* tab = reinterpret_cast<const float2*>(a.lut);
    if constexpr (LDS) {
        stage_to_lds<8>(tab, a.NP, [&](int i, float2 v) { s_tab[i] = v; });
        __syncthreads();
        tab = s_tab;
    }
    FwdTile t;
    if (!fwd_tile<false>(a, MR, t)) return;
    fwd_body<MR, kFwdORR, false>(a, MeasuredFwdCell<PAIR>{reinterpret_cast<const char*>(tab)}, a.xrec, a.wsT, t);
}

template <bool PAIR, bool LDS>
__global__ __launch_bounds__(1024) void bwd_measured_kernel(BwdArgs a) {
    extern __shared__ float4 s_mtab[];
    const float2* tab = reinterpret_cast<const float2*>(a.lut);
    if constexpr (LDS) {
        float2* s2 = reinterpret_cast<float2*>(s_mtab);
        stage_to_lds<8>(tab, a.NP, [&](int i, float2 v) { s2[i] = v; });
        __syncthreads();
        tab = s2;
    }
    const int waves = blockDim.x >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int item = blockIdx.x * waves + wave;
    if (item >= a.n_items) return;
    // dX partials reduced with lane exchanges: the LDS holds only the codebook
    bwd_body<kBwdKRExact, true, false, MeasuredBwdCell<PAIR>, true>(a, MeasuredBwdCell<PAIR>{reinterpret_cast<const char*>(tab)},
                                                       a.xrec, a.wsT, nullptr, item);
}

// dX[m,k] = scale * sum over output blocks, in block order (deterministic); scale is 1 for
// the LUT path and the derivative constant of the exact cells. With an input mapping
// v = clamp(x * s + b) in front of the layer (in_affine), dX is the gradient for v and the
// reduction applies the mapping's backward (cim.py:37-39 under autograd: mask where
// lo <= x*s + b <= hi, dx = mask * dv * s) and writes per-block partial sums of
// mask*dv*x (ds) and mask*dv (db) to aff_part[block] for the glue reduction.
// range_mask (no in_affine): dx = dv where lo <= x <= hi, else 0 (torch.clamp's backward of
// the measured path's input clamp).
constexpr int kDxReduceBlocks = 1024;  // blocks of a dX reduction, at most (aff_part entries)

struct DxReduceArgs {
    const float* part;  // [n_planes][n]
    int n_planes;
    int64_t n;          // M * K
    float scale;
    float* dx;
    const float* x;
    const float* in_affine;
    float in_lo, in_hi;
    float2* aff_part;   // [blocks] (in_affine)
    int range_mask;
};

// Block b of nb (grid-stride over the elements).
__device__ inline void dx_reduce_block(const DxReduceArgs& a, int b, int nb) {
    const float aff_s = a.in_affine ? a.in_affine[0] : 1.0f;
    const float aff_b = a.in_affine ? a.in_affine[1] : 0.0f;
    float ds = 0.0f, db = 0.0f;
    auto finish = [&](float s, float xv) {
        s *= a.scale;
        if (a.range_mask) {
            s = (xv >= a.in_lo && xv <= a.in_hi) ? s : 0.0f;
        } else if (a.in_affine) {
            const float pre = mapped_pre(xv, aff_s, aff_b);
            const float g = (pre >= a.in_lo && pre <= a.in_hi) ? s : 0.0f;
            ds = fmaf(g, xv, ds);
            db += g;
            s = g * aff_s;
        }
        return s;
    };
    const bool need_x = a.range_mask || a.in_affine;
    const int64_t n = a.n;
    const int64_t stride = (int64_t)nb * blockDim.x;
    const bool vec4 = (n & 3) == 0 && (((uintptr_t)a.part | (uintptr_t)a.dx) & 15) == 0 &&
                      (!need_x || ((uintptr_t)a.x & 15) == 0);
    if (vec4) {  // 16-byte vectors
        const int64_t n4 = n >> 2;
        const float4* p4 = reinterpret_cast<const float4*>(a.part);
        for (int64_t e = (int64_t)b * blockDim.x + threadIdx.x; e < n4; e += stride) {
            float4 s = p4[e];
            for (int q = 1; q < a.n_planes; ++q) {
                const float4 v = p4[(size_t)q * n4 + e];
                s.x += v.x;
                s.y += v.y;
                s.z += v.z;
                s.w += v.w;
            }
            const float4 xv = need_x ? reinterpret_cast<const float4*>(a.x)[e] : make_float4(0.f, 0.f, 0.f, 0.f);
            reinterpret_cast<float4*>(a.dx)[e] =
                make_float4(finish(s.x, xv.x), finish(s.y, xv.y), finish(s.z, xv.z), finish(s.w, xv.w));
        }
    } else {
        for (int64_t e = (int64_t)b * blockDim.x + threadIdx.x; e < n; e += stride) {
            float s = a.part[e];
            for (int q = 1; q < a.n_planes; ++q) s += a.part[(size_t)q * n + e];
            a.dx[e] = finish(s, need_x ? a.x[e] : 0.0f);
        }
    }
    if (a.in_affine) {
        __shared__ float s_ds[4], s_db[4];
        for (int off = 32; off > 0; off >>= 1) {
            ds += __shfl_xor(ds, off);
            db += __shfl_xor(db, off);
        }
        const int wave = threadIdx.x >> 6;
        if ((threadIdx.x & 63) == 0) {
            s_ds[wave] = ds;
            s_db[wave] = db;
        }
        __syncthreads();
        if (threadIdx.x == 0)
            a.aff_part[b] = make_float2((s_ds[0] + s_ds[1]) + (s_ds[2] + s_ds[3]),
                                        (s_db[0] + s_db[1]) + (s_db[2] + s_db[3]));
    }
}

// Blocks of a dX reduction over n elements: enough for one 16-byte vector per thread, at most
// kDxReduceBlocks.
int dx_reduce_blocks(int64_t n) {
    return (int)std::max<int64_t>(1, std::min<int64_t>(kDxReduceBlocks, ((n + 3) / 4 + 255) / 256));
}

__global__ __launch_bounds__(256) void dx_reduce_kernel(DxReduceArgs a) { dx_reduce_block(a, blockIdx.x, gridDim.x); }

// dVth+[o,k] = -scale * sum_s P[s][0][k][o], dVth-[o,k] = +scale * sum_s P[s][1][k][o]
// (splits summed in order s = 0, 1, ...). Tiles of 64 outputs x 8 inputs, one thread per
// (plane, input, 4 outputs): 16-byte loads along o, eight splits' loads in flight per
// thread, the tile transposed through LDS, stores along k.
struct DvReduceArgs {
    const float* part;  // [n_split][2][Kp][Op]
    int n_split, K, O, Kp, Op;
    float scale;
    float* dvp;
    float* dvn;
    // a table backward that may run ranked: its mode word, and the planes the ranked launch
    // writes (it merges token splits) when the word says it ran
    const int* mode_word;
    int ranked_planes;
};

constexpr int kDvTileK = 8;

int dv_reduce_tiles(int64_t K, int64_t O) { return (int)(((O + 63) / 64) * ((K + kDvTileK - 1) / kDvTileK)); }

__device__ inline void dv_reduce_block(const DvReduceArgs& a, int b, int nb) {
    __shared__ float tile[2][kDvTileK][65];
    const int n_ot = (a.O + 63) / 64, n_kt = (a.K + kDvTileK - 1) / kDvTileK;
    const int t = threadIdx.x;
    const int c4 = t & 15, row = (t >> 4) & (kDvTileK - 1), plane = t >> 7;  // loads
    const int kl = t & (kDvTileK - 1), orow = t >> 3;                          // stores: 8 x 32
    const size_t plane_floats = (size_t)a.Kp * a.Op;
    const float sg = plane == 0 ? -a.scale : a.scale;
    const int n_split =
        a.mode_word && __builtin_amdgcn_readfirstlane(*a.mode_word) == kModeRanked ? a.ranked_planes : a.n_split;
    for (int tile_id = b; tile_id < n_ot * n_kt; tile_id += nb) {
        const int ot = tile_id % n_ot, kt = tile_id / n_ot;
        const int k = kt * kDvTileK + row;
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
        if (k < a.K) {  // ot * 64 + 63 < Op: Op is O rounded up to 256
            const float4* src =
                reinterpret_cast<const float4*>(a.part + plane * plane_floats + (size_t)k * a.Op + ot * 64 + c4 * 4);
            const size_t split4 = 2 * plane_floats / 4;
#pragma unroll 8
            for (int sidx = 0; sidx < n_split; ++sidx) {
                const float4 v = src[(size_t)sidx * split4];
                acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
            }
        }
        float* tp = &tile[plane][row][c4 * 4];
        tp[0] = acc.x * sg; tp[1] = acc.y * sg; tp[2] = acc.z * sg; tp[3] = acc.w * sg;
        __syncthreads();
        for (int orr = orow; orr < 64; orr += 32) {
            const int o = ot * 64 + orr, kk = kt * kDvTileK + kl;
            if (o < a.O && kk < a.K) {
                a.dvp[(size_t)o * a.K + kk] = tile[0][kl][orr];
                a.dvn[(size_t)o * a.K + kk] = tile[1][kl][orr];
            }
        }
        __syncthreads();
    }
}

// ----------------------------------------------------------------------------------
// Layer glue backward (the reverse of layer_tia and layer_adc, cim.py:190-193 and :243 under
// autograd).
// For every (m, o) with G the gradient of the layer output:
//   gy = G * adc_scale[o]                        (G without an ADC affine)
//   y0 = idiff * r_tia, mask = lo <= y0 <= hi    (torch.clamp's backward mask)
//   G_eff[m, o] = mask * gy * r_tia               (the CIM backward's upstream gradient)
//   d r_tia   += mask * gy * idiff,   d adc_scale[o] += G * clamp(y0),   d adc_shift[o] += G
// A block owns a contiguous row range (one of kGlueBlocks) and 256 padded outputs (one of
// Op / 256): 4 row lanes x 64 output lanes, each thread 4 outputs 64 apart so every load
// instruction of a wave reads 64 consecutive floats. Per-block partials are combined in
// block order by the glue reduction, so every result is reproducible. G_eff is written
// [M][Op] with zeros in the padded outputs.
// ----------------------------------------------------------------------------------

constexpr int kGlueBlocks = 256;  // row ranges

struct GlueGradArgs {
    const float* g;          // [M][O]
    const float* idiff;      // [M][O]
    int64_t M, O, Op;
    const float* r_tia;      // the gain is tia_gain(r_tia, r_log_scale, r_log_lo, r_log_hi)
    const float* r_log_scale;
    float r_log_lo, r_log_hi;
    float y_lo, y_hi;
    const float* adc_scale;  // [O] or null
    float* geff;             // [M][Op]
    float* col_part;         // [kGlueBlocks][2][Op] (d adc_scale, d adc_shift)
    float* r_part;           // [kGlueBlocks * (Op / 256)]
};

// Glue block (row range rg, output block ob); n_gob = Op / 256 output blocks.
__device__ inline void glue_grad_block(const GlueGradArgs& a, int rg, int ob, int n_gob) {
    const bool has_r = a.r_tia != nullptr;
    const float r = has_r ? tia_gain(a.r_tia, a.r_log_scale, a.r_log_lo, a.r_log_hi) : 1.0f;
    const int lane_o = threadIdx.x & 63, row_lane = threadIdx.x >> 6;
    const int64_t rows = (a.M + kGlueBlocks - 1) / kGlueBlocks;
    const int64_t m_begin = (int64_t)rg * rows, m_end = m_begin + rows < a.M ? m_begin + rows : a.M;
    float da[4] = {0.0f, 0.0f, 0.0f, 0.0f}, dc[4] = {0.0f, 0.0f, 0.0f, 0.0f}, as[4];
    int64_t o[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        o[c] = (int64_t)ob * 256 + c * 64 + lane_o;
        as[c] = (a.adc_scale && o[c] < a.O) ? a.adc_scale[o[c]] : 1.0f;
    }
    float racc = 0.0f;
    for (int64_t m = m_begin + row_lane; m < m_end; m += 4) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            float ge = 0.0f;
            if (o[c] < a.O) {
                const float gz = a.g[m * a.O + o[c]];
                const float id = a.idiff[m * a.O + o[c]];
                const float y0 = id * r;
                const bool pass = !has_r || (y0 >= a.y_lo && y0 <= a.y_hi);
                if (a.adc_scale) {
                    const float y = !has_r ? id : (y0 != y0 ? y0 : fminf(fmaxf(y0, a.y_lo), a.y_hi));
                    da[c] = fmaf(gz, y, da[c]);
                    dc[c] += gz;
                }
                const float gy = a.adc_scale ? gz * as[c] : gz;
                const float gm = pass ? gy : 0.0f;
                racc = fmaf(gm, id, racc);
                ge = gm * r;
            }
            a.geff[m * a.Op + o[c]] = ge;
        }
    }
    __shared__ float s_da[4][256], s_dc[4][256], s_r[4];
    if (a.adc_scale) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            s_da[row_lane][c * 64 + lane_o] = da[c];
            s_dc[row_lane][c * 64 + lane_o] = dc[c];
        }
    }
    for (int off = 32; off > 0; off >>= 1) racc += __shfl_xor(racc, off);
    if (lane_o == 0) s_r[row_lane] = racc;
    __syncthreads();
    if (a.adc_scale) {
        const int t = threadIdx.x;  // one output of the block each
        const float sa = (s_da[0][t] + s_da[1][t]) + (s_da[2][t] + s_da[3][t]);
        const float sc = (s_dc[0][t] + s_dc[1][t]) + (s_dc[2][t] + s_dc[3][t]);
        const int64_t oo = (int64_t)ob * 256 + (t & 63) + (t >> 6) * 64;
        a.col_part[(size_t)rg * 2 * a.Op + oo] = sa;
        a.col_part[(size_t)rg * 2 * a.Op + a.Op + oo] = sc;
    }
    if (has_r && threadIdx.x == 0) a.r_part[(size_t)rg * n_gob + ob] = (s_r[0] + s_r[1]) + (s_r[2] + s_r[3]);
}

// Grid (kGlueBlocks, Op / 256).
__global__ __launch_bounds__(256) void glue_grad_kernel(GlueGradArgs a) {
    glue_grad_block(a, blockIdx.x, blockIdx.y, gridDim.y);
}

// The table backward's prep and the glue gradient pass in one launch (independent work:
// the prep reads x and the thresholds, the glue pass G and idiff): blocks
// [0, kPrepBlocksX + kPrepBlocksW) prep, then, when g.geff is set, kGlueBlocks x (Op / 256)
// glue blocks, row range fastest.
__global__ __launch_bounds__(256) void bwd_prep_kernel(PrepArgs a, GlueGradArgs g) {
    constexpr int kPrep = kPrepBlocksX + kPrepBlocksW;
    if (blockIdx.x < kPrep) {
        prep_block(a, blockIdx.x);
        return;
    }
    const int b = blockIdx.x - kPrep;
    glue_grad_block(g, b % kGlueBlocks, b / kGlueBlocks, (int)(g.Op / 256));
}

// Final sums of the glue partials in fixed order: d adc_scale/shift[o] over glue blocks,
// d r_tia over glue blocks and output blocks, d {scale, shift} of the input mapping over
// the dX reduction's blocks. Blocks: ceil(O / 64) column blocks (64 outputs x 4 quarters of
// the glue blocks each, quarters combined in LDS), then one block for the three scalars
// (strided partial sums per thread, then a tree in LDS).
struct GlueReduceArgs {
    const float* col_part;
    const float* r_part;
    const float2* aff_part;
    int n_aff;  // aff_part entries (the dX reduction's blocks)
    int64_t O, Op;
    float* d_adc_scale;
    float* d_adc_shift;
    float* d_r_tia;
    float* d_affine;
    // d r_log_scale = d r * r_tia[0] * exp(clamp(log_scale)) where lo <= log_scale <= hi, else
    // 0: autograd through cim.py:77 (mul, exp, clamp backward), op by op
    const float* r_tia;
    const float* r_log_scale;
    float r_log_lo, r_log_hi;
    float* d_r_log_scale;
};

int glue_reduce_blocks(int64_t O) { return (int)((O + 63) / 64 + 1); }

__device__ inline void glue_reduce_block(const GlueReduceArgs& a, int b) {
    __shared__ float red[3][256];
    const int t = threadIdx.x;
    const int64_t n_col_blocks = (a.O + 63) / 64;
    if ((int64_t)b < n_col_blocks) {
        if (!a.d_adc_scale && !a.d_adc_shift) return;
        const int64_t o = (int64_t)b * 64 + (t & 63);
        constexpr int kQuarter = kGlueBlocks / 4;
        const int b0 = (t >> 6) * kQuarter;
        float sa = 0.0f, sc = 0.0f;
        if (o < a.O) {
            for (int q = b0; q < b0 + kQuarter; ++q) {
                sa += a.col_part[(size_t)q * 2 * a.Op + o];
                sc += a.col_part[(size_t)q * 2 * a.Op + a.Op + o];
            }
        }
        red[0][t] = sa;
        red[1][t] = sc;
        __syncthreads();
        if (t < 64 && o < a.O) {
            if (a.d_adc_scale) a.d_adc_scale[o] = (red[0][t] + red[0][t + 64]) + (red[0][t + 128] + red[0][t + 192]);
            if (a.d_adc_shift) a.d_adc_shift[o] = (red[1][t] + red[1][t + 64]) + (red[1][t + 128] + red[1][t + 192]);
        }
        return;
    }
    const int n_rpart = kGlueBlocks * (int)(a.Op / 256);
    float sr = 0.0f, ss = 0.0f, sb = 0.0f;
    if (a.d_r_tia || a.d_r_log_scale)
        for (int q = t; q < n_rpart; q += 256) sr += a.r_part[q];
    if (a.d_affine)
        for (int q = t; q < a.n_aff; q += 256) {
            ss += a.aff_part[q].x;
            sb += a.aff_part[q].y;
        }
    red[0][t] = sr;
    red[1][t] = ss;
    red[2][t] = sb;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (t < w) {
            red[0][t] += red[0][t + w];
            red[1][t] += red[1][t + w];
            red[2][t] += red[2][t + w];
        }
        __syncthreads();
    }
    if (t == 0) {
        if (a.d_r_tia) a.d_r_tia[0] = red[0][0];
        if (a.d_r_log_scale) {
#pragma clang fp contract(off)
            const float ls = a.r_log_scale[0];
            const bool pass = ls >= a.r_log_lo && ls <= a.r_log_hi;  // torch.clamp's backward mask
            const float ge = red[0][0] * a.r_tia[0];                  // mul backward: d r * base
            a.d_r_log_scale[0] = pass ? ge * expf(ls) : 0.0f;          // exp backward: * exp(ls)
        }
        if (a.d_affine) {
            a.d_affine[0] = red[1][0];
            a.d_affine[1] = red[2][0];
        }
    }
}

__global__ __launch_bounds__(256) void glue_reduce_kernel(GlueReduceArgs a) { glue_reduce_block(a, blockIdx.x); }

// The backward's final reductions in one launch: dx_blocks dX blocks, then dv_blocks dVth
// blocks, then (gl_blocks > 0) the glue sums, which must not need the dX blocks' aff_part
// (no input mapping). A part with zero blocks is skipped.
__global__ __launch_bounds__(256) void grad_reduce_kernel(DxReduceArgs dx, int dx_blocks, DvReduceArgs dv,
                                                          int dv_blocks, GlueReduceArgs gl) {
    int b = blockIdx.x;
    if (b < dx_blocks) {
        dx_reduce_block(dx, b, dx_blocks);
        return;
    }
    b -= dx_blocks;
    if (b < dv_blocks) {
        dv_reduce_block(dv, b, dv_blocks);
        return;
    }
    glue_reduce_block(gl, b - dv_blocks);
}

// ----------------------------------------------------------------------------------
// LDS gather probe (measurement aid for the LDS roofline of the table kernels). Two
// 1024-thread blocks per CU each hold a 64 KB table; every lane issues gathers of REC-byte
// records (ds_read_b64 or ds_read_b128, the instructions the table kernels use) at 8 fixed
// indices drawn uniformly from [0, window) per lane, i.e. the pattern of one table gather
// whose lanes see thresholds spread over `window` records. Eight gathers are in flight per
// wave between waits; 32 waves per CU overlap them. The results are summed into out so the
// reads stay live. Indices are < window <= kProbeLdsBytes / REC, inside the table.
// ----------------------------------------------------------------------------------

typedef float probe_f2 __attribute__((ext_vector_type(2)));
typedef float probe_f4 __attribute__((ext_vector_type(4)));

// The table is dynamic LDS sized at launch (kProbeLdsBytes): a static array that only the
// inline-asm reads use would be removed by the compiler, leaving the reads outside the
// workgroup's allocation.
constexpr int kProbeLdsBytes = 65536;
constexpr int kProbeBlocksPerCU = 2;  // 32 waves per CU, as the table kernels run

template <int REC>
__global__ __launch_bounds__(1024) void lds_gather_probe_kernel(int window, int iters, unsigned seed, float* out,
                                                                 long long* clocks) {
    extern __shared__ float4 probe_table[];
    for (int i = threadIdx.x; i < kProbeLdsBytes / 16; i += blockDim.x)
        probe_table[i] = make_float4(i, 0.5f * i, 0.25f * i, 1.0f);
    __syncthreads();
    // shader-clock cycles (clock64) and constant-rate wall-clock ticks (wall_clock64) over this
    // wave's gather loop: their ratio is the sustained shader clock while the CU gathers
    const long long c0 = clocks ? clock64() : 0, w0 = clocks ? wall_clock64() : 0;
    unsigned h = (threadIdx.x + 1) * 2654435761u ^ seed ^ blockIdx.x * 40503u;
    unsigned addr[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        h ^= h << 13;
        h ^= h >> 17;
        h ^= h << 5;
        addr[i] = (h % (unsigned)window) * REC;
    }
    float acc = 0.0f;
    for (int it = 0; it < iters; ++it) {
        if constexpr (REC == 8) {
            probe_f2 v0, v1, v2, v3, v4, v5, v6, v7;
            asm volatile("ds_read_b64 %0, %1" : "=v"(v0) : "v"(addr[0]));
            asm volatile("ds_read_b64 %0, %1" : "=v"(v1) : "v"(addr[1]));
            asm volatile("ds_read_b64 %0, %1" : "=v"(v2) : "v"(addr[2]));
            asm volatile("ds_read_b64 %0, %1" : "=v"(v3) : "v"(addr[3]));
            asm volatile("ds_read_b64 %0, %1" : "=v"(v4) : "v"(addr[4]));
            asm volatile("ds_read_b64 %0, %1" : "=v"(v5) : "v"(addr[5]));
            asm volatile("ds_read_b64 %0, %1" : "=v"(v6) : "v"(addr[6]));
            asm volatile("ds_read_b64 %0, %1" : "=v"(v7) : "v"(addr[7]));
            asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(v0));
            asm volatile("" : "+v"(v1));
            asm volatile("" : "+v"(v2));
            asm volatile("" : "+v"(v3));
            asm volatile("" : "+v"(v4));
            asm volatile("" : "+v"(v5));
            asm volatile("" : "+v"(v6));
            asm volatile("" : "+v"(v7));
            acc += ((v0.x + v1.x) + (v2.x + v3.x)) + ((v4.x + v5.x) + (v6.x + v7.x));
        } else {
            probe_f4 v0, v1, v2, v3, v4, v5, v6, v7;
            asm volatile("ds_read_b128 %0, %1" : "=v"(v0) : "v"(addr[0]));
            asm volatile("ds_read_b128 %0, %1" : "=v"(v1) : "v"(addr[1]));
            asm volatile("ds_read_b128 %0, %1" : "=v"(v2) : "v"(addr[2]));
            asm volatile("ds_read_b128 %0, %1" : "=v"(v3) : "v"(addr[3]));
            asm volatile("ds_read_b128 %0, %1" : "=v"(v4) : "v"(addr[4]));
            asm volatile("ds_read_b128 %0, %1" : "=v"(v5) : "v"(addr[5]));
            asm volatile("ds_read_b128 %0, %1" : "=v"(v6) : "v"(addr[6]));
            asm volatile("ds_read_b128 %0, %1" : "=v"(v7) : "v"(addr[7]));
            asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(v0));
            asm volatile("" : "+v"(v1));
            asm volatile("" : "+v"(v2));
            asm volatile("" : "+v"(v3));
            asm volatile("" : "+v"(v4));
            asm volatile("" : "+v"(v5));
            asm volatile("" : "+v"(v6));
            asm volatile("" : "+v"(v7));
            acc += ((v0.x + v1.x) + (v2.x + v3.x)) + ((v4.x + v5.x) + (v6.x + v7.x));
        }
    }
    out[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = acc;
    if (clocks && threadIdx.x == 0) {
        const long long c1 = clock64(), w1 = wall_clock64();
        clocks[2 * blockIdx.x] = c1 - c0;
        clocks[2 * blockIdx.x + 1] = w1 - w0;
    }
}

// ----------------------------------------------------------------------------------
// VALU issue probe (isa_ekv_probe_valu_issue), a measurement aid: the table kernels' VALU
// instruction mixes replayed on registers only, no LDS or memory in the loop, at the
// kernels' occupancy, timed per block with clock64 (shader cycles) and wall_clock64. The
// wave-instructions a CU issues per cycle in this replay bound what the kernel itself can
// issue: its measured ceiling, which on gfx950 exceeds one instruction per CU-cycle (the
// second VALU pipe). Mixes, with the VALU wave-instructions of one loop iteration:
//   0  32 independent fma chains: the raw issue rate (32);
//   1  the ranked backward's branch-token body (bwd_ranked_kernel's group: per slot and token
//      coordinate, cvt, address, L_I and L_D, G r, the dVth and the two dX fmas), 8 slots x 4
//      tokens, token records by scalar loads, 16-wave blocks, two per CU (288);
//   2  the forward's cell (LutFwdCell on an LDS table: per branch coordinate, the float add and
//      the mask of its record address, interpolation; the difference and the accumulate),
//      8 tokens x 4 outputs, 8-wave blocks, two per CU (320);
//   3  mix 2 with the integer record address (v_cvt_u32_f32 and v_lshl_add_u32, as
//      table[(unsigned)c] compiles and the other LUT kernels issue), for comparison (320).
// The counts are the instructions the compiler emits for these loops (the replay's own
// SQ_INSTS_VALU agrees); the addresses are kept live by empty asm statements, not consumed.
// A CU's waves do not share its issue evenly (older waves go first, so some finish long before
// others), so the rate is a CU's: each block records the span to its last wave's end, its
// start and its CU, and the caller divides a CU's instructions by the interval its two blocks
// kept it busy.
// ----------------------------------------------------------------------------------

constexpr int kValuProbeTokens = 64;  // token records the replay cycles through (uniform loads)
constexpr int kValuMixInstr[4] = {32, 288, 320, 320};
constexpr int kValuMixWaves[4] = {16, 16, 8, 8};  // waves per block; two blocks per CU

__device__ inline void keep_live(unsigned v) { asm volatile("" ::"v"(v)); }

template <int MIX>
__global__ __launch_bounds__(1024, 8) void valu_probe_kernel(int iters, const float4* __restrict__ tok, float* out,
                                                            long long* clocks) {
    extern __shared__ float valu_probe_lds[];  // sized at launch to hold two blocks per CU; untouched
    (void)valu_probe_lds;
    const int lane = threadIdx.x & 63;
    const float lf = (float)lane;
    const long long c0 = clock64(), w0 = wall_clock64();
    float res = 0.0f;
    if constexpr (MIX == 0) {
        float acc[32];
#pragma unroll
        for (int j = 0; j < 32; ++j) acc[j] = lf + j;
        const float m = 0.999f + 1e-6f * lf, b = 1e-3f * lf;  // VGPR operands, as the kernels' fmas
        for (int it = 0; it < iters; ++it) {
#pragma unroll
            for (int j = 0; j < 32; ++j) acc[j] = fmaf(acc[j], m, b);
        }
#pragma unroll
        for (int j = 0; j < 32; ++j) res += acc[j];
    } else if constexpr (MIX == 1) {
        float ws[8], acc[8], q[8];
#pragma unroll
        for (int s2 = 0; s2 < 8; ++s2) {
            ws[s2] = 8.0f + 0.37f * s2 + 0.01f * lf;
            acc[s2] = 0.0f;
            q[s2] = 1.0f + 0.01f * (lf + s2);
        }
        // the records' intercepts and slopes (LDS reads in the kernel): VGPR operands
        const float t0 = 0.5f + 1e-3f * lf, t1 = 0.25f + 1e-7f * lf, t2 = 0.125f + 1e-3f * lf,
                    t3 = 0.0625f + 1e-7f * lf;
        const unsigned base = (unsigned)lane * 4u;
        float tvs = 0.0f;
        for (int it = 0; it < iters; ++it) {
            const int m0 = (it * 4) & (kValuProbeTokens - 1);
            float xs[4], rr[4], zz[4], tv[4];
#pragma unroll
            for (int mm = 0; mm < 4; ++mm) {
                const float4 xv = load_uniform4(tok + m0 + mm);
                xs[mm] = xv.x;
                rr[mm] = xv.y;
                zz[mm] = xv.z;
                tv[mm] = 0.0f;
            }
#pragma unroll
            for (int s2 = 0; s2 < 8; ++s2) {
#pragma unroll
                for (int mm = 0; mm < 4; ++mm) {
                    const float cc = xs[mm] - ws[s2];
                    const unsigned i = (unsigned)cc;
                    keep_live((i << 3) + base);
                    const float li = fmaf(cc, t1, t0);
                    const float ld = fmaf(cc, t3, t2);
                    const float gr = q[s2] * rr[mm];
                    acc[s2] = fmaf(gr, ld, acc[s2]);
                    tv[mm] = fmaf(gr, fmaf(zz[mm], li, ld), tv[mm]);
                }
                asm volatile("" : "+v"(acc[s2]));
            }
            // (the kernel sums tv across the wave here; the replay keeps one lane's sums live)
#pragma unroll
            for (int mm = 0; mm < 4; ++mm) asm volatile("" : "+v"(tv[mm]));
            tvs = tv[0];
        }
        res = tvs;
#pragma unroll
        for (int s2 = 0; s2 < 8; ++s2) res += acc[s2];
    } else {
        float wp[4], wn[4], acc[8][4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            wp[j] = 0.3f * j + 0.01f * lf;
            wn[j] = 0.2f * j + 0.02f * lf;
        }
#pragma unroll
        for (int mm = 0; mm < 8; ++mm)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[mm][j] = 0.0f;
        const float t0 = 0.5f + 1e-3f * lf, t1 = 0.25f + 1e-7f * lf;
        const float bias = rec_addr_bias((int)(lf * 0.0f));  // 0: a VGPR operand, as the kernel's
        const unsigned base = (unsigned)lane * 4u;
        for (int it = 0; it < iters; ++it) {
            const int m0 = (it * 8) & (kValuProbeTokens - 1);
#pragma unroll
            for (int mm = 0; mm < 8; ++mm) {
                const float4 xv = load_uniform4(tok + m0 + mm);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float cp = xv.x - wp[j], cn = xv.x - wn[j];
                    if constexpr (MIX == 2) {
                        keep_live(__float_as_uint(cp + bias) & kRecAddrMask);
                        keep_live(__float_as_uint(cn + bias) & kRecAddrMask);
                    } else {
                        keep_live(((unsigned)cp << 3) + base);
                        keep_live(((unsigned)cn << 3) + base);
                    }
                    acc[mm][j] = fmaf(fmaf(cp, t1, t0) - fmaf(cn, t1, t0), xv.y, acc[mm][j]);
                }
            }
#pragma unroll
            for (int mm = 0; mm < 8; ++mm)
#pragma unroll
                for (int j = 0; j < 4; ++j) asm volatile("" : "+v"(acc[mm][j]));
        }
#pragma unroll
        for (int mm = 0; mm < 8; ++mm)
#pragma unroll
            for (int j = 0; j < 4; ++j) res += acc[mm][j];
    }
    out[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = res;
    if (clocks) __syncthreads();  // the block's span ends with its last wave (the oldest wave ends first)
    if (clocks && threadIdx.x == 0) {
        const long long c1 = clock64(), w1 = wall_clock64();
        // the CU the block ran on: HW_ID's CU, shader array and engine fields (bits 8-14) and
        // the XCC (XCC_ID bits 0-3), read from the hardware registers
        const unsigned hw = __builtin_amdgcn_s_getreg((31 << 11) | (0 << 6) | 4);
        const unsigned xcc = __builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20);
        clocks[4 * blockIdx.x] = c1 - c0;
        clocks[4 * blockIdx.x + 1] = w1 - w0;
        clocks[4 * blockIdx.x + 2] = w0;
        clocks[4 * blockIdx.x + 3] = (long long)((xcc << 8) | ((hw >> 8) & 0x7Fu));
    }
}

// ----------------------------------------------------------------------------------
// Host-side planning shared by the workspace queries and the launches.
// ----------------------------------------------------------------------------------

struct FwdPlan {
    int64_t Kp, Op;
    int mr, n_mt, n_ot, blocks;
    int n_split, k_chunk;  // K split of small problems (n_split = 1: none)
    int wpb;               // waves per block
    size_t off_xrec, off_wsT, off_xrec_alt, off_wsT_alt, off_part, off_stat, off_mode, off_split, bytes;
};

#ifndef ISA_EKV_BWD_MIN_SPLIT_M
#define ISA_EKV_BWD_MIN_SPLIT_M 16
#endif
constexpr int64_t kBwdMinSplitTokens = ISA_EKV_BWD_MIN_SPLIT_M;  // tokens per backward token split, at least
#ifndef ISA_EKV_FWD_MIN_SPLIT_K
#define ISA_EKV_FWD_MIN_SPLIT_K 32
#endif
constexpr int kFwdMaxSplit = 8;
constexpr int kFwdMinSplitInputs = ISA_EKV_FWD_MIN_SPLIT_K;  // padded inputs per K split, at least
// Small-problem plans (too little work for the chip at any MR and K split of the usual plan)
// weigh a wave's work as its chunk (padded inputs, forward; tokens, backward) plus this much
// per-wave setup (threshold records, partial-plane stores, pipeline fill), in the same units.
#ifndef ISA_EKV_FWD_WAVE_COST
#define ISA_EKV_FWD_WAVE_COST 8
#endif
#ifndef ISA_EKV_FWD_INPUT_COST  // forward: per padded input of a wave, in token-input units
#define ISA_EKV_FWD_INPUT_COST 0
#endif
#ifndef ISA_EKV_FWD_SMALL_MR_MIN  // forward small plans: tokens per wave considered
#define ISA_EKV_FWD_SMALL_MR_MIN 2
#endif
#ifndef ISA_EKV_FWD_SMALL_MR_MAX
#define ISA_EKV_FWD_SMALL_MR_MAX 2
#endif
#ifndef ISA_EKV_BWD_ITEM_COST
#define ISA_EKV_BWD_ITEM_COST 2
#endif
#ifndef ISA_EKV_BWD_SMALL_ROUNDS  // backward plans by the cost model below this many possible rounds
#define ISA_EKV_BWD_SMALL_ROUNDS 8
#endif
constexpr int64_t kBwdSmallRounds = ISA_EKV_BWD_SMALL_ROUNDS;
// ... and a CU holding one block where it could hold two runs its waves at this percentage of
// the full rate (fewer waves to hide the LDS and memory latencies)
#ifndef ISA_EKV_LONE_BLOCK_RATE
#define ISA_EKV_LONE_BLOCK_RATE 70
#endif

// Relative duration of a launch of `blocks` equal blocks of `work` units each (at most one
// round), `resident` blocks fitting a CU: its busiest CU's work at that CU's rate.
int64_t small_launch_cost(int64_t blocks, int64_t work, int resident) {
    const int64_t per_cu = (blocks + kCUs - 1) / kCUs;
    if (per_cu == 1 && resident > 1) return work * 100 / ISA_EKV_LONE_BLOCK_RATE;
    return per_cu * work;
}

FwdPlan plan_forward(int64_t M, int64_t K, int64_t O, bool exact, bool allow_split = true, int wpb = kFwdWaves) {
    FwdPlan p{};
    p.wpb = wpb;
    p.Kp = round_up(K > 0 ? K : 1, 8);
    p.Op = round_up(O > 0 ? O : 1, 64 * kFwdORR);
    p.n_ot = (int)(p.Op / (64 * kFwdORR));
    // Tokens per wave and K split. Each wave streams its 256 outputs' threshold records once
    // per input for its MR tokens, so MR sets the threshold traffic per cell (8 / MR bytes
    // from L2); take the largest MR whose waves, times a K split, cover the chip
    // ISA_EKV_FWD_WT times over (MR = 2 and the largest split when none does). Each K split
    // sums k_chunk padded inputs into its own partial plane, finished by split_reduce_kernel.
    const int64_t waves_target = (int64_t)ISA_EKV_FWD_WT * 256 * 16;
    int sp_max = 1;
    while (allow_split && sp_max < kFwdMaxSplit && p.Kp / (2 * sp_max) >= kFwdMinSplitInputs) sp_max *= 2;
    int split = 1;
    bool small = false;
    for (p.mr = 8;; p.mr /= 2) {
        const int64_t waves = round_up(M, (int64_t)wpb * p.mr) / p.mr * p.n_ot;
        if (p.mr == 2 || waves * sp_max >= waves_target) {
            small = waves * sp_max < waves_target;
            while (split < sp_max && waves * split < waves_target) split *= 2;
            break;
        }
    }
    const int64_t tokens_per_block = (int64_t)wpb * p.mr;
    p.n_mt = (int)((M + tokens_per_block - 1) / tokens_per_block);
    if (small && allow_split) {
        // Too few waves to cover the chip even at the largest split: one round of blocks at
        // most, and the launch lasts as long as its busiest CU. Take the tokens per wave and
        // split count (any count up to kFwdMaxSplit whose chunks hold at least 8 padded
        // inputs) that minimise small_launch_cost of blocks of waves costing MR x (chunk +
        // per-wave setup) + chunk x the per-input threshold-record cost; ties go to fewer
        // tokens per wave, then fewer splits.
        int64_t best_cost = -1;
        for (int mr = ISA_EKV_FWD_SMALL_MR_MIN; mr <= ISA_EKV_FWD_SMALL_MR_MAX; mr *= 2) {
            const int64_t n_mt = (M + (int64_t)wpb * mr - 1) / ((int64_t)wpb * mr);
            const int64_t tiles = n_mt * p.n_ot;
            for (int sp = 1; sp <= kFwdMaxSplit; ++sp) {
                const int64_t chunk = round_up((p.Kp + sp - 1) / sp, 8);
                const int64_t n_sp = (p.Kp + chunk - 1) / chunk;
                if (n_sp != sp) continue;  // the same plan as a smaller count
                const int64_t work = 100 * (mr * (chunk + ISA_EKV_FWD_WAVE_COST) + ISA_EKV_FWD_INPUT_COST * chunk);
                const int64_t cost = small_launch_cost(tiles * n_sp, work, wpb == kFwdWaves ? 2 : 1);
                if (best_cost < 0 || cost < best_cost) {
                    best_cost = cost;
                    split = sp;
                    p.mr = mr;
                    p.n_mt = (int)n_mt;
                }
            }
        }
    }
    p.k_chunk = (int)round_up((p.Kp + split - 1) / split, 8);
    p.n_split = (int)((p.Kp + p.k_chunk - 1) / p.k_chunk);
    p.blocks = p.n_mt * p.n_ot * p.n_split;
    const size_t xrec_bytes = (size_t)round_up((int64_t)M * p.Kp * 8, 256);
    const size_t wsT_bytes = (size_t)round_up(p.Kp * p.Op * 8, 256);
    size_t off = 0;
    p.off_xrec = off;
    off += xrec_bytes;
    p.off_wsT = off;
    off += wsT_bytes;
    p.off_xrec_alt = off;
    if (exact) off += xrec_bytes;
    p.off_wsT_alt = off;
    if (exact) off += wsT_bytes;
    p.off_part = off;
    off += (size_t)round_up((kPrepBlocksX + kPrepBlocksW) * 8, 256);
    p.off_stat = off;
    off += 256;
    p.off_mode = off;  // the table-copy mode word
    off += 256;
    p.off_split = off;
    if (p.n_split > 1) off += (size_t)round_up((int64_t)p.n_split * M * O * 4, 256);
    p.bytes = round_up((int64_t)off, 256);
    return p;
}

struct BwdPlan {
    int64_t Kp, Op;
    int n_ob, n_kb, n_split, m_chunk, n_items, waves_per_block, blocks;
    int dv_planes;  // dVth partial planes: n_split, or n_split / kDvGroup with dv_group
    bool dv_group;
    bool grad_padded, split, lane_red, gtab, halves;
    bool copies;  // at least ISA_EKV_OPT_COPY_MIN_CELLS cells: the second table copy may pay
    bool ranked;  // the copies' launches may include the ranked backward (its branch-deal arrays)
    int mc_max;   // split tables with the copies' launches: most windowed copies of the two-copy launch (0: none)
    size_t off_xrec, off_wsT, off_xrec_alt, off_wsT_alt, off_part, off_mode, off_gpad, off_dx, off_dv, off_glue,
        off_rank_ws, off_rank_branch, bytes, lds_bytes;
    int rank_merge;  // ranked launch: token splits summed per block
};

bool bwd_may_use_copies(const BwdPlan& p, bool exact, bool need_x);

// n_entries = 0 plans the exact-formula backward (no LDS table, general-loop records).
// glue: the layer backward (G_eff always written [M][Op], plus the glue partial sums).
BwdPlan plan_backward(int64_t M, int64_t K, int64_t O, int n_entries, bool need_x, bool need_w,
                      bool glue = false) {
    BwdPlan p{};
    const bool exact = n_entries == 0;
    p.Kp = round_up(K > 0 ? K : 1, 8);
    p.Op = round_up(O > 0 ? O : 1, 64 * kBwdORR);
    p.n_ob = (int)(p.Op / (64 * kBwdORR));
    // inputs per wave: the table kernels take kBwdKR, the exact and measured kernels (planned
    // with n_entries = 0) kBwdKRExact
    const int kr = exact ? kBwdKRExact : kBwdKR;
    const int mb = kRedSlots / kr;  // tokens per dX batch
    p.n_kb = (int)(p.Kp / kr);
    const size_t red_bytes = (size_t)kRedSlots * kRedStride * 4;
    p.gtab = !exact && n_entries > kMaxEntriesBwdHalf;  // table read from global memory
    // past the one-table limit: a D pass and an I pass, each with one record half in LDS
    p.halves = !exact && !p.gtab && n_entries > kMaxEntriesBwd;
    p.split = !exact && !p.gtab && !p.halves && ISA_EKV_BWD_SPLIT && lut_records(n_entries) <= kSplitRecords;
    const size_t lut_bytes = exact || p.gtab ? 0
                             : p.halves     ? (size_t)lut_records(n_entries) * 8
                                            : (size_t)(p.split ? kSplitRecords : lut_records(n_entries)) * 16;
    // dX reduction across the wave: lane exchanges (no LDS; measured 5% faster at N = 4096
    // and, with the 8192-entry table, the only way to keep 16 waves per block), or the LDS
    // transpose buffers
    p.lane_red = !exact && need_x &&
                 (p.gtab || p.halves || ISA_EKV_BWD_LANE_RED == 1 ||
                  (ISA_EKV_BWD_LANE_RED == 2 && lut_bytes + 16 * red_bytes > (size_t)kLdsBytes));
    // (a dVth-only launch has no dX to reduce: no buffers, so every gradient subset gets the
    // same blocks and token splits, and the same dVth sums)
    const size_t per_wave = p.lane_red || !need_x ? 0 : red_bytes;
    int wpb = 16;
    while (wpb > 1 && lut_bytes + wpb * per_wave > (size_t)kLdsBytes) wpb /= 2;
    p.waves_per_block = wpb;
    p.lds_bytes = lut_bytes + (size_t)wpb * per_wave;
    // Token splits. One block runs per CU at a time (the LDS table), and blocks of equal
    // work finish together, so the launch takes ceil(blocks / CUs) rounds. Among the split
    // counts from ~2 rounds up, take the smallest whose block count fills its rounds to
    // within 0.5% of the best fill (each split adds a dVth partial plane and per-item
    // setup, measured at well under the 1.6% a 98.4%-filled last round costs).
    // blocks resident per CU: the table kernels fit ISA_EKV_BWD_MIN_BLOCKS 16-wave blocks in
    // their VGPR budget when the LDS holds that many tables; the exact kernels fit one
    const int64_t resident =
        exact ? 1
              : std::max<int64_t>(1, std::min<int64_t>(ISA_EKV_BWD_MIN_BLOCKS,
                                                       (int64_t)(kLdsBytes / std::max<size_t>(p.lds_bytes, 1))));
    const int64_t base_items = (int64_t)p.n_ob * p.n_kb;
    const int64_t max_splits = std::max<int64_t>(1, (M + kBwdMinSplitTokens - 1) / kBwdMinSplitTokens);
    const int64_t min_splits =
        std::min<int64_t>(max_splits, (2 * kCUs * resident * wpb + base_items - 1) / base_items);
    const int64_t top_splits = std::min<int64_t>(max_splits, 4 * min_splits + 8);
    auto fill_of = [&](int64_t sp) {
        const int64_t chunk = round_up((M + sp - 1) / sp, mb);
        const int64_t n_sp = (M + chunk - 1) / chunk;
        const int64_t blocks = (base_items * n_sp + wpb - 1) / wpb;
        const int64_t slots = kCUs * resident;  // blocks resident per round
        const int64_t rounds = (blocks + slots - 1) / slots;
        return (double)blocks / (double)(rounds * slots);
    };
    // interleaved tables (past kSplitRecords entries) may run the persistent two-copy launch
    // instead (one 16-wave block per CU, kBwdKRTwoCopies inputs per wave, decided on the
    // device): fill the rounds of both
    p.copies = copies_pay(M, K, O);
    const bool pair =
        !exact && p.copies && !p.gtab && !p.halves && !p.split && p.lane_red && wpb == 16 && kBwdORR == kFwdORR;
    auto fill_pair = [&](int64_t sp) {
        const double f1 = fill_of(sp);
        if (!pair) return f1;
        const int64_t chunk = round_up((M + sp - 1) / sp, mb);
        const int64_t n_sp = (M + chunk - 1) / chunk;
        const int64_t items = (int64_t)p.n_ob * (p.Kp / kBwdKRTwoCopies) * n_sp;
        const int64_t slots = (int64_t)kCUs * 16;
        const int64_t rounds = (items + slots - 1) / slots;
        return std::min(f1, (double)items / (double)(rounds * slots));
    };
    double best_fill = 0.0;
    for (int64_t sp = min_splits; sp <= top_splits; ++sp) best_fill = std::max(best_fill, fill_pair(sp));
    int64_t best_splits = min_splits;
    while (best_splits < top_splits && fill_pair(best_splits) < best_fill - 0.005) ++best_splits;
    p.m_chunk = (int)round_up((M + best_splits - 1) / best_splits, mb);
    if (p.m_chunk < mb) p.m_chunk = mb;
    // Problems with too few tokens for many rounds of blocks take their token splits from the
    // launch cost model instead of the fill rule (whose chunks of whole dX batches leave a
    // round two-thirds empty at a few rounds)
    const bool small = !pair && base_items * max_splits < kBwdSmallRounds * kCUs * resident * wpb;
    // Small plans of the one-shot table kernel sum each block's dVth partials over groups of
    // kDvGroup token splits in LDS (bwd_item's grouped order), writing a quarter of the planes:
    // token-split counts are then multiples of kDvGroup, and every block is full.
    const bool grouped = small && need_w && !exact && !p.gtab && !p.halves && !p.copies && wpb == 16 &&
                         base_items % (16 / kDvGroup) == 0;
    if (small) {
        // The launch lasts as long as its busiest CU. The token loop masks the tokens past a
        // chunk, so any chunk length works; take the one (of at least 8 tokens) minimising
        // small_launch_cost of blocks of (chunk + per-item setup); ties go to fewer splits.
        const int64_t min_chunk = std::max<int64_t>(8, mb);
        int64_t best_cost = -1;
        for (int64_t sp = 1; sp <= (M + min_chunk - 1) / min_chunk; ++sp) {
            if (grouped && sp % kDvGroup) continue;
            const int64_t chunk = (M + sp - 1) / sp;
            if ((M + chunk - 1) / chunk != sp) continue;  // the same plan as a smaller count
            const int64_t blocks = (base_items * sp + wpb - 1) / wpb;
            const int64_t cost = small_launch_cost(blocks, 100 * (chunk + ISA_EKV_BWD_ITEM_COST), (int)resident);
            if (best_cost < 0 || cost < best_cost) {
                best_cost = cost;
                p.m_chunk = (int)chunk;
            }
        }
    }
    p.n_split = (int)((M + p.m_chunk - 1) / p.m_chunk);
    if (p.n_split < 1) p.n_split = 1;
    p.n_items = (int)(base_items * p.n_split);
    p.blocks = (p.n_items + wpb - 1) / wpb;
    p.dv_group = grouped && p.n_split % kDvGroup == 0 && p.n_items % wpb == 0;
    p.dv_planes = p.dv_group ? p.n_split / kDvGroup : p.n_split;
    p.grad_padded = glue || (O % (64 * kBwdORR)) != 0;
    const size_t xrec_bytes = (size_t)round_up((int64_t)M * p.Kp * 16, 256);
    const size_t wsT_bytes = (size_t)round_up(p.Kp * p.Op * 8, 256);
    size_t off = 0;
    p.off_xrec = off;
    off += xrec_bytes;
    p.off_wsT = off;
    off += wsT_bytes;
    p.off_xrec_alt = off;
    if (exact) off += xrec_bytes;
    p.off_wsT_alt = off;
    if (exact) off += wsT_bytes;
    p.off_part = off;
    off += (size_t)round_up((kPrepBlocksX + kPrepBlocksW) * 8, 256);
    p.off_mode = off;  // the table-copy mode word
    off += 256;
    p.off_gpad = off;
    if (p.grad_padded) off += (size_t)round_up((int64_t)M * p.Op * 4, 256);
    p.off_dx = off;  // the half-table passes write a plane each
    if (need_x) off += (size_t)round_up((int64_t)(p.halves ? 2 : 1) * p.n_ob * M * (K > 0 ? K : 1) * 4, 256);
    p.off_dv = off;
    if (need_w) off += (size_t)round_up((int64_t)p.dv_planes * 2 * p.Kp * p.Op * 4, 256);
    p.off_glue = off;  // col_part [kGlueBlocks][2][Op], r_part [kGlueBlocks][Op/256], aff_part [kDxReduceBlocks]
    if (glue)
        off += (size_t)round_up((int64_t)kGlueBlocks * 2 * p.Op * 4, 256) +
               (size_t)round_up((int64_t)kGlueBlocks * (p.Op / 256) * 4, 256) +
               (size_t)round_up(kDxReduceBlocks * 8, 256);
    // the ranked backward rides with the copies' launch pair (decided on the device)
    p.ranked = bwd_may_use_copies(p, exact, need_x) && kBwdORR == 4 && g_ranked.load(std::memory_order_relaxed) != 0;
    {
        const int64_t mc = std::min<int64_t>(g_window_copies.load(std::memory_order_relaxed), kMultiMax);
        p.mc_max = bwd_may_use_copies(p, exact, need_x) && p.split && mc >= kModeMultiMin ? (int)mc : 0;
    }
    // The ranked launch (16 inputs per block, two blocks per CU) has twice the one-copy
    // launch's blocks at the same token splits; it merges r consecutive splits per block (r
    // dividing the split count) when its rounds stay as well filled and number at least 4:
    // fewer dVth partial planes to write and reduce, and fewer table loads.
    p.rank_merge = 1;
    if (p.ranked) {
        const int64_t n_kg = (p.Kp + kRankWaves - 1) / kRankWaves, slots = kCUs * 2;
        auto fill = [&](int64_t r, int64_t& rounds) {
            const int64_t blocks = n_kg * p.n_ob * (p.n_split / r);
            rounds = (blocks + slots - 1) / slots;
            return (double)blocks / (double)(rounds * slots);
        };
        int64_t rounds1 = 0;
        const double f1 = fill(1, rounds1);
        for (int r = 2; r <= ISA_EKV_RANK_MERGE_MAX; r *= 2) {
            int64_t rounds = 0;
            if (p.n_split % r == 0 && fill(r, rounds) >= f1 - 0.005 && rounds >= 4) p.rank_merge = r;
        }
    }
    p.off_rank_ws = off;
    if (p.ranked) off += (size_t)round_up(p.Kp * p.n_ob * 64 * 8 * 4, 256);
    p.off_rank_branch = off;
    if (p.ranked) off += (size_t)round_up(p.Kp * p.n_ob * 64 * 8, 256);
    p.bytes = round_up((int64_t)off, 256);
    return p;
}

__global__ __launch_bounds__(256) void pad_grad_kernel(const float* __restrict__ g, int64_t M, int64_t O,
                                                       int64_t Op, float* __restrict__ gp) {
    const int64_t total = M * Op;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t m = e / Op, o = e - m * Op;
        gp[e] = o < O ? g[m * O + o] : 0.0f;  // padded outputs contribute nothing to dX
    }
}

// Zero fill by kernel (not hipMemsetAsync), so a caller may capture the call in a graph.
__global__ __launch_bounds__(256) void zero_kernel(float* __restrict__ p, int64_t n) {
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x)
        p[e] = 0.0f;
}

template <bool SPLITS>
void launch_forward_split(bool exact, bool gtab, int mr, int wpb, dim3 grid, size_t lds, hipStream_t s,
                          const FwdArgs& fa) {
    const dim3 block(wpb * 64);
    if (gtab) {
        if (mr == 8)
            hipLaunchKernelGGL((fwd_global_kernel<8, SPLITS>), grid, block, 0, s, fa);
        else if (mr == 4)
            hipLaunchKernelGGL((fwd_global_kernel<4, SPLITS>), grid, block, 0, s, fa);
        else
            hipLaunchKernelGGL((fwd_global_kernel<2, SPLITS>), grid, block, 0, s, fa);
        return;
    }
    if (exact) {
        if (mr == 8)
            hipLaunchKernelGGL((fwd_exact_kernel<8, SPLITS>), grid, block, 0, s, fa);
        else if (mr == 4)
            hipLaunchKernelGGL((fwd_exact_kernel<4, SPLITS>), grid, block, 0, s, fa);
        else
            hipLaunchKernelGGL((fwd_exact_kernel<2, SPLITS>), grid, block, 0, s, fa);
        return;
    }
    if (fa.copy_window > 0 || fa.mc_budget > 0 || ISA_EKV_FWD_SMALL_WIN) {
        if (mr == 8)
            hipLaunchKernelGGL((fwd_kernel<8, SPLITS, true>), grid, block, lds, s, fa);
        else if (mr == 4)
            hipLaunchKernelGGL((fwd_kernel<4, SPLITS, true>), grid, block, lds, s, fa);
        else
            hipLaunchKernelGGL((fwd_kernel<2, SPLITS, true>), grid, block, lds, s, fa);
        return;
    }
    if (mr == 8)
        hipLaunchKernelGGL((fwd_kernel<8, SPLITS>), grid, block, lds, s, fa);
    else if (mr == 4)
        hipLaunchKernelGGL((fwd_kernel<4, SPLITS>), grid, block, lds, s, fa);
    else
        hipLaunchKernelGGL((fwd_kernel<2, SPLITS>), grid, block, lds, s, fa);
}

// The LDS-table forward kernels read their table at LDS address 0 (lds_record): their dynamic
// LDS starts there only while they declare no static LDS. Checked once per process.
template <class Kernel>
bool no_static_lds(Kernel kernel) {
    hipFuncAttributes at{};
    return hipFuncGetAttributes(&at, reinterpret_cast<const void*>(kernel)) == hipSuccess && at.sharedSizeBytes == 0;
}

bool fwd_tables_at_lds_zero() {
    static const bool ok = no_static_lds(fwd_kernel<8, false>) && no_static_lds(fwd_kernel<4, false>) &&
                           no_static_lds(fwd_kernel<2, false>) && no_static_lds(fwd_kernel<8, true>) &&
                           no_static_lds(fwd_kernel<4, true>) && no_static_lds(fwd_kernel<2, true>) &&
                           no_static_lds(fwd_kernel<8, false, true>) && no_static_lds(fwd_kernel<4, false, true>) &&
                           no_static_lds(fwd_kernel<2, false, true>) && no_static_lds(fwd_kernel<8, true, true>) &&
                           no_static_lds(fwd_kernel<4, true, true>) && no_static_lds(fwd_kernel<2, true, true>);
    return ok;
}

void launch_forward(bool exact, bool gtab, int mr, int wpb, dim3 grid, size_t lds, hipStream_t s,
                    const FwdArgs& fa) {
    if (fa.n_split > 1)
        launch_forward_split<true>(exact, gtab, mr, wpb, grid, lds, s, fa);
    else
        launch_forward_split<false>(exact, gtab, mr, wpb, grid, lds, s, fa);
}

template <bool SPLIT, bool LANE_RED>
void launch_backward_layout(bool need_x, bool need_w, dim3 grid, dim3 block, size_t lds, hipStream_t s,
                            const BwdArgs& ba) {
    if (need_x && need_w)
        hipLaunchKernelGGL((bwd_kernel<true, true, SPLIT, LANE_RED>), grid, block, lds, s, ba);
    else if (need_x)
        hipLaunchKernelGGL((bwd_kernel<true, false, SPLIT, LANE_RED>), grid, block, lds, s, ba);
    else
        hipLaunchKernelGGL((bwd_kernel<false, true, SPLIT, false>), grid, block, lds, s, ba);
}

// The split-layout lane-exchange backward as a pair of launches (kBwdOneCopy, kBwdTwoCopies)
// of which the device runs one; the same plan (grid, token splits, partial planes) serves both.
void launch_backward_copies(bool split, bool need_w, dim3 grid, dim3 block, size_t lds, hipStream_t s,
                            const BwdArgs& ba0, size_t lds2) {
    const dim3 grid2(std::min<unsigned>(grid.x, kCUs));  // persistent: one block per CU
    BwdArgs ba2 = ba0;  // the two-copy kernel's inputs per wave
    ba2.n_kb = ba0.Kp / kBwdKRTwoCopies;
    ba2.n_items = ba0.n_ob * ba2.n_kb * ba0.n_split;
    const BwdArgs& ba = ba0;
    if (need_w) {
        if (split)
            hipLaunchKernelGGL((bwd_kernel<true, true, true, true, kBwdOneCopy>), grid, block, lds, s, ba);
        else
            hipLaunchKernelGGL((bwd_kernel<true, true, false, true, kBwdOneCopy>), grid, block, lds, s, ba);
        if (split)
            hipLaunchKernelGGL((bwd_two_copies_kernel<true, true, true>), grid2, block, lds2, s, ba2);
        else
            hipLaunchKernelGGL((bwd_two_copies_kernel<true, true, false>), grid2, block, kBwdTwoCopiesLdsI,
                               s, ba2);
    } else {
        if (split)
            hipLaunchKernelGGL((bwd_kernel<true, false, true, true, kBwdOneCopy>), grid, block, lds, s, ba);
        else
            hipLaunchKernelGGL((bwd_kernel<true, false, false, true, kBwdOneCopy>), grid, block, lds, s, ba);
        if (split)
            hipLaunchKernelGGL((bwd_two_copies_kernel<true, false, true>), grid2, block, lds2, s, ba2);
        else
            hipLaunchKernelGGL((bwd_two_copies_kernel<true, false, false>), grid2, block, kBwdTwoCopiesLdsI,
                               s, ba2);
    }
}

// The half-table backward: the D pass (dVth and, with dX, its main term), then the I pass.
void launch_backward_halves(bool need_x, bool need_w, dim3 grid, dim3 block, size_t lds, hipStream_t s,
                            const BwdArgs& ba) {
    if (need_x && need_w)
        hipLaunchKernelGGL((bwd_half_kernel<0, true, true>), grid, block, lds, s, ba);
    else if (need_x)
        hipLaunchKernelGGL((bwd_half_kernel<0, true, false>), grid, block, lds, s, ba);
    else
        hipLaunchKernelGGL((bwd_half_kernel<0, false, true>), grid, block, lds, s, ba);
    if (need_x) hipLaunchKernelGGL((bwd_half_kernel<1, true, false>), grid, block, lds, s, ba);
}

void launch_backward(bool exact, bool gtab, bool need_x, bool need_w, bool split, bool lane_red, dim3 grid,
                     dim3 block, size_t lds, hipStream_t s, const BwdArgs& ba) {
    if (gtab) {
        if (need_x && need_w)
            hipLaunchKernelGGL((bwd_global_kernel<true, true>), grid, block, lds, s, ba);
        else if (need_x)
            hipLaunchKernelGGL((bwd_global_kernel<true, false>), grid, block, lds, s, ba);
        else
            hipLaunchKernelGGL((bwd_global_kernel<false, true>), grid, block, lds, s, ba);
    } else if (exact) {
        if (need_x && need_w)
            hipLaunchKernelGGL((bwd_exact_kernel<true, true>), grid, block, lds, s, ba);
        else if (need_x)
            hipLaunchKernelGGL((bwd_exact_kernel<true, false>), grid, block, lds, s, ba);
        else
            hipLaunchKernelGGL((bwd_exact_kernel<false, true>), grid, block, lds, s, ba);
    } else if (split) {
        if (lane_red)
            launch_backward_layout<true, true>(need_x, need_w, grid, block, lds, s, ba);
        else
            launch_backward_layout<true, false>(need_x, need_w, grid, block, lds, s, ba);
    } else {
        if (lane_red)
            launch_backward_layout<false, true>(need_x, need_w, grid, block, lds, s, ba);
        else
            launch_backward_layout<false, false>(need_x, need_w, grid, block, lds, s, ba);
    }
}

int check_shapes(const float* x, const float* wp, const float* wn, int64_t M, int64_t K, int64_t O, float v_sat) {
    if (M < 0 || K < 0 || O < 0) return fail(ISA_EKV_EINVAL, "negative shape (M=%lld, K=%lld, O=%lld)",
                                             (long long)M, (long long)K, (long long)O);
    if (M > INT32_MAX / 2 || K > INT32_MAX / 2 || O > INT32_MAX / 2)
        return fail(ISA_EKV_EINVAL, "shape too large for 32-bit tile indices");
    if (!(v_sat != 0.0f)) return fail(ISA_EKV_EINVAL, "V_sat must be nonzero");
    if (M * K > 0 && !x) return fail(ISA_EKV_EINVAL, "x is null");
    if (O * K > 0 && (!wp || !wn)) return fail(ISA_EKV_EINVAL, "vth_pos/vth_neg is null");
    return 0;
}

int check_common(const float* x, const float* wp, const float* wn, const void* lut, int64_t M, int64_t K,
                 int64_t O, int n_entries, float delta_min, float delta_max, float v_sat) {
    if (M < 0 || K < 0 || O < 0) return fail(ISA_EKV_EINVAL, "negative shape (M=%lld, K=%lld, O=%lld)",
                                             (long long)M, (long long)K, (long long)O);
    if (n_entries < 1) return fail(ISA_EKV_EINVAL, "LUT_DELTA_SIZE must be >= 1 (got %d)", n_entries);
    if (!(delta_max > delta_min)) return fail(ISA_EKV_EINVAL, "LUT range must satisfy delta_max > delta_min");
    const int rc = check_shapes(x, wp, wn, M, K, O, v_sat);
    if (rc) return rc;
    if (!lut) return fail(ISA_EKV_EINVAL, "lut is null");
    return 0;
}

// Operand transform of one call: LUT coordinates, or the exact formula's log2-unit operands.
struct CallSetup {
    bool exact;
    const void* lut;  // LUT records
    int n_entries;
    float delta_min, delta_max;
    double a_log2;    // exact: log2(e) / (2 n U_T)
    float k2, c2;     // exact: 2^(-V_D a_log2), V_D a_log2
    double cur_scale; // exact: I_S ln2^2 (current constant of the cells)
    double der_scale; // exact: 2 I_S ln2 / (2 n U_T) (derivative constant of the cells)
};

CallSetup lut_setup(const void* lut, int n_entries, float delta_min, float delta_max) {
    CallSetup cs{};
    cs.lut = lut;
    cs.n_entries = n_entries;
    cs.delta_min = delta_min;
    cs.delta_max = delta_max;
    return cs;
}

int exact_setup(const double* params, CallSetup* cs) {
    if (!params) return fail(ISA_EKV_EINVAL, "params is null");
    const double n = params[0], u_t = params[1], i_s = params[2], v_d = params[3];
    if (!(n > 0.0) || !(u_t > 0.0) || !std::isfinite(n * u_t))
        return fail(ISA_EKV_EINVAL, "n and U_T must be positive and finite");
    if (!std::isfinite(i_s) || !std::isfinite(v_d)) return fail(ISA_EKV_EINVAL, "I_S and V_D must be finite");
    const double ln2 = 0.69314718055994530942;
    const double inv_2nut = 1.0 / (2.0 * n * u_t);
    *cs = CallSetup{};
    cs->exact = true;
    cs->a_log2 = inv_2nut / ln2;
    cs->c2 = (float)(v_d * cs->a_log2);
    cs->k2 = (float)std::exp2(-v_d * cs->a_log2);
    cs->cur_scale = i_s * ln2 * ln2;
    cs->der_scale = 2.0 * i_s * inv_2nut * ln2;
    if (!(cs->a_log2 < 1e30)) return fail(ISA_EKV_EINVAL, "2 n U_T too small");
    return 0;
}

PrepArgs make_prep(const CallSetup& cs, const float* x, const float* wp, const float* wn, int64_t M, int64_t K,
                   int64_t O, int64_t Kp, int64_t Op, float v_sat, int rec_floats, char* ws, size_t off_xrec,
                   size_t off_wsT, size_t off_xrec_alt, size_t off_wsT_alt, size_t off_part,
                   const isa_ekv_glue* glue) {
    PrepArgs pa{};
    if (glue && glue->in_affine) {
        pa.in_affine = glue->in_affine;
        pa.in_lo = glue->in_lo;
        pa.in_hi = glue->in_hi;
    }
    pa.x = x;
    pa.wp = wp;
    pa.wn = wn;
    pa.M = M;
    pa.K = K;
    pa.O = O;
    pa.Kp = Kp;
    pa.Op = Op;
    pa.v_sat = v_sat;
    pa.rec_floats = rec_floats;
    pa.xrec = reinterpret_cast<float*>(ws + off_xrec);
    pa.wsT = reinterpret_cast<float2*>(ws + off_wsT);
    pa.partials = reinterpret_cast<float2*>(ws + off_part);
    if (!cs.exact) {
        const int n = cs.n_entries;
        const double scale_d = n > 1 ? (double)(n - 1) / ((double)cs.delta_max - (double)cs.delta_min) : 0.0;
        pa.xoff = cs.delta_min;
        pa.scale = (float)scale_d;
        pa.xadd = (float)kPad;
        pa.scale_d = scale_d;
        pa.z_div = v_sat;
        pa.pad_coord = (float)kPad + 1.0f;
        pa.exact = 0;
    } else {
        pa.xoff = 0.0f;
        pa.scale = (float)cs.a_log2;
        pa.xadd = 0.0f;
        pa.scale_d = cs.a_log2;
        pa.z_div = (float)((double)v_sat * cs.der_scale / cs.cur_scale);
        pa.pad_coord = 0.0f;
        pa.exact = 1;
        pa.xrec_slow = reinterpret_cast<float*>(ws + off_xrec_alt);
        pa.wsT_slow = reinterpret_cast<float2*>(ws + off_wsT_alt);
    }
    return pa;
}

// Folds one forward's max |y| (bit pattern from the epilogue's atomic max) into the caller's
// running statistics as cim.py:194-198 does: abs_max = maximum(abs_max, max|y|), NaN
// propagating like torch.maximum; total += count.
__global__ void stat_merge_kernel(const unsigned* bits, float* abs_max, double* total, double count) {
    if (threadIdx.x != 0) return;
    if (abs_max) {
        const float m = __uint_as_float(*bits), cur = *abs_max;
        *abs_max = cur != cur ? cur : (m != m || m > cur) ? m : cur;
    }
    if (total) *total += count;
}

// Finishes a K-split forward (fwd_body wrote each split's partial sums): the splits are summed
// in split order, then clamped (LUT) or scaled (exact, measured) and given the layer glue
// exactly as fwd_body's epilogue does. Grid-stride over the [M][O] outputs, VEC of them per
// thread (VEC = 4 when O and every pointer allow 16-byte accesses).
template <int VEC>
__global__ __launch_bounds__(256) void split_reduce_kernel(FwdArgs a, int clamp_out) {
    const int64_t n = (int64_t)a.M * a.O;
    const int64_t nv = n / VEC;
    const bool has_r = a.glue && a.r_tia != nullptr;
    const float r = has_r ? tia_gain(a.r_tia, a.r_log_scale, a.r_log_lo, a.r_log_hi) : 1.0f;
    unsigned ymax = 0;
    for (int64_t ev = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; ev < nv; ev += (int64_t)gridDim.x * blockDim.x) {
        float v[VEC], id[VEC];
        if constexpr (VEC == 4) {
            float4 t = reinterpret_cast<const float4*>(a.split_part)[ev];
            for (int sp = 1; sp < a.n_split; ++sp) {
                const float4 u = reinterpret_cast<const float4*>(a.split_part + (size_t)sp * n)[ev];
                t.x += u.x;
                t.y += u.y;
                t.z += u.z;
                t.w += u.w;
            }
            v[0] = t.x;
            v[1] = t.y;
            v[2] = t.z;
            v[3] = t.w;
        } else {
            v[0] = a.split_part[ev];
            for (int sp = 1; sp < a.n_split; ++sp) v[0] += a.split_part[(size_t)sp * n + ev];
        }
#pragma unroll
        for (int i = 0; i < VEC; ++i)
            id[i] = clamp_out ? fminf(fmaxf(v[i], a.out_min), a.out_max) : v[i] * a.out_scale;
        const int64_t e = ev * VEC;
        if (!a.glue) {
            if constexpr (VEC == 4)
                reinterpret_cast<float4*>(a.out)[ev] = make_float4(id[0], id[1], id[2], id[3]);
            else
                a.out[e] = id[0];
            continue;
        }
        const int o0 = (int)(e % a.O);  // VEC divides O: the VEC outputs share a row
        float y[VEC];
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
            const float yt = layer_tia(id[i], r, has_r, a.y_lo, a.y_hi);
            ymax = max(ymax, layer_stat_bits(yt));
            y[i] = layer_adc(yt, a.adc_scale, a.adc_shift, o0 + i);
        }
        if constexpr (VEC == 4) {
            if (a.idiff) reinterpret_cast<float4*>(a.idiff)[ev] = make_float4(id[0], id[1], id[2], id[3]);
            reinterpret_cast<float4*>(a.out)[ev] = make_float4(y[0], y[1], y[2], y[3]);
        } else {
            if (a.idiff) a.idiff[e] = id[0];
            a.out[e] = y[0];
        }
    }
    if (a.stat_bits) {  // every lane of the wave is here: the loop has no early exit
#pragma unroll
        for (int d = 32; d >= 1; d >>= 1) ymax = max(ymax, (unsigned)__shfl_xor((int)ymax, d, 64));
        if ((threadIdx.x & 63) == 0) atomicMax(a.stat_bits, ymax);
    }
}

// Points a forward launch at the plan's K split (no-op without one).
void set_split(const FwdPlan& p, char* ws, FwdArgs& fa) {
    fa.n_split = p.n_split;
    fa.k_chunk = p.k_chunk;
    fa.split_part = p.n_split > 1 ? reinterpret_cast<float*>(ws + p.off_split) : nullptr;
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

hipError_t finish_split(const FwdPlan& p, const FwdArgs& fa, bool clamp_out, hipStream_t s) {
    if (p.n_split <= 1) return hipSuccess;
    const int64_t n = (int64_t)fa.M * fa.O;
    const bool vec4 = fa.O % 4 == 0 && aligned16(fa.out) && aligned16(fa.split_part) &&
                      (!fa.glue || !fa.idiff || aligned16(fa.idiff));
    const int64_t work = vec4 ? n / 4 : n;
    const unsigned blocks = (unsigned)std::min<int64_t>((work + 255) / 256, 8192);
    if (vec4)
        hipLaunchKernelGGL(split_reduce_kernel<4>, dim3(blocks), dim3(256), 0, s, fa, clamp_out ? 1 : 0);
    else
        hipLaunchKernelGGL(split_reduce_kernel<1>, dim3(blocks), dim3(256), 0, s, fa, clamp_out ? 1 : 0);
    return hipGetLastError();
}

// The forward plan of a call. LUT tables past 4096 entries hold their two copies (132 KB) in
// one 16-wave block per CU, the same 16 waves per CU as two 8-wave blocks of one copy; that
// pays when each wave sums a long K range (measured: 768 inputs per wave -7%, 64 or 128 +9%:
// the block's table load, barrier and tail are spread over less work).
FwdPlan plan_forward_call(bool exact, int n_entries, int64_t M, int64_t K, int64_t O) {
    FwdPlan p = plan_forward(M, K, O, exact, true, kFwdWaves);
    if (!exact && copies_pay(M, K, O) && fwd_copy_lds(n_entries) > kFwdCopyLdsBytes &&
        fwd_copy_lds(n_entries) <= (size_t)kLdsBytes) {
        const FwdPlan p16 = plan_forward(M, K, O, false, true, 2 * kFwdWaves);
        if (p16.k_chunk >= kFwdCopyMinInputs16) p = p16;
    }
    return p;
}

// Table placement of a LUT forward launch with wpb waves per block: LDS bytes, and the second
// table copy (copy_offset > 0: the launch may use it, decided on the device from the range
// partials and recorded in the mode word; copy_window > 0: the copies hold only the
// coordinate window, of at most that many records). copies = false (calls below
// ISA_EKV_OPT_COPY_MIN_CELLS): one copy.
struct FwdTableCfg {
    bool gtab;  // table read from global memory
    size_t lds;
    int copy_offset, copy_window;
    int mc_budget, mc_max;  // windowed copies (mc_budget > 0): LDS records of the allocation, most copies
};

FwdTableCfg fwd_table_cfg(int n_entries, int wpb, bool copies) {
    FwdTableCfg t{};
    t.gtab = n_entries > kMaxEntriesFwd;
    t.lds = t.gtab ? 0 : (size_t)lut_records(n_entries) * 8;
    if (t.gtab || !copies) return t;
    // the second table copy (used when the thresholds spread wide) when both copies still
    // leave room for two forward blocks per CU
    int t1 = fwd_copy_offset(n_entries);
    size_t lds2 = fwd_copy_lds(n_entries);
    const size_t lds_cap = wpb == kFwdWaves ? kFwdCopyLdsBytes : (size_t)kLdsBytes;
    // tables whose two full copies do not fit copy only the coordinate window the launch
    // reaches (the allocation also holds the whole table for the one-copy case)
    const size_t lds_win = std::max(t.lds, (size_t)(kFwdWinOffset + kSplitRecords) * 8);
    if (lds2 > lds_cap && lds_win <= lds_cap) {
        t1 = kFwdWinOffset;
        lds2 = lds_win;
        t.copy_window = kSplitRecords;
    }
    if (lds2 <= lds_cap) {
        t.copy_offset = t1;
        t.lds = lds2;
    }
    // the windowed copies, in an allocation of at least the block shape's share of the CU's
    // LDS (the device takes as many copies as fit the launch's window)
    const int64_t mc_max = std::min<int64_t>(g_window_copies.load(std::memory_order_relaxed), 32);
    if (mc_max >= kModeMultiMin) {
        t.lds = std::max(t.lds, lds_cap);
        t.mc_budget = (int)(t.lds / 8);
        t.mc_max = (int)mc_max;
    }
    return t;
}

int run_forward(const CallSetup& cs, const float* x, const float* vth_pos, const float* vth_neg, int64_t M,
                int64_t K, int64_t O, float v_sat, float out_min, float out_max, float* out, void* workspace,
                size_t workspace_bytes, hipStream_t s, const isa_ekv_glue* glue = nullptr,
                float* idiff = nullptr, bool timed = true) {
    if (M == 0 || O == 0) return 0;
    if (!out) return fail(ISA_EKV_EINVAL, "out is null");
    const FwdPlan p = plan_forward_call(cs.exact, cs.n_entries, M, K, O);
    if (!workspace || workspace_bytes < p.bytes)
        return fail(ISA_EKV_EINVAL, "forward workspace too small (%zu < %zu bytes)", workspace_bytes, p.bytes);
    char* ws = static_cast<char*>(workspace);
    CallTimer call_timer(s, 2, timed);
    PrepArgs pa = make_prep(cs, x, vth_pos, vth_neg, M, K, O, p.Kp, p.Op, v_sat, 2, ws, p.off_xrec, p.off_wsT,
                            p.off_xrec_alt, p.off_wsT_alt, p.off_part, glue);
    const bool stats = glue && (glue->stat_abs_max || glue->stat_total);
    unsigned* stat_bits = stats ? reinterpret_cast<unsigned*>(ws + p.off_stat) : nullptr;
    pa.stat_bits = stat_bits;
    hipLaunchKernelGGL(prep_kernel, dim3(kPrepBlocksX + kPrepBlocksW), dim3(256), 0, s, pa);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return hip_fail(err, "forward prep launch");
    FwdArgs fa{};
    fa.xrec = reinterpret_cast<const float2*>(ws + p.off_xrec);
    fa.wsT = reinterpret_cast<const float2*>(ws + p.off_wsT);
    fa.xrec_alt = reinterpret_cast<const float2*>(ws + p.off_xrec_alt);
    fa.wsT_alt = reinterpret_cast<const float2*>(ws + p.off_wsT_alt);
    fa.partials = reinterpret_cast<const float2*>(ws + p.off_part);
    fa.out = out;
    fa.M = (int)M;
    fa.O = (int)O;
    fa.Kp = (int)p.Kp;
    fa.Op = (int)p.Op;
    fa.n_mt = p.n_mt;
    fa.n_ot = p.n_ot;
    fa.out_min = out_min;
    fa.out_max = out_max;
    if (glue) {
        fa.glue = 1;
        fa.idiff = idiff;
        fa.r_tia = glue->r_tia;
        fa.r_log_scale = glue->r_log_scale;
        fa.r_log_lo = glue->r_log_lo;
        fa.r_log_hi = glue->r_log_hi;
        fa.y_lo = glue->y_lo;
        fa.y_hi = glue->y_hi;
        fa.adc_scale = glue->adc_scale;
        fa.adc_shift = glue->adc_shift;
        fa.stat_bits = stat_bits;
    }
    size_t lds = 0;
    bool gtab = false;
    if (cs.exact) {
        fa.out_scale = (float)cs.cur_scale;
        fa.k2 = cs.k2;
        fa.c2 = cs.c2;
    } else {
        fa.lut = static_cast<const float2*>(cs.lut);
        fa.NP = cs.n_entries + 2 * kPad;
        fa.cmin = (float)kPad;
        fa.cmax = (float)(kPad + cs.n_entries - 1);
        fa.out_scale = 1.0f;
        const FwdTableCfg tc = fwd_table_cfg(cs.n_entries, p.wpb, copies_pay(M, K, O));
        gtab = tc.gtab;
        lds = tc.lds;
        fa.copy_offset = tc.copy_offset;
        fa.copy_window = tc.copy_window;
        fa.mc_budget = tc.mc_budget;
        fa.mc_max = tc.mc_max;
        int* mode = reinterpret_cast<int*>(ws + p.off_mode);
        const int64_t problems = p.Kp * (p.Op / (64 * kFwdORR)) * kFwdORR * 4;
        const dim3 agrid((unsigned)((problems + kAssignThreads - 1) / kAssignThreads));
        if (tc.mc_budget > 0) {
            hipLaunchKernelGGL(fwd_multi_assign_kernel, dim3((unsigned)((problems + kMcProblems - 1) / kMcProblems)),
                               dim3(kMcThreads), 0, s,
                               reinterpret_cast<float2*>(ws + p.off_wsT), fa.partials, fa.NP, tc.mc_budget,
                               tc.mc_max, mode, p.Kp, p.Op, 0, fa.NP, 0, 0.0f);
            err = hipGetLastError();
            if (err != hipSuccess) return hip_fail(err, "forward windowed-copy assignment launch");
        }
        if (tc.copy_offset > 0) {
            hipLaunchKernelGGL(fwd_copy_assign_kernel<32>, agrid, dim3(kAssignThreads), 0, s,
                               reinterpret_cast<float2*>(ws + p.off_wsT), fa.partials, fa.NP,
                               fa.copy_window > 0 ? fa.copy_window : fa.NP, mode, p.Kp, p.Op, tc.copy_offset,
                               tc.mc_budget > 0 ? kModeMultiMin : 0);
            err = hipGetLastError();
            if (err != hipSuccess) return hip_fail(err, "forward copy assignment launch");
        }
    }
    set_split(p, ws, fa);
    if (!cs.exact && !gtab && !fwd_tables_at_lds_zero())
        return fail(ISA_EKV_EINVAL, "forward: the LDS-table kernels declare static LDS, so their table is not "
                                          "at LDS address 0 (rebuild without static __shared__ in fwd_kernel)");
    ProfiledLaunch* prof = nullptr;
    if (timed) prof_start(s, 0, &prof);
    if (timed && !cs.exact) fa.clock_acc = clock_acc(0);
    launch_forward(cs.exact, gtab, p.mr, p.wpb, dim3(p.blocks), lds, s, fa);
    err = hipGetLastError();
    if (err == hipSuccess) err = finish_split(p, fa, !cs.exact, s);
    prof_stop(s, prof);
    if (err != hipSuccess) return hip_fail(err, "forward launch");
    if (stats) {
        hipLaunchKernelGGL(stat_merge_kernel, dim3(1), dim3(64), 0, s, stat_bits, glue->stat_abs_max,
                           glue->stat_total, (double)M * (double)O);
        err = hipGetLastError();
        if (err != hipSuccess) return hip_fail(err, "output statistics launch");
    }
    return 0;
}

// Whether a table backward enqueues the second-copy pair of launches (the device then picks
// one and records it in the mode word): split layout with lane-exchange dX, whose LDS holds
// only the table, so both copies fit one block per CU; tables past the split layout's length
// (the 8192-entry ones) take the copies when the coordinate window the launch reaches fits
// that length, which the device decides.
bool bwd_may_use_copies(const BwdPlan& p, bool exact, bool need_x) {
    return kBwdORR == kFwdORR && !exact && p.copies && !p.gtab && !p.halves && p.lane_red && need_x &&
           (p.split ? p.lds_bytes <= kBwdTwoCopiesLds / 2 : true) && p.waves_per_block == 16;
}

void zero_fill(float* p, int64_t n, hipStream_t s) {
    if (p && n > 0) hipLaunchKernelGGL(zero_kernel, dim3(256), dim3(256), 0, s, p, n);
}

// glue / glue_grads: the layer backward (null for the plain projection backward).
int run_backward(const CallSetup& cs, const float* x, const float* vth_pos, const float* vth_neg,
                 const float* grad_out, int64_t M, int64_t K, int64_t O, float v_sat, float* grad_x,
                 float* grad_vth_pos, float* grad_vth_neg, void* workspace, size_t workspace_bytes, hipStream_t s,
                 const isa_ekv_glue* glue = nullptr, const float* idiff = nullptr,
                 const isa_ekv_glue_grads* gg = nullptr) {
    const bool need_x = grad_x != nullptr;
    const bool need_w = grad_vth_pos != nullptr || grad_vth_neg != nullptr;
    if (need_w && (grad_vth_pos == nullptr || grad_vth_neg == nullptr))
        return fail(ISA_EKV_EINVAL, "grad_vth_pos and grad_vth_neg must both be given or both be null");
    const bool need_glue = gg && (gg->in_affine || gg->r_tia || gg->adc_scale || gg->adc_shift || gg->r_log_scale);
    if (!need_x && !need_w && !need_glue) return 0;
    hipError_t err;
    // degenerate shapes: empty reductions give zero gradients (with glue and K == 0 the
    // glue still acts on idiff = 0 and its gradients are computed below)
    if (M == 0 || O == 0 || (K == 0 && !glue)) {
        if (need_x) zero_fill(grad_x, M * K, s);
        if (need_w) {
            zero_fill(grad_vth_pos, O * K, s);
            zero_fill(grad_vth_neg, O * K, s);
        }
        if (gg) {
            zero_fill(gg->in_affine, 2, s);
            zero_fill(gg->r_tia, 1, s);
            zero_fill(gg->r_log_scale, 1, s);
            zero_fill(gg->adc_scale, O, s);
            zero_fill(gg->adc_shift, O, s);
        }
        err = hipGetLastError();
        if (err != hipSuccess) return hip_fail(err, "zero fill launch");
        return 0;
    }
    if (!grad_out) return fail(ISA_EKV_EINVAL, "grad_out is null");
    const BwdPlan p = plan_backward(M, K, O, cs.exact ? 0 : cs.n_entries, need_x, need_w, glue != nullptr);
    if (!workspace || workspace_bytes < p.bytes)
        return fail(ISA_EKV_EINVAL, "backward workspace too small (%zu < %zu bytes)", workspace_bytes, p.bytes);
    char* ws = static_cast<char*>(workspace);
    CallTimer call_timer(s, 3);
    float* col_part = reinterpret_cast<float*>(ws + p.off_glue);
    float* r_part = col_part + (size_t)round_up((int64_t)kGlueBlocks * 2 * p.Op * 4, 256) / 4;
    float2* aff_part =
        reinterpret_cast<float2*>(r_part + (size_t)round_up((int64_t)kGlueBlocks * (p.Op / 256) * 4, 256) / 4);
    GlueGradArgs ga{};
    if (glue) {
        ga = GlueGradArgs{grad_out, idiff, M, O, p.Op, glue->r_tia, glue->r_log_scale, glue->r_log_lo,
                          glue->r_log_hi, glue->y_lo, glue->y_hi, glue->adc_scale,
                          reinterpret_cast<float*>(ws + p.off_gpad), col_part, r_part};
        if (K == 0) {  // nothing reaches x or the thresholds
            hipLaunchKernelGGL(glue_grad_kernel, dim3(kGlueBlocks, (unsigned)(p.Op / 256)), dim3(256), 0, s, ga);
            if (gg) zero_fill(gg->in_affine, 2, s);
            if (gg && (gg->r_tia || gg->adc_scale || gg->adc_shift || gg->r_log_scale)) {
                const GlueReduceArgs gr{col_part, r_part, aff_part, 0, O, p.Op, gg->adc_scale, gg->adc_shift,
                                        gg->r_tia, nullptr, glue->r_tia, glue->r_log_scale, glue->r_log_lo,
                                        glue->r_log_hi, gg->r_log_scale};
                hipLaunchKernelGGL(glue_reduce_kernel, dim3((unsigned)glue_reduce_blocks(O)), dim3(256), 0, s, gr);
            }
            err = hipGetLastError();
            if (err != hipSuccess) return hip_fail(err, "glue gradient launch");
            return 0;
        }
    }
    // the prep, and with the layer glue its gradient pass (G_eff for the main kernel)
    const PrepArgs pa = make_prep(cs, x, vth_pos, vth_neg, M, K, O, p.Kp, p.Op, v_sat, 4, ws, p.off_xrec, p.off_wsT,
                                  p.off_xrec_alt, p.off_wsT_alt, p.off_part, glue);
    const int64_t glue_blocks = glue ? (int64_t)kGlueBlocks * (p.Op / 256) : 0;
    hipLaunchKernelGGL(bwd_prep_kernel, dim3((unsigned)(kPrepBlocksX + kPrepBlocksW + glue_blocks)), dim3(256), 0, s,
                       pa, ga);
    err = hipGetLastError();
    if (err != hipSuccess) return hip_fail(err, "backward prep launch");
    const float* g = grad_out;
    int ldg = (int)O;
    if (glue) {
        g = reinterpret_cast<const float*>(ws + p.off_gpad);
        ldg = (int)p.Op;
    } else if (p.grad_padded) {
        float* gp = reinterpret_cast<float*>(ws + p.off_gpad);
        hipLaunchKernelGGL(pad_grad_kernel, dim3(1024), dim3(256), 0, s, grad_out, M, O, p.Op, gp);
        err = hipGetLastError();
        if (err != hipSuccess) return hip_fail(err, "grad pad launch");
        g = gp;
        ldg = (int)p.Op;
    }
    BwdArgs ba{};
    ba.xrec = reinterpret_cast<const float4*>(ws + p.off_xrec);
    ba.wsT = reinterpret_cast<const float2*>(ws + p.off_wsT);
    ba.xrec_alt = reinterpret_cast<const float4*>(ws + p.off_xrec_alt);
    ba.wsT_alt = reinterpret_cast<const float2*>(ws + p.off_wsT_alt);
    ba.grad = g;
    ba.partials = reinterpret_cast<const float2*>(ws + p.off_part);
    ba.dx_part = reinterpret_cast<float*>(ws + p.off_dx);
    ba.dv_part = reinterpret_cast<float*>(ws + p.off_dv);
    ba.M = (int)M;
    ba.K = (int)K;
    ba.O = (int)O;
    ba.Kp = (int)p.Kp;
    ba.Op = (int)p.Op;
    ba.ldg = ldg;
    ba.n_ob = p.n_ob;
    ba.n_kb = p.n_kb;
    ba.n_split = p.n_split;
    ba.m_chunk = p.m_chunk;
    ba.n_items = p.n_items;
    ba.dv_group = p.dv_group ? 1 : 0;
    float scale = 1.0f;
    if (cs.exact) {
        ba.k2 = cs.k2;
        ba.c2 = cs.c2;
        scale = (float)cs.der_scale;
    } else {
        ba.lut = static_cast<const float4*>(cs.lut);
        ba.NP = cs.n_entries + 2 * kPad;
        ba.cmin = (float)kPad;
        ba.cmax = (float)(kPad + cs.n_entries - 1);
    }
    const dim3 grid(p.blocks), block(p.waves_per_block * 64);
    const bool copies = bwd_may_use_copies(p, cs.exact, need_x);
    const float rank_max_spread = (float)g_rank_max_spread.load(std::memory_order_relaxed);
    if (copies) {
        int* mode = reinterpret_cast<int*>(ws + p.off_mode);
        if (p.ranked) {  // the branch deal first: it records the ranked mode when that launch works
            const RankArgs ra{reinterpret_cast<const float2*>(ws + p.off_wsT),
                              reinterpret_cast<float*>(ws + p.off_rank_ws),
                              reinterpret_cast<uint2*>(ws + p.off_rank_branch), ba.partials, mode,
                              (int)p.Kp, (int)p.Op, p.n_ob, ba.NP, rank_max_spread,
                              (float)g_rank_greedy_min.load(std::memory_order_relaxed)};
            const int64_t threads = p.Kp * p.n_ob * kRankClasses;
            hipLaunchKernelGGL(bwd_rank_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, ra);
            // the greedy deal of spreads past greedy_min (exits at once when the rank deal
            // applies); not launched when no spread the ranked mode takes can exceed greedy_min
            const int64_t problems_q = p.Kp * p.n_ob;
            if (ra.greedy_min < ra.max_spread)
                hipLaunchKernelGGL(bwd_deal_kernel, dim3((unsigned)((problems_q + kDealProblems - 1) / kDealProblems)),
                                   dim3(kDealWaves * 64), 0, s, ra);
        }
        // split tables: 8-byte records (half-wave banks); interleaved: 16-byte (quarter-wave)
        const int64_t problems = p.Kp * (p.Op / (64 * kBwdORR)) * kBwdORR * (p.split ? 4 : 8);
        const dim3 agrid((unsigned)((problems + kAssignThreads - 1) / kAssignThreads));
        if (p.mc_max > 0) {  // then the windowed copies of the two-copy launch, unless ranked
            ba.mc_budget = kBwdWinBudget;
            ba.mc_max = p.mc_max;
            hipLaunchKernelGGL(fwd_multi_assign_kernel, dim3((unsigned)((problems + kMcProblems - 1) / kMcProblems)),
                               dim3(kMcThreads), 0, s, reinterpret_cast<float2*>(ws + p.off_wsT), ba.partials,
                               ba.NP, kBwdWinBudget, p.mc_max, mode, p.Kp, p.Op, kBwdWinDOffset, kBwdWinWindow,
                               kBwdWinWideDOffset, p.ranked ? rank_max_spread : 0.0f);
        }
        // (a pass before it recorded the ranked mode or the windowed copies: skip_from)
        const int skip_from = p.ranked ? kModeRanked : p.mc_max > 0 ? kModeMultiMin : 0;
        if (p.split)
            hipLaunchKernelGGL(fwd_copy_assign_kernel<32>, agrid, dim3(kAssignThreads), 0, s,
                               reinterpret_cast<float2*>(ws + p.off_wsT), ba.partials, ba.NP, kSplitRecords, mode,
                               p.Kp, p.Op, kBwdCopyOffset, skip_from);
        else
            hipLaunchKernelGGL(fwd_copy_assign_kernel<16>, agrid, dim3(kAssignThreads), 0, s,
                               reinterpret_cast<float2*>(ws + p.off_wsT), ba.partials, ba.NP, kSplitRecords, mode,
                               p.Kp, p.Op, kBwdCopyOffsetI, skip_from);
        ba.copy_mode = mode;
        err = hipGetLastError();
        if (err != hipSuccess) return hip_fail(err, "backward copy assignment launch");
    }
    ProfiledLaunch* prof;
    prof_start(s, 1, &prof);
    if (!cs.exact) ba.clock_acc = clock_acc(1);
    if (p.halves)
        launch_backward_halves(need_x, need_w, grid, block, p.lds_bytes, s, ba);
    else if (copies) {
        launch_backward_copies(p.split, need_w, grid, block, p.lds_bytes, s, ba,
                               p.mc_max > 0 ? (size_t)kLdsBytes : kBwdTwoCopiesLds);
        if (p.ranked) {
            // the ranked launch sums p.rank_merge consecutive token splits per block
            BwdArgs br = ba;
            br.xcd_order = g_rank_xcd_order.load(std::memory_order_relaxed) != 0 ? 1 : 0;
            br.n_split = p.n_split / p.rank_merge;
            br.m_chunk = p.m_chunk * p.rank_merge;
            const dim3 rgrid((unsigned)(((p.Kp + kRankWaves - 1) / kRankWaves) * p.n_ob * br.n_split));
            const float* rws = reinterpret_cast<const float*>(ws + p.off_rank_ws);
            const uint2* rbr = reinterpret_cast<const uint2*>(ws + p.off_rank_branch);
            if (need_w)
                hipLaunchKernelGGL(bwd_ranked_kernel<true>, rgrid, dim3(kRankWaves * 64), kRankLds, s, br, rws, rbr);
            else
                hipLaunchKernelGGL(bwd_ranked_kernel<false>, rgrid, dim3(kRankWaves * 64), kRankLds, s, br, rws, rbr);
        }
    }
    else
        launch_backward(cs.exact, p.gtab, need_x, need_w, p.split, p.lane_red, grid, block, p.lds_bytes, s, ba);
    err = hipGetLastError();
    prof_stop(s, prof);
    if (err != hipSuccess) return hip_fail(err, "backward launch");
    // dX and dVth reductions in one launch, with the glue sums unless they need the dX
    // reduction's input-mapping partials (a second launch then follows)
    DxReduceArgs dxa{};
    int dx_blocks = 0;
    if (need_x) {
        dxa = DxReduceArgs{reinterpret_cast<const float*>(ws + p.off_dx), (p.halves ? 2 : 1) * p.n_ob, M * K, scale,
                           grad_x, x, glue ? glue->in_affine : nullptr, glue ? glue->in_lo : 0.0f,
                           glue ? glue->in_hi : 0.0f, aff_part, 0};
        dx_blocks = dx_reduce_blocks(M * K);
    }
    DvReduceArgs dva{};
    int dv_blocks = 0;
    if (need_w) {
        dva = DvReduceArgs{reinterpret_cast<const float*>(ws + p.off_dv), p.dv_planes, (int)K, (int)O, (int)p.Kp,
                           (int)p.Op, scale, grad_vth_pos, grad_vth_neg,
                           p.ranked && copies ? reinterpret_cast<const int*>(ws + p.off_mode) : nullptr,
                           p.n_split / p.rank_merge};
        dv_blocks = std::min(dv_reduce_tiles(K, O), 4096);
    }
    GlueReduceArgs gra{};
    int gl_blocks = 0;
    if (need_glue) {
        gra = GlueReduceArgs{col_part, r_part, aff_part, dx_blocks, O, p.Op, gg->adc_scale, gg->adc_shift,
                             gg->r_tia, gg->in_affine, glue->r_tia, glue->r_log_scale, glue->r_log_lo,
                             glue->r_log_hi, gg->r_log_scale};
        gl_blocks = glue_reduce_blocks(O);
    }
    const bool glue_after = gg && gg->in_affine;  // needs aff_part from the dX blocks
    const int first_blocks = dx_blocks + dv_blocks + (glue_after ? 0 : gl_blocks);
    if (first_blocks > 0)
        hipLaunchKernelGGL(grad_reduce_kernel, dim3((unsigned)first_blocks), dim3(256), 0, s, dxa, dx_blocks, dva,
                           dv_blocks, gra);
    if (need_glue && glue_after)
        hipLaunchKernelGGL(glue_reduce_kernel, dim3((unsigned)gl_blocks), dim3(256), 0, s, gra);
    err = hipGetLastError();
    if (err != hipSuccess) return hip_fail(err, "gradient reduction launch");
    return 0;
}

// need_x: whether grad_x is given (or has no elements, M * K == 0)
int check_glue(const isa_ekv_glue* glue, const isa_ekv_glue_grads* gg, bool need_x) {
    if (!glue) return fail(ISA_EKV_EINVAL, "glue is null");
    if (glue->adc_scale && !glue->adc_shift) return fail(ISA_EKV_EINVAL, "adc_scale needs adc_shift");
    if (glue->in_affine && !(glue->in_hi >= glue->in_lo)) return fail(ISA_EKV_EINVAL, "input range needs in_hi >= in_lo");
    if (glue->r_tia && !(glue->y_hi >= glue->y_lo)) return fail(ISA_EKV_EINVAL, "output range needs y_hi >= y_lo");
    if (glue->r_log_scale && !glue->r_tia) return fail(ISA_EKV_EINVAL, "r_log_scale needs r_tia (the base gain)");
    if (glue->r_log_scale && !(glue->r_log_hi >= glue->r_log_lo))
        return fail(ISA_EKV_EINVAL, "log-gain range needs r_log_hi >= r_log_lo");
    if (gg) {
        if (gg->in_affine && !glue->in_affine) return fail(ISA_EKV_EINVAL, "input-mapping gradient without in_affine");
        if (gg->in_affine && !need_x)
            return fail(ISA_EKV_EINVAL, "the input-mapping gradient needs grad_x (it is formed from dX)");
        if (gg->r_tia && !glue->r_tia) return fail(ISA_EKV_EINVAL, "r_tia gradient without r_tia");
        if (gg->r_log_scale && !glue->r_log_scale)
            return fail(ISA_EKV_EINVAL, "r_log_scale gradient without r_log_scale");
        if ((gg->adc_scale || gg->adc_shift) && !glue->adc_scale)
            return fail(ISA_EKV_EINVAL, "ADC affine gradient without adc_scale/adc_shift");
    }
    return 0;
}


// ----------------------------------------------------------------------------------
// Measured-codebook calls.
// ----------------------------------------------------------------------------------

constexpr size_t kMeasuredBwdLdsTableBytes = 128 * 1024;  // the dX reduction needs no LDS

size_t measured_table_bytes(int n_seg, int n_rows) {
    return (size_t)round_up(((int64_t)n_seg * n_rows + 1) * 8, 256);
}

int check_codebook(const isa_ekv_codebook* cb, const short* ids_a) {
    if (!cb) return fail(ISA_EKV_EINVAL, "codebook is null");
    if (cb->n_seg < 1 || cb->n_rows < 1) return fail(ISA_EKV_EINVAL, "codebook needs n_seg >= 1 and n_rows >= 1");
    if ((int64_t)cb->n_seg * cb->n_rows > (int64_t)INT32_MAX / 16)
        return fail(ISA_EKV_EINVAL, "codebook too large (n_seg * n_rows records)");
    if (!cb->slopes || !cb->intercepts) return fail(ISA_EKV_EINVAL, "codebook slopes/intercepts are null");
    if (cb->seg_mode < ISA_EKV_SEG_UNIFORM || cb->seg_mode > ISA_EKV_SEG_ROUND)
        return fail(ISA_EKV_EINVAL, "unknown segment mode %d", cb->seg_mode);
    if (cb->seg_mode == ISA_EKV_SEG_SEARCH && !cb->vg) return fail(ISA_EKV_EINVAL, "segment search needs vg");
    if (!(cb->lookup_max >= cb->lookup_min)) return fail(ISA_EKV_EINVAL, "lookup range needs lookup_max >= lookup_min");
    if (!ids_a) return fail(ISA_EKV_EINVAL, "ids_a is null");
    return 0;
}

MeasuredPrepArgs measured_prep(const isa_ekv_codebook* cb, const float* x, const short* ids_a, const short* ids_b,
                               int64_t M, int64_t K, int64_t O, int64_t Kp, int64_t Op, int rec_floats, float* xrec,
                               float2* idT, float2* table) {
    MeasuredPrepArgs pa{};
    pa.x = x;
    pa.ids_a = ids_a;
    pa.ids_b = ids_b;
    pa.slopes = cb->slopes;
    pa.intercepts = cb->intercepts;
    pa.vg = cb->vg;
    pa.M = M;
    pa.K = K;
    pa.O = O;
    pa.Kp = Kp;
    pa.Op = Op;
    pa.n_seg = cb->n_seg;
    pa.n_rows = cb->n_rows;
    pa.seg_mode = cb->seg_mode;
    pa.voltage_min = cb->voltage_min;
    pa.inverse_step = cb->inverse_step;
    pa.lookup_min = cb->lookup_min;
    pa.lookup_max = cb->lookup_max;
    pa.rec_floats = rec_floats;
    pa.xrec = xrec;
    pa.idT = idT;
    pa.table = table;
    return pa;
}

template <bool PAIR>
void launch_fwd_measured(bool lds, int mr, dim3 grid, size_t lds_bytes, hipStream_t s, const FwdArgs& fa) {
    const dim3 block(kFwdWaves * 64);
    if (lds) {
        if (mr == 8) hipLaunchKernelGGL((fwd_measured_kernel<8, PAIR, true>), grid, block, lds_bytes, s, fa);
        else if (mr == 4) hipLaunchKernelGGL((fwd_measured_kernel<4, PAIR, true>), grid, block, lds_bytes, s, fa);
        else hipLaunchKernelGGL((fwd_measured_kernel<2, PAIR, true>), grid, block, lds_bytes, s, fa);
    } else {
        if (mr == 8) hipLaunchKernelGGL((fwd_measured_kernel<8, PAIR, false>), grid, block, 0, s, fa);
        else if (mr == 4) hipLaunchKernelGGL((fwd_measured_kernel<4, PAIR, false>), grid, block, 0, s, fa);
        else hipLaunchKernelGGL((fwd_measured_kernel<2, PAIR, false>), grid, block, 0, s, fa);
    }
}

int run_measured_forward(const float* x, const short* ids_a, const short* ids_b, int64_t M, int64_t K, int64_t O,
                         const isa_ekv_codebook* cb, float current_scale, const float* r_tia, float out_min,
                         float out_max, float* out_pre, float* out, void* workspace, size_t workspace_bytes,
                         hipStream_t s) {
    if (M == 0 || O == 0) return 0;
    if (!out) return fail(ISA_EKV_EINVAL, "out is null");
    const FwdPlan p = plan_forward(M, K, O, false, false);
    const size_t tbytes = measured_table_bytes(cb->n_seg, cb->n_rows);
    const size_t need = p.bytes + tbytes;
    if (!workspace || workspace_bytes < need)
        return fail(ISA_EKV_EINVAL, "forward workspace too small (%zu < %zu bytes)", workspace_bytes, need);
    char* ws = static_cast<char*>(workspace);
    CallTimer call_timer(s, 2);
    float2* table = reinterpret_cast<float2*>(ws + p.bytes);
    const MeasuredPrepArgs pa = measured_prep(cb, x, ids_a, ids_b, M, K, O, p.Kp, p.Op, 2,
                                              reinterpret_cast<float*>(ws + p.off_xrec),
                                              reinterpret_cast<float2*>(ws + p.off_wsT), table);
    hipLaunchKernelGGL(measured_prep_kernel, dim3(kPrepBlocksX + 2 * kPrepBlocksW), dim3(256), 0, s, pa);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return hip_fail(err, "measured prep launch");
    FwdArgs fa{};
    fa.xrec = reinterpret_cast<const float2*>(ws + p.off_xrec);
    fa.wsT = reinterpret_cast<const float2*>(ws + p.off_wsT);
    fa.lut = table;
    fa.out = out;
    fa.M = (int)M;
    fa.O = (int)O;
    fa.Kp = (int)p.Kp;
    fa.Op = (int)p.Op;
    fa.NP = cb->n_seg * cb->n_rows + 1;
    fa.n_mt = p.n_mt;
    fa.n_ot = p.n_ot;
    fa.out_scale = current_scale;
    fa.glue = 1;
    fa.idiff = out_pre;
    fa.r_tia = r_tia;
    fa.y_lo = out_min;
    fa.y_hi = out_max;
    const size_t lds_bytes = (size_t)fa.NP * 8;
    const bool lds = lds_bytes <= kMeasuredLdsBytes;
    ProfiledLaunch* prof;
    prof_start(s, 0, &prof);
    if (ids_b)
        launch_fwd_measured<false>(lds, p.mr, dim3(p.blocks), lds_bytes, s, fa);
    else
        launch_fwd_measured<true>(lds, p.mr, dim3(p.blocks), lds_bytes, s, fa);
    err = hipGetLastError();
    prof_stop(s, prof);
    if (err != hipSuccess) return hip_fail(err, "measured forward launch");
    return 0;
}

int run_measured_backward(const float* x, const short* ids_a, const short* ids_b, int64_t M, int64_t K, int64_t O,
                          const isa_ekv_codebook* cb, float current_scale, const float* grad_out,
                          const float* out_pre,
                          const float* r_tia, float out_min, float out_max, float* grad_x, void* workspace,
                          size_t workspace_bytes, hipStream_t s) {
    if (!grad_x) return 0;
    hipError_t err;
    if (M == 0 || K == 0 || O == 0) {
        zero_fill(grad_x, M * K, s);
        err = hipGetLastError();
        if (err != hipSuccess) return hip_fail(err, "zero fill launch");
        return 0;
    }
    if (!grad_out || !out_pre) return fail(ISA_EKV_EINVAL, "grad_out/out_pre is null");
    BwdPlan p = plan_backward(M, K, O, 0, true, false, true);
    const size_t tbytes = measured_table_bytes(cb->n_seg, cb->n_rows);
    const size_t need = p.bytes + tbytes;
    if (!workspace || workspace_bytes < need)
        return fail(ISA_EKV_EINVAL, "backward workspace too small (%zu < %zu bytes)", workspace_bytes, need);
    char* ws = static_cast<char*>(workspace);
    CallTimer call_timer(s, 3);
    float2* table = reinterpret_cast<float2*>(ws + p.bytes);
    const MeasuredPrepArgs pa = measured_prep(cb, x, ids_a, ids_b, M, K, O, p.Kp, p.Op, 4,
                                              reinterpret_cast<float*>(ws + p.off_xrec),
                                              reinterpret_cast<float2*>(ws + p.off_wsT), table);
    hipLaunchKernelGGL(measured_prep_kernel, dim3(kPrepBlocksX + 2 * kPrepBlocksW), dim3(256), 0, s, pa);
    err = hipGetLastError();
    if (err != hipSuccess) return hip_fail(err, "measured prep launch");
    float* col_part = reinterpret_cast<float*>(ws + p.off_glue);
    float* r_part = col_part + (size_t)round_up((int64_t)kGlueBlocks * 2 * p.Op * 4, 256) / 4;
    GlueGradArgs ga{grad_out, out_pre, M, O, p.Op, r_tia, nullptr, 0.0f, 0.0f, out_min, out_max, nullptr,
                    reinterpret_cast<float*>(ws + p.off_gpad), col_part, r_part};
    hipLaunchKernelGGL(glue_grad_kernel, dim3(kGlueBlocks, (unsigned)(p.Op / 256)), dim3(256), 0, s, ga);
    err = hipGetLastError();
    if (err != hipSuccess) return hip_fail(err, "measured grad prep launch");
    const int np = cb->n_seg * cb->n_rows + 1;
    const bool lds = (size_t)np * 8 <= kMeasuredBwdLdsTableBytes;
    BwdArgs ba{};
    ba.xrec = reinterpret_cast<const float4*>(ws + p.off_xrec);
    ba.wsT = reinterpret_cast<const float2*>(ws + p.off_wsT);
    ba.grad = reinterpret_cast<const float*>(ws + p.off_gpad);
    ba.lut = reinterpret_cast<const float4*>(table);
    ba.dx_part = reinterpret_cast<float*>(ws + p.off_dx);
    ba.M = (int)M;
    ba.K = (int)K;
    ba.O = (int)O;
    ba.Kp = (int)p.Kp;
    ba.Op = (int)p.Op;
    ba.ldg = (int)p.Op;
    ba.NP = np;
    ba.n_ob = p.n_ob;
    ba.n_kb = p.n_kb;
    ba.n_split = p.n_split;
    ba.m_chunk = p.m_chunk;
    ba.n_items = p.n_items;
    const size_t lds_bytes = lds ? round_up((int64_t)np * 8, 16) : 0;
    const dim3 grid(p.blocks), block(p.waves_per_block * 64);
    ProfiledLaunch* prof;
    prof_start(s, 1, &prof);
    if (ids_b) {
        if (lds) hipLaunchKernelGGL((bwd_measured_kernel<false, true>), grid, block, lds_bytes, s, ba);
        else hipLaunchKernelGGL((bwd_measured_kernel<false, false>), grid, block, lds_bytes, s, ba);
    } else {
        if (lds) hipLaunchKernelGGL((bwd_measured_kernel<true, true>), grid, block, lds_bytes, s, ba);
        else hipLaunchKernelGGL((bwd_measured_kernel<true, false>), grid, block, lds_bytes, s, ba);
    }
    err = hipGetLastError();
    prof_stop(s, prof);
    if (err != hipSuccess) return hip_fail(err, "measured backward launch");
    const DxReduceArgs dxa{reinterpret_cast<const float*>(ws + p.off_dx), p.n_ob, M * K, current_scale, grad_x, x,
                           nullptr, cb->lookup_min, cb->lookup_max, nullptr, 1};
    hipLaunchKernelGGL(dx_reduce_kernel, dim3((unsigned)dx_reduce_blocks(M * K)), dim3(256), 0, s, dxa);
    err = hipGetLastError();
    if (err != hipSuccess) return hip_fail(err, "dx reduce launch");
    return 0;
}
}  // namespace

// ----------------------------------------------------------------------------------
// No-allocation forward (isa_ekv_forward_noalloc). Its workspace is `scratch`, a file-scope
// device array of kScratchBytes that every device the library runs on holds from module load
// to process end, so a caller that cannot allocate (HIP graph capture, serving loops) still
// gets the forward. In host code `scratch` names a host-side stand-in, not device memory: the
// array's address on the current device comes from hipGetSymbolAddress, resolved once per
// device on the first call there and kept in g_scratch_ptr, and only that pointer is handed to
// kernels. Every workspace byte the forward reads is written earlier in the same call (token
// and threshold records, range partials, the table-copy mode word, K-split planes), so nothing
// needs clearing between calls; calls that overlap on one device share the array and race.
// ----------------------------------------------------------------------------------

constexpr size_t kScratchBytes = ISA_EKV_NOALLOC_MAX_BYTES;  // 128 MiB per device (the GPT-L fc1 forward needs 66)
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kScratchMaxDevices = 64;
std::mutex g_scratch_lock;
void* g_scratch_ptr[kScratchMaxDevices] = {};

// The current device's address of `scratch` (resolved on the first call on that device).
int scratch_for_current_device(void** ptr) {
    int dev = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) return hip_fail(err, "hipGetDevice");
    if (dev < 0 || dev >= kScratchMaxDevices)
        return fail(ISA_EKV_EINVAL, "device %d is past the %d devices the scratch table covers", dev,
                    kScratchMaxDevices);
    std::lock_guard<std::mutex> guard(g_scratch_lock);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (err != hipSuccess) return hip_fail(err, "hipGetSymbolAddress(scratch)");
        if (!p) return fail(ISA_EKV_EINVAL, "hipGetSymbolAddress(scratch) returned null");
        g_scratch_ptr[dev] = p;
    }
    *ptr = g_scratch_ptr[dev];
    return 0;
}

}  // namespace

// ----------------------------------------------------------------------------------
// C ABI
// ----------------------------------------------------------------------------------

extern "C" {

int isa_ekv_abi_version(void) { return ISA_EKV_ABI_VERSION; }

const char* isa_ekv_last_error(void) { return g_last_error; }

int isa_ekv_lut_pad(void) { return kPad; }

size_t isa_ekv_lut_bytes(int n_entries, int layout) {
    if (n_entries < 1) return 0;
    switch (layout) {
        case ISA_EKV_LUT_PLAIN_F32: return (size_t)n_entries * 2 * 4;
        case ISA_EKV_LUT_PLAIN_BF16: return (size_t)n_entries * 2 * 2;
        case ISA_EKV_LUT_FWD: return (size_t)lut_records(n_entries) * 8;
        case ISA_EKV_LUT_BWD: return (size_t)lut_records(n_entries) * 16;
        default: return 0;
    }
}

int isa_ekv_lut_build(const double params[4], double delta_min, double delta_max, int n_entries, int layout,
                      void* dst, void* stream) {
    if (!params) return fail(ISA_EKV_EINVAL, "params is null");
    if (!dst) return fail(ISA_EKV_EINVAL, "dst is null");
    if (n_entries < 1) return fail(ISA_EKV_EINVAL, "LUT_DELTA_SIZE must be >= 1 (got %d)", n_entries);
    if (!(delta_max > delta_min)) return fail(ISA_EKV_EINVAL, "LUT range must satisfy delta_max > delta_min");
    if (isa_ekv_lut_bytes(n_entries, layout) == 0) return fail(ISA_EKV_EINVAL, "unknown LUT layout %d", layout);
    if (!(params[0] > 0.0) || !(params[1] > 0.0))
        return fail(ISA_EKV_EINVAL, "n and U_T must be positive");
    DeviceParams p{params[0], params[1], params[2], params[3], delta_min, delta_max, n_entries};
    const int total = (layout == ISA_EKV_LUT_PLAIN_F32 || layout == ISA_EKV_LUT_PLAIN_BF16)
                          ? n_entries
                          : n_entries + 2 * kPad;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(lut_build_kernel, dim3((total + 255) / 256), dim3(256), 0, s, p, layout, dst);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return hip_fail(err, "lut_build launch");
    return 0;
}

int isa_ekv_lut_pack(const void* table_i, const void* table_ddelta, int n_entries, int src_dtype, int layout,
                     void* dst, void* stream) {
    if (!table_i || !dst) return fail(ISA_EKV_EINVAL, "table_i/dst is null");
    if (layout == ISA_EKV_LUT_BWD && !table_ddelta) return fail(ISA_EKV_EINVAL, "table_ddelta is null");
    if (n_entries < 1) return fail(ISA_EKV_EINVAL, "LUT_DELTA_SIZE must be >= 1 (got %d)", n_entries);
    if (layout != ISA_EKV_LUT_FWD && layout != ISA_EKV_LUT_BWD)
        return fail(ISA_EKV_EINVAL, "pack layout must be ISA_EKV_LUT_FWD or ISA_EKV_LUT_BWD (got %d)", layout);
    if (src_dtype != ISA_EKV_DTYPE_F32 && src_dtype != ISA_EKV_DTYPE_BF16)
        return fail(ISA_EKV_EINVAL, "unknown table dtype %d", src_dtype);
    const int total = n_entries + 2 * kPad;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(lut_pack_kernel, dim3((total + 255) / 256), dim3(256), 0, s, table_i, table_ddelta, n_entries,
                       src_dtype == ISA_EKV_DTYPE_BF16 ? 1 : 0, layout, dst);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return hip_fail(err, "lut_pack launch");
    return 0;
}

int isa_ekv_profile_begin(void) {
    for (int i = 0; i < g_prof_count; ++i) {
        (void)hipEventDestroy(g_prof[i].start);
        (void)hipEventDestroy(g_prof[i].stop);
    }
    g_prof_count = 0;
    int dev = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) {  // no device: event timing only (nothing will launch)
        (void)hipGetLastError();
        g_profiling = true;
        return 0;
    }
    if (dev >= 0 && dev < kClockMaxDevices) {
        const size_t bytes = 3 * kClockKinds * sizeof(unsigned long long);
        if (!g_clock_buf[dev]) {
            err = hipMalloc(reinterpret_cast<void**>(&g_clock_buf[dev]), bytes);
            if (err != hipSuccess) {
                g_clock_buf[dev] = nullptr;
                return hip_fail(err, "clock sample buffer");
            }
        }
        err = hipMemset(g_clock_buf[dev], 0, bytes);  // synchronous: before any profiled launch
        if (err != hipSuccess) return hip_fail(err, "clock sample buffer clear");
    }
    g_profiling = true;
    return 0;
}

int isa_ekv_profile_clock(double* out) {
    static_assert(kClockKinds == 4, "isa_ekv_profile_clock writes 12 values");
    if (!out) return fail(ISA_EKV_EINVAL, "out is null");
    for (int i = 0; i < 3 * kClockKinds; ++i) out[i] = 0.0;
    int dev = 0, khz = 0;
    if (hipGetDevice(&dev) != hipSuccess) {  // no device: nothing was sampled
        (void)hipGetLastError();
        return 0;
    }
    if (dev < 0 || dev >= kClockMaxDevices || !g_clock_buf[dev]) return 0;
    hipError_t err = hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev);
    if (err != hipSuccess) return hip_fail(err, "wall clock rate query");
    if (khz <= 0) return 0;
    unsigned long long h[3 * kClockKinds];
    err = hipMemcpy(h, g_clock_buf[dev], sizeof(h), hipMemcpyDeviceToHost);  // after the profiled work
    if (err != hipSuccess) return hip_fail(err, "clock sample read");
    for (int k = 0; k < kClockKinds; ++k) {
        out[3 * k] = (double)h[3 * k];
        out[3 * k + 1] = (double)h[3 * k + 1] / (1e3 * khz);
        out[3 * k + 2] = (double)h[3 * k + 2];
    }
    return 0;
}

int isa_ekv_profile_end(double* ms, int* launches) {
    g_profiling = false;
    double t[kProfKinds] = {0.0, 0.0, 0.0, 0.0};
    int c[kProfKinds] = {0, 0, 0, 0};
    int rc = 0;
    for (int i = 0; i < g_prof_count; ++i) {
        float ms = 0.0f;
        hipError_t err = hipEventSynchronize(g_prof[i].stop);
        if (err == hipSuccess) err = hipEventElapsedTime(&ms, g_prof[i].start, g_prof[i].stop);
        if (err != hipSuccess && rc == 0) rc = hip_fail(err, "profile event");
        t[g_prof[i].kind] += ms;
        c[g_prof[i].kind] += 1;
        (void)hipEventDestroy(g_prof[i].start);
        (void)hipEventDestroy(g_prof[i].stop);
    }
    g_prof_count = 0;
    for (int k = 0; k < kProfKinds; ++k) {
        if (ms) ms[k] = t[k];
        if (launches) launches[k] = c[k];
    }
    return rc;
}

size_t isa_ekv_forward_workspace(int64_t M, int64_t K, int64_t O) {
    if (M < 0 || K < 0 || O < 0) return 0;
    // the table size is not an argument: cover both block shapes run_forward may plan
    return std::max(plan_forward(M, K, O, false).bytes, plan_forward(M, K, O, false, true, 2 * kFwdWaves).bytes);
}

int isa_ekv_forward(const float* x, const float* vth_pos, const float* vth_neg, const void* lut_fwd, int64_t M,
                    int64_t K, int64_t O, int n_entries, float delta_min, float delta_max, float v_sat,
                    float out_min, float out_max, float* out, void* workspace, size_t workspace_bytes,
                    void* stream) {
    const int rc = check_common(x, vth_pos, vth_neg, lut_fwd, M, K, O, n_entries, delta_min, delta_max, v_sat);
    if (rc) return rc;
    if (n_entries > kMaxEntriesGlobal)
        return fail(ISA_EKV_EINVAL, "LUT forward supports LUT_DELTA_SIZE <= %d (got %d)", kMaxEntriesGlobal,
                    n_entries);
    return run_forward(lut_setup(lut_fwd, n_entries, delta_min, delta_max), x, vth_pos, vth_neg, M, K, O, v_sat,
                       out_min, out_max, out, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

int isa_ekv_forward_noalloc(const float* x, const float* vth_pos, const float* vth_neg, const void* lut_fwd,
                            int64_t M, int64_t K, int64_t O, int n_entries, float delta_min, float delta_max,
                            float v_sat, float out_min, float out_max, float* out, void* stream) {
    const int rc = check_common(x, vth_pos, vth_neg, lut_fwd, M, K, O, n_entries, delta_min, delta_max, v_sat);
    if (rc) return rc;
    if (n_entries > kMaxEntriesGlobal)
        return fail(ISA_EKV_EINVAL, "LUT forward supports LUT_DELTA_SIZE <= %d (got %d)", kMaxEntriesGlobal,
                    n_entries);
    if (M == 0 || O == 0) return 0;
    const size_t need = plan_forward_call(false, n_entries, M, K, O).bytes;
    if (need > kScratchBytes)
        return fail(ISA_EKV_EINVAL,
                    "isa_ekv_forward_noalloc: shape (M=%lld, K=%lld, O=%lld) needs %zu bytes of scratch, more "
                    "than its %zu-byte maximum; use isa_ekv_forward with a workspace",
                    (long long)M, (long long)K, (long long)O, need, kScratchBytes);
    void* ws = nullptr;
    const int src = scratch_for_current_device(&ws);
    if (src) return src;
    return run_forward(lut_setup(lut_fwd, n_entries, delta_min, delta_max), x, vth_pos, vth_neg, M, K, O, v_sat,
                       out_min, out_max, out, ws, kScratchBytes, static_cast<hipStream_t>(stream), nullptr, nullptr,
                       false);
}

size_t isa_ekv_backward_workspace(int64_t M, int64_t K, int64_t O, int n_entries, int need_grad_x,
                                  int need_grad_w) {
    if (M < 0 || K < 0 || O < 0 || n_entries < 1) return 0;
    return plan_backward(M, K, O, n_entries, need_grad_x != 0, need_grad_w != 0).bytes;
}

int isa_ekv_backward(const float* x, const float* vth_pos, const float* vth_neg, const float* grad_out,
                     const void* lut_bwd, int64_t M, int64_t K, int64_t O, int n_entries, float delta_min,
                     float delta_max, float v_sat, float* grad_x, float* grad_vth_pos, float* grad_vth_neg,
                     void* workspace, size_t workspace_bytes, void* stream) {
    const int rc = check_common(x, vth_pos, vth_neg, lut_bwd, M, K, O, n_entries, delta_min, delta_max, v_sat);
    if (rc) return rc;
    if (n_entries > kMaxEntriesGlobal)
        return fail(ISA_EKV_EINVAL, "LUT backward supports LUT_DELTA_SIZE <= %d (got %d)", kMaxEntriesGlobal,
                    n_entries);
    return run_backward(lut_setup(lut_bwd, n_entries, delta_min, delta_max), x, vth_pos, vth_neg, grad_out, M, K,
                        O, v_sat, grad_x, grad_vth_pos, grad_vth_neg, workspace, workspace_bytes,
                        static_cast<hipStream_t>(stream));
}

size_t isa_ekv_exact_forward_workspace(int64_t M, int64_t K, int64_t O) {
    if (M < 0 || K < 0 || O < 0) return 0;
    return plan_forward(M, K, O, true).bytes;
}

int isa_ekv_exact_forward(const float* x, const float* vth_pos, const float* vth_neg, int64_t M, int64_t K,
                          int64_t O, const double params[4], float v_sat, float* out, void* workspace,
                          size_t workspace_bytes, void* stream) {
    int rc = check_shapes(x, vth_pos, vth_neg, M, K, O, v_sat);
    if (rc) return rc;
    CallSetup cs;
    rc = exact_setup(params, &cs);
    if (rc) return rc;
    return run_forward(cs, x, vth_pos, vth_neg, M, K, O, v_sat, -INFINITY, INFINITY, out, workspace,
                       workspace_bytes, static_cast<hipStream_t>(stream));
}

size_t isa_ekv_exact_backward_workspace(int64_t M, int64_t K, int64_t O, int need_grad_x, int need_grad_w) {
    if (M < 0 || K < 0 || O < 0) return 0;
    return plan_backward(M, K, O, 0, need_grad_x != 0, need_grad_w != 0).bytes;
}

int isa_ekv_exact_backward(const float* x, const float* vth_pos, const float* vth_neg, const float* grad_out,
                           int64_t M, int64_t K, int64_t O, const double params[4], float v_sat, float* grad_x,
                           float* grad_vth_pos, float* grad_vth_neg, void* workspace, size_t workspace_bytes,
                           void* stream) {
    int rc = check_shapes(x, vth_pos, vth_neg, M, K, O, v_sat);
    if (rc) return rc;
    CallSetup cs;
    rc = exact_setup(params, &cs);
    if (rc) return rc;
    return run_backward(cs, x, vth_pos, vth_neg, grad_out, M, K, O, v_sat, grad_x, grad_vth_pos, grad_vth_neg,
                        workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

size_t isa_ekv_layer_forward_workspace(int64_t M, int64_t K, int64_t O) {
    return isa_ekv_forward_workspace(M, K, O);
}

size_t isa_ekv_layer_backward_workspace(int64_t M, int64_t K, int64_t O, int n_entries, int need_grad_x,
                                        int need_grad_w) {
    if (M < 0 || K < 0 || O < 0 || n_entries < 1) return 0;
    return plan_backward(M, K, O, n_entries, need_grad_x != 0, need_grad_w != 0, true).bytes;
}

int isa_ekv_layer_forward(const float* x, const float* vth_pos, const float* vth_neg, const void* lut_fwd, int64_t M,
                          int64_t K, int64_t O, int n_entries, float delta_min, float delta_max, float v_sat,
                          float idiff_min, float idiff_max, const isa_ekv_glue* glue, float* idiff, float* out,
                          void* workspace, size_t workspace_bytes, void* stream) {
    int rc = check_common(x, vth_pos, vth_neg, lut_fwd, M, K, O, n_entries, delta_min, delta_max, v_sat);
    if (rc) return rc;
    rc = check_glue(glue, nullptr, false);
    if (rc) return rc;
    if (n_entries > kMaxEntriesGlobal)
        return fail(ISA_EKV_EINVAL, "LUT forward supports LUT_DELTA_SIZE <= %d (got %d)", kMaxEntriesGlobal,
                    n_entries);
    return run_forward(lut_setup(lut_fwd, n_entries, delta_min, delta_max), x, vth_pos, vth_neg, M, K, O, v_sat,
                       idiff_min, idiff_max, out, workspace, workspace_bytes, static_cast<hipStream_t>(stream), glue,
                       idiff);
}

int isa_ekv_layer_backward(const float* x, const float* vth_pos, const float* vth_neg, const float* grad_out,
                           const float* idiff, const void* lut_bwd, int64_t M, int64_t K, int64_t O, int n_entries,
                           float delta_min, float delta_max, float v_sat, const isa_ekv_glue* glue, float* grad_x,
                           float* grad_vth_pos, float* grad_vth_neg, const isa_ekv_glue_grads* glue_grads,
                           void* workspace, size_t workspace_bytes, void* stream) {
    int rc = check_common(x, vth_pos, vth_neg, lut_bwd, M, K, O, n_entries, delta_min, delta_max, v_sat);
    if (rc) return rc;
    rc = check_glue(glue, glue_grads, grad_x != nullptr || M * K == 0);
    if (rc) return rc;
    if (n_entries > kMaxEntriesGlobal)
        return fail(ISA_EKV_EINVAL, "LUT backward supports LUT_DELTA_SIZE <= %d (got %d)", kMaxEntriesGlobal,
                    n_entries);
    if (M * O > 0 && !idiff) return fail(ISA_EKV_EINVAL, "idiff is null");
    return run_backward(lut_setup(lut_bwd, n_entries, delta_min, delta_max), x, vth_pos, vth_neg, grad_out, M, K,
                        O, v_sat, grad_x, grad_vth_pos, grad_vth_neg, workspace, workspace_bytes,
                        static_cast<hipStream_t>(stream), glue, idiff, glue_grads);
}

size_t isa_ekv_measured_forward_workspace(int64_t M, int64_t K, int64_t O, int n_seg, int n_rows) {
    if (M < 0 || K < 0 || O < 0 || n_seg < 1 || n_rows < 1) return 0;
    return plan_forward(M, K, O, false, false).bytes + measured_table_bytes(n_seg, n_rows);
}

size_t isa_ekv_measured_backward_workspace(int64_t M, int64_t K, int64_t O, int n_seg, int n_rows) {
    if (M < 0 || K < 0 || O < 0 || n_seg < 1 || n_rows < 1) return 0;
    return plan_backward(M, K, O, 0, true, false, true).bytes + measured_table_bytes(n_seg, n_rows);
}

int isa_ekv_measured_forward(const float* x, const int16_t* ids_a, const int16_t* ids_b, int64_t M, int64_t K,
                             int64_t O, const isa_ekv_codebook* codebook, float current_scale, const float* r_tia,
                             float out_min, float out_max, float* out_pre, float* out, void* workspace,
                             size_t workspace_bytes, void* stream) {
    int rc = check_codebook(codebook, reinterpret_cast<const short*>(ids_a));
    if (rc) return rc;
    // the id arrays stand where the threshold arrays are checked
    rc = check_shapes(x, reinterpret_cast<const float*>(ids_a), reinterpret_cast<const float*>(ids_a), M, K, O, 1.0f);
    if (rc) return rc;
    if (!r_tia) return fail(ISA_EKV_EINVAL, "r_tia is null");
    if (!(out_max >= out_min)) return fail(ISA_EKV_EINVAL, "output range needs out_max >= out_min");
    return run_measured_forward(x, reinterpret_cast<const short*>(ids_a), reinterpret_cast<const short*>(ids_b), M,
                                K, O, codebook, current_scale, r_tia, out_min, out_max, out_pre, out, workspace,
                                workspace_bytes, static_cast<hipStream_t>(stream));
}

int isa_ekv_measured_backward(const float* x, const int16_t* ids_a, const int16_t* ids_b, int64_t M, int64_t K,
                              int64_t O, const isa_ekv_codebook* codebook, float current_scale,
                              const float* grad_out, const float* out_pre, const float* r_tia, float out_min,
                              float out_max, float* grad_x, void* workspace, size_t workspace_bytes, void* stream) {
    int rc = check_codebook(codebook, reinterpret_cast<const short*>(ids_a));
    if (rc) return rc;
    // the id arrays stand where the threshold arrays are checked
    rc = check_shapes(x, reinterpret_cast<const float*>(ids_a), reinterpret_cast<const float*>(ids_a), M, K, O, 1.0f);
    if (rc) return rc;
    if (!r_tia) return fail(ISA_EKV_EINVAL, "r_tia is null");
    if (!(out_max >= out_min)) return fail(ISA_EKV_EINVAL, "output range needs out_max >= out_min");
    return run_measured_backward(x, reinterpret_cast<const short*>(ids_a), reinterpret_cast<const short*>(ids_b), M,
                                 K, O, codebook, current_scale, grad_out, out_pre, r_tia, out_min, out_max, grad_x,
                                 workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

int isa_ekv_plan_info(int which, int64_t M, int64_t K, int64_t O, int n_entries, int need_grad_x, int need_grad_w,
                      int64_t* info, int n_info) {
    if (!info || n_info < 1) return fail(ISA_EKV_EINVAL, "info is null");
    if (M < 0 || K < 0 || O < 0) return fail(ISA_EKV_EINVAL, "negative shape");
    if (n_entries < 1 || n_entries > kMaxEntriesGlobal)
        return fail(ISA_EKV_EINVAL, "LUT_DELTA_SIZE must be in [1, %d] (got %d)", kMaxEntriesGlobal, n_entries);
    int64_t v[ISA_EKV_PLAN_INFO_LEN];
    if (which == ISA_EKV_PLAN_FORWARD) {
        const FwdPlan p = plan_forward_call(false, n_entries, M, K, O);
        const FwdTableCfg tc = fwd_table_cfg(n_entries, p.wpb, copies_pay(M, K, O));
        v[0] = (int64_t)p.bytes;
        v[1] = tc.copy_offset > 0 || tc.mc_budget > 0 ? (int64_t)p.off_mode : -1;
        v[2] = p.n_split;
        v[3] = p.mr;
        v[4] = p.blocks;
        v[5] = p.wpb;
        v[6] = (int64_t)tc.lds;
        v[7] = 0;
    } else if (which == ISA_EKV_PLAN_BACKWARD || which == ISA_EKV_PLAN_LAYER_BACKWARD) {
        const bool nx = need_grad_x != 0, nw = need_grad_w != 0;
        const BwdPlan p = plan_backward(M, K, O, n_entries, nx, nw, which == ISA_EKV_PLAN_LAYER_BACKWARD);
        v[0] = (int64_t)p.bytes;
        v[1] = bwd_may_use_copies(p, false, nx) ? (int64_t)p.off_mode : -1;
        v[2] = p.n_split;
        v[3] = p.Kp / p.n_kb;
        v[4] = p.blocks;
        v[5] = p.waves_per_block;
        v[6] = (int64_t)p.lds_bytes;
        v[7] = nw ? p.dv_planes : 0;
    } else {
        return fail(ISA_EKV_EINVAL, "unknown plan kind %d", which);
    }
    for (int i = 0; i < n_info; ++i) info[i] = i < ISA_EKV_PLAN_INFO_LEN ? v[i] : 0;
    return 0;
}

int isa_ekv_set_option(int option, int64_t value, int64_t* previous) {
    std::atomic<int64_t>* opt = option == ISA_EKV_OPT_COPY_MIN_CELLS      ? &g_copy_min_cells
                                : option == ISA_EKV_OPT_RANKED          ? &g_ranked
                                : option == ISA_EKV_OPT_WINDOW_COPIES   ? &g_window_copies
                                : option == ISA_EKV_OPT_RANK_MAX_SPREAD ? &g_rank_max_spread
                                : option == ISA_EKV_OPT_RANK_GREEDY_MIN ? &g_rank_greedy_min
                                : option == ISA_EKV_OPT_RANK_XCD_ORDER  ? &g_rank_xcd_order
                                                                        : nullptr;
    if (!opt) return fail(ISA_EKV_EINVAL, "unknown option %d", option);
    const int64_t old = value >= 0 ? opt->exchange(value) : opt->load();
    if (previous) *previous = old;
    return 0;
}

int isa_ekv_probe_lds_gather(int window_records, int record_bytes, int iterations, float* out, int64_t out_floats,
                             int* gathers_per_cu, int64_t* clocks, int* wall_clock_khz, void* stream) {
    if (record_bytes != 8 && record_bytes != 16)
        return fail(ISA_EKV_EINVAL, "record_bytes must be 8 or 16 (got %d)", record_bytes);
    if (window_records < 1 || window_records > kProbeLdsBytes / record_bytes)
        return fail(ISA_EKV_EINVAL, "window_records must be in [1, %d] (got %d)", kProbeLdsBytes / record_bytes,
                    window_records);
    if (iterations < 1 || iterations > (1 << 20))
        return fail(ISA_EKV_EINVAL, "iterations must be in [1, 2^20] (got %d)", iterations);
    int dev = 0, cus = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err == hipSuccess) err = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (err != hipSuccess) return hip_fail(err, "device query");
    const int blocks = kProbeBlocksPerCU * cus;
    if (!out || out_floats < (int64_t)blocks * 1024)
        return fail(ISA_EKV_EINVAL, "out needs %lld floats (one per thread of %d blocks)", (long long)blocks * 1024,
                    blocks);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (wall_clock_khz) {
        err = hipDeviceGetAttribute(wall_clock_khz, hipDeviceAttributeWallClockRate, dev);
        if (err != hipSuccess) return hip_fail(err, "wall clock rate query");
    }
    long long* clk = reinterpret_cast<long long*>(clocks);
    if (record_bytes == 8)
        hipLaunchKernelGGL(lds_gather_probe_kernel<8>, dim3(blocks), dim3(1024), kProbeLdsBytes, s, window_records,
                           iterations, 12345u, out, clk);
    else
        hipLaunchKernelGGL(lds_gather_probe_kernel<16>, dim3(blocks), dim3(1024), kProbeLdsBytes, s, window_records,
                           iterations, 12345u, out, clk);
    err = hipGetLastError();
    if (err != hipSuccess) return hip_fail(err, "lds probe launch");
    if (gathers_per_cu) *gathers_per_cu = kProbeBlocksPerCU * 16 * 8 * iterations;
    return 0;
}

int isa_ekv_probe_valu_issue(int mix, int iterations, const float* tokens, float* out, int64_t out_floats,
                             int64_t* clocks, double* instr_per_cu, int* wall_clock_khz, void* stream) {
    if (mix < 0 || mix > 3) return fail(ISA_EKV_EINVAL, "mix must be 0, 1, 2 or 3 (got %d)", mix);
    if (iterations < 1 || iterations > (1 << 20))
        return fail(ISA_EKV_EINVAL, "iterations must be in [1, 2^20] (got %d)", iterations);
    if (!tokens) return fail(ISA_EKV_EINVAL, "tokens is null (%d float4 token records)", kValuProbeTokens);
    int dev = 0, cus = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err == hipSuccess) err = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (err != hipSuccess) return hip_fail(err, "device query");
    const int blocks = 2 * cus, threads = kValuMixWaves[mix] * 64;
    if (!out || out_floats < (int64_t)blocks * threads)
        return fail(ISA_EKV_EINVAL, "out needs %lld floats (one per thread of %d blocks)",
                    (long long)blocks * threads, blocks);
    if (wall_clock_khz) {
        err = hipDeviceGetAttribute(wall_clock_khz, hipDeviceAttributeWallClockRate, dev);
        if (err != hipSuccess) return hip_fail(err, "wall clock rate query");
    }
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const float4* tok = reinterpret_cast<const float4*>(tokens);
    long long* clk = reinterpret_cast<long long*>(clocks);
    // half the CU's LDS per block (unused by the loops): exactly two blocks fit a CU, as the
    // table kernels run, so the blocks of a CU overlap and each CU holds two
    const size_t lds = (size_t)kLdsBytes / 2;
    if (mix == 0)
        hipLaunchKernelGGL(valu_probe_kernel<0>, dim3(blocks), dim3(threads), lds, s, iterations, tok, out, clk);
    else if (mix == 1)
        hipLaunchKernelGGL(valu_probe_kernel<1>, dim3(blocks), dim3(threads), lds, s, iterations, tok, out, clk);
    else if (mix == 2)
        hipLaunchKernelGGL(valu_probe_kernel<2>, dim3(blocks), dim3(threads), lds, s, iterations, tok, out, clk);
    else
        hipLaunchKernelGGL(valu_probe_kernel<3>, dim3(blocks), dim3(threads), lds, s, iterations, tok, out, clk);
    err = hipGetLastError();
    if (err != hipSuccess) return hip_fail(err, "valu probe launch");
    // VALU wave-instructions each CU issues in the loops: two blocks per CU
    if (instr_per_cu) *instr_per_cu = 2.0 * kValuMixWaves[mix] * (double)kValuMixInstr[mix] * iterations;
    return 0;
}

}  // extern "C"
