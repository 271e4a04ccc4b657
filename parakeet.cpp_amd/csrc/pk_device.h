// pk_device.h -- device code of the MI355X transducer greedy decode.
//
// Included once, by pk_decode.hip.  See that file for the host side and the
// overall structure; this file holds the data layout, the building blocks
// (MFMA tiles over q8_0 / f16 weights, argmax keys, domain barrier, coherent
// loads and stores) and the kernels.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "parakeet_hip.h"

namespace pkdev {

constexpr int kWave = 64;
constexpr int kBlock = 512;                 // 8 waves per workgroup, one workgroup per CU
constexpr int kWaves = kBlock / kWave;
constexpr int kTile = 16;                   // MFMA tile edge (rows = outputs, columns = utterances)
constexpr int kMaxNT = 2;                   // utterance tiles per domain
constexpr int kDomCap = kTile * kMaxNT;     // utterances per domain
constexpr int kColCap = kDomCap;            // joint columns per domain and iteration (argmax key slots)
constexpr int kSmallB = 4;                  // LSTM batch at or below which layer 0 runs redundantly
constexpr int kIdxBits = 14;                // argmax key: index field
constexpr int kStampShift = 46;             // argmax key: 14 index + 32 value bits below the stamp
constexpr unsigned kMaxStamp = (1u << 18) - 1;
constexpr int kFlagStride = 64;             // words between barrier flags (256 B)
// error word of a launch whose ordinary dispatch was not co-resident (never returned to a caller:
// the host relaunches the call cooperatively)
constexpr int kStatusNotResident = 0x7001;
constexpr int kShards = 32;                 // argmax keys: most max targets per utterance and head
constexpr int kSlotCols = 2;                // one-domain launches with at most this many joint columns
                                            // exchange argmax keys through per-workgroup slots
constexpr int kKPad = 8;                    // halves of padding per staged row (bank spread)

// Flags in the per-utterance control word.
constexpr int kFlagZeroHC = 1;              // LSTM input state is zero (init / EOU reset)
constexpr int kFlagTokOverflow = 2;
constexpr int kFlagSegOverflow = 4;
constexpr int kFlagTraceOverflow = 8;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// A weight matrix [rows][K] laid out as MFMA fragments: for row tile t and
// K block kb (32 columns), lane l holds the 8 consecutive weights of row
// 16t + l%16 starting at column 32kb + 8(l/16).  f16: 8 halves per lane,
// [t][kb][lane]; f32: two f16 planes holding hi = f16(w), lo = f16(w - hi).
// q8_0: 8 bytes q ^ 0x80 per lane and block (the int8 values offset by 128, so
// the conversion needs no xor), stored per unit of kQ8Unit = 5 blocks as one
// kQ8UnitBytes record [t][unit]: lane l's 16 bytes of blocks 0-1 (1 KB for the
// 64 lanes), of blocks 2-3 (1 KB), its 8 bytes of block 4 (512 B), then the
// block scales (the stored f16 bits), 16 bytes per row r = d[16t + r] of
// blocks 0-4 and three zeros.  A unit is then 4 wave loads (16 + 16 + 8 bytes
// of quants, 16 bytes of scales per lane) instead of 10: the products are paced
// by the number of vector memory instructions per CU, not by bytes.
//
// Products are computed transposed: the staged activations are the MFMA A
// operand (rows = utterances) and the weight fragment the B operand (columns =
// weight rows), so a D fragment lane holds ONE weight row (l%16) for four
// utterances (4(l/16) .. +3) and a q8_0 block needs one scale per lane.
struct TMat {
    const void *a;                 // fragment plane (f32 weights: the hi plane, then the lo plane)
    const void *a_lo;              // f32 weights: the lo plane (a + one plane)
    const unsigned short *scale;   // q8_0 block scales, f16 bits
    int type;                      // PK_TYPE_Q8_0, PK_TYPE_F16, PK_TYPE_F32
    int rows, tiles, KB;           // KB: stored K blocks of 32 per tile row (q8_0: padded to whole units)
    int KBa;                       // K blocks that hold weights (K / 32); blocks KBa .. KB-1 are zero
    int lds_off;                   // byte offset of this workgroup's tiles in its LDS weight cache, -1: not cached
};

constexpr int kQ8Unit = 5, kQ8UnitBytes = 2 * 1024 + 512 + 16 * 16;   // q8_0 unit record (see TMat)
constexpr int kQ8Scales = 2560;                                        // offset of its scales

// Bytes of one tile row of a matrix (KB stored blocks), as stored and as cached
// in LDS: q8_0 unit records; f16 fragments; f32 hi then lo fragments.
__host__ __device__ constexpr int tile_bytes(int type, int KB) {
    return type == PK_TYPE_Q8_0 ? KB / kQ8Unit * kQ8UnitBytes : type == PK_TYPE_F16 ? KB * 1024 : KB * 2048;
}

struct KParams {
    int kind, H, L, J, V1, Dn, Vo, blank, eou, eob, max_sym, n_dur;
    int durations[PK_MAX_DURATIONS];
    const float *eproj;                      // [V1][4H] W_ih0 . embed[v] + b_ih0 + b_hh0, unit-major
    TMat w_ih[PK_MAX_LAYERS], w_hh[PK_MAX_LAYERS];   // unit-major gate rows (w_ih[0] unused)
    const float *b_lstm[PK_MAX_LAYERS];      // b_ih + b_hh (unit-major), layers >= 1
    TMat w_pred, w_out;
    const float *b_pred, *b_out;
    const unsigned char *special;
    int n_special;
    // slot state (persistent between calls)
    float *slot_h;       // [slots][L][H]
    float *slot_c;       // [slots][L][H]
    float *slot_pp;      // [slots][J]  b_p + W_p . h[L-1]
    float *slot_r;       // [slots][L][4H]  W_hh . h (no bias), unit-major rows
    int *slot_ctrl;      // [slots][PK_CTRL_N]
    // batch
    int n_utts;
    const float *encp;           // [rows][J] b_e + W_e . enc
    long long encp_rows;
    const long long *encp_row;   // [n_utts]
    const int *T;
    const int *slot;
    const float *blank_bias;     // nullable
    const int *tokens_base;      // nullable
    int *tokens; int token_cap;
    int *n_tokens; int *steps;
    int *segs; int seg_cap; int *n_segs;
    int *trace; int trace_cap;
    float *logits; int logit_steps;   // nullable debug tap [n_utts][logit_steps][Vo]
    float *lcol;                 // tap staging [n_dom][kColCap][Vo]: each joint column's logits of one
                                 // iteration, copied to the row of the step that takes the column
    const int *reset;            // nullable [n_utts]: 1 = fresh state whatever the slot holds
    int *ctrl_out;               // nullable [n_utts][PK_CTRL_N]: control words after the call
    // exchange buffers of one launch (batch-indexed, written/read coherently)
    float *hx;           // [2][L][n][H] ping-pong by utterance parity
    float *cx;           // [2][L][n][H]
    float *ppx;          // [n][J]
    float *rx;           // [2][L][n][4H]  W_hh . h (no bias), unit-major rows, ping-pong like hx
    unsigned xchg_bytes; // hx, cx, ppx, rx: one allocation in this order, from hx
    // domains: independent utterance groups, each on dom_size workgroups
    int n_dom, dom_size, nt;
    const int *dom_n;            // [n_dom] utterances per domain
    const int *dom_list;         // [n_dom][kDomCap] batch indices
    const int *wg_dom;           // [nwg] domain of a workgroup
    const int *wg_rank;          // [nwg] rank inside its domain
    const int *dom_wg;           // [n_dom][dom_size] workgroup of each rank
    // sync
    unsigned *flags;             // [nwg * kFlagStride]
    unsigned long long *keys;    // [2][n_dom][kColCap][shards][2] best keys per joint column, by iteration parity
    int shards;                  // power of two <= kShards: ranks per shard ~ 8
    int *status;                 // [0] error code, [1] iterations, [2] overflow, [3] trace overflow,
                                 // [9] co-residency decision (cleared per launch)
    unsigned arrive_ticks;       // ordinary dispatch: limit of the arrival wait (100 MHz ticks); 0: none
    int spec;                    // blank-run columns: spare joint columns evaluate later frames
    int max_iter;
    int red_slots;               // LDS partial slots: a phase runs in passes of red_slots / (units per item) items
    int st_n, st_k;              // LDS state of layers >= 1: utterance and owned-tile capacity
    int bias_floats;             // LDS bias table size (floats)
    int wcache_bytes;            // LDS weight cache per workgroup (0: weights are read from L2)
    unsigned long long *prof;    // nullable: per-phase wall-clock totals of workgroup 0 (100 MHz ticks)
    unsigned long long *slots;   // nullable (one-domain launches): [2][P][kSlotCols][2] stamped best keys
                                 // of each workgroup, by iteration parity
};

// Phase timers (workgroup 0 only, when p.prof is set): totals kept in LDS,
// written to p.prof when the loop ends.
enum { kPrL0 = 0, kPrSync0, kPrL1, kPrSync1, kPrPred, kPrSync2, kPrJStage, kPrJCompute, kPrJSync, kPrDecide,
       kPrStageL, kPrN };

// ---------------------------------------------------------------- memory helpers

// Buffer resource over [base, base + bytes): out-of-range lanes read 0 and
// drop stores, so a bad index cannot fault.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *base, unsigned bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}

// Agent-coherent (SC1) loads / stores: used for every buffer written by one
// workgroup and read by another inside a launch.  Plain loads elsewhere keep
// weights cached in L2 (nothing in the loop invalidates the L2).
constexpr int kSC1 = 16;
__device__ __forceinline__ float4 ld4_coh(__amdgpu_buffer_rsrc_t r, unsigned byte_off) {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, kSC1));
}
__device__ __forceinline__ void st4_coh(__amdgpu_buffer_rsrc_t r, unsigned byte_off, float4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned, v), r,
                                           byte_off, 0, kSC1);
}
// Offset past every buffer range: loads return 0 and stores are dropped.
constexpr unsigned kBad = 0x80000000u;
__device__ __forceinline__ float4 ld4(__amdgpu_buffer_rsrc_t r, unsigned byte_off) {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0));
}
__device__ __forceinline__ float ld1_coh(__amdgpu_buffer_rsrc_t r, unsigned byte_off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, kSC1));
}
__device__ __forceinline__ float ld_coh(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coh(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Workgroup barrier for LDS traffic only: each wave waits for its own LDS
// operations (lgkmcnt 0) but not for its global loads and stores, which stay
// in flight across it (s_barrier carries no implicit wait on gfx950).  Every
// exchange between workgroups goes through dom_sync, which drains them.  The
// signal fences keep the compiler from moving memory accesses across it.
__device__ __forceinline__ void lds_sync() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);   // gfx9 encoding: lgkmcnt(0), vmcnt and expcnt unconstrained
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// ---------------------------------------------------------------- MFMA tiles

// 8 int8 stored as q ^ 0x80 = q + 128 (two dwords) -> 8 exact f16: the byte
// becomes the low mantissa byte of 1024.0 (0x64xx), then 1152 is subtracted.
__device__ __forceinline__ half8 q8_to_half8(uint2 q) {
    const unsigned x0 = q.x, x1 = q.y;
    const half2v off = {(_Float16)1152.0f, (_Float16)1152.0f};
    half2v p0 = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, x0, 0x04010400u)) - off;
    half2v p1 = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, x0, 0x04030402u)) - off;
    half2v p2 = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, x1, 0x04010400u)) - off;
    half2v p3 = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, x1, 0x04030402u)) - off;
    return half8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

__device__ __forceinline__ void split_f16(float x, _Float16 &hi, _Float16 &lo) {
    hi = (_Float16)x;
    lo = (_Float16)(x - (float)hi);
}

// DPP quad permutation of a float: lane i of each quad reads quad lane perm_i.
template <int CTRL>
__device__ __forceinline__ float quad_perm(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
// 4x4 transpose inside each quad of lanes: afterwards element j of quad lane p
// is what element p of quad lane j was.  Two butterfly stages (partner p^1,
// then p^2), each exchanging the two elements whose index bit differs from p's.
__device__ __forceinline__ f32x4 quad_transpose(f32x4 a) {
    const int p = threadIdx.x & 3;
    {
        const bool odd = p & 1;
        const float r0 = quad_perm<0xB1>(odd ? a[0] : a[1]);   // quad_perm [1,0,3,2]
        const float r1 = quad_perm<0xB1>(odd ? a[2] : a[3]);
        if (odd) { a[0] = r0; a[2] = r1; } else { a[1] = r0; a[3] = r1; }
    }
    {
        const bool hi = p & 2;
        const float r0 = quad_perm<0x4E>(hi ? a[0] : a[2]);    // quad_perm [2,3,0,1]
        const float r1 = quad_perm<0x4E>(hi ? a[1] : a[3]);
        if (hi) { a[0] = r0; a[1] = r1; } else { a[2] = r0; a[3] = r1; }
    }
    return a;
}

// Staged activation block: 16 utterance rows of K values as f16 (hi, lo).
// Only rows 0 .. n-1 are staged; product columns n .. 15 are not used.
struct Act {
    _Float16 *hi, *lo;
    int kp;     // row stride in halves (K + kKPad)
    int n;      // live rows
};

// Four values split as in split_f16 (packed conversions).
__device__ __forceinline__ void put4(const Act &x, int row, int k, float4 v) {
    const f32x4 f = {v.x, v.y, v.z, v.w};
    const half4 h = __builtin_convertvector(f, half4);
    const half4 l = __builtin_convertvector(f - __builtin_convertvector(h, f32x4), half4);
    *reinterpret_cast<half4 *>(x.hi + row * x.kp + k) = h;
    *reinterpret_cast<half4 *>(x.lo + row * x.kp + k) = l;
}

// ---------------------------------------------------------------- argmax keys

// Order-preserving map of an f32 onto u32 (-0 folded onto +0).
__device__ __forceinline__ unsigned ordered_bits(float v) {
    if (v == 0.0f) v = 0.0f;
    const unsigned b = __float_as_uint(v);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
// Larger key = larger value, then smaller index: the reference's first-index rule.
__device__ __forceinline__ unsigned long long make_key(float v, int idx) {
    return ((unsigned long long)ordered_bits(v) << kIdxBits) | (unsigned long long)((1 << kIdxBits) - 1 - idx);
}
__device__ __forceinline__ int key_index(unsigned long long key) {
    return (1 << kIdxBits) - 1 - (int)(key & ((1u << kIdxBits) - 1));
}
__device__ __forceinline__ unsigned key_stamp(unsigned long long key) { return (unsigned)(key >> kStampShift); }

// Gate nonlinearities from the hardware base-2 exponential (v_exp_f32) and
// reciprocal (v_rcp_f32), each within about 1 ulp: sigmoid(x) = 1 / (1 + e^-x),
// tanh(x) = 2 sigmoid(2x) - 1.  Absolute error stays below ~1e-7, far inside
// the state tolerance, and saturates correctly for large |x| (e^-x -> inf / 0).
__device__ __forceinline__ float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }
__device__ __forceinline__ float sigmoidf_(float x) { return __builtin_amdgcn_rcpf(1.0f + exp_fast(-x)); }
__device__ __forceinline__ float tanh_fast(float x) { return 2.0f * sigmoidf_(2.0f * x) - 1.0f; }

__device__ __forceinline__ void cell(float gi, float gf, float gg, float go, float c_prev, float &c_new, float &h_new) {
    c_new = sigmoidf_(gf) * c_prev + sigmoidf_(gi) * tanh_fast(gg);
    h_new = sigmoidf_(go) * tanh_fast(c_new);
}

// ---------------------------------------------------------------- prepare-time kernels

// out[v][r] = bias0[r] + bias1[r] + W[r, :] . E[v, :] in f32: the layer-0
// input projection of every vocabulary row (W_ih0 . embed[v] + b_ih0 + b_hh0).
// Operands are dense f32 here (dequantised on the host from the stored bytes).
__global__ void __launch_bounds__(256) embed_proj_kernel(const float *__restrict w, const float *__restrict e,
                                                         int rows, int V, int K, const float *__restrict b0,
                                                         const float *__restrict b1, float *__restrict out) {
    const int v0 = blockIdx.x * 16, r0 = blockIdx.y * 64;
    __shared__ float es[16][65];
    __shared__ float ws[64][65];
    const int tid = threadIdx.x;
    const int tv = tid / 16, tr = tid % 16;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < K; k0 += 64) {
        for (int i = tid; i < 16 * 64; i += 256) {
            const int vv = i / 64, k = i % 64;
            es[vv][k] = (v0 + vv < V && k0 + k < K) ? e[(size_t)(v0 + vv) * K + k0 + k] : 0.0f;
        }
        for (int i = tid; i < 64 * 64; i += 256) {
            const int rr = i / 64, k = i % 64;
            ws[rr][k] = (r0 + rr < rows && k0 + k < K) ? w[(size_t)(r0 + rr) * K + k0 + k] : 0.0f;
        }
        __syncthreads();
        for (int k = 0; k < 64; ++k) {
            const float x = es[tv][k];
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[j] = fmaf(ws[tr * 4 + j][k], x, acc[j]);
        }
        __syncthreads();
    }
    const int v = v0 + tv;
    if (v >= V) return;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int r = r0 + tr * 4 + j;
        if (r < rows) out[(size_t)v * rows + r] = acc[j] + (b0[r] + b1[r]);
    }
}

// Zero n 32-bit words (clears the flags, keys and status words of a call).
__global__ void __launch_bounds__(256) fill_zero_kernel(unsigned *__restrict p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) p[i] = 0u;
}

// ---------------------------------------------------------------- enc_proj

// encp[rows of utterance u] = b_e + W_e . enc[row] for every frame: an MFMA
// GEMM with f32 accuracy.  Frames (f32) are split into f16 hi + lo when staged
// in LDS; W_e arrives as f16 hi / lo planes [J][D] (split once at load).
// Each 16x16 output tile takes hi.hi + lo.hi + hi.lo (the lo.lo term is below
// f32 rounding).  Workgroup: 64 output rows x 64 outputs, 4 waves of 16 rows;
// K steps of 32.  d_enc % 32 == 0.  Output rows are the frames of all
// utterances packed in order (utterance u owns rows dst_row[u] ..
// dst_row[u] + T[u]), so short windows of many utterances share tiles; a
// row's utterance is the last u with dst_row[u] <= row.
constexpr int kEpTile = 64, kEpK = 32, kEpStride = kEpK + 8;   // LDS row stride in halves
// The global loads of K step k+1 are issued before the products of step k (one
// register set ahead), so each step waits for LDS and the matrix cores rather
// than for memory.  Threads of the whole grid also zero `clear_words` 32-bit
// words at `clear` (the decode loop's status, barrier flags and argmax keys),
// which saves the loop a separate fill.
__global__ void __launch_bounds__(256) enc_proj_kernel(const _Float16 *__restrict whi, const _Float16 *__restrict wlo,
                                                       int J, const float *__restrict bias,
                                                       const float *__restrict enc, int d_enc,
                                                       const long long *__restrict src_row,
                                                       const long long *__restrict dst_row, int n_utts,
                                                       long long rows, float *__restrict out,
                                                       unsigned *__restrict clear, size_t clear_words) {
    __shared__ __attribute__((aligned(16))) _Float16 ah[kEpTile * kEpStride], al[kEpTile * kEpStride];
    __shared__ __attribute__((aligned(16))) _Float16 bh[kEpTile * kEpStride], bl[kEpTile * kEpStride];
    {
        const size_t nthreads = (size_t)gridDim.x * gridDim.z * 256;
        const size_t gtid = ((size_t)blockIdx.z * gridDim.x + blockIdx.x) * 256 + threadIdx.x;
        for (size_t i = gtid; i < clear_words; i += nthreads) clear[i] = 0u;
    }
    const long long m0 = (long long)blockIdx.x * kEpTile;
    const int n0 = blockIdx.z * kEpTile;
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
    const int sr = tid / 4, sc = (tid % 4) * 8;   // staging: row / column of this thread's 8 values
    // the source frame of this thread's staging row
    const long long r = m0 + sr;
    const bool live = r < rows;
    const float *src = enc;
    if (live) {
        int lo = 0, hi = n_utts - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (dst_row[mid] <= r) lo = mid;
            else hi = mid - 1;
        }
        src = enc + (size_t)(src_row[lo] + (r - dst_row[lo])) * d_enc;
    }
    const int j = n0 + sr;
    // one K step's global operands of this thread: 8 frame values, 8 W_e values (hi, lo)
    float4 v0 = make_float4(0.f, 0.f, 0.f, 0.f), v1 = v0;
    half8 wh = half8{}, wl = half8{};
    auto fetch = [&](int k0) {
        if (live) {
            v0 = *reinterpret_cast<const float4 *>(src + k0 + sc);
            v1 = *reinterpret_cast<const float4 *>(src + k0 + sc + 4);
        }
        if (j < J) {
            wh = *reinterpret_cast<const half8 *>(whi + (size_t)j * d_enc + k0 + sc);
            wl = *reinterpret_cast<const half8 *>(wlo + (size_t)j * d_enc + k0 + sc);
        }
    };
    f32x4 acc[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    fetch(0);
    for (int k0 = 0; k0 < d_enc; k0 += kEpK) {
        {
            const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
            half8 h, l;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                h[i] = (_Float16)v[i];
                l[i] = (_Float16)(v[i] - (float)h[i]);
            }
            *reinterpret_cast<half8 *>(ah + sr * kEpStride + sc) = h;
            *reinterpret_cast<half8 *>(al + sr * kEpStride + sc) = l;
            *reinterpret_cast<half8 *>(bh + sr * kEpStride + sc) = wh;
            *reinterpret_cast<half8 *>(bl + sr * kEpStride + sc) = wl;
        }
        __syncthreads();
        if (k0 + kEpK < d_enc) fetch(k0 + kEpK);   // in flight during this step's products
        const int ao = (wave * 16 + (lane & 15)) * kEpStride + (lane >> 4) * 8;
        const half8 a_h = *reinterpret_cast<const half8 *>(ah + ao);
        const half8 a_l = *reinterpret_cast<const half8 *>(al + ao);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int bo = (t * 16 + (lane & 15)) * kEpStride + (lane >> 4) * 8;
            const half8 b_h = *reinterpret_cast<const half8 *>(bh + bo);
            const half8 b_l = *reinterpret_cast<const half8 *>(bl + bo);
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_h, b_h, acc[t], 0, 0, 0);
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_l, b_h, acc[t], 0, 0, 0);
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_h, b_l, acc[t], 0, 0, 0);
        }
        __syncthreads();
    }
    // D fragment: lane holds output column 16t + lane % 16 of rows 4 (lane / 16) .. +3
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const int col = n0 + t * 16 + (lane & 15);
        if (col >= J) continue;
        const float bc = bias[col];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const long long row = m0 + wave * 16 + (lane >> 4) * 4 + i;
            if (row < rows) out[(size_t)row * J + col] = acc[t][i] + bc;
        }
    }
}

// enc_proj for few rows (streaming chunks, short windows).  There the tiled
// kernel above runs on a few dozen workgroups, each paying two workgroup
// barriers and an LDS round trip per K step.  Here each wave owns one 16x16
// output block and loads its operands straight into MFMA fragment registers,
// kEnSteps K steps per batch, the next batch in flight while the current one is
// multiplied: no LDS and no barrier.  Each block takes exactly the
// instructions of enc_proj_kernel, in the same order: per K step of 32 the same
// lane layout (row lane % 16, K slice 8 (lane / 16)), the same f16 hi / lo split
// of the frames, hi.hi + lo.hi + hi.lo into one accumulator in K order, then +
// bias.  So the two kernels' outputs are bit-identical, and the host chooses
// between them by row count alone.  Workgroup: 4 waves, 16 rows x 64 outputs.
constexpr int kEnSteps = 4;   // K steps per batch of the narrow kernel
__global__ void __launch_bounds__(256) enc_proj_narrow_kernel(const _Float16 *__restrict whi,
                                                              const _Float16 *__restrict wlo, int J,
                                                              const float *__restrict bias,
                                                              const float *__restrict enc, int d_enc,
                                                              const long long *__restrict src_row,
                                                              const long long *__restrict dst_row, int n_utts,
                                                              long long rows, float *__restrict out,
                                                              unsigned *__restrict clear, size_t clear_words) {
    {
        const size_t nthreads = (size_t)gridDim.x * gridDim.z * 256;
        const size_t gtid = ((size_t)blockIdx.z * gridDim.x + blockIdx.x) * 256 + threadIdx.x;
        for (size_t i = gtid; i < clear_words; i += nthreads) clear[i] = 0u;
    }
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const long long m0 = (long long)blockIdx.x * 16;
    const int n0 = (blockIdx.z * 4 + wave) * 16;
    if (n0 >= J) return;
    const long long r = m0 + (lane & 15);
    const bool live = r < rows;
    const float *src = enc;
    if (live) {
        int lo = 0, hi = n_utts - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (dst_row[mid] <= r) lo = mid;
            else hi = mid - 1;
        }
        src = enc + (size_t)(src_row[lo] + (r - dst_row[lo])) * d_enc;
    }
    const int col = n0 + (lane & 15);
    const bool cl = col < J;
    const int ks = (lane >> 4) * 8;
    const int nsteps = d_enc / kEpK, nb = (nsteps + kEnSteps - 1) / kEnSteps;
    // Every lane loads: a row past the last reads frame row 0 and a column past J reads
    // W_e row J - 1.  Row i of an MFMA product depends only on row i of A, and column j
    // only on column j of B, so those lanes' values reach only outputs never stored.
    const _Float16 *bhp = whi + (size_t)(cl ? col : J - 1) * d_enc + ks;
    const _Float16 *blp = wlo + (size_t)(cl ? col : J - 1) * d_enc + ks;
    src += ks;
    struct Batch {
        float4 a0[kEnSteps], a1[kEnSteps];
        half8 bh[kEnSteps], bl[kEnSteps];
    };
    // batch b's operands (a batch past the last reloads the last one, so no load sits
    // behind a branch and the compiler's wait counts stay exact)
    auto load = [&](int b, Batch &x) {
        b = b < nb ? b : nb - 1;
#pragma unroll
        for (int s = 0; s < kEnSteps; ++s) {
            int st = b * kEnSteps + s;
            st = st < nsteps ? st : nsteps - 1;
            const int k = st * kEpK;
            x.a0[s] = *reinterpret_cast<const float4 *>(src + k);
            x.a1[s] = *reinterpret_cast<const float4 *>(src + k + 4);
            x.bh[s] = *reinterpret_cast<const half8 *>(bhp + k);
            x.bl[s] = *reinterpret_cast<const half8 *>(blp + k);
        }
    };
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
    auto mul = [&](int b, const Batch &x) {
#pragma unroll
        for (int s = 0; s < kEnSteps; ++s) {
            if (b * kEnSteps + s >= nsteps) break;
            const float v[8] = {x.a0[s].x, x.a0[s].y, x.a0[s].z, x.a0[s].w,
                                x.a1[s].x, x.a1[s].y, x.a1[s].z, x.a1[s].w};
            half8 h, l;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                h[i] = (_Float16)v[i];
                l[i] = (_Float16)(v[i] - (float)h[i]);
            }
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(h, x.bh[s], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(l, x.bh[s], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(h, x.bl[s], acc, 0, 0, 0);
        }
    };
    Batch X, Y;
    load(0, X);
    for (int b = 0; b < nb; b += 2) {
        load(b + 1, Y);
        mul(b, X);
        load(b + 2, X);
        if (b + 1 < nb) mul(b + 1, Y);
    }
    if (!cl) return;
    const float bc = bias[col];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const long long row = m0 + (lane >> 4) * 4 + i;
        if (row < rows) out[(size_t)row * J + col] = acc[i] + bc;
    }
}

// ---------------------------------------------------------------- decode loop

struct Ctl {                      // per-workgroup copy of its domain's control state
    int b[kDomCap];               // batch index of each domain utterance
    int t[kDomCap], T[kDomCap], sym[kDomCap], pend[kDomCap], flags[kDomCap];
    int ntok[kDomCap], steps[kDomCap], nseg[kDomCap], segst[kDomCap], last[kDomCap], cur[kDomCap];
    int lst[kDomCap], jst[kDomCap];
    // joint columns: column i < nj is joint-list utterance i at its frame t; columns
    // sbase[i] .. sbase[i] + sn[i] - 1 are the same utterance at frames t + 1 .. t + sn[i]
    int cu[kColCap], co[kColCap], sbase[kDomCap], sn[kDomCap];
    long long crow[kColCap];      // encp row of each column (utterance's first row + t + offset)
    int cb[kColCap];              // batch index of each column's utterance
    int brun[kDomCap];            // 1: the utterance's last decision kept the prediction output
    int ncol;
    long long erow[kDomCap];      // first encp row of each utterance
    float bbias[kDomCap];         // blank logit offset of each utterance
    int tbase[kDomCap];           // tokens before this call (EOU segment indices)
    int dur[PK_MAX_DURATIONS];    // duration values (the decision step reads them from LDS)
    int n, nl, nj;
    int dom, rank, P;
    // this workgroup's tiles of an LSTM matrix, of W_p and of W_o (fixed for the
    // launch; computed once, since each is an integer division)
    int own_lstm, own_pred, own_out;
    int pass[PK_MAX_LAYERS + 1];  // items per pass of the phase consuming layer l's output (l < L), of W_o (L)
    unsigned mag_p, mag_h, mag_units;   // udiv multipliers for P, H and 4 * own_lstm
    unsigned wmask;               // bit ul: this workgroup writes utterance ul's outputs (ul % P == rank)
    int tq_n, tq_col[kColCap], tq_b[kColCap], tq_step[kColCap];   // logit tap: (column, utterance, step)
                                                                  // of this iteration's decisions
    unsigned long long wgkey[kColCap][2];   // this workgroup's best key per joint column and head
    unsigned long long prof[kPrN];
};

__device__ __forceinline__ void pmark(const KParams &p, Ctl &s, unsigned long long &last, int k) {
    if (!p.prof) return;
    lds_sync();
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        const unsigned long long now = __builtin_amdgcn_s_memrealtime();
        s.prof[k] += now - last;
        last = now;
    }
}

// Checkpoint timeline (built with -DPK_TIMELINE, read with PK_PROFILE_PHASES=1):
// workgroup 0 sums, per wave and checkpoint, the time since the start of the
// iteration over iterations 40 .. 295; the host prints the per-wave means.
// TL(k) is relative to the phase base set by TLBASE, TLA(k) absolute.  The
// checkpoints add LDS traffic and waits of their own, so their times are
// upper bounds.
constexpr int kTl = 32;
#ifdef PK_TIMELINE
__device__ __forceinline__ unsigned long long *tl_sum() { __shared__ unsigned long long b[kWaves * kTl]; return b; }
__device__ __forceinline__ int *tl_ctl() { __shared__ int c[2 + kTl]; return c; }
__device__ __forceinline__ unsigned long long *tl_t0() { __shared__ unsigned long long t; return &t; }
#define TLX(k, rel) do { int *c_ = tl_ctl(); if (c_[0]) { const int w_ = threadIdx.x >> 6; \
    if ((threadIdx.x & 63) == 0) { const int kk_ = ((rel) ? c_[1] : 0) + (k); \
    tl_sum()[w_ * kTl + kk_] += __builtin_amdgcn_s_memrealtime() - *tl_t0(); if (w_ == 0) c_[2 + kk_]++; } } } while (0)
#define TLBASE(b) do { if (threadIdx.x == 0) tl_ctl()[1] = (b); } while (0)
#else
#define TLX(k, rel) do { } while (0)
#define TLBASE(b) do { } while (0)
#endif
#define TL(k) TLX(k, 1)
#define TLA(k) TLX(k, 0)

// Compact the LSTM list (pending token) and the joint list (frames left).
// Then the joint columns: one per joint-list utterance at its frame t, and
// (spec) the column tiles' spare columns dealt out evenly as frames t + 1,
// t + 2, ... to the utterances in a run of blanks (last decision kept the
// prediction output), up to their last frame.  A blank decision keeps the
// prediction output, so the logits of the next frame are already in a spare
// column: the decision step walks a run of blanks in one iteration instead of
// one iteration per blank.
__device__ __forceinline__ void build_lists(Ctl &s, bool spec) {
    if (threadIdx.x < kWave) {
        const int lane = threadIdx.x;
        const bool fl = lane < s.n && s.pend[lane] >= 0;
        const bool fj = lane < s.n && s.t[lane] < s.T[lane];
        const unsigned long long bl = __ballot(fl), bj = __ballot(fj);
        const unsigned long long below = (lane == 0) ? 0ull : (~0ull >> (kWave - lane));
        const int il = __popcll(bl & below), ij = __popcll(bj & below);
        if (fl) s.lst[il] = lane;
        if (fj) s.jst[ij] = lane;
        const int nj = __popcll(bj);
        // an utterance in a blank run takes q spare columns: an even share of the
        // spare columns of the tiles, capped at the frames it has left
        const int spare = spec && nj > 0 ? ((nj + kTile - 1) / kTile) * kTile - nj : 0;
        const bool fe = fj && spare > 0 && s.brun[lane] != 0;
        const unsigned long long be = __ballot(fe);
        int total = 0;
        if (fj) {
            s.cu[ij] = lane;
            s.co[ij] = 0;
            s.crow[ij] = s.erow[lane] + s.t[lane];
            s.cb[ij] = s.b[lane];
        }
        if (be != 0ull) {   // some utterance is in a run of blanks (wave-uniform)
            const int ne = __popcll(be), ie = __popcll(be & below);
            int q = 0;
            if (fe) {
                q = spare / ne + (ie < spare % ne ? 1 : 0);
                q = min(q, s.T[lane] - s.t[lane] - 1);
            }
            // exclusive prefix sum of q over the joint list (lanes in list order)
            int incl = q;
#pragma unroll
            for (int d = 1; d < kWave; d <<= 1) {
                const int v = __shfl_up(incl, d, kWave);
                if (lane >= d) incl += v;
            }
            if (fj) {
                const int base = nj + incl - q;
                s.sbase[ij] = base;
                s.sn[ij] = q;
                for (int o = 1; o <= q; ++o) {
                    s.cu[base + o - 1] = lane;
                    s.co[base + o - 1] = o;
                    s.crow[base + o - 1] = s.erow[lane] + s.t[lane] + o;
                    s.cb[base + o - 1] = s.b[lane];
                }
            }
            total = __shfl(incl, kWave - 1, kWave);
        }
        if (lane == 0) {
            s.nl = __popcll(bl);
            s.nj = nj;
            s.ncol = nj + total;
        }
    }
    lds_sync();
}

// Domain barrier: every member publishes its epoch in its own flag word and
// every member polls all members' flags (thread t polls rank t).  No
// cache-wide fences: cross-workgroup data is stored and loaded coherently
// (SC1), and each thread waits for its own stores (s_waitcnt 0) before
// arriving.  Returns false if the error word is set or the wait exceeds ~2 s.
__device__ __forceinline__ bool dom_sync(const KParams &p, const Ctl &s, unsigned &epoch) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    __shared__ int s_ok;
    ++epoch;
    if (threadIdx.x == 0) {
        s_ok = 1;
        __hip_atomic_store(p.flags + (size_t)blockIdx.x * kFlagStride, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (threadIdx.x < s.P) {
        // tight poll; the error word and the clock are checked every 64 polls
        unsigned *f = p.flags + (size_t)p.dom_wg[s.dom * s.P + threadIdx.x] * kFlagStride;
        const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
        unsigned n = 0;
        while (__hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < epoch) {
            if ((++n & 63) != 0) continue;
            if (__hip_atomic_load(p.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) { s_ok = 0; break; }
            if (__builtin_amdgcn_s_memrealtime() - t0 > 200000000ull) {   // 100 MHz clock: 2 s
                __hip_atomic_store(p.status, PK_ERR_TIMEOUT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                s_ok = 0;
                break;
            }
        }
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __syncthreads();
    return s_ok != 0;
}

// Exchange-buffer offsets (floats).
__device__ __forceinline__ size_t hx_off(const KParams &p, int buf, int layer, int b) {
    return (((size_t)buf * p.L + layer) * p.n_utts + b) * p.H;
}
__device__ __forceinline__ size_t rx_off(const KParams &p, int buf, int layer, int b) {
    return (((size_t)buf * p.L + layer) * p.n_utts + b) * 4 * p.H;
}

struct Bufs {
    __amdgpu_buffer_rsrc_t hx, cx, ppx, rx, ep, encp;
};

// One utterance's slot state in float4 chunks: h of every layer, c_0, pp,
// R_0 (c and R of layers >= 1 live in the LDS state during a launch).  Chunk
// q is at `slot` in its slot array and at float offset `x` from p.hx in the
// exchange buffers (hx, cx, ppx, rx are consecutive).
struct StateChunk {
    float *slot;
    long long x;
};
__device__ __forceinline__ int state_chunks(const KParams &p) { return (p.L * p.H + p.H + p.J + 4 * p.H) / 4; }
__device__ __forceinline__ StateChunk state_chunk(const KParams &p, int q, int slot, int b, int buf) {
    const int H = p.H, L = p.L, J = p.J;
    int i = 4 * q;
    if (i < L * H) {
        const int l = i / H;
        return {p.slot_h + (size_t)slot * L * H + i, (long long)hx_off(p, buf, l, b) + (i - l * H)};
    }
    i -= L * H;
    if (i < H) return {p.slot_c + (size_t)slot * L * H + i, (long long)(p.cx - p.hx) + (long long)hx_off(p, buf, 0, b) + i};
    i -= H;
    if (i < J) return {p.slot_pp + (size_t)slot * J + i, (long long)(p.ppx - p.hx) + (long long)b * J + i};
    i -= J;
    return {p.slot_r + (size_t)slot * L * 4 * H + i, (long long)(p.rx - p.hx) + (long long)rx_off(p, buf, 0, b) + i};
}
constexpr int kCopyB = 4;   // float4 per thread in flight when copying state

// Stage vectors of length K for n <= 16 utterances into an activation block:
// row u <- src(off(u)) via coherent loads; rows n .. 15 are zero.  Every
// thread issues all of its loads before converting any of them.
// Staging: 32 threads per row, so a 512-thread block covers 16 rows per
// round; each thread resolves its row once and moves float4 chunks sub,
// sub + 32, ... (kStageMax per thread in flight: 160 float4 = K 640 per pass).
constexpr int kStageMax = 5, kStageTpr = 32;
template <class OffFn>
__device__ __forceinline__ void stage_act(const Act &x, int K, int n, __amdgpu_buffer_rsrc_t r, OffFn off) {
    const int per = K / 4, sub = threadIdx.x % kStageTpr;
    for (int u0 = 0; u0 < n; u0 += kBlock / kStageTpr) {
        const int u = u0 + threadIdx.x / kStageTpr;
        const bool live = u < n;
        const unsigned row = (unsigned)(off(live ? u : n - 1) * 4);   // byte offset of the row
        for (int k0 = 0; k0 < per; k0 += kStageTpr * kStageMax) {
            float4 v[kStageMax];
#pragma unroll
            for (int j = 0; j < kStageMax; ++j) {
                const int k4 = k0 + sub + kStageTpr * j;
                v[j] = ld4_coh(r, live && k4 < per ? row + (unsigned)k4 * 16 : kBad);
            }
#pragma unroll
            for (int j = 0; j < kStageMax; ++j) {
                const int k4 = k0 + sub + kStageTpr * j;
                if (live && k4 < per) put4(x, u, k4 * 4, v[j]);
            }
        }
    }
}

// ---------------------------------------------------------------- MFMA phase engine
//
// A phase multiplies weight row tiles ("items") by one staged 16-utterance
// activation block.  Items 0 .. n_a-1 are tiles rank, rank+P, ... of matrix A,
// items n_a .. n_items-1 the same of matrix B (same storage type and K).  Each
// item's K blocks are cut into S units of kUnitOf blocks (f32 weights count
// every K block twice, once per f16 plane).  Items are taken in passes of as
// many items as the LDS partial slots hold.  Within a pass the units are
// numbered K-major -- unit u = chunk * nj + item -- and every wave takes a
// contiguous range of them, so a wave reads one chunk's activation fragments
// from LDS once and reuses them from registers for every item of its range.
// Each unit leaves one 16x16 partial in LDS slot (item - j0) * S + chunk; the
// pass's reduce sums an item's partials in chunk order (a fixed order, so
// results do not depend on timing) and runs the epilogue.  The weight
// fragments of a wave's next unit are loaded before its current unit is
// multiplied, so one unit's L2 latency hides behind the previous unit's
// products.

// K blocks per unit, by weight storage.  Measured: q8_0 5 (beats 4, 8 and 10 at B=1/64/256);
// f16 and f32 4 (TDT-1.1b f16 at B=256: 49.9 vs 60.5 ms per launch with 5).
template <bool Q8> constexpr int kUnitOf = Q8 ? 5 : 4;
__host__ __device__ constexpr int unit_blocks(int type) { return type == PK_TYPE_Q8_0 ? 5 : 4; }

// One matrix's fragment sources for a phase: buffer descriptors (q8_0: the
// quants and the block scales; f16: the plane twice; f32: the hi and lo
// planes) and the base of this workgroup's LDS-cached tiles, set up once.
struct MatSrc {
    __amdgpu_buffer_rsrc_t r0, r1;
    const unsigned char *lds;
    int KB;
    unsigned plane;   // f32: bytes of the hi plane (the lo plane's offset)
};
template <bool Q8, bool CACHED>
__device__ __forceinline__ MatSrc mat_src(const TMat &m, bool two, const unsigned char *wc) {
    MatSrc s;
    if (Q8) {
        s.r0 = rsrc(m.a, (unsigned)m.tiles * (unsigned)tile_bytes(PK_TYPE_Q8_0, m.KB));
        s.r1 = s.r0;
    } else {   // f32: both planes under one descriptor (the lo plane follows the hi plane)
        const unsigned bytes = (unsigned)m.tiles * m.KB * kWave * 16u;
        s.r0 = rsrc(m.a, two ? 2 * bytes : bytes);
        s.r1 = s.r0;
    }
    s.lds = CACHED ? wc + m.lds_off : nullptr;
    s.KB = m.KB;
    s.plane = (unsigned)m.tiles * m.KB * kWave * 16u;
    return s;
}

// Fragments of one unit, blocks sb0 .. sb0+kUnitOf-1 of tile `tile` (local index
// li in the LDS cache).  q8_0: the unit's record, four loads.  f16 / f32: FULL,
// all kUnitOf blocks exist (K is a whole number of units), so every offset is a
// lane constant plus a wave-uniform base plus an immediate; otherwise blocks
// past nb read as zero (buffer loads past the range return 0; cached blocks are
// zeroed).  Matrices are stored in whole units, so only FULL is instantiated.
template <bool Q8, bool CACHED, bool FULL>
__device__ __forceinline__ void unit_load_src(const MatSrc &m, bool two, int tile, int li, int sb0, int nb, int lane,
                                              uint4 (&f)[kUnitOf<Q8>]) {
    if constexpr (Q8) {   // one unit record (matrices are stored in whole units: every block exists)
        static_assert(kUnitOf<Q8> == kQ8Unit, "q8_0 units are the stored records");
        const int uc = sb0 / kQ8Unit;
        uint4 qa, qb, sc;
        uint2 qc;
        if (CACHED) {
            const unsigned char *rec = m.lds + ((size_t)li * (m.KB / kQ8Unit) + uc) * kQ8UnitBytes;
            qa = *reinterpret_cast<const uint4 *>(rec + lane * 16);
            qb = *reinterpret_cast<const uint4 *>(rec + 1024 + lane * 16);
            qc = *reinterpret_cast<const uint2 *>(rec + 2048 + lane * 8);
            sc = *reinterpret_cast<const uint4 *>(rec + kQ8Scales + (lane & 15) * 16);
        } else {
            const int rec = (tile * (m.KB / kQ8Unit) + uc) * kQ8UnitBytes;   // wave-uniform
            qa = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(m.r0, lane * 16, rec, 0));
            qb = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(m.r0, lane * 16 + 1024, rec, 0));
            qc = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(m.r0, lane * 8 + 2048, rec, 0));
            sc = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(m.r0, (lane & 15) * 16 + kQ8Scales,
                                                                                 rec, 0));
        }
        f[0] = make_uint4(qa.x, qa.y, sc.x & 0xffffu, 0u);
        f[1] = make_uint4(qa.z, qa.w, sc.x >> 16, 0u);
        f[2] = make_uint4(qb.x, qb.y, sc.y & 0xffffu, 0u);
        f[3] = make_uint4(qb.z, qb.w, sc.y >> 16, 0u);
        f[4] = make_uint4(qc.x, qc.y, sc.z & 0xffffu, 0u);
        return;
    }
    if (CACHED) {
#pragma unroll
        for (int j = 0; j < kUnitOf<Q8>; ++j) {
            const bool ok = FULL || j < nb;
            const int sb = ok ? sb0 + j : sb0;
            uint4 v;
            {
                const int kb = two ? sb >> 1 : sb;
                const int plane = two ? (sb & 1) : 0;
                v = *reinterpret_cast<const uint4 *>(m.lds + (((size_t)li * m.KB + kb) * (two ? 2 : 1) + plane) * 1024 +
                                                     lane * 16);
            }
            f[j] = ok ? v : make_uint4(0u, 0u, 0u, 0u);
        }
        return;
    }
    {
#pragma unroll
        for (int j = 0; j < kUnitOf<Q8>; ++j) {
            const int sb = sb0 + j;
            const int kb = two ? sb >> 1 : sb;
            const bool ok = FULL || j < nb;
            // f32: odd sub-blocks read the lo plane, m.plane bytes past the hi plane
            const unsigned o = ok ? (unsigned)(((tile * m.KB + kb) * kWave + lane) * 16) +
                                        ((two && (sb & 1)) ? m.plane : 0u)
                                  : kBad;
            f[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(m.r0, o, 0, 0));
        }
    }
}

// The activation fragments of a unit's K blocks (all reads issued at once).
template <int U>
__device__ __forceinline__ void unit_act(const Act &x, int xo, bool two, int sb0, int nb, half8 (&ah)[U],
                                         half8 (&al)[U]) {
#pragma unroll
    for (int j = 0; j < U; ++j) {
        const int sb = min(sb0 + j, sb0 + nb - 1);
        const int kb = two ? sb >> 1 : sb;
        ah[j] = *reinterpret_cast<const half8 *>(x.hi + xo + kb * 32);
        al[j] = *reinterpret_cast<const half8 *>(x.lo + xo + kb * 32);
    }
}

// acc += (unit's weight blocks) . (activation blocks), transposed (lane: one
// weight row, four utterances).  Zero blocks past nb add nothing.  q8_0: the
// products of all blocks are issued first (independent MFMA pairs), then each
// is scaled by its block's d; f16/f32: two independent accumulation chains (hi
// and lo activations) added at the end.
template <bool Q8>
__device__ __forceinline__ f32x4 unit_mma(const uint4 (&f)[kUnitOf<Q8>], const half8 (&ah)[kUnitOf<Q8>],
                                          const half8 (&al)[kUnitOf<Q8>],
                                          bool two, int sb0, f32x4 acc) {
    if (Q8) {
        f32x4 p[kUnitOf<Q8>];
#pragma unroll
        for (int j = 0; j < kUnitOf<Q8>; ++j) {
            const half8 w = q8_to_half8(make_uint2(f[j].x, f[j].y));
            p[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[j], w, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            p[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[j], w, p[j], 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < kUnitOf<Q8>; ++j) {
            const float d = (float)__builtin_bit_cast(_Float16, (unsigned short)f[j].z);
            acc += d * p[j];
        }
        return acc;
    }
    // f16 weights: hi and lo activations; f32 weights: the lo plane (odd
    // sub-blocks) skips the lo activations (lo x lo is below f32 rounding)
    f32x4 lo = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < kUnitOf<Q8>; ++j) {
        const half8 w = __builtin_bit_cast(half8, f[j]);
        const half8 b2 = (two && ((sb0 + j) & 1)) ? half8{} : al[j];
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[j], w, acc, 0, 0, 0);
        lo = __builtin_amdgcn_mfma_f32_16x16x32_f16(b2, w, lo, 0, 0, 0);
    }
    return acc + lo;
}

// Wavefront-reduction GEMV form of unit_mma for column tiles with at most
// kGemvCols live utterances (q8_0 weights): VALU dot products instead of a
// 16-column MFMA tile of which at most kGemvCols columns are live.  Lane l
// takes weight row l % 16 and the K slice 8 (l / 16) .. +7 of every block (the
// fragment it loaded), multiplies it with each live utterance's activations
// (hi + lo, exact in f32) in f32, scales by the block's d, and the four lanes
// of a row sum their slices with two shuffles.  The partial lands in the
// layout unit_mma produces (lane l < 16: row l, utterances 0 .. 3), so the
// reduce and the epilogues are the same; columns 4 .. 15 read as zero.
constexpr int kGemvCols = 4;
template <int U>
__device__ __forceinline__ f32x4 unit_gemv(const uint4 (&f)[U], const Act &x, int sb0, int nb, int lane) {
    const int g = lane >> 4;
    float acc[kGemvCols] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < U; ++j) {
        const unsigned q0 = f[j].x, q1 = f[j].y;
        // the stored bytes are q + 128: exact small integers in f32
        const float w[8] = {(float)(q0 & 0xffu) - 128.f, (float)((q0 >> 8) & 0xffu) - 128.f,
                            (float)((q0 >> 16) & 0xffu) - 128.f, (float)(q0 >> 24) - 128.f,
                            (float)(q1 & 0xffu) - 128.f, (float)((q1 >> 8) & 0xffu) - 128.f,
                            (float)((q1 >> 16) & 0xffu) - 128.f, (float)(q1 >> 24) - 128.f};
        const float d = (float)__builtin_bit_cast(_Float16, (unsigned short)f[j].z);
        // blocks past the weights' K (zero scales, matrices padded to whole units) read the last
        // real block's activations, which are finite
        const int ko = (sb0 + min(j, nb - 1)) * 32 + g * 8;
#pragma unroll
        for (int u = 0; u < kGemvCols; ++u) {
            if (u >= x.n) break;   // wave-uniform
            const half8 h = *reinterpret_cast<const half8 *>(x.hi + u * x.kp + ko);
            const half8 l = *reinterpret_cast<const half8 *>(x.lo + u * x.kp + ko);
            float sum = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) sum = fmaf(w[i], (float)h[i] + (float)l[i], sum);
            acc[u] = fmaf(d, sum, acc[u]);
        }
    }
#pragma unroll
    for (int u = 0; u < kGemvCols; ++u) {
        acc[u] += __shfl_xor(acc[u], 16, kWave);
        acc[u] += __shfl_xor(acc[u], 32, kWave);
    }
    return lane < kTile ? f32x4{acc[0], acc[1], acc[2], acc[3]} : f32x4{0.f, 0.f, 0.f, 0.f};
}

// Wave w's unit range [c0, c1) of N units.  Waves w and w + 4 share SIMD w & 3,
// and the older one (w < 4) wins the issue arbitration: for equal ranges the
// younger one finishes 15-30 % later, and the reduce waits for it.  So each SIMD
// gets an even quarter of the units, and its older wave takes the odd unit and,
// with at least 12 units per SIMD, 19 % more than half (76 / 128).  Partials are
// reduced in chunk order, so the split does not change results.  Measured
// against an even split over the 8 waves (two A/Bs chained): B=256, ragged
// B=512 and TDT-1.1b f16 about -3 %, B=64 -0.5 %, B=1 +1.5 %; a 28 % skew
// gained no more.
static_assert(kWaves == 8, "wave_range pairs waves w and w + 4 on SIMD w & 3");
__device__ __forceinline__ void wave_range(int N, int w, int &c0, int &c1) {
    const int j = w & 3, a = (N * j) >> 2, b = (N * (j + 1)) >> 2, len = b - a;
    const int d = N >= 48 ? 12 : 0;
    const int o = (len * (64 + d) + 64) >> 7;   // the older wave's share of its SIMD's range
    c0 = w < 4 ? a : a + o;
    c1 = w < 4 ? a + o : b;
}

// Partials of items j0 .. j1-1 (one pass), K-major, next unit's weights prefetched.
template <bool Q8, bool CACHED, bool FULL, bool GV = false>
__device__ __forceinline__ void phase_partials(const TMat &A, int n_a, const TMat &Bm, int j0, int j1, int rank, int P,
                                               const Act &x, f32x4 *red, const unsigned char *wc) {
    // wave-uniform unit bookkeeping: the weight buffer descriptors stay in SGPRs
    const int lane = threadIdx.x & (kWave - 1), wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const bool two = !Q8 && A.type == PK_TYPE_F32;
    const int KBe = two ? 2 * A.KB : A.KB;
    const int KBa = two ? 2 * A.KBa : A.KBa;          // blocks with weights (activations past them are never read)
    constexpr int U = kUnitOf<Q8>;
    const int S = (KBe + U - 1) / U;                  // units per item
    const int nj = j1 - j0, N = nj * S;
    int c0, c1;
    wave_range(N, wave, c0, c1);
    if (c0 >= c1) return;
    // Column c of the product depends only on row c of the activations; rows
    // past x.n are not staged (they hold older values) and the columns they
    // feed are never read.
    const int xo = (lane & 15) * x.kp + (lane >> 4) * 8;
    const MatSrc sA = mat_src<Q8, CACHED>(A, two, wc), sB = mat_src<Q8, CACHED>(Bm, two, wc);
    auto load = [&](int item, int c, uint4 (&f)[U]) {
        const bool in_a = item < n_a;
        const int li = in_a ? item : item - n_a;
        const int sb0 = c * U;
        unit_load_src<Q8, CACHED, FULL>(in_a ? sA : sB, two, rank + li * P, li, sb0, min(U, KBe - sb0), lane, f);
    };
    half8 ah[U], al[U];
    uint4 fa[U], fb[U];
    // u = c * nj + i: c < S, so short wave-uniform loops instead of divisions
    int u = c0, c = 0, i = c0, cur = -1;
    while (i >= nj) {
        i -= nj;
        ++c;
    }
    // f16 / f32 from L2: the prefetch past the range reloads the wave's last unit,
    // an address the compiler cannot equate with the set in flight (reloading the
    // current unit, it copies that set instead, waiting for its loads)
    int cl = 0, il = c1 - 1;
    while (il >= nj) {
        il -= nj;
        ++cl;
    }
    load(j0 + i, c, fa);
    // one unit: issue the next unit's loads into fn, then multiply fc
    auto step = [&](uint4 (&fc)[U], uint4 (&fn)[U]) {
        int nc = c, ni = i + 1;
        if (ni == nj) {
            ni = 0;
            ++nc;
        }
        // q8_0 from L2: issued on every step (the last one reloads the current
        // unit).  With a conditional prefetch the compiler's wait counts after
        // the join assume no prefetch, so each unit's products would also wait
        // for the next unit's first loads.  (Measured: B=256 q8_0 -6 %; the f16
        // and LDS-cached paths are faster with the conditional form.)
        if (u + 1 < c1) load(j0 + ni, nc, fn);
        else if (Q8 && !CACHED) load(j0 + i, c, fn);
        else if (!CACHED) load(j0 + il, cl, fn);   // f16 / f32: the wave's last unit (see below)
        const int sb0 = c * U;
        if constexpr (GV) {
            red[(i * S + c) * kWave + lane] = unit_gemv<U>(fc, x, sb0, min(U, KBa - sb0), lane);
        } else {
            if (c != cur) {
                unit_act(x, xo, two, sb0, min(U, KBa - sb0), ah, al);
                cur = c;
            }
            red[(i * S + c) * kWave + lane] = unit_mma<Q8>(fc, ah, al, two, sb0, f32x4{0.f, 0.f, 0.f, 0.f});
        }
        ++u;
        c = nc;
        i = ni;
    };
    while (true) {
        step(fa, fb);
        if (u >= c1) break;
        step(fb, fa);
        if (u >= c1) break;
    }
    TL(2);
}

// Sum each item's partials of one pass in chunk order and run epi(item, acc);
// items are dealt round robin over the waves.  Opens with a barrier (all
// partials written); the caller's next barrier (before any new partials or
// staging) closes it.
template <class EpiFn>
__device__ __forceinline__ void phase_reduce(int j0, int j1, int S, const f32x4 *red, EpiFn epi) {
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    lds_sync();
    TL(3);
    for (int it = j0 + wave; it < j1; it += kWaves) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        for (int c = 0; c < S; ++c) acc += red[((it - j0) * S + c) * kWave + lane];
        epi(it, acc);
    }
    TL(4);
}

// Weight classes the decode loop is compiled for: each instantiation carries
// only the phase engines its matrices need (a smaller kernel with its own
// register allocation).  kWcAny serves models whose phases mix storage types.
// kWcQ8Gemv: all-q8_0 decoders with the wavefront-reduction GEMV form for column
// tiles of at most kGemvCols live utterances (its own instantiation, so the
// default kernels keep their registers; selected by PK_GEMV=1 for comparisons:
// the MFMA form measured faster at every batch size).
enum { kWcQ8 = 0, kWcHalf = 1, kWcAny = 2, kWcQ8Gemv = 3 };

// Products of one phase for this workgroup, then the epilogue per item, in
// passes of at most `batch` items (red_slots / S, computed once per launch).
template <int WC, class EpiFn>
__device__ __forceinline__ void run_phase(const TMat &A, int n_a, const TMat &Bm, int n_items, int rank, int P,
                                          const Act &x, f32x4 *red, const unsigned char *wc, int batch, EpiFn epi) {
    if (n_items <= 0) return;
    // both matrices of a phase are in the LDS weight cache or neither
    const bool cached = wc != nullptr && A.lds_off >= 0;
    const int KBe = A.type == PK_TYPE_F32 ? 2 * A.KB : A.KB;
    const int U = (WC == kWcQ8 || WC == kWcQ8Gemv) ? kUnitOf<true> : WC == kWcHalf ? kUnitOf<false> : unit_blocks(A.type);
    const int S = (KBe + U - 1) / U;
    for (int j0 = 0; j0 < n_items; j0 += batch) {
        const int j1 = min(n_items, j0 + batch);
        if (j0 > 0) lds_sync();   // the previous pass's reduce has read its slots
        // matrices are stored with whole units of K blocks (zero blocks past
        // K / 32), so unit loads are never masked
        auto q8 = [&]() {
            if (WC == kWcQ8Gemv && x.n <= kGemvCols) {
                if (cached) phase_partials<true, true, true, true>(A, n_a, Bm, j0, j1, rank, P, x, red, wc);
                else phase_partials<true, false, true, true>(A, n_a, Bm, j0, j1, rank, P, x, red, wc);
            } else if (cached) {
                phase_partials<true, true, true>(A, n_a, Bm, j0, j1, rank, P, x, red, wc);
            } else {
                phase_partials<true, false, true>(A, n_a, Bm, j0, j1, rank, P, x, red, wc);
            }
        };
        auto half = [&]() {
            if (cached) phase_partials<false, true, true>(A, n_a, Bm, j0, j1, rank, P, x, red, wc);
            else phase_partials<false, false, true>(A, n_a, Bm, j0, j1, rank, P, x, red, wc);
        };
        if constexpr (WC == kWcQ8 || WC == kWcQ8Gemv) q8();
        else if constexpr (WC == kWcHalf) half();
        else if (A.type == PK_TYPE_Q8_0) q8();
        else half();
        phase_reduce(j0, j1, S, red, epi);
    }
}

// Tiles of a matrix with `tiles` row tiles owned by rank r of P: t = r, r+P, ...
__device__ __forceinline__ int owned(int tiles, int r, int P) { return tiles > r ? (tiles - r + P - 1) / P : 0; }

// n / d without a division, for n * d < 2^32: with m = floor(2^32 / d) + 1,
// floor(n * m / 2^32) = floor(n / d + n * e / 2^32) (0 < e <= 1), and the added
// term stays below 1 / d, the distance from n / d up to the next integer.
__host__ __device__ inline unsigned udiv_magic(unsigned d) { return d <= 1 ? 0u : (unsigned)(0x100000000ull / d + 1); }
__device__ __forceinline__ int udiv(int n, unsigned m, int d) { return d <= 1 ? n : (int)__umulhi((unsigned)n, m); }

// Units (kUnitOf K blocks) per tile row of a matrix.
__device__ __forceinline__ int units_per_item(const TMat &m) {
    const int KBe = m.type == PK_TYPE_F32 ? 2 * m.KB : m.KB, U = unit_blocks(m.type);
    return (KBe + U - 1) / U;
}

// LSTM state of layers >= 1 kept in LDS by the workgroup that owns the units:
// for layer l, utterance ul (domain index) and owned tile k (tile rank + kP,
// units 4t .. 4t+3): R_l rows 16t .. 16t+15 (W_hh_l . h_l, unit-major), then
// c_l of the 4 units.  Those units' gates are produced (the recurrent product
// of the phase that consumes h_l) and consumed (the cell update) by the same
// workgroup, so they never travel through memory inside a launch.
constexpr int kStFloats = kTile + 4;

struct Lds {
    Act act[1 + PK_MAX_LAYERS];   // staged activation blocks
    float *st;                    // [L-1][st_n][st_k][kStFloats] LDS state of layers >= 1
    float *bias;                  // epilogue bias rows of this workgroup's tiles (see bias_table)
    f32x4 *red;                   // [red_slots][kWave] per-(item, chunk) partials of one pass
    const unsigned char *wcache;  // weight cache (nullptr when the tiles do not fit)
};

// Epilogue bias rows of this workgroup's tiles, in LDS for the whole launch:
// the 16 rows of each owned tile of W_ih_l (b_ih_l + b_hh_l, l = 1 .. L-1;
// 4H/16 tiles each), then of W_p (b_p; J/16 tiles), then of W_o (b_o).
// The rows of matrix m start at float kTile * m * own_lstm (m = 0 .. L-2 the
// LSTM layers 1 .. L-1, m = L-1 W_p) and W_o's at kTile * ((L-1) * own_lstm +
// own_pred): H and J are multiples of 32, so own_lstm and own_pred count the
// 4H/16 and J/16 tiles used here.
__device__ __forceinline__ void bias_table(const KParams &p, int rank, int P, float *tab) {
    const int n_lstm = owned(p.H / 4, rank, P), n_pred = owned(p.J / kTile, rank, P);
    const int n_out = owned(p.w_out.tiles, rank, P);
    const int nl = (p.L - 1) * n_lstm * kTile, np = n_pred * kTile, no = n_out * kTile;
    for (int i = threadIdx.x; i < nl + np + no; i += kBlock) {
        float v;
        if (i < nl) {
            const int l = 1 + i / (n_lstm * kTile), r = i % (n_lstm * kTile);
            v = p.b_lstm[l][(rank + (r / kTile) * P) * kTile + r % kTile];
        } else if (i < nl + np) {
            const int r = i - nl;
            v = p.b_pred[(rank + (r / kTile) * P) * kTile + r % kTile];
        } else {
            const int r = i - nl - np;
            const int row = (rank + (r / kTile) * P) * kTile + r % kTile;
            v = row < p.Vo ? p.b_out[row] : 0.0f;
        }
        tab[i] = v;
    }
}

// Copy this workgroup's tiles of m (rank, rank+P, ...) into its LDS cache:
// per K block the fragment, then (q8_0) the 16 block scales.  kCacheB 16-byte
// chunks per thread are loaded before any is stored.
constexpr int kCacheB = 8;
// 16-byte chunk c of this workgroup's cached image of m: its tiles in order,
// each as stored (q8_0 unit records, f16 fragments; f32: per K block the hi
// then the lo fragment).
__device__ __forceinline__ const unsigned char *cache_src(const TMat &m, int rank, int P, int chunks, int c) {
    const int ch = c % chunks, li = c / chunks;   // chunks: of one tile
    const size_t t = (size_t)(rank + li * P);      // global tile
    if (m.type != PK_TYPE_F32) return static_cast<const unsigned char *>(m.a) + t * (size_t)chunks * 16 + ch * 16;
    const int kb = ch / 128, part = ch % 128;      // f32: 128 chunks per block (64 hi, 64 lo)
    return static_cast<const unsigned char *>(part < 64 ? m.a : m.a_lo) + (t * m.KB + kb) * 1024 + (part % 64) * 16;
}
__device__ __forceinline__ void cache_matrix(const TMat &m, int rank, int P, unsigned char *wc) {
    if (m.lds_off < 0) return;
    const int n = owned(m.tiles, rank, P);
    const int chunks = tile_bytes(m.type, m.KB) / 16;
    const int nchunk = n * chunks;
    if (nchunk == 0) return;
    for (int base = 0; base < nchunk; base += kCacheB * kBlock) {
        uint4 v[kCacheB];
#pragma unroll
        for (int j = 0; j < kCacheB; ++j)   // clamped: chunks past the end reload the last one
            v[j] = *reinterpret_cast<const uint4 *>(cache_src(m, rank, P, chunks, min(base + (int)threadIdx.x + j * kBlock, nchunk - 1)));
#pragma unroll
        for (int j = 0; j < kCacheB; ++j) {
            const int c = base + threadIdx.x + j * kBlock;
            if (c < nchunk) *reinterpret_cast<uint4 *>(wc + m.lds_off + (size_t)c * 16) = v[j];
        }
    }
}

// A one-domain launch with at most kSlotCols joint columns exchanges the argmax
// keys through per-workgroup slots instead of atomics, a barrier and a gather:
// each workgroup stores its stamped best key per column and head in its own
// slot, and every workgroup polls all slots until each carries this
// iteration's stamp (the stamp is the arrival signal).  One round trip instead
// of two.  The condition is the same in every workgroup of the domain; ONE
// launches (one domain, p.slots set) run their own instantiation of the loop.
template <bool ONE>
__device__ __forceinline__ bool slot_mode(const Ctl &s) {
    return ONE && s.ncol <= kSlotCols;
}

// Joint + argmax for this workgroup's output tiles.  Utterances are processed
// 16 at a time (one MFMA column tile).
// The encp rows of the joint's first staging round (column tile 0, chunks
// sub, sub + 32, ...), loaded at the start of the iteration: the list rebuild
// has fixed every column's frame, and the loads complete during layer 0, whose
// own loads take as long, instead of at the joint's staging.
__device__ __forceinline__ void encp_prefetch(const KParams &p, const Ctl &s, const Bufs &B, float4 (&e)[kStageMax]) {
    const int J = p.J, per = J / 4, sub = threadIdx.x % kStageTpr, u = threadIdx.x / kStageTpr;
    const int nc = min(kTile, s.ncol);
    const bool live = u < nc;
    const unsigned erow = (unsigned)((size_t)s.crow[live ? u : 0] * J * 4);
#pragma unroll
    for (int j = 0; j < kStageMax; ++j) {
        const int k4 = sub + kStageTpr * j;
        e[j] = ld4(B.encp, live && k4 < per ? erow + (unsigned)k4 * 16 : kBad);
    }
}

template <int WC, bool ONE>
__device__ __forceinline__ void joint_phase(const KParams &p, Ctl &s, const Bufs &B, const Lds &S, unsigned stamp,
                            const float4 (&epre)[kStageMax], unsigned long long &tlast) {
    const int J = p.J, lane = threadIdx.x & (kWave - 1);
    if (threadIdx.x < 2 * kColCap) s.wgkey[threadIdx.x / 2][threadIdx.x % 2] = 0ull;
    const int n_out = s.own_out;
    for (int c0 = 0; c0 < s.ncol; c0 += kTile) {
        const int nc = min(kTile, s.ncol - c0);
        Act x = S.act[0];
        x.n = nc;
        // stage hidden = relu(encp[t] + pp) for this column tile (row mapping as in stage_act)
        {
            const int per = J / 4, sub = threadIdx.x % kStageTpr;
            for (int u0 = 0; u0 < nc; u0 += kBlock / kStageTpr) {
                const int u = u0 + threadIdx.x / kStageTpr;
                const bool live = u < nc;
                const int col = c0 + (live ? u : nc - 1);
                const unsigned erow = (unsigned)((size_t)s.crow[col] * J * 4);
                const unsigned prow = (unsigned)((size_t)s.cb[col] * J * 4);
                for (int k0 = 0; k0 < per; k0 += kStageTpr * kStageMax) {
                    float4 e[kStageMax], q[kStageMax];
#pragma unroll
                    for (int j = 0; j < kStageMax; ++j) {
                        const int k4 = k0 + sub + kStageTpr * j;
                        const bool ok = live && k4 < per;
                        e[j] = (c0 == 0 && k0 == 0) ? epre[j] : ld4(B.encp, ok ? erow + (unsigned)k4 * 16 : kBad);
                        q[j] = ld4_coh(B.ppx, ok ? prow + (unsigned)k4 * 16 : kBad);
                    }
#pragma unroll
                    for (int j = 0; j < kStageMax; ++j) {
                        const int k4 = k0 + sub + kStageTpr * j;
                        if (live && k4 < per) {
                            float4 v = make_float4(e[j].x + q[j].x, e[j].y + q[j].y, e[j].z + q[j].z, e[j].w + q[j].w);
                            v.x = (0.0f < v.x) ? v.x : 0.0f;
                            v.y = (0.0f < v.y) ? v.y : 0.0f;
                            v.z = (0.0f < v.z) ? v.z : 0.0f;
                            v.w = (0.0f < v.w) ? v.w : 0.0f;
                            put4(x, u, k4 * 4, v);
                        }
                    }
                }
            }
        }
        TLBASE(21);
        lds_sync();
        TL(0);
        pmark(p, s, tlast, kPrJStage);
        // after the epilogue's quad transpose (see quad_transpose) a lane holds
        // rows 4g .. 4g+3 of a tile for utterance u of the column tile; its blank
        // offset is loaded before the products
        const int u = 4 * (lane >> 4) + (lane & 3), g = (lane >> 2) & 3;
        const float bb = u < nc ? s.bbias[s.cu[c0 + u]] : 0.0f;
        // (b_out is zero-padded to whole tiles)
        const float *btab = S.bias + kTile * ((p.L - 1) * s.own_lstm + s.own_pred);
        TL(1);
        // debug logit tap: this lane's column (spare columns included) into the staging rows;
        // the decision step copies a column to the row of the step that takes it
        float *ltap = nullptr;
        if (p.logits && u < nc) ltap = p.lcol + ((size_t)s.dom * kColCap + c0 + u) * p.Vo;
        // each lane keeps its best key per head over all its rows; the four
        // lanes of one utterance then combine, and one LDS atomic per utterance
        // and head follows
        unsigned long long best0 = 0ull, best1 = 0ull;
        run_phase<WC>(p.w_out, n_out, p.w_out, n_out, s.rank, s.P, x, S.red, S.wcache, s.pass[p.L],
                  [&](int k, f32x4 acc) {
                      acc = quad_transpose(acc);   // every lane of the wave takes part
                      if (u >= nc) return;
                      const int tile = s.rank + k * s.P;
                      const float4 bias4 = *reinterpret_cast<const float4 *>(btab + k * kTile + g * 4);
#pragma unroll
                      for (int i = 0; i < 4; ++i) {
                          const int row = tile * kTile + g * 4 + i;
                          if (row >= p.Vo) continue;
                          const float bias = i == 0 ? bias4.x : i == 1 ? bias4.y : i == 2 ? bias4.z : bias4.w;
                          float v = acc[i] + bias;
                          if (row == p.blank) v += bb;
                          if (ltap) st_coh(ltap + row, v);
                          if (row < p.V1) {
                              const unsigned long long key = make_key(v, row);
                              best0 = key > best0 ? key : best0;
                          } else {
                              const unsigned long long key = make_key(v, row - p.V1);
                              best1 = key > best1 ? key : best1;
                          }
                      }
                  });
#pragma unroll
        for (int m = 4; m < kTile; m <<= 1) {   // the lanes of utterance u differ in bits 2 and 3
            const unsigned long long o0 = __shfl_xor(best0, m, kWave), o1 = __shfl_xor(best1, m, kWave);
            best0 = o0 > best0 ? o0 : best0;
            best1 = o1 > best1 ? o1 : best1;
        }
        if (g == 0 && u < nc) {
            if (best0) atomicMax(&s.wgkey[c0 + u][0], best0);
            if (best1) atomicMax(&s.wgkey[c0 + u][1], best1);
        }
        lds_sync();
        TLA(27);
        pmark(p, s, tlast, kPrJCompute);
    }
    if (slot_mode<ONE>(s)) {   // this workgroup's stamped best keys into its own slot
        if (threadIdx.x < 2 * s.ncol) {
            const int u = threadIdx.x / 2, head = threadIdx.x % 2;
            __hip_atomic_store(p.slots + (((size_t)(stamp & 1) * s.P + s.rank) * kSlotCols + u) * 2 + head,
                               ((unsigned long long)stamp << kStampShift) | s.wgkey[u][head], __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
        TLA(28);
        return;
    }
    // one device-scope max per utterance and head into shard rank % kShards
    // (spreads the atomics of many workgroups over several words); the stamp
    // keeps keys of iteration `stamp` above every older key in the same parity
    unsigned long long *keys = p.keys + (size_t)(stamp & 1) * p.n_dom * kColCap * p.shards * 2;
    if (threadIdx.x < 2 * s.ncol) {
        const int u = threadIdx.x / 2, head = threadIdx.x % 2;
        const unsigned long long k = s.wgkey[u][head];
        if (k != 0ull)
            __hip_atomic_fetch_max(&keys[((size_t)(s.dom * kColCap + u) * p.shards + (s.rank & (p.shards - 1))) * 2 + head],
                                   ((unsigned long long)stamp << kStampShift) | k, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
    }
    TLA(28);
}

// Layer 0 from the precomputed input projection: gates = E'[token] + R0,
// elementwise per unit.  redundant: every unit for every listed utterance,
// h' also written into the layer-1 activation block; otherwise only this
// workgroup's unit tiles.
// Owners store h', c' coherently.
// Each thread issues the loads of up to kL0 units before computing any.
constexpr int kL0 = 3;
__device__ __forceinline__ void lstm_layer0(const KParams &p, Ctl &s, const Lds &S, const Bufs &B, bool redundant) {
    const int H = p.H;
    const int n_own = s.own_lstm;
    const int nunits = redundant ? H : 4 * n_own;
    const unsigned mag = redundant ? s.mag_h : s.mag_units;
    const int n_work = s.nl * nunits;
    for (int base = 0; base < n_work; base += kL0 * kBlock) {
        float4 e[kL0], r[kL0];
        float c_prev[kL0];
        int uq[kL0], jq[kL0];
#pragma unroll
        for (int q = 0; q < kL0; ++q) {   // no branches: unused loads take kBad and return 0
            const int i = base + threadIdx.x + q * kBlock;
            const int ic = min(i, n_work - 1);
            const int u = udiv(ic, mag, nunits), jj = ic - u * nunits;   // ic * nunits < 2^32 (H <= 4096)
            const int j = redundant ? jj : 4 * (s.rank + (jj / 4) * s.P) + (jj & 3);
            uq[q] = u;
            jq[q] = j;
            const bool ok = i < n_work && j < H;
            const int ul = s.lst[u], b = s.b[ul], cur = s.cur[ul];
            const bool st = ok && !(s.flags[ul] & kFlagZeroHC);
            e[q] = ld4(B.ep, ok ? (unsigned)(((size_t)s.pend[ul] * 4 * H + 4 * j) * 4) : kBad);
            r[q] = ld4_coh(B.rx, st ? (unsigned)((rx_off(p, cur, 0, b) + 4 * j) * 4) : kBad);
            c_prev[q] = ld1_coh(B.cx, st ? (unsigned)((hx_off(p, cur, 0, b) + j) * 4) : kBad);
        }
#pragma unroll
        for (int q = 0; q < kL0; ++q) {
            const int i = base + threadIdx.x + q * kBlock;
            const int u = uq[q], j = jq[q];
            if (i >= n_work || j >= H) continue;
            const int ul = s.lst[u], b = s.b[ul], cur = s.cur[ul];
            float c_new, h_new;
            cell(e[q].x + r[q].x, e[q].y + r[q].y, e[q].z + r[q].z, e[q].w + r[q].w, c_prev[q], c_new, h_new);
            if (redundant) {   // straight into the layer-1 activation block
                const Act &x = S.act[1];
                split_f16(h_new, x.hi[u * x.kp + j], x.lo[u * x.kp + j]);
            }
            // owner of unit group j / 4 (always, when only this workgroup's units are listed)
            if (!redundant || (j >> 2) - udiv(j >> 2, s.mag_p, s.P) * s.P == s.rank) {
                st_coh(p.cx + hx_off(p, cur ^ 1, 0, b) + j, c_new);
                st_coh(p.hx + hx_off(p, cur ^ 1, 0, b) + j, h_new);
            }
        }
    }
}

// Items of the phase that consumes layer lc's new output h_lc' (staged in x):
//   consumer tiles   W_ih_{lc+1} (LSTM layer lc+1, cell update in the epilogue:
//                    the four rows a lane holds are the four gates of one unit)
//                    or W_p (pred projection) when lc is the last layer;
//   recurrent tiles  W_hh_lc . h_lc' -> R_lc for the utterance's next step
//                    (stored in the other ping-pong half of rx).
// Column tile: utterances lst[c0 .. c0+nc).
// Both matrices have K = H and the same storage type.
// LDS state of layer l (>= 1), utterance ul, owned tile k.
__device__ __forceinline__ float *st_at(const KParams &p, const Lds &S, int l, int ul, int k) {
    return S.st + ((size_t)((l - 1) * p.st_n + ul) * p.st_k + k) * kStFloats;
}

template <int WC>
__device__ __forceinline__ void consume_layer(const KParams &p, Ctl &s, const Lds &S, const Bufs &B, const Act &x,
                                              int lc, int c0, int nc) {
    const int lane = threadIdx.x & (kWave - 1);
    const bool last = lc == p.L - 1;
    const TMat &wc = last ? p.w_pred : p.w_ih[lc + 1];
    const TMat &wr = p.w_hh[lc];
    const int n_c = last ? s.own_pred : s.own_lstm, n_r = s.own_lstm;
    // the epilogue quad-transposes the (transposed) D fragment, after which a
    // lane holds rows 4g .. 4g+3 of a tile (the four gates of one unit, or four
    // pred rows) for one utterance u of the column tile
    const int layer = lc + 1, u = 4 * (lane >> 4) + (lane & 3), g = (lane >> 2) & 3;
    // this lane's utterance (a valid index for every lane; lanes u >= nc store nothing)
    const int ul = s.lst[c0 + min(u, nc - 1)], b = s.b[ul], cur = s.cur[ul];
    const bool zero = s.flags[ul] & kFlagZeroHC;
    // bias rows of the consumer tiles (LDS table): lane rows row0 .. row0+3 are
    // the pred rows, or the four gates of unit j = row0 / 4
    const float *btab = S.bias + kTile * lc * s.own_lstm;
    TL(1);
    run_phase<WC>(wc, n_c, wr, n_c + n_r, s.rank, s.P, x, S.red, S.wcache, s.pass[lc],
              [&](int it, f32x4 acc) {
                  acc = quad_transpose(acc);   // every lane of the wave takes part
                  if (u >= nc) return;
                  if (it >= n_c) {          // recurrent product for the next step
                      const int k = it - n_c;
                      if (lc == 0) {        // R_0: read by the layer-0 update of every workgroup (global)
                          const int row0 = (s.rank + k * s.P) * kTile + g * 4;
                          st4_coh(B.rx, (unsigned)((rx_off(p, cur ^ 1, 0, b) + row0) * 4),
                                  make_float4(acc[0], acc[1], acc[2], acc[3]));
                      } else {              // R_lc: LDS state of this workgroup
                          *reinterpret_cast<float4 *>(st_at(p, S, lc, ul, k) + g * 4) =
                              make_float4(acc[0], acc[1], acc[2], acc[3]);
                      }
                      return;
                  }
                  const int row0 = (s.rank + it * s.P) * kTile + g * 4;
                  const float4 bias = *reinterpret_cast<const float4 *>(btab + it * kTile + g * 4);
                  if (last) {               // pred projection: rows row0 .. row0+3 of pp
                      st4_coh(B.ppx, (unsigned)(((size_t)b * p.J + row0) * 4),
                              make_float4(acc[0] + bias.x, acc[1] + bias.y, acc[2] + bias.z, acc[3] + bias.w));
                      return;
                  }
                  // cell update of unit j = row0 / 4 of layer `layer`: R and c_prev from the LDS state
                  float *st = st_at(p, S, layer, ul, it);
                  float4 r = *reinterpret_cast<const float4 *>(st + g * 4);
                  float c_prev = st[kTile + g];
                  if (zero) {
                      r = make_float4(0.f, 0.f, 0.f, 0.f);
                      c_prev = 0.0f;
                  }
                  float c_new, h_new;
                  cell((acc[0] + r.x) + bias.x, (acc[1] + r.y) + bias.y, (acc[2] + r.z) + bias.z,
                       (acc[3] + r.w) + bias.w, c_prev, c_new, h_new);
                  st[kTile + g] = c_new;
                  st_coh(p.hx + hx_off(p, cur ^ 1, layer, b) + row0 / 4, h_new);
              });
}

// One LSTM step (all layers), the pred projection and the recurrent products
// for every utterance of the LSTM list.  A small list in a whole-device
// domain runs layer 0 redundantly in every workgroup (no barrier between
// layers 0 and 1); otherwise layer 0 is split by unit tiles and followed by a
// barrier.  Each later phase stages one layer's full new output and runs the
// tiles that consume it.
template <int WC>
__device__ __forceinline__ bool lstm_and_pred(const KParams &p, Ctl &s, const Bufs &B, const Lds &S, unsigned &epoch,
                              unsigned long long &tlast) {
    const int H = p.H, L = p.L;
    const bool redundant = s.nl <= kSmallB && p.n_dom == 1;
    lstm_layer0(p, s, S, B, redundant);
    TLA(1);
    pmark(p, s, tlast, kPrL0);
    for (int lc = 0; lc < L; ++lc) {
        const bool local = lc == 0 && redundant;     // h_0' is in LDS already
        if (!local) {
            if (!dom_sync(p, s, epoch)) return false;
            TLA(18 + lc);
            pmark(p, s, tlast, lc == 0 ? kPrSync0 : kPrSync1);
        }
        for (int c0 = 0; c0 < s.nl; c0 += kTile) {
            const int nc = min(kTile, s.nl - c0);
            Act x = S.act[1];
            x.n = nc;
            if (!local) {   // (redundant layer 0 wrote h_0' into the block itself)
                stage_act(x, H, nc, B.hx, [&](int u) { const int ul = s.lst[c0 + u]; return hx_off(p, s.cur[ul] ^ 1, lc, s.b[ul]); });
            }
            TLBASE(2 + 8 * lc);
            lds_sync();
            TL(0);
            pmark(p, s, tlast, kPrStageL);
            consume_layer<WC>(p, s, S, B, x, lc, c0, nc);
            TL(6);
        }
        pmark(p, s, tlast, lc == L - 1 ? kPrPred : kPrL1);
    }
    for (int i = threadIdx.x; i < s.nl; i += kBlock) {   // the new state becomes current
        const int ul = s.lst[i];
        s.cur[ul] ^= 1;
        s.pend[ul] = -1;
        s.flags[ul] &= ~kFlagZeroHC;
    }
    const bool ok = dom_sync(p, s, epoch);
    TLA(20);
    pmark(p, s, tlast, kPrSync2);
    return ok;
}

// Apply the argmax results of iteration `stamp` to every utterance of the joint
// list: src/parakeet_tdt.cpp:936-967 (TDT) and src/parakeet_eou.cpp:275-332 (EOU).
// The domain's best key per joint column and head: the maximum over the
// shards that carry this iteration's stamp (shards no rank wrote this
// iteration hold older stamps and are skipped).  Lane groups of p.shards
// reduce one (column, head) with shuffles; results go to s.wgkey.
__device__ __forceinline__ void gather_shards(const KParams &p, Ctl &s, unsigned stamp) {
    const int G = p.shards, lg = __builtin_ctz((unsigned)G);   // a power of two
    const unsigned long long *keys = p.keys + (size_t)(stamp & 1) * p.n_dom * kColCap * G * 2;
    const int lane = threadIdx.x & (kWave - 1);
    const int n = s.ncol * 2 * G;
    for (int e0 = 0; e0 < n; e0 += kBlock) {      // e = (pair, shard); whole waves stay together
        const int e = e0 + threadIdx.x;
        unsigned long long k = 0ull;
        if (e < n) {
            const int pair = e >> lg, sh = e & (G - 1);
            const size_t col = (size_t)s.dom * kColCap + (pair >> 1);
            k = __hip_atomic_load(&keys[(col * G + sh) * 2 + (pair & 1)], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (key_stamp(k) != stamp) k = 0ull;
        }
        for (int m = 1; m < G; m <<= 1) {
            const unsigned long long o = __shfl_xor(k, m, kWave);
            k = o > k ? o : k;
        }
        if (e < n && (lane & (G - 1)) == 0) {
            const int pair = e >> lg;
            s.wgkey[pair >> 1][pair & 1] = k;
        }
    }
    lds_sync();
}

// The domain's best key per joint column and head from the workgroups' slots
// (slot mode): thread e polls slot (pair e / P, rank e % P) until it carries
// stamp, each wave takes the maximum per pair, and one LDS atomic max per wave
// and pair lands in s.wgkey (stamped keys are above the unstamped local ones it
// holds).  Bounded like dom_sync: false on an error or a ~2 s wait.
__device__ __forceinline__ bool gather_slots(const KParams &p, Ctl &s, unsigned stamp) {
    __shared__ int s_ok;
    if (threadIdx.x == 0) s_ok = 1;
    lds_sync();   // this workgroup's slot stores have read s.wgkey
    const int P = s.P, npair = 2 * s.ncol, n = npair * P;
    const unsigned long long *sl = p.slots + (size_t)(stamp & 1) * P * kSlotCols * 2;
    const int lane = threadIdx.x & (kWave - 1);
    for (int e0 = 0; e0 < n; e0 += kBlock) {   // whole waves stay together
        const int e = e0 + threadIdx.x;
        unsigned long long k = 0ull;
        int pair = -1;
        if (e < n) {
            pair = udiv(e, s.mag_p, P);
            const int r = e - pair * P;
            const unsigned long long *w = sl + ((size_t)r * kSlotCols + (pair >> 1)) * 2 + (pair & 1);
            const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
            unsigned m = 0;
            while (key_stamp(k = __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) != stamp) {
                if ((++m & 63) != 0) continue;
                if (__hip_atomic_load(p.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) { s_ok = 0; break; }
                if (__builtin_amdgcn_s_memrealtime() - t0 > 200000000ull) {   // 100 MHz clock: 2 s
                    __hip_atomic_store(p.status, PK_ERR_TIMEOUT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    s_ok = 0;
                    break;
                }
            }
        }
        for (int q = 0; q < npair; ++q) {
            unsigned long long v = pair == q ? k : 0ull;
#pragma unroll
            for (int m = 1; m < kWave; m <<= 1) {
                const unsigned long long o = __shfl_xor(v, m, kWave);
                v = o > v ? o : v;
            }
            if (lane == 0 && v != 0ull) atomicMax(&s.wgkey[q >> 1][q & 1], v);
        }
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    lds_sync();
    return s_ok != 0;
}

// One utterance per thread.  Its first decision is column i (frame t); while
// the decision keeps the prediction output (a TDT blank; an EOU blank, <EOB>
// or special piece) and the next frame's column was evaluated, the walk goes
// on with that column, one step per column, exactly as later iterations would.
// CHAIN: spare columns were evaluated this iteration (otherwise sbase / sn are
// stale and every utterance takes exactly one step).
template <bool CHAIN>
__device__ __forceinline__ void decide_steps(const KParams &p, Ctl &s, unsigned stamp) {
    for (int i = threadIdx.x; i < s.nj; i += kBlock) {
        const int ul = s.jst[i], b = s.b[ul];
        const bool writer = ((s.wmask >> ul) & 1u) != 0u;
        const int t0 = s.t[ul];
        int col = i;
        while (true) {
            const unsigned long long kt = s.wgkey[col][0], kd = s.wgkey[col][1];
            if (key_stamp(kt) != stamp || (p.Dn > 0 && key_stamp(kd) != stamp)) {
                __hip_atomic_store(p.status, PK_ERR_DEVICE, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                s.t[ul] = s.T[ul];
                break;
            }
            const int tok = key_index(kt);
            const int di = p.Dn > 0 ? key_index(kd) : -1;
            const int step = s.steps[ul]++;
            if (p.logits && step < p.logit_steps) {
                const int q = atomicAdd(&s.tq_n, 1);
                s.tq_col[q] = col;
                s.tq_b[q] = b;
                s.tq_step[q] = step;
            }
            if (writer && p.trace) {
                if (step < p.trace_cap) {
                    p.trace[((size_t)b * p.trace_cap + step) * 2] = tok;
                    p.trace[((size_t)b * p.trace_cap + step) * 2 + 1] = di;
                } else {
                    s.flags[ul] |= kFlagTraceOverflow;
                }
            }
            bool keep = false;   // the prediction output stays: the next frame may follow at once
            if (p.kind == PK_KIND_TDT) {
                const int dur = p.n_dur > 0 ? s.dur[di] : di;
                const int adv = dur > 1 ? dur : 1;
                if (tok == p.blank) {
                    s.t[ul] += adv;
                    s.sym[ul] = 0;
                    keep = true;
                } else {
                    const int n = s.ntok[ul]++;
                    if (writer) {
                        if (n < p.token_cap) p.tokens[(size_t)b * p.token_cap + n] = tok;
                        else s.flags[ul] |= kFlagTokOverflow;
                    }
                    s.pend[ul] = tok;
                    s.sym[ul] += 1;
                    if (dur > 0 || s.sym[ul] >= p.max_sym) {
                        s.t[ul] += adv;
                        s.sym[ul] = 0;
                    }
                }
            } else {
                const int max_syms = p.max_sym > 1 ? p.max_sym : 1;
                bool frame_done = false;
                if (tok == p.blank || tok == p.eob) {
                    frame_done = true;
                    keep = true;
                } else if (tok == p.eou) {
                    const int total = s.tbase[ul] + s.ntok[ul];
                    if (total > s.segst[ul]) {
                        const int ns = s.nseg[ul]++;
                        if (writer) {
                            if (p.segs && ns < p.seg_cap) p.segs[(size_t)b * p.seg_cap + ns] = total;
                            else s.flags[ul] |= kFlagSegOverflow;
                        }
                        s.segst[ul] = total;
                    }
                    s.flags[ul] |= kFlagZeroHC;
                    s.pend[ul] = p.blank;
                    s.last[ul] = p.blank;
                    frame_done = true;
                } else if (tok >= 0 && tok < p.n_special && p.special[tok]) {
                    frame_done = true;
                    keep = true;
                } else {
                    const int n = s.ntok[ul]++;
                    if (writer) {
                        if (n < p.token_cap) p.tokens[(size_t)b * p.token_cap + n] = tok;
                        else s.flags[ul] |= kFlagTokOverflow;
                    }
                    s.pend[ul] = tok;
                    s.last[ul] = tok;
                    s.sym[ul] += 1;
                    if (s.sym[ul] >= max_syms) frame_done = true;
                }
                if (frame_done) {          // the next frame starts with sym = 0 (src/parakeet_eou.cpp:269)
                    s.t[ul] += 1;
                    if (s.t[ul] < s.T[ul]) s.sym[ul] = 0;
                }
            }
            // the next decision's frame offset from t0, if its column was evaluated
            s.brun[ul] = keep ? 1 : 0;
            if (!CHAIN || !keep || s.t[ul] >= s.T[ul]) break;
            const int o = s.t[ul] - t0;
            if (o > s.sn[i]) break;
            col = s.sbase[i] + o - 1;
        }
    }
}

// Logit tap: the staged logits of each column a decision took go to the row of
// that decision's step.  Every workgroup copies the rows of its own W_o tiles,
// the ones it staged (so no other workgroup's stores are read).
__device__ __forceinline__ void tap_copy(const KParams &p, Ctl &s) {
    __builtin_amdgcn_s_waitcnt(0);   // this workgroup's staging stores are complete
    lds_sync();
    const int rows = s.own_out * kTile;
    for (int e = threadIdx.x; e < s.tq_n * rows; e += kBlock) {
        const int q = e / rows, r = e - q * rows;
        const int row = (s.rank + (r / kTile) * s.P) * kTile + r % kTile;
        if (row >= p.Vo) continue;
        const float v = ld_coh(p.lcol + ((size_t)s.dom * kColCap + s.tq_col[q]) * p.Vo + row);
        p.logits[((size_t)s.tq_b[q] * p.logit_steps + s.tq_step[q]) * p.Vo + row] = v;
    }
    lds_sync();
    if (threadIdx.x == 0) s.tq_n = 0;
}

__device__ __forceinline__ void decide(const KParams &p, Ctl &s, unsigned stamp, bool gathered) {
    if (!gathered) gather_shards(p, s, stamp);
    TLA(30);
    if (s.ncol > s.nj) decide_steps<true>(p, s, stamp);
    else decide_steps<false>(p, s, stamp);
    if (p.logits) tap_copy(p, s);
}

// Co-residency of an ordinary dispatch.  The loop's barriers need every
// workgroup of the grid resident at once, which a cooperative launch
// guarantees and an ordinary dispatch does not (a long kernel on another
// stream may hold CUs).  Each workgroup stores an arrival flag (word 1 of its
// barrier flag slot).  Workgroup 0 watches every flag, one thread per
// workgroup, for up to p.arrive_ticks, and proposes "go" if all arrived,
// "abort" if not; any other workgroup that has waited twice that long for a
// decision proposes "abort" (workgroup 0 itself may be the one not resident).
// One compare-and-swap on the decision word settles it, and every workgroup
// follows it.  On "abort" no workgroup has written anything but these words;
// the winner of the abort sets the error word to kStatusNotResident, and the
// host relaunches the call cooperatively.  A workgroup that starts after the
// decision reads it and leaves.  Every wait is bounded by the tick limit.
constexpr unsigned kArriveGo = 1u, kArriveAbort = 2u;
__device__ __forceinline__ void propose(const KParams &p, unsigned *dec, unsigned want) {
    unsigned z = 0u;
    if (__hip_atomic_compare_exchange_strong(dec, &z, want, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT) &&
        want == kArriveAbort)
        __hip_atomic_store(p.status, kStatusNotResident, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool coresident(const KParams &p) {
    __shared__ unsigned s_dec;
    __shared__ int s_all;
    unsigned *dec = reinterpret_cast<unsigned *>(p.status + 9);
    if (threadIdx.x == 0) {
        s_all = 1;
        __hip_atomic_store(p.flags + (size_t)blockIdx.x * kFlagStride + 1, 1u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
    if (blockIdx.x == 0) {   // the decider (gridDim.x <= the block size)
        __syncthreads();
        if (threadIdx.x < gridDim.x) {
            const unsigned *f = p.flags + (size_t)threadIdx.x * kFlagStride + 1;
            const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
            while (__hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0u) {
                if (__builtin_amdgcn_s_memrealtime() - t0 > p.arrive_ticks) {
                    s_all = 0;
                    break;
                }
            }
        }
        __syncthreads();
        if (threadIdx.x == 0) propose(p, dec, s_all ? kArriveGo : kArriveAbort);
    }
    if (threadIdx.x == 0) {
        const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
        unsigned d;
        while ((d = __hip_atomic_load(dec, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) == 0u)
            if (__builtin_amdgcn_s_memrealtime() - t0 > 2ull * p.arrive_ticks) propose(p, dec, kArriveAbort);
        s_dec = d;
    }
    __syncthreads();
    return s_dec == kArriveGo;
}

template <int WC, bool ONE>
__global__ void __launch_bounds__(kBlock) decode_loop_kernel(KParams p) {
    extern __shared__ __attribute__((aligned(16))) unsigned char lds_raw[];
    __shared__ Ctl s;
    if (p.arrive_ticks != 0u && !coresident(p)) return;
    const int wg = blockIdx.x;
    const int H = p.H, L = p.L, J = p.J, n_all = p.n_utts;
    unsigned epoch = 0;
    Bufs B;
    B.hx = rsrc(p.hx, (unsigned)((size_t)2 * L * n_all * H * 4));
    B.cx = rsrc(p.cx, (unsigned)((size_t)2 * L * n_all * H * 4));
    B.ppx = rsrc(p.ppx, (unsigned)((size_t)n_all * J * 4));
    B.rx = rsrc(p.rx, (unsigned)((size_t)2 * L * n_all * 4 * H * 4));
    B.ep = rsrc(p.eproj, (unsigned)((size_t)p.V1 * 4 * H * 4));
    B.encp = rsrc(p.encp, (unsigned)(p.encp_rows * J * 4));

    // LDS: one activation block (the joint's hidden block and the LSTM phases'
    // block are never live together), per-(item, wave) partials, then the
    // weight cache
    Lds S;
    unsigned char *wcache = nullptr;
    {
        unsigned char *q = lds_raw;
        for (int a = 0; a <= 1; ++a) {
            const int K = a == 0 ? J : H;
            const int kp = K + kKPad;
            S.act[a].hi = reinterpret_cast<_Float16 *>(q);
            S.act[a].lo = S.act[a].hi + kTile * kp;
            S.act[a].kp = kp;
            S.act[a].n = kTile;
        }
        q += (size_t)kTile * ((J > H ? J : H) + kKPad) * 2 * 2;
        S.st = reinterpret_cast<float *>(q);
        q += (size_t)(L - 1) * p.st_n * p.st_k * kStFloats * 4;
        S.bias = reinterpret_cast<float *>(q);
        q += (size_t)p.bias_floats * 4;
        S.red = reinterpret_cast<f32x4 *>(q);
        q += (size_t)p.red_slots * kWave * sizeof(f32x4);
        if (p.wcache_bytes > 0) wcache = q;
        S.wcache = wcache;
    }

    if (threadIdx.x < kPrN) s.prof[threadIdx.x] = 0ull;
    if (threadIdx.x == 0) s.tq_n = 0;
#ifdef PK_TIMELINE
    if (threadIdx.x < kWaves * kTl) tl_sum()[threadIdx.x] = 0ull;
    if (threadIdx.x < 2 + kTl) tl_ctl()[threadIdx.x] = 0;
#endif
    if (threadIdx.x == 0) {
        s.dom = p.wg_dom[wg];
        s.rank = p.wg_rank[wg];
        s.P = p.dom_size;
        s.n = p.dom_n[s.dom];
        s.own_lstm = owned(p.w_hh[0].tiles, s.rank, s.P);
        s.own_pred = owned(p.w_pred.tiles, s.rank, s.P);
        s.own_out = owned(p.w_out.tiles, s.rank, s.P);
        for (int lc = 0; lc < p.L; ++lc)
            s.pass[lc] = p.red_slots / units_per_item(lc == p.L - 1 ? p.w_pred : p.w_ih[lc + 1]);
        s.pass[p.L] = p.red_slots / units_per_item(p.w_out);
        s.mag_p = udiv_magic(s.P);
        s.mag_h = udiv_magic(p.H);
        s.mag_units = udiv_magic(4 * s.own_lstm);
        unsigned wm = 0;
        for (int ul = 0; ul < kDomCap; ++ul) wm |= (ul % s.P == s.rank ? 1u : 0u) << ul;
        s.wmask = wm;
    }
    if (threadIdx.x < PK_MAX_DURATIONS) s.dur[threadIdx.x] = threadIdx.x < p.n_dur ? p.durations[threadIdx.x] : 0;
    __syncthreads();
    for (int ul = threadIdx.x; ul < s.n; ul += kBlock) {
        const int b = p.dom_list[s.dom * kDomCap + ul];
        const int slot = p.slot[b];
        const int *ctrl = p.slot_ctrl + (size_t)slot * PK_CTRL_N;
        const bool init = ctrl[PK_CTRL_INIT] != 0 && !(p.reset && p.reset[b]);
        s.b[ul] = b;
        s.T[ul] = p.T[b];
        s.erow[ul] = p.encp_row[b];
        s.bbias[ul] = p.blank_bias ? p.blank_bias[b] : 0.0f;
        s.tbase[ul] = p.tokens_base ? p.tokens_base[b] : 0;
        s.ntok[ul] = 0;
        s.steps[ul] = 0;
        s.nseg[ul] = 0;
        s.cur[ul] = 0;
        s.sym[ul] = init ? ctrl[PK_CTRL_SYM] : 0;
        if (p.kind == PK_KIND_EOU && s.T[ul] > 0) s.sym[ul] = 0;   // reset per frame (src/parakeet_eou.cpp:269)
        s.last[ul] = init ? ctrl[PK_CTRL_LAST] : -1;
        s.segst[ul] = init ? ctrl[PK_CTRL_SEGSTART] : 0;
        const int carry = init ? ctrl[PK_CTRL_CARRY] : 0;
        s.pend[ul] = init ? -1 : p.blank;
        s.flags[ul] = init ? 0 : kFlagZeroHC;
        s.brun[ul] = 0;
        if (p.kind == PK_KIND_TDT) s.t[ul] = carry > 0 ? min(carry, s.T[ul]) : 0;
        else s.t[ul] = 0;
    }
    __syncthreads();
    // copy the slot state of this workgroup's utterances into the exchange
    // buffers (kCopyB loads in flight per thread, then the stores)
    const __amdgpu_buffer_rsrc_t bx = rsrc(p.hx, p.xchg_bytes);
    const int nq = state_chunks(p);
    for (int ul = s.rank; ul < s.n; ul += s.P) {
        const int b = s.b[ul], slot = p.slot[b];
        for (int q0 = 0; q0 < nq; q0 += kCopyB * kBlock) {
            float4 v[kCopyB];
            long long xo[kCopyB];
#pragma unroll
            for (int j = 0; j < kCopyB; ++j) {
                const int q = q0 + threadIdx.x + j * kBlock;
                if (q < nq) {
                    const StateChunk c = state_chunk(p, q, slot, b, 0);
                    v[j] = *reinterpret_cast<const float4 *>(c.slot);
                    xo[j] = c.x;
                }
            }
#pragma unroll
            for (int j = 0; j < kCopyB; ++j)
                if (q0 + threadIdx.x + j * kBlock < nq) st4_coh(bx, (unsigned)(xo[j] * 4), v[j]);
        }
    }
    bias_table(p, s.rank, s.P, S.bias);
    // LDS state of layers >= 1: R and c of this workgroup's unit tiles for every utterance of the domain
    if (L > 1) {
        const int n_own = owned(p.w_hh[1].tiles, s.rank, s.P);
        const int n_st = (L - 1) * s.n * n_own * kStFloats;
        for (int i = threadIdx.x; i < n_st; i += kBlock) {
            const int e = i % kStFloats, k = (i / kStFloats) % n_own, ul = (i / kStFloats / n_own) % s.n;
            const int l = 1 + i / (kStFloats * n_own * s.n);
            const int slot = p.slot[s.b[ul]], t = s.rank + k * s.P;
            st_at(p, S, l, ul, k)[e] = e < kTile ? p.slot_r[((size_t)slot * L + l) * 4 * H + t * kTile + e]
                                                 : p.slot_c[((size_t)slot * L + l) * H + t * 4 + (e - kTile)];
        }
    }
    if (wcache) {      // this workgroup's weight tiles, read from LDS for the whole launch
        for (int l = 1; l < L; ++l) cache_matrix(p.w_ih[l], s.rank, s.P, wcache);
        for (int l = 0; l < L; ++l) cache_matrix(p.w_hh[l], s.rank, s.P, wcache);
        cache_matrix(p.w_pred, s.rank, s.P, wcache);
        cache_matrix(p.w_out, s.rank, s.P, wcache);
    }
    build_lists(s, p.spec != 0);
    bool ok = dom_sync(p, s, epoch);

    unsigned iter = 0;
    unsigned long long tlast = __builtin_amdgcn_s_memrealtime();
    while (ok) {
        if (s.nl == 0 && s.nj == 0) break;
        if ((int)iter >= p.max_iter) {
            if (threadIdx.x == 0)
                __hip_atomic_store(p.status, PK_ERR_TIMEOUT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            ok = false;
            break;
        }
        ++iter;
#ifdef PK_TIMELINE
        if (p.prof) {
            if (threadIdx.x == 0) {
                tl_ctl()[0] = (blockIdx.x == 0 && iter >= 40 && iter < 40 + 256) ? 1 : 0;
                *tl_t0() = __builtin_amdgcn_s_memrealtime();
            }
            lds_sync();
        }
#endif
        float4 epre[kStageMax];
        if (s.nj > 0) encp_prefetch(p, s, B, epre);
        if (s.nl > 0) {
            ok = lstm_and_pred<WC>(p, s, B, S, epoch, tlast);
            if (!ok) break;
        }
        if (s.nj > 0) {
            joint_phase<WC, ONE>(p, s, B, S, iter, epre, tlast);
            const bool slots = slot_mode<ONE>(s);
            ok = slots ? gather_slots(p, s, iter) : dom_sync(p, s, epoch);
            TLA(29);
            pmark(p, s, tlast, kPrJSync);
            if (!ok) break;
            decide(p, s, iter, slots);
        }
        lds_sync();
        build_lists(s, p.spec != 0);
        TLA(31);
        pmark(p, s, tlast, kPrDecide);
    }
    if (p.prof && wg == 0 && threadIdx.x < kPrN) p.prof[threadIdx.x] = s.prof[threadIdx.x];
#ifdef PK_TIMELINE
    if (p.prof && wg == 0 && threadIdx.x < kWaves * kTl) p.prof[kPrN + threadIdx.x] = tl_sum()[threadIdx.x];
    if (p.prof && wg == 0 && threadIdx.x < kTl) p.prof[kPrN + kWaves * kTl + threadIdx.x] = tl_ctl()[2 + threadIdx.x];
#endif
    if (!ok) return;

    if (L > 1) {       // layers >= 1: R and c of this workgroup's unit tiles, from its LDS state
        const int n_own = owned(p.w_hh[1].tiles, s.rank, s.P);
        const int n_st = (L - 1) * s.n * n_own * kStFloats;
        for (int i = threadIdx.x; i < n_st; i += kBlock) {
            const int e = i % kStFloats, k = (i / kStFloats) % n_own, ul = (i / kStFloats / n_own) % s.n;
            const int l = 1 + i / (kStFloats * n_own * s.n);
            const int slot = p.slot[s.b[ul]], t = s.rank + k * s.P;
            const float v = st_at(p, S, l, ul, k)[e];
            if (e < kTile) p.slot_r[((size_t)slot * L + l) * 4 * H + t * kTile + e] = v;
            else p.slot_c[((size_t)slot * L + l) * H + t * 4 + (e - kTile)] = v;
        }
    }
    for (int ul = s.rank; ul < s.n; ul += s.P) {
        const int b = s.b[ul], slot = p.slot[b];
        const int cur = s.cur[ul];
        for (int q0 = 0; q0 < nq; q0 += kCopyB * kBlock) {
            float4 v[kCopyB];
            float *dst[kCopyB];
#pragma unroll
            for (int j = 0; j < kCopyB; ++j) {
                const int q = q0 + threadIdx.x + j * kBlock;
                const StateChunk c = state_chunk(p, min(q, nq - 1), slot, b, cur);
                v[j] = ld4_coh(bx, q < nq ? (unsigned)(c.x * 4) : kBad);
                dst[j] = c.slot;
            }
#pragma unroll
            for (int j = 0; j < kCopyB; ++j)
                if (q0 + threadIdx.x + j * kBlock < nq) *reinterpret_cast<float4 *>(dst[j]) = v[j];
        }
        if (threadIdx.x < PK_CTRL_N) {   // the slot's control words (and the caller's copy)
            const int k = threadIdx.x;
            const int v = k == PK_CTRL_INIT ? 1
                        : k == PK_CTRL_SYM ? s.sym[ul]
                        : k == PK_CTRL_CARRY ? ((p.kind == PK_KIND_TDT) ? max(0, s.t[ul] - s.T[ul]) : 0)
                        : k == PK_CTRL_LAST ? s.last[ul]
                        : k == PK_CTRL_SEGSTART ? s.segst[ul] : 0;
            p.slot_ctrl[(size_t)slot * PK_CTRL_N + k] = v;
            if (p.ctrl_out) p.ctrl_out[(size_t)b * PK_CTRL_N + k] = v;
        }
        if (threadIdx.x == 0) {
            p.n_tokens[b] = s.ntok[ul];
            p.steps[b] = s.steps[ul];
            if (p.n_segs) p.n_segs[b] = s.nseg[ul];
            if (s.flags[ul] & (kFlagTokOverflow | kFlagSegOverflow))
                __hip_atomic_store(p.status + 2, PK_ERR_OVERFLOW, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (s.flags[ul] & kFlagTraceOverflow)
                __hip_atomic_store(p.status + 3, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if (threadIdx.x == 0) atomicMax(p.status + 1, (int)iter);
}

}  // namespace pkdev
