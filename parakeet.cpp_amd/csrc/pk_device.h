// pk_device.h -- device code of the MI355X transducer greedy decode.
//
// Included once, by pk_decode.hip.  See that file for the host side and the
// overall structure; this file holds the data layout, the building blocks
// (weight loads, wave reductions, argmax keys, grid barrier, coherent loads
// and stores) and the kernels.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "parakeet_hip.h"

namespace pkdev {

constexpr int kWave = 64;
constexpr int kBlock = 512;                 // 8 waves per workgroup, one workgroup per CU
constexpr int kWaves = kBlock / kWave;
constexpr int kMaxBatch = PK_MAX_BATCH;
constexpr int kUC = 8;                      // utterances per register tile
constexpr int kSmallB = 4;                  // LSTM batch at or below which layer 0 runs redundantly
constexpr int kIdxBits = 14;                // argmax key: index field
constexpr int kStampShift = 46;             // argmax key: 14 index + 32 value bits below the stamp
constexpr unsigned kMaxStamp = (1u << 18) - 1;
constexpr int kFlagStride = 64;             // words between barrier flags (256 B)

// Flags in the per-utterance control word.
constexpr int kFlagZeroHC = 1;              // LSTM input state is zero (init / EOU reset)
constexpr int kFlagTokOverflow = 2;
constexpr int kFlagSegOverflow = 4;
constexpr int kFlagTraceOverflow = 8;

struct DMat {
    const void *w;       // int8 / f16 / f32 plane [rows][cols]
    const float *d;      // q8_0 block scales [rows][cols/32], else null
    int type;
    int rows, cols;
};

struct KParams {
    int kind, H, L, J, V1, Dn, Vo, blank, eou, eob, max_sym, n_dur;
    int durations[PK_MAX_DURATIONS];
    const float *eproj;                      // [V1][4H] W_ih0 . embed[v] + b_ih0 + b_hh0, unit-major
    DMat w_ih[PK_MAX_LAYERS], w_hh[PK_MAX_LAYERS];   // unit-major gate rows
    const float *b_lstm[PK_MAX_LAYERS];      // b_ih + b_hh (unit-major), layers >= 1
    DMat w_pred, w_out;
    const float *b_pred, *b_out;
    const unsigned char *special;
    int n_special;
    // slot state (persistent between calls)
    float *slot_h;       // [slots][L][H]
    float *slot_c;       // [slots][L][H]
    float *slot_pp;      // [slots][J]  b_p + W_p . h[L-1]
    int *slot_ctrl;      // [slots][PK_CTRL_N]
    // batch
    int n_utts;
    const float *encp;           // [rows][J] b_e + W_e . enc
    const long long *encp_row;   // [n_utts]
    const int *T;
    const int *slot;
    const float *blank_bias;     // nullable
    const int *tokens_base;      // nullable
    int *tokens; int token_cap;
    int *n_tokens; int *steps;
    int *segs; int seg_cap; int *n_segs;
    int *trace; int trace_cap;
    // exchange buffers of one launch (batch-indexed, written/read coherently)
    float *hx;           // [2][L][n][H] ping-pong by utterance parity
    float *cx;           // [2][L][n][H]
    float *ppx;          // [n][J]
    float *rx;           // [L][n][4H]  W_hh . h (no bias), unit-major rows
    // sync
    unsigned *flags;             // [nwg * kFlagStride]
    unsigned long long *keys;    // [2][n_utts][2]
    int *status;                 // [0] error code, [1] iterations, [2] overflow, [3] trace overflow
    int max_iter;
};

// ---------------------------------------------------------------- memory helpers

// Buffer resource over [base, base + bytes): out-of-range lanes read 0 and
// drop stores, so a bad index cannot fault.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *base, unsigned bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}

// Agent-coherent (SC1) 16-byte load / store: used for every buffer written by
// one workgroup and read by another inside a launch.  Plain loads elsewhere
// keep weights cached in L2 (no cache-wide invalidation anywhere in the loop).
constexpr int kSC1 = 16;
__device__ __forceinline__ float4 ld4_coh(__amdgpu_buffer_rsrc_t r, unsigned byte_off) {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, kSC1));
}
__device__ __forceinline__ float ld_coh(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coh(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float4 load_w4(const DMat &m, int r, int k) {
    if (m.type == PK_TYPE_Q8_0) {
        const int packed = *reinterpret_cast<const int *>(static_cast<const signed char *>(m.w) + (size_t)r * m.cols + k);
        const float d = m.d[(size_t)r * (m.cols >> 5) + (k >> 5)];
        return make_float4(d * (float)(signed char)(packed), d * (float)(signed char)(packed >> 8),
                           d * (float)(signed char)(packed >> 16), d * (float)(signed char)(packed >> 24));
    } else if (m.type == PK_TYPE_F16) {
        const uint2 raw = *reinterpret_cast<const uint2 *>(static_cast<const __half *>(m.w) + (size_t)r * m.cols + k);
        const float2 fa = __half22float2(*reinterpret_cast<const __half2 *>(&raw.x));
        const float2 fb = __half22float2(*reinterpret_cast<const __half2 *>(&raw.y));
        return make_float4(fa.x, fa.y, fb.x, fb.y);
    }
    return *reinterpret_cast<const float4 *>(static_cast<const float *>(m.w) + (size_t)r * m.cols + k);
}

__device__ __forceinline__ float load_w1(const DMat &m, int r, int k) {
    if (m.type == PK_TYPE_Q8_0) {
        const signed char q = static_cast<const signed char *>(m.w)[(size_t)r * m.cols + k];
        return m.d[(size_t)r * (m.cols >> 5) + (k >> 5)] * (float)q;
    } else if (m.type == PK_TYPE_F16) {
        return __half2float(static_cast<const __half *>(m.w)[(size_t)r * m.cols + k]);
    }
    return static_cast<const float *>(m.w)[(size_t)r * m.cols + k];
}

// ---------------------------------------------------------------- wave reductions

// Butterfly reduction of N per-lane partial sums over the 64 lanes of a wave:
// each exchange halves the values a lane carries.  On return lane l holds the
// total of value index (l >> (6 - log2 N)).  Partners add the same two
// operands, so every lane holding an index holds the same bits.
template <int N, int M>
struct Bfly {
    static __device__ __forceinline__ void run(float *v, int lane) {
        if constexpr (M == 0) {
            return;
        } else if constexpr (N > 1) {
            const bool up = (lane & M) != 0;
#pragma unroll
            for (int i = 0; i < N / 2; ++i) {
                const float send = up ? v[i] : v[i + N / 2];
                const float keep = up ? v[i + N / 2] : v[i];
                v[i] = keep + __shfl_xor(send, M, kWave);
            }
            Bfly<N / 2, M / 2>::run(v, lane);
        } else {
            v[0] = v[0] + __shfl_xor(v[0], M, kWave);
            Bfly<1, M / 2>::run(v, lane);
        }
    }
};

template <int N>
constexpr int ilog2() { return N <= 1 ? 0 : 1 + ilog2<N / 2>(); }

template <int N>
__device__ __forceinline__ float wave_reduce_n(float (&v)[N], int lane) {
    Bfly<N, 32>::run(v, lane);
    return v[0];
}

// acc[r*UC+u] += W[r0+r, :] . xs[u*xstride + :] for R rows (nrows valid), nu <= UC utterances.
template <int R, int UC>
__device__ __forceinline__ void dot_rows(const DMat &m, int r0, int nrows, const float *xs, int xstride, int nu,
                                         float *acc, int lane) {
    for (int k = lane * 4; k < m.cols; k += 4 * kWave) {
        float4 w[R];
#pragma unroll
        for (int r = 0; r < R; ++r) w[r] = (r < nrows) ? load_w4(m, r0 + r, k) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int u = 0; u < UC; ++u) {
            if (u < nu) {
                const float4 x = *reinterpret_cast<const float4 *>(xs + u * xstride + k);
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    float a = acc[r * UC + u];
                    a = fmaf(w[r].x, x.x, a);
                    a = fmaf(w[r].y, x.y, a);
                    a = fmaf(w[r].z, x.z, a);
                    a = fmaf(w[r].w, x.w, a);
                    acc[r * UC + u] = a;
                }
            }
        }
    }
}

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }

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

// ---------------------------------------------------------------- grid barrier

// Every workgroup publishes its epoch in its own flag word and every workgroup
// polls all flags (thread t polls flag t).  No cache-wide fences: data that
// crosses workgroups is stored and loaded agent-coherently (SC1), and each
// thread waits for its own stores (s_waitcnt 0) before arriving.  Returns
// false if the error word is set or the wait exceeds ~2 s of wall clock.
__device__ __forceinline__ bool grid_sync(const KParams &p, unsigned &epoch) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    __shared__ int s_ok;
    ++epoch;
    if (threadIdx.x == 0) {
        s_ok = 1;
        __hip_atomic_store(p.flags + (size_t)blockIdx.x * kFlagStride, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (threadIdx.x < gridDim.x) {
        unsigned *f = p.flags + (size_t)threadIdx.x * kFlagStride;
        const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
        while (__hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < epoch) {
            __builtin_amdgcn_s_sleep(1);
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

__device__ __forceinline__ int split_begin(int i, int total, int parts) {
    return (int)(((long long)i * total) / parts);
}

// ---------------------------------------------------------------- prepare-time kernels

// out[v][r] = bias0[r] + bias1[r] + W[r, :] . E[v, :]: the layer-0 input
// projection of every vocabulary row (W_ih0 . embed[v] + b_ih0 + b_hh0).
__global__ void __launch_bounds__(256) embed_proj_kernel(DMat w, DMat e, const float *__restrict b0,
                                                         const float *__restrict b1, float *__restrict out) {
    const int v0 = blockIdx.x * 16, r0 = blockIdx.y * 64;
    const int K = w.cols;
    __shared__ float es[16][65];
    __shared__ float ws[64][65];
    const int tid = threadIdx.x;
    const int tv = tid / 16, tr = tid % 16;       // 16 vocab rows x 16 thread columns (4 outputs each)
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < K; k0 += 64) {
        for (int i = tid; i < 16 * 64; i += 256) {
            const int vv = i / 64, k = i % 64;
            es[vv][k] = (v0 + vv < e.rows && k0 + k < K) ? load_w1(e, v0 + vv, k0 + k) : 0.0f;
        }
        for (int i = tid; i < 64 * 64; i += 256) {
            const int rr = i / 64, k = i % 64;
            ws[rr][k] = (r0 + rr < w.rows && k0 + k < K) ? load_w1(w, r0 + rr, k0 + k) : 0.0f;
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
    if (v >= e.rows) return;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int r = r0 + tr * 4 + j;
        if (r < w.rows) out[(size_t)v * w.rows + r] = acc[j] + (b0[r] + b1[r]);
    }
}

// ---------------------------------------------------------------- enc_proj

// encp[rows of utterance u] = b_e + W_e . enc[row]  (f32), 64x64 tiles, K step 32.
__global__ void __launch_bounds__(256) enc_proj_kernel(DMat w, const float *__restrict bias,
                                                       const float *__restrict enc, int d_enc,
                                                       const long long *__restrict src_row,
                                                       const long long *__restrict dst_row,
                                                       const int *__restrict T, float *__restrict out) {
    const int u = blockIdx.y;
    const int Tu = T[u];
    const int m0 = blockIdx.x * 64;
    if (m0 >= Tu) return;
    const int n0 = blockIdx.z * 64;
    const int J = w.rows;
    __shared__ float xs[32][65];
    __shared__ float ws[32][65];
    const int tid = threadIdx.x;
    const int tr = tid / 16, tc = tid % 16;     // 16x16 threads, 4x4 outputs each
    float acc[4][4] = {};
    const float *src = enc + (size_t)src_row[u] * d_enc;
    for (int k0 = 0; k0 < d_enc; k0 += 32) {
        for (int i = tid; i < 64 * 32; i += 256) {
            const int r = i / 32, k = i % 32;
            const int m = m0 + r, n = n0 + r;
            xs[k][r] = (m < Tu && k0 + k < d_enc) ? src[(size_t)m * d_enc + k0 + k] : 0.0f;
            ws[k][r] = (n < J && k0 + k < d_enc) ? load_w1(w, n, k0 + k) : 0.0f;
        }
        __syncthreads();
#pragma unroll 8
        for (int k = 0; k < 32; ++k) {
            float a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) { a[i] = xs[k][tr * 4 + i]; b[i] = ws[k][tc * 4 + i]; }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
        }
        __syncthreads();
    }
    float *dst = out + (size_t)dst_row[u] * J;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = m0 + tr * 4 + i;
        if (m >= Tu) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int n = n0 + tc * 4 + j;
            if (n < J) dst[(size_t)m * J + n] = bias[n] + acc[i][j];
        }
    }
}

// ---------------------------------------------------------------- decode loop

struct Ctl {                      // per-workgroup copy of the control state
    int t[kMaxBatch], T[kMaxBatch], sym[kMaxBatch], pend[kMaxBatch], flags[kMaxBatch];
    int ntok[kMaxBatch], steps[kMaxBatch], nseg[kMaxBatch], segst[kMaxBatch], last[kMaxBatch];
    int cur[kMaxBatch];
    int lst[kMaxBatch], jst[kMaxBatch];
    int cnt_l[kMaxBatch / kWave], cnt_j[kMaxBatch / kWave];
    int nl, nj;
    unsigned long long wgkey[kUC][2];
};

__device__ void build_lists(Ctl &s, int n) {
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int nblk = (n + kWave - 1) / kWave;
    for (int b = wave; b < nblk; b += kWaves) {
        const int u = b * kWave + lane;
        const bool fl = u < n && s.pend[u] >= 0;
        const bool fj = u < n && s.t[u] < s.T[u];
        const unsigned long long bl = __ballot(fl), bj = __ballot(fj);
        if (lane == 0) { s.cnt_l[b] = __popcll(bl); s.cnt_j[b] = __popcll(bj); }
    }
    __syncthreads();
    for (int b = wave; b < nblk; b += kWaves) {
        int base_l = 0, base_j = 0;
        for (int i = 0; i < b; ++i) { base_l += s.cnt_l[i]; base_j += s.cnt_j[i]; }
        const int u = b * kWave + lane;
        const bool fl = u < n && s.pend[u] >= 0;
        const bool fj = u < n && s.t[u] < s.T[u];
        const unsigned long long bl = __ballot(fl), bj = __ballot(fj);
        const unsigned long long below = (lane == 0) ? 0ull : (~0ull >> (kWave - lane));
        if (fl) s.lst[base_l + __popcll(bl & below)] = u;
        if (fj) s.jst[base_j + __popcll(bj & below)] = u;
    }
    if (threadIdx.x == 0) {
        int nl = 0, nj = 0;
        for (int i = 0; i < nblk; ++i) { nl += s.cnt_l[i]; nj += s.cnt_j[i]; }
        s.nl = nl;
        s.nj = nj;
    }
    __syncthreads();
}

// Exchange-buffer offsets (floats).
__device__ __forceinline__ size_t hx_off(const KParams &p, int buf, int layer, int b) {
    return (((size_t)buf * p.L + layer) * p.n_utts + b) * p.H;
}
__device__ __forceinline__ size_t rx_off(const KParams &p, int layer, int b) {
    return ((size_t)layer * p.n_utts + b) * 4 * p.H;
}

struct Bufs {                       // buffer resources of the exchange buffers
    __amdgpu_buffer_rsrc_t hx, cx, ppx, rx;
};

// Stage nu utterances' vectors of length len (multiple of 4) from an exchange
// buffer into LDS: dst[u*dstride + k] = src[off(u) + k], coherent loads.
template <class OffFn>
__device__ __forceinline__ void stage_coh(float *dst, int dstride, int nu, int len, __amdgpu_buffer_rsrc_t r,
                                          OffFn off) {
    const int per = len / 4;
    for (int i = threadIdx.x; i < nu * per; i += kBlock) {
        const int u = i / per, k = (i - u * per) * 4;
        *reinterpret_cast<float4 *>(dst + u * dstride + k) = ld4_coh(r, (unsigned)((off(u) + k) * 4));
    }
}

__device__ __forceinline__ void cell(float gi, float gf, float gg, float go, float c_prev, float &c_new, float &h_new) {
    c_new = sigmoidf_(gf) * c_prev + sigmoidf_(gi) * tanhf(gg);
    h_new = sigmoidf_(go) * tanhf(c_new);
}

// LSTM layers >= 1 for this workgroup's units: gates = W_ih . x (staged) +
// R (rx, computed in the joint phase) + b_ih + b_hh, cell update, coherent
// stores of h', c' into the other ping-pong buffer.  xs holds the layer input
// for nu utterances (stride xstride).
__device__ void lstm_upper_layer(const KParams &p, Ctl &s, const Bufs &B, const float *xs, int xstride, int layer,
                                 int c0, int nu, int wg, int nwg) {
    const int H = p.H, lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int j0 = split_begin(wg, H, nwg), j1 = split_begin(wg + 1, H, nwg);
    for (int j = j0 + wave; j < j1; j += kWaves) {
        float acc[4 * kUC];
#pragma unroll
        for (int i = 0; i < 4 * kUC; ++i) acc[i] = 0.0f;
        dot_rows<4, kUC>(p.w_ih[layer], 4 * j, 4, xs, xstride, nu, acc, lane);
        wave_reduce_n<4 * kUC>(acc, lane);
        constexpr int kShift = 6 - ilog2<4 * kUC>();
        float g[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) g[q] = __shfl(acc[0], ((q * kUC + (lane % kUC)) << kShift), kWave);
        if (lane < nu) {
            const int b = s.lst[c0 + lane];
            const bool zero = s.flags[b] & kFlagZeroHC;
            const int cur = s.cur[b];
            const float *bl = p.b_lstm[layer];
            float gate[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float r = zero ? 0.0f : ld_coh(p.rx + rx_off(p, layer, b) + 4 * j + q);
                gate[q] = (g[q] + r) + bl[4 * j + q];
            }
            const float c_prev = zero ? 0.0f : ld_coh(p.cx + hx_off(p, cur, layer, b) + j);
            float c_new, h_new;
            cell(gate[0], gate[1], gate[2], gate[3], c_prev, c_new, h_new);
            st_coh(p.cx + hx_off(p, cur ^ 1, layer, b) + j, c_new);
            st_coh(p.hx + hx_off(p, cur ^ 1, layer, b) + j, h_new);
        }
    }
}

// Layer 0 from the precomputed input projection: gates = E'[token] + R0.
// redundant == true: every workgroup computes every unit (into h0s, LDS,
// stride H) and the unit owners store h', c'; otherwise only own units.
__device__ void lstm_layer0(const KParams &p, Ctl &s, float *h0s, int c0, int nu, bool redundant, int wg, int nwg) {
    const int H = p.H;
    const int j0 = split_begin(wg, H, nwg), j1 = split_begin(wg + 1, H, nwg);
    const int ja = redundant ? 0 : j0, jn = redundant ? H : j1 - j0;
    for (int i = threadIdx.x; i < nu * jn; i += kBlock) {
        const int uu = i / jn, j = ja + (i - uu * jn);
        const int b = s.lst[c0 + uu];
        const bool zero = s.flags[b] & kFlagZeroHC;
        const int cur = s.cur[b];
        const float4 e = *reinterpret_cast<const float4 *>(p.eproj + (size_t)s.pend[b] * 4 * H + 4 * j);
        float4 r = make_float4(0.f, 0.f, 0.f, 0.f);
        float c_prev = 0.0f;
        if (!zero) {
            const float *rp = p.rx + rx_off(p, 0, b) + 4 * j;
            r = make_float4(ld_coh(rp), ld_coh(rp + 1), ld_coh(rp + 2), ld_coh(rp + 3));
            c_prev = ld_coh(p.cx + hx_off(p, cur, 0, b) + j);
        }
        float c_new, h_new;
        cell(e.x + r.x, e.y + r.y, e.z + r.z, e.w + r.w, c_prev, c_new, h_new);
        if (redundant) h0s[uu * H + j] = h_new;
        if (j >= j0 && j < j1) {
            st_coh(p.cx + hx_off(p, cur ^ 1, 0, b) + j, c_new);
            st_coh(p.hx + hx_off(p, cur ^ 1, 0, b) + j, h_new);
        }
    }
}

// pp = b_p + W_p . h[L-1]' for this workgroup's rows; hs holds h[L-1]' (stride H).
__device__ void pred_rows(const KParams &p, Ctl &s, const float *hs, int c0, int nu, int wg, int nwg) {
    const int H = p.H, J = p.J, lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int r0 = split_begin(wg, J, nwg), r1 = split_begin(wg + 1, J, nwg);
    constexpr int R = 2;
    for (int r = r0 + wave * R; r < r1; r += kWaves * R) {
        float acc[R * kUC];
#pragma unroll
        for (int i = 0; i < R * kUC; ++i) acc[i] = 0.0f;
        dot_rows<R, kUC>(p.w_pred, r, min(R, r1 - r), hs, H, nu, acc, lane);
        wave_reduce_n<R * kUC>(acc, lane);
        constexpr int kShift = 6 - ilog2<R * kUC>();
        const int idx = lane >> kShift;
        const int rr = idx / kUC, uu = idx % kUC;
        if ((lane & ((1 << kShift) - 1)) == 0 && uu < nu && r + rr < r1) {
            const int b = s.lst[c0 + uu];
            st_coh(p.ppx + (size_t)b * J + r + rr, p.b_pred[r + rr] + acc[0]);
        }
    }
}

// Joint + argmax for this workgroup's output rows, plus the recurrent products
// R_l = W_hh_l . h_l of its LSTM units for the next step (off the critical path).
__device__ void joint_phase(const KParams &p, Ctl &s, const Bufs &B, float *stage, unsigned stamp, int wg, int nwg) {
    const int J = p.J, H = p.H, L = p.L, lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int r0 = split_begin(wg, p.Vo, nwg), r1 = split_begin(wg + 1, p.Vo, nwg);
    const int j0 = split_begin(wg, H, nwg), j1 = split_begin(wg + 1, H, nwg);
    const int xstride = J + L * H;
    constexpr int R = 2;
    unsigned long long *keys = p.keys + (size_t)(stamp & 1) * p.n_utts * 2;
    for (int c0 = 0; c0 < s.nj; c0 += kUC) {
        const int nu = min(kUC, s.nj - c0);
        // stage: hidden = relu(encp[t] + pp) and h_l for every layer
        const int per = J / 4;
        for (int i = threadIdx.x; i < nu * per; i += kBlock) {
            const int uu = i / per, k = (i - uu * per) * 4;
            const int b = s.jst[c0 + uu];
            const float4 e = *reinterpret_cast<const float4 *>(p.encp + (size_t)(p.encp_row[b] + s.t[b]) * J + k);
            const float4 q = ld4_coh(B.ppx, (unsigned)(((size_t)b * J + k) * 4));
            float4 v = make_float4(e.x + q.x, e.y + q.y, e.z + q.z, e.w + q.w);
            v.x = (0.0f < v.x) ? v.x : 0.0f;
            v.y = (0.0f < v.y) ? v.y : 0.0f;
            v.z = (0.0f < v.z) ? v.z : 0.0f;
            v.w = (0.0f < v.w) ? v.w : 0.0f;
            *reinterpret_cast<float4 *>(stage + uu * xstride + k) = v;
        }
        for (int l = 0; l < L; ++l)
            stage_coh(stage + J + l * H, xstride, nu, H, B.hx,
                      [&](int uu) { const int b = s.jst[c0 + uu]; return hx_off(p, s.cur[b], l, b); });
        if (threadIdx.x < 2 * kUC) s.wgkey[threadIdx.x / 2][threadIdx.x % 2] = 0ull;
        __syncthreads();
        for (int r = r0 + wave * R; r < r1; r += kWaves * R) {
            float acc[R * kUC];
#pragma unroll
            for (int i = 0; i < R * kUC; ++i) acc[i] = 0.0f;
            dot_rows<R, kUC>(p.w_out, r, min(R, r1 - r), stage, xstride, nu, acc, lane);
            wave_reduce_n<R * kUC>(acc, lane);
            constexpr int kShift = 6 - ilog2<R * kUC>();
            const int idx = lane >> kShift;
            const int rr = idx / kUC, uu = idx % kUC;
            const int row = r + rr;
            if ((lane & ((1 << kShift) - 1)) == 0 && uu < nu && row < r1) {
                float v = acc[0] + p.b_out[row];
                const int b = s.jst[c0 + uu];
                if (row == p.blank && p.blank_bias) v += p.blank_bias[b];
                const int head = row < p.V1 ? 0 : 1;
                atomicMax(&s.wgkey[uu][head], make_key(v, head ? row - p.V1 : row));
            }
        }
        // recurrent products for the next LSTM step of these utterances
        for (int job = wave; job < L * (j1 - j0); job += kWaves) {
            const int l = job / (j1 - j0), j = j0 + job % (j1 - j0);
            float acc[4 * kUC];
#pragma unroll
            for (int i = 0; i < 4 * kUC; ++i) acc[i] = 0.0f;
            dot_rows<4, kUC>(p.w_hh[l], 4 * j, 4, stage + J + l * H, xstride, nu, acc, lane);
            wave_reduce_n<4 * kUC>(acc, lane);
            constexpr int kShift = 6 - ilog2<4 * kUC>();
            const int idx = lane >> kShift;
            const int q = idx / kUC, uu = idx % kUC;
            if ((lane & ((1 << kShift) - 1)) == 0 && uu < nu)
                st_coh(p.rx + rx_off(p, l, s.jst[c0 + uu]) + 4 * j + q, acc[0]);
        }
        __syncthreads();
        if (threadIdx.x < 2 * nu) {
            const int uu = threadIdx.x / 2, head = threadIdx.x % 2;
            const unsigned long long k = s.wgkey[uu][head];
            if (k != 0ull)
                __hip_atomic_fetch_max(&keys[(size_t)s.jst[c0 + uu] * 2 + head],
                                       ((unsigned long long)stamp << kStampShift) | k, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
    }
}

// Apply the argmax results of iteration `stamp` to every utterance of the joint
// list: src/parakeet_tdt.cpp:936-967 (TDT) and src/parakeet_eou.cpp:275-332 (EOU).
__device__ void decide(const KParams &p, Ctl &s, unsigned stamp, int wg, int nwg) {
    const unsigned long long *keys = p.keys + (size_t)(stamp & 1) * p.n_utts * 2;
    for (int i = threadIdx.x; i < s.nj; i += kBlock) {
        const int b = s.jst[i];
        const unsigned long long kt = __hip_atomic_load(&keys[(size_t)b * 2], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const unsigned long long kd =
            __hip_atomic_load(&keys[(size_t)b * 2 + 1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (key_stamp(kt) != stamp || (p.Dn > 0 && key_stamp(kd) != stamp)) {
            __hip_atomic_store(p.status, PK_ERR_DEVICE, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s.t[b] = s.T[b];
            continue;
        }
        const int tok = key_index(kt);
        const int di = p.Dn > 0 ? key_index(kd) : -1;
        const bool writer = (b % nwg) == wg;
        const int step = s.steps[b]++;
        if (writer && p.trace) {
            if (step < p.trace_cap) {
                p.trace[((size_t)b * p.trace_cap + step) * 2] = tok;
                p.trace[((size_t)b * p.trace_cap + step) * 2 + 1] = di;
            } else {
                s.flags[b] |= kFlagTraceOverflow;
            }
        }
        if (p.kind == PK_KIND_TDT) {
            const int dur = p.n_dur > 0 ? p.durations[di] : di;
            const int adv = dur > 1 ? dur : 1;
            if (tok == p.blank) {
                s.t[b] += adv;
                s.sym[b] = 0;
                continue;
            }
            const int n = s.ntok[b]++;
            if (writer) {
                if (n < p.token_cap) p.tokens[(size_t)b * p.token_cap + n] = tok;
                else s.flags[b] |= kFlagTokOverflow;
            }
            s.pend[b] = tok;
            s.sym[b] += 1;
            if (dur > 0 || s.sym[b] >= p.max_sym) {
                s.t[b] += adv;
                s.sym[b] = 0;
            }
        } else {
            const int max_syms = p.max_sym > 1 ? p.max_sym : 1;
            bool frame_done = false;
            if (tok == p.blank || tok == p.eob) {
                frame_done = true;
            } else if (tok == p.eou) {
                const int total = (p.tokens_base ? p.tokens_base[b] : 0) + s.ntok[b];
                if (total > s.segst[b]) {
                    const int ns = s.nseg[b]++;
                    if (writer) {
                        if (p.segs && ns < p.seg_cap) p.segs[(size_t)b * p.seg_cap + ns] = total;
                        else s.flags[b] |= kFlagSegOverflow;
                    }
                    s.segst[b] = total;
                }
                s.flags[b] |= kFlagZeroHC;
                s.pend[b] = p.blank;
                s.last[b] = p.blank;
                frame_done = true;
            } else if (tok >= 0 && tok < p.n_special && p.special[tok]) {
                frame_done = true;
            } else {
                const int n = s.ntok[b]++;
                if (writer) {
                    if (n < p.token_cap) p.tokens[(size_t)b * p.token_cap + n] = tok;
                    else s.flags[b] |= kFlagTokOverflow;
                }
                s.pend[b] = tok;
                s.last[b] = tok;
                s.sym[b] += 1;
                if (s.sym[b] >= max_syms) frame_done = true;
            }
            if (frame_done) {          // the next frame starts with sym = 0 (src/parakeet_eou.cpp:269)
                s.t[b] += 1;
                if (s.t[b] < s.T[b]) s.sym[b] = 0;
            }
        }
    }
}

// One LSTM step (all layers) and the pred projection for every utterance of
// the LSTM list.  Small lists run layer 0 redundantly in every workgroup
// (no barrier between layer 0 and layer 1); larger lists split every layer
// by units with a barrier after each.
__device__ bool lstm_and_pred(const KParams &p, Ctl &s, const Bufs &B, float *stage, unsigned &epoch, int wg,
                              int nwg) {
    const int H = p.H, L = p.L;
    const bool small = s.nl <= kSmallB;
    if (small) {
        // stage layout: [h_0' (nu x H)] [h_1' ...]: layer l's output is layer l+1's input
        const int nu = s.nl;
        lstm_layer0(p, s, stage, 0, nu, true, wg, nwg);
        __syncthreads();
        for (int l = 1; l < L; ++l) {
            if (l > 1) {     // deeper layers need the full h_{l-1}' from every owner
                if (!grid_sync(p, epoch)) return false;
                stage_coh(stage, H, nu, H, B.hx,
                          [&](int uu) { const int b = s.lst[uu]; return hx_off(p, s.cur[b] ^ 1, l - 1, b); });
                __syncthreads();
            }
            lstm_upper_layer(p, s, B, stage, H, l, 0, nu, wg, nwg);
        }
        if (L > 1) {
            if (!grid_sync(p, epoch)) return false;
            stage_coh(stage, H, nu, H, B.hx,
                      [&](int uu) { const int b = s.lst[uu]; return hx_off(p, s.cur[b] ^ 1, L - 1, b); });
        }
        __syncthreads();
        pred_rows(p, s, stage, 0, nu, wg, nwg);
    } else {
        for (int c0 = 0; c0 < s.nl; c0 += kUC * 4) {
            const int nu = min(kUC * 4, s.nl - c0);
            lstm_layer0(p, s, nullptr, c0, nu, false, wg, nwg);
        }
        if (!grid_sync(p, epoch)) return false;
        for (int l = 1; l < L; ++l) {
            for (int c0 = 0; c0 < s.nl; c0 += kUC) {
                const int nu = min(kUC, s.nl - c0);
                stage_coh(stage, H, nu, H, B.hx,
                          [&](int uu) { const int b = s.lst[c0 + uu]; return hx_off(p, s.cur[b] ^ 1, l - 1, b); });
                __syncthreads();
                lstm_upper_layer(p, s, B, stage, H, l, c0, nu, wg, nwg);
                __syncthreads();
            }
            if (!grid_sync(p, epoch)) return false;
        }
        for (int c0 = 0; c0 < s.nl; c0 += kUC) {
            const int nu = min(kUC, s.nl - c0);
            stage_coh(stage, H, nu, H, B.hx,
                      [&](int uu) { const int b = s.lst[c0 + uu]; return hx_off(p, s.cur[b] ^ 1, L - 1, b); });
            __syncthreads();
            pred_rows(p, s, stage, c0, nu, wg, nwg);
            __syncthreads();
        }
    }
    // the new state becomes current
    __syncthreads();
    for (int i = threadIdx.x; i < s.nl; i += kBlock) {
        const int b = s.lst[i];
        s.cur[b] ^= 1;
        s.pend[b] = -1;
        s.flags[b] &= ~kFlagZeroHC;
    }
    return grid_sync(p, epoch);
}

__global__ void __launch_bounds__(kBlock) decode_loop_kernel(KParams p) {
    extern __shared__ float stage[];
    __shared__ Ctl s;
    const int wg = blockIdx.x, nwg = gridDim.x;
    const int n = p.n_utts, H = p.H, L = p.L, J = p.J;
    unsigned epoch = 0;
    Bufs B;
    B.hx = rsrc(p.hx, (unsigned)((size_t)2 * L * n * H * 4));
    B.cx = rsrc(p.cx, (unsigned)((size_t)2 * L * n * H * 4));
    B.ppx = rsrc(p.ppx, (unsigned)((size_t)n * J * 4));
    B.rx = rsrc(p.rx, (unsigned)((size_t)L * n * 4 * H * 4));

    for (int b = threadIdx.x; b < n; b += kBlock) {
        const int slot = p.slot[b];
        const int *ctrl = p.slot_ctrl + (size_t)slot * PK_CTRL_N;
        const bool init = ctrl[PK_CTRL_INIT] != 0;
        s.T[b] = p.T[b];
        s.ntok[b] = 0;
        s.steps[b] = 0;
        s.nseg[b] = 0;
        s.cur[b] = 0;
        s.sym[b] = init ? ctrl[PK_CTRL_SYM] : 0;
        if (p.kind == PK_KIND_EOU && s.T[b] > 0) s.sym[b] = 0;   // reset per frame (src/parakeet_eou.cpp:269)
        s.last[b] = init ? ctrl[PK_CTRL_LAST] : -1;
        s.segst[b] = init ? ctrl[PK_CTRL_SEGSTART] : 0;
        const int carry = init ? ctrl[PK_CTRL_CARRY] : 0;
        s.pend[b] = init ? -1 : p.blank;
        s.flags[b] = init ? 0 : kFlagZeroHC;
        if (p.kind == PK_KIND_TDT) s.t[b] = carry > 0 ? min(carry, s.T[b]) : 0;
        else s.t[b] = 0;
    }
    // copy the slot state of this workgroup's utterances into the exchange buffers
    for (int b = wg; b < n; b += nwg) {
        const int slot = p.slot[b];
        for (int i = threadIdx.x; i < L * H; i += kBlock) {
            const int l = i / H, k = i - l * H;
            st_coh(p.hx + hx_off(p, 0, l, b) + k, p.slot_h[(size_t)slot * L * H + i]);
            st_coh(p.cx + hx_off(p, 0, l, b) + k, p.slot_c[(size_t)slot * L * H + i]);
        }
        for (int i = threadIdx.x; i < J; i += kBlock) st_coh(p.ppx + (size_t)b * J + i, p.slot_pp[(size_t)slot * J + i]);
    }
    __syncthreads();
    build_lists(s, n);
    bool ok = grid_sync(p, epoch);

    unsigned iter = 0;
    while (ok) {
        if (s.nl == 0 && s.nj == 0) break;
        if ((int)iter >= p.max_iter) {
            if (wg == 0 && threadIdx.x == 0)
                __hip_atomic_store(p.status, PK_ERR_TIMEOUT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            ok = false;
            break;
        }
        ++iter;
        if (s.nl > 0) {
            ok = lstm_and_pred(p, s, B, stage, epoch, wg, nwg);
            if (!ok) break;
        }
        if (s.nj > 0) {
            joint_phase(p, s, B, stage, iter, wg, nwg);
            ok = grid_sync(p, epoch);
            if (!ok) break;
            decide(p, s, iter, wg, nwg);
        }
        __syncthreads();
        build_lists(s, n);
    }
    if (!ok) return;

    for (int b = wg; b < n; b += nwg) {
        const int slot = p.slot[b];
        const int cur = s.cur[b];
        for (int i = threadIdx.x; i < L * H; i += kBlock) {
            const int l = i / H, k = i - l * H;
            p.slot_h[(size_t)slot * L * H + i] = ld_coh(p.hx + hx_off(p, cur, l, b) + k);
            p.slot_c[(size_t)slot * L * H + i] = ld_coh(p.cx + hx_off(p, cur, l, b) + k);
        }
        for (int i = threadIdx.x; i < J; i += kBlock) p.slot_pp[(size_t)slot * J + i] = ld_coh(p.ppx + (size_t)b * J + i);
        if (threadIdx.x == 0) {
            int *ctrl = p.slot_ctrl + (size_t)slot * PK_CTRL_N;
            ctrl[PK_CTRL_INIT] = 1;
            ctrl[PK_CTRL_SYM] = s.sym[b];
            ctrl[PK_CTRL_CARRY] = (p.kind == PK_KIND_TDT) ? max(0, s.t[b] - s.T[b]) : 0;
            ctrl[PK_CTRL_LAST] = s.last[b];
            ctrl[PK_CTRL_SEGSTART] = s.segst[b];
            ctrl[PK_CTRL_CUR] = 0;
            p.n_tokens[b] = s.ntok[b];
            p.steps[b] = s.steps[b];
            if (p.n_segs) p.n_segs[b] = s.nseg[b];
            if (s.flags[b] & (kFlagTokOverflow | kFlagSegOverflow))
                __hip_atomic_store(p.status + 2, PK_ERR_OVERFLOW, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (s.flags[b] & kFlagTraceOverflow)
                __hip_atomic_store(p.status + 3, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if (wg == 0 && threadIdx.x == 0) p.status[1] = (int)iter;
}

}  // namespace pkdev
