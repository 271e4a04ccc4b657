// pk_decode.hip -- MI355X (gfx950) transducer greedy decode: host side + C ABI.
//
// Replaces the decode loop of parakeet.cpp (tdt_decode_window,
// src/parakeet_tdt.cpp:865-981; eou_decode_window, src/parakeet_eou.cpp:232-336)
// with one persistent, batch-over-utterances kernel (pk_device.h):
//
//   enc_proj_kernel     b_e + W_e . enc[t] for every frame of every utterance,
//                       once per window (src/parakeet_tdt.cpp:433-483 computes
//                       the same projection as a ggml graph; the CPU path
//                       recomputes it per step at :167-168).  At most
//                       kNarrowRows rows: enc_proj_narrow_kernel instead
//                       (bit-identical outputs).
//   decode_loop_kernel  all lockstep iterations of all utterances in one
//                       launch (an ordinary dispatch whose workgroups first
//                       check that the whole grid is resident, relaunched
//                       cooperatively if not; see launch_loop).  The batch is split into
//                       independent domains (16 or 32 utterances, each on
//                       nwg/C workgroups with its own barrier); one iteration
//                       of a domain is
//                         LSTM layer 0        gates = E'[token] + W_hh0 . h0
//                         LSTM layers >= 1    MFMA tiles, cell update in the epilogue
//                         pred projection     pp = b_p + W_p . h[L-1]
//                         joint + argmax      logits = b_o + W_o . relu(encp[t] + pp),
//                                             and W_hh_l . h_l for the next step
//                         decisions           token / duration / frame advance,
//                                             symbol cap, EOU reset, compaction
//                       with a barrier after each dependent phase.
//
// Weights stay at their stored precision.  Matrices used per step are tiled
// as MFMA A fragments (16 rows x 32 columns per fragment); q8_0 integers go
// through the matrix cores exactly as f16 and the block scale d is applied in
// f32 per 32-column block; activations enter as f16 pairs (hi + lo = x to
// about 2^-22 relative).  The layer-0 input projection of every token,
// E'[v] = W_ih0 . embed[v] + b_ih0 + b_hh0, is computed once at load in f32.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cerrno>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <numeric>
#include <string>
#include <vector>

#include <fcntl.h>
#include <sys/file.h>
#include <sys/stat.h>
#include <unistd.h>

extern char **environ;

#include "parakeet_hip.h"
#include "pk_device.h"

namespace {

using pkdev::KParams;
using pkdev::TMat;
using pkdev::kBlock;
using pkdev::kDomCap;
using pkdev::kFlagStride;
using pkdev::kIdxBits;
using pkdev::kKPad;
using pkdev::kMaxStamp;
using pkdev::kSmallB;
using pkdev::kTile;
using pkdev::kWave;
using pkdev::kWaves;

constexpr int kMaxBatch = PK_MAX_BATCH;
// host outputs up to this size come back whole with the counters (one stream wait per call)
constexpr size_t kEagerCopyBytes = 256 << 10;
// host frames up to this size go up through a pinned staging block of the decoder
constexpr size_t kPinnedFrames = 64ull << 20;
// windows shorter than this many frames do not fill the LDS weight cache
constexpr int kCacheMinFrames = 16;
// enc_proj over at most this many rows runs the narrow kernel (one wave per 16x16 block;
// measured faster up to 256 rows, slower from 750 on)
constexpr long long kNarrowRows = 256;

thread_local std::string g_err;

// Decode-loop launches of this process, per device: the loop's workgroups
// wait on one another, so two loops must never share a device.  Every launch
// waits for the previous one on the same device: on the same stream by stream
// order, from another stream through an event recorded on the previous loop's
// stream at this launch (its work so far, the loop included).
struct LoopOrder {
    std::mutex mu;
    std::map<int, hipStream_t> last_stream;   // per device: the stream of the latest loop launch
    std::map<int, hipEvent_t> last;       // per device: event for a wait across streams
    std::map<int, bool> coop_refused;     // per device: cooperative launches refused once
    std::map<int, int> coop_left;         // per device: launches still cooperative after a grid
                                          // found not co-resident
};
LoopOrder g_loops;
// set by an atexit handler: process teardown has begun
std::atomic<bool> g_exiting{false};

int fail(int rc, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return rc;
}

#define HIP_TRY(expr)                                                                          \
    do {                                                                                       \
        hipError_t e_ = (expr);                                                                \
        if (e_ != hipSuccess) return fail(PK_ERR_DEVICE, "%s: %s", #expr, hipGetErrorString(e_)); \
    } while (0)

float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t mant = h & 0x3FFu, bits;
    if (e == 0) {
        if (mant == 0) bits = sign;
        else {
            int k = -1;
            do { ++k; mant <<= 1; } while ((mant & 0x400u) == 0);
            bits = sign | ((uint32_t)(127 - 15 - k) << 23) | ((mant & 0x3FFu) << 13);
        }
    } else if (e == 0x1F) bits = sign | 0x7F800000u | (mant << 13);
    else bits = sign | ((e + 127 - 15) << 23) | (mant << 13);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

struct DevBuf {
    void *p = nullptr;
    size_t n = 0;
    DevBuf() = default;
    DevBuf(const DevBuf &) = delete;
    DevBuf &operator=(const DevBuf &) = delete;
    ~DevBuf() { if (p) (void)hipFree(p); }
    int ensure(size_t bytes) {
        if (bytes <= n) return 0;
        if (p) (void)hipFree(p);
        p = nullptr;
        n = 0;
        if (hipMalloc(&p, bytes) != hipSuccess) { p = nullptr; return fail(PK_ERR_NOMEM, "hipMalloc(%zu) failed", bytes); }
        n = bytes;
        return 0;
    }
    template <class T> T *as() const { return static_cast<T *>(p); }
};

// Pinned host memory, grown on demand (staging of the outputs copied back).
struct HostBuf {
    void *p = nullptr;
    size_t n = 0;
    HostBuf() = default;
    HostBuf(const HostBuf &) = delete;
    HostBuf &operator=(const HostBuf &) = delete;
    ~HostBuf() { if (p) (void)hipHostFree(p); }
    int ensure(size_t bytes) {
        if (bytes <= n) return 0;
        if (p) (void)hipHostFree(p);
        p = nullptr;
        n = 0;
        if (hipHostMalloc(&p, bytes, hipHostMallocDefault) != hipSuccess) {
            p = nullptr;
            return fail(PK_ERR_NOMEM, "hipHostMalloc(%zu) failed", bytes);
        }
        n = bytes;
        return 0;
    }
    template <class T> T *as() const { return static_cast<T *>(p); }
};

// Block-quantized ggml types: 32 weights per block, one f16 scale d, weight = d * q.
//   q8_0 {f16 d; int8 q[32]}                      q in -128 .. 127 (34 bytes)
//   q5_0 {f16 d; u8 qh[4]; u8 qs[16]}             q = (nibble | high bit << 4) - 16 (22 bytes)
//   q4_0 {f16 d; u8 qs[16]}                       q = nibble - 8 (18 bytes)
// Nibbles: qs[j] & 15 is weight j, qs[j] >> 4 is weight j + 16; bit j of the
// little-endian word qh is the high bit of weight j (ggml's block formats; the
// reference converter writes all three, scripts/convert-nemo-to-gguf.py:90-103).
bool quantized(int type) { return type == PK_TYPE_Q8_0 || type == PK_TYPE_Q5_0 || type == PK_TYPE_Q4_0; }
int block_bytes(int type) { return type == PK_TYPE_Q8_0 ? 34 : type == PK_TYPE_Q5_0 ? 22 : 18; }

// One block as its scale bits and 32 exact int8 weights: q4_0 and q5_0 blocks
// become q8_0 blocks with the same scale, so the device runs one exact path.
void block_q(const uint8_t *blk, int type, uint16_t &dh, int8_t (&q)[32]) {
    memcpy(&dh, blk, 2);
    if (type == PK_TYPE_Q8_0) {
        memcpy(q, blk + 2, 32);
        return;
    }
    uint32_t qh = 0;
    const uint8_t *qs = blk + 2;
    if (type == PK_TYPE_Q5_0) {
        memcpy(&qh, blk + 2, 4);
        qs = blk + 6;
    }
    const int bias = type == PK_TYPE_Q5_0 ? 16 : 8;
    for (int j = 0; j < 16; ++j) {
        const int lo = (qs[j] & 15) | (int)(((qh >> j) & 1u) << 4);
        const int hi = (qs[j] >> 4) | (int)(((qh >> (j + 16)) & 1u) << 4);
        q[j] = (int8_t)(lo - bias);
        q[j + 16] = (int8_t)(hi - bias);
    }
}

int check_tensor(const pk_tensor &t, int rows, int cols, const char *name) {
    if (!t.data) return fail(PK_ERR_TENSOR, "missing tensor %s", name);
    if (t.ne0 != cols || t.ne1 != rows)
        return fail(PK_ERR_TENSOR, "%s: ne=[%lld,%lld], expected [%d,%d]", name, (long long)t.ne0, (long long)t.ne1,
                    cols, rows);
    if (t.type != PK_TYPE_F32 && t.type != PK_TYPE_F16 && !quantized(t.type))
        return fail(PK_ERR_UNSUPPORTED, "%s: ggml type %d not supported", name, t.type);
    if (quantized(t.type) && cols % 32) return fail(PK_ERR_TENSOR, "%s: block-quantized row length %d", name, cols);
    return 0;
}

// Stored row sr of a tensor as f32 (ggml to_float: d*q per block, f16 -> f32).
void row_f32(const pk_tensor &t, int cols, int sr, float *out) {
    const uint8_t *src = static_cast<const uint8_t *>(t.data);
    if (quantized(t.type)) {
        const int bb = block_bytes(t.type);
        const uint8_t *row = src + (size_t)sr * (cols / 32) * bb;
        for (int b = 0; b < cols / 32; ++b) {
            uint16_t dh;
            int8_t q[32];
            block_q(row + (size_t)bb * b, t.type, dh, q);
            const float d = f16_to_f32(dh);
            for (int j = 0; j < 32; ++j) out[32 * b + j] = (float)q[j] * d;
        }
    } else if (t.type == PK_TYPE_F16) {
        const uint16_t *row = reinterpret_cast<const uint16_t *>(src) + (size_t)sr * cols;
        for (int j = 0; j < cols; ++j) out[j] = f16_to_f32(row[j]);
    } else {
        memcpy(out, reinterpret_cast<const float *>(src) + (size_t)sr * cols, 4 * (size_t)cols);
    }
}

// Dense f32 copy [rows][cols] of a stored matrix; map[r] = stored row placed at r.
int dense_f32(const pk_tensor &t, int rows, int cols, const std::vector<int> *map, std::vector<float> &out,
              const char *name) {
    if (int rc = check_tensor(t, rows, cols, name)) return rc;
    out.resize((size_t)rows * cols);
    for (int r = 0; r < rows; ++r) row_f32(t, cols, map ? (*map)[r] : r, out.data() + (size_t)r * cols);
    return 0;
}

int vec_f32(const pk_tensor &t, int n, const std::vector<int> *map, std::vector<float> &out, const char *name) {
    if (!t.data) return fail(PK_ERR_TENSOR, "missing tensor %s", name);
    if (t.ne0 * t.ne1 != n)
        return fail(PK_ERR_TENSOR, "%s: %lld elements, expected %d", name, (long long)(t.ne0 * t.ne1), n);
    if (t.type != PK_TYPE_F32 && t.type != PK_TYPE_F16) return fail(PK_ERR_UNSUPPORTED, "%s: bias type %d", name, t.type);
    std::vector<float> tmp(n);
    row_f32(t, n, 0, tmp.data());
    out.resize(n);
    for (int i = 0; i < n; ++i) out[i] = tmp[map ? (*map)[i] : i];
    return 0;
}

// A matrix tiled as MFMA A fragments (see TMat in pk_device.h), host side.
struct HostTiled {
    int type = 0, rows = 0, tiles = 0, KB = 0, KBa = 0;
    std::vector<uint8_t> a;   // f32: the hi plane, then the lo plane
    std::vector<uint16_t> scale;   // (unused: q8_0 block scales live in the unit records of `a`)
};

int tile_matrix(const pk_tensor &t, int rows, int cols, const std::vector<int> *map, HostTiled &out, const char *name) {
    if (int rc = check_tensor(t, rows, cols, name)) return rc;
    if (cols % 32) return fail(PK_ERR_UNSUPPORTED, "%s: row length %d not a multiple of 32", name, cols);
    out.type = quantized(t.type) ? PK_TYPE_Q8_0 : t.type;   // q4_0 / q5_0 repacked exactly as q8_0
    out.rows = rows;
    out.tiles = (rows + kTile - 1) / kTile;
    out.KBa = cols / 32;
    // stored with whole units of K blocks (zero weights and scales past K / 32; an f32
    // block counts twice, once per plane), so the decode loop's products never mask a unit
    const int ub = out.type == PK_TYPE_F32 ? pkdev::unit_blocks(out.type) / 2 : pkdev::unit_blocks(out.type);
    out.KB = (out.KBa + ub - 1) / ub * ub;
    const size_t frags = (size_t)out.tiles * out.KB;
    const uint8_t *src = static_cast<const uint8_t *>(t.data);
    if (quantized(t.type)) {
        // unit records (pkdev::TMat): per tile and unit of 5 blocks, lane l's bytes of blocks
        // 0-1, of blocks 2-3, of block 4, then 16 bytes of block scales per row
        const int bb = block_bytes(t.type);
        const int units = out.KB / pkdev::kQ8Unit;
        out.a.assign((size_t)out.tiles * units * pkdev::kQ8UnitBytes, 0);
        for (int tile = 0; tile < out.tiles; ++tile)
            for (int r = 0; r < kTile; ++r) {
                const int row = tile * kTile + r;
                if (row >= rows) continue;
                const uint8_t *srow = src + (size_t)(map ? (*map)[row] : row) * out.KBa * bb;
                for (int kb = 0; kb < out.KBa; ++kb) {
                    const int uc = kb / pkdev::kQ8Unit, j = kb % pkdev::kQ8Unit;
                    uint8_t *rec = out.a.data() + ((size_t)tile * units + uc) * pkdev::kQ8UnitBytes;
                    uint16_t dh;
                    int8_t q[32];
                    block_q(srow + (size_t)bb * kb, t.type, dh, q);
                    memcpy(rec + pkdev::kQ8Scales + r * 16 + j * 2, &dh, 2);
                    for (int g = 0; g < 4; ++g) {   // lane r + 16 g holds q[8g .. 8g+8) as q ^ 0x80
                        const int lane = r + 16 * g;
                        uint8_t *dst = j < 4 ? rec + (j / 2) * 1024 + lane * 16 + (j % 2) * 8 : rec + 2048 + lane * 8;
                        for (int i = 0; i < 8; ++i) dst[i] = (uint8_t)q[8 * g + i] ^ 0x80;
                    }
                }
            }
    } else {
        std::vector<float> row(cols);
        const size_t plane = frags * kWave * 16;   // bytes of one f16 plane
        out.a.assign(t.type == PK_TYPE_F32 ? 2 * plane : plane, 0);
        for (int tile = 0; tile < out.tiles; ++tile)
            for (int r = 0; r < kTile; ++r) {
                const int rr = tile * kTile + r;
                if (rr >= rows) continue;
                row_f32(t, cols, map ? (*map)[rr] : rr, row.data());
                for (int kb = 0; kb < out.KBa; ++kb) {
                    const size_t f = (size_t)tile * out.KB + kb;
                    for (int g = 0; g < 4; ++g)
                        for (int i = 0; i < 8; ++i) {
                            const float w = row[32 * kb + 8 * g + i];
                            const _Float16 hi = (_Float16)w;
                            const size_t at = ((f * kWave + r + 16 * g) * 8 + i) * 2;
                            memcpy(&out.a[at], &hi, 2);
                            if (t.type == PK_TYPE_F32) {
                                const _Float16 lo = (_Float16)(w - (float)hi);
                                memcpy(&out.a[plane + at], &lo, 2);
                            }
                        }
                }
            }
    }
    return 0;
}

// ---------------------------------------------------------------- fixed scratch
//
// pk_decode_noalloc takes every device buffer of a call beyond its inputs and
// outputs (descriptor block, enc_proj rows, status / barrier flags / argmax
// keys, exchange buffers) from this array instead of allocating.  Each device
// holds its own copy for the life of the process; host code never uses the
// symbol itself, only the address hipGetSymbolAddress returns for the current
// device (kept per device in g_scratch).
constexpr size_t kScratchBytes = (size_t)32 << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

struct ScratchTable {
    std::mutex mu;
    std::map<int, unsigned char *> ptr;   // device -> address of its scratch array
};
ScratchTable g_scratch;

// The current device's scratch address, resolved once per device.
int scratch_address(int device, unsigned char **out) {
    std::lock_guard<std::mutex> lk(g_scratch.mu);
    auto it = g_scratch.ptr.find(device);
    if (it != g_scratch.ptr.end()) {
        *out = it->second;
        return 0;
    }
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
        return fail(PK_ERR_DEVICE, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    g_scratch.ptr[device] = static_cast<unsigned char *>(ptr);
    *out = static_cast<unsigned char *>(ptr);
    return 0;
}

}  // namespace

struct pk_decoder {
    KParams kp{};              // weights + dims (batch fields filled per call)
    pk_decoder_desc desc{};    // host copy of the description (tensor pointers not kept)
    const _Float16 *w_enc_hi = nullptr, *w_enc_lo = nullptr;   // joint.enc [J][D] as f16 hi + lo planes
    const float *b_enc = nullptr;                               // joint.enc bias
    int n_slots = 0;
    int device = 0;
    int n_cu = 0, lds_block = 0;
    int nwg = 0;               // decode-loop workgroups
    size_t lds_bytes = 0;      // dynamic LDS limit of the decode loop
    size_t lds_fixed = 0;      // activation blocks + redundant layer-0 output
    hipStream_t stream = nullptr;
    hipEvent_t ev[3] = {};
    bool timing = true;        // record ev[] in each call (pk_decoder_set_timing)
    bool timed = false;        // the last call recorded them
    DevBuf arena;              // weights
    DevBuf eproj;              // [V1][4H] layer-0 input projection of every token
    DevBuf slots_h, slots_c, slots_pp, slots_r, slots_ctrl;
    DevBuf special;
    // per-call scratch
    DevBuf d_desc, d_encp, d_clear, d_enc, d_out, d_xchg, d_prof, d_lcol;   // d_clear: status, barrier flags, argmax keys
    std::vector<uint8_t> h_desc;
    HostBuf h_pin;             // pinned: 16 B of status read back, the descriptor block, then the
                               // per-utterance counters read back (sized at creation for n_slots
                               // utterances, so these copies are asynchronous and no call allocates)
    size_t pin_cnt = 0;        // offset of the counters in h_pin (the descriptor block ends there)
    HostBuf h_out;             // staging of host-memory outputs
    HostBuf h_frames;          // staging of host-memory frames (up to kPinnedFrames bytes)
    unsigned char *scratch = nullptr;   // this device's fixed scratch array (pk_decode_noalloc)
    int last_iters = 0;
    // a call decoded in several launches (decode_chained): the kernels' times and the
    // lockstep iterations summed over its launches, which pk_last_timing then reports
    bool chained = false;
    float chain_ep_ms = 0.f, chain_loop_ms = 0.f;
    int chain_iters = 0;
    int lock_fd = -1;          // this GPU's cross-process loop lock (see DeviceLoopLock), -1: none
    const void *loop_fn[2] = {};   // the decode-loop instantiations for this decoder's weight storage:
                                   // several domains, one domain (argmax key slots)
    // Drop every device and pinned allocation without freeing it (process exit).
    void forget_device() {
        for (DevBuf *b : {&arena, &eproj, &slots_h, &slots_c, &slots_pp, &slots_r, &slots_ctrl, &special, &d_desc,
                          &d_encp, &d_clear, &d_enc, &d_out, &d_xchg, &d_prof, &d_lcol}) {
            b->p = nullptr;
            b->n = 0;
        }
        for (HostBuf *b : {&h_pin, &h_out, &h_frames}) {
            b->p = nullptr;
            b->n = 0;
        }
    }
};

namespace {

// One device arena for every weight plane and bias.
struct Arena {
    std::vector<std::pair<const void *, size_t>> parts;
    std::vector<const void **> dst;
    void add(const void *host, size_t bytes, const void **where) {
        parts.emplace_back(host, bytes);
        dst.push_back(where);
    }
    int upload(DevBuf &buf) {
        auto align = [](size_t x) { return (x + 255) & ~(size_t)255; };
        size_t total = 0;
        for (auto &p : parts) total += align(p.second);
        if (int rc = buf.ensure(std::max<size_t>(total, 256))) return rc;
        size_t off = 0;
        for (size_t i = 0; i < parts.size(); ++i) {
            uint8_t *d = buf.as<uint8_t>() + off;
            if (parts[i].second) HIP_TRY(hipMemcpy(d, parts[i].first, parts[i].second, hipMemcpyHostToDevice));
            *dst[i] = parts[i].second ? d : nullptr;
            off += align(parts[i].second);
        }
        return 0;
    }
};

void arena_tiled(Arena &ar, HostTiled &h, TMat &m) {
    m.type = h.type;
    m.rows = h.rows;
    m.tiles = h.tiles;
    m.KB = h.KB;
    m.KBa = h.KBa;
    ar.add(h.a.data(), h.a.size(), &m.a);
    ar.add(h.scale.data(), h.scale.size() * 2, reinterpret_cast<const void **>(&m.scale));
}

// Domain plan for m utterances over nwg workgroups (see KParams::n_dom).
struct Plan {
    int n_dom = 1, P = 0, nt = 1;
    std::vector<int> dom_n, dom_list, wg_dom, wg_rank, dom_wg;
};

Plan plan_domains(int m, int nwg, const std::vector<int32_t> &T) {
    Plan pl;
    int C, nt;
    // one 16-utterance column tile per domain up to 256 utterances (at 129..256 this beats
    // 32-utterance domains: each staging moves half the rows and runs once per phase);
    // beyond that, 16 workgroups per domain is the least that keeps the products short
    if (m <= kTile) { C = 1; nt = 1; }
    else if (m <= 16 * kTile) { nt = 1; C = 1; while (C * kTile < m) C *= 2; }
    else { nt = 2; C = 1; while (C * 2 * kTile < m) C *= 2; }
    while (C > 1 && nwg / C < 8) C /= 2;      // at least 8 workgroups per domain
    pl.n_dom = C;
    pl.nt = nt;
    pl.P = nwg / C;
    // utterances dealt longest-first round robin, so every domain sees a similar length mix
    std::vector<int> order(m);
    std::iota(order.begin(), order.end(), 0);
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return T[a] > T[b]; });
    pl.dom_n.assign(C, 0);
    pl.dom_list.assign((size_t)C * kDomCap, 0);
    for (int i = 0; i < m; ++i) {
        const int d = i % C;
        if (pl.dom_n[d] < kDomCap) pl.dom_list[(size_t)d * kDomCap + pl.dom_n[d]] = order[i];
        ++pl.dom_n[d];
    }
    // workgroup -> (domain, rank); with 8 XCDs dispatched round robin, rank r
    // of every domain sits on XCD r % 8, so the weight tiles of rank r share
    // one L2 across domains
    pl.wg_dom.assign(nwg, 0);
    pl.wg_rank.assign(nwg, 0);
    pl.dom_wg.assign((size_t)C * pl.P, 0);
    const bool xcd = nwg % (8 * C) == 0;
    for (int wg = 0; wg < C * pl.P; ++wg) {
        int d, r;
        if (xcd) {
            const int x = wg % 8, j = wg / 8;
            d = j % C;
            r = x + 8 * (j / C);
        } else {
            d = wg / pl.P;
            r = wg % pl.P;
        }
        pl.wg_dom[wg] = d;
        pl.wg_rank[wg] = r;
        pl.dom_wg[(size_t)d * pl.P + r] = wg;
    }
    return pl;
}

// One call's device buffers beyond inputs and outputs: grown handle buffers, or
// (fixed != nullptr) consecutive 256-byte aligned pieces of the fixed scratch array.
struct CallScratch {
    unsigned char *fixed = nullptr;
    size_t cap = 0, used = 0;
    int get(DevBuf &buf, size_t bytes, void **out) {
        if (!fixed) {
            if (int rc = buf.ensure(std::max<size_t>(bytes, 1))) return rc;
            *out = buf.p;
            return 0;
        }
        const size_t at = (used + 255) & ~(size_t)255;
        if (at + bytes > cap)
            return fail(PK_ERR_UNSUPPORTED, "batch needs more than the %zu B fixed scratch (pk_decode_noalloc limit)",
                        cap);
        *out = fixed + at;
        used = at + bytes;
        return 0;
    }
};

int decode_impl(pk_decoder *dec, const pk_batch *bt, bool keep_empty, CallScratch cs = CallScratch{});
int decode_chained(pk_decoder *dec, const pk_batch *bt, int W, const std::vector<int32_t> &launches);
// Longest piece of a window split over several launches (bounds the per-launch host staging).
constexpr int kChainFrames = 8192;
int open_loop_lock(int device);

}  // namespace

extern "C" {

PK_API const char *pk_last_error(void) { return g_err.c_str(); }

PK_API int pk_device_info(int32_t *n_cu, int32_t *lds_per_block, int32_t *wave_size) {
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev));
    hipDeviceProp_t prop;
    HIP_TRY(hipGetDeviceProperties(&prop, dev));
    if (n_cu) *n_cu = prop.multiProcessorCount;
    if (lds_per_block) *lds_per_block = (int32_t)prop.sharedMemPerBlock;
    if (wave_size) *wave_size = prop.warpSize;
    return 0;
}

PK_API int pk_decoder_create(const pk_decoder_desc *d, int32_t n_slots, pk_decoder **out) {
    g_err.clear();
    // registered after any static that holds this decoder has been constructed, so at exit
    // it runs before that static's destructor (which then makes no HIP call)
    static std::once_flag exit_hook;
    std::call_once(exit_hook, [] { std::atexit([] { g_exiting.store(true); }); });
    if (!d || !out || n_slots <= 0) return fail(PK_ERR_ARG, "pk_decoder_create: bad arguments");
    *out = nullptr;
    const int H = d->pred_hidden, L = d->pred_rnn_layers, J = d->joint_hidden, D = d->d_enc;
    const int V1 = d->vocab_size + 1;
    const int Dn = d->kind == PK_KIND_TDT ? d->num_durations : 0;
    const int Vo = V1 + Dn;
    if (d->kind != PK_KIND_TDT && d->kind != PK_KIND_EOU) return fail(PK_ERR_ARG, "unknown decoder kind %d", d->kind);
    if (H <= 0 || J <= 0 || D <= 0 || L <= 0 || L > PK_MAX_LAYERS || d->vocab_size <= 0)
        return fail(PK_ERR_ARG, "bad dims H=%d L=%d J=%d D=%d V=%d", H, L, J, D, d->vocab_size);
    if (H % 32 || J % 32 || D % 32)
        return fail(PK_ERR_UNSUPPORTED, "pred_hidden, joint_hidden and d_enc must be multiples of 32");
    if (d->kind == PK_KIND_TDT && (Dn <= 0 || Dn > PK_MAX_DURATIONS))
        return fail(PK_ERR_UNSUPPORTED, "TDT num_durations %d", Dn);
    if (d->kind == PK_KIND_TDT && d->n_duration_values > 0 && d->n_duration_values < Dn)
        return fail(PK_ERR_ARG, "durations table (%d) shorter than num_durations (%d)", d->n_duration_values, Dn);
    if (V1 > (1 << kIdxBits) - 1) return fail(PK_ERR_UNSUPPORTED, "vocab %d exceeds the argmax key index field", V1);
    if (d->blank_id < 0 || d->blank_id >= V1) return fail(PK_ERR_ARG, "blank_id %d outside [0,%d)", d->blank_id, V1);

    auto *dec = new pk_decoder();
    auto cleanup = [&](int rc) { delete dec; return rc; };
    dec->desc = *d;
    dec->desc.special = nullptr;
    dec->n_slots = n_slots;
    KParams &kp = dec->kp;
    kp.kind = d->kind; kp.H = H; kp.L = L; kp.J = J; kp.V1 = V1; kp.Dn = Dn; kp.Vo = Vo;
    kp.blank = d->blank_id;
    kp.eou = d->eou_id >= 0 ? d->eou_id : d->vocab_size - 2;
    kp.eob = d->eob_id >= 0 ? d->eob_id : d->vocab_size - 1;
    kp.n_dur = d->kind == PK_KIND_TDT ? d->n_duration_values : 0;
    for (int i = 0; i < PK_MAX_DURATIONS; ++i) kp.durations[i] = d->durations[i];

    if (hipGetDevice(&dec->device) != hipSuccess) return cleanup(fail(PK_ERR_DEVICE, "no HIP device"));
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dec->device) != hipSuccess) return cleanup(fail(PK_ERR_DEVICE, "device props"));
    dec->n_cu = prop.multiProcessorCount;
    dec->lds_block = (int)prop.sharedMemPerBlock;

    // unit-major gate rows: row 4j+g <- stored row g*H + j
    std::vector<int> gmap(4 * H);
    for (int j = 0; j < H; ++j)
        for (int g = 0; g < 4; ++g) gmap[4 * j + g] = g * H + j;

    int rc;
    Arena ar;
    std::vector<HostTiled> tiled(2 * L + 2);
    std::vector<std::vector<float>> vecs(L + 2);
    for (int l = 0; l < L; ++l) {
        if (l > 0) {
            if ((rc = tile_matrix(d->w_ih[l], 4 * H, H, &gmap, tiled[2 * l], "predict.lstm.w_ih"))) return cleanup(rc);
            arena_tiled(ar, tiled[2 * l], kp.w_ih[l]);
            std::vector<float> bh;
            if ((rc = vec_f32(d->b_ih[l], 4 * H, &gmap, vecs[l], "predict.lstm.b_ih"))) return cleanup(rc);
            if ((rc = vec_f32(d->b_hh[l], 4 * H, &gmap, bh, "predict.lstm.b_hh"))) return cleanup(rc);
            for (int i = 0; i < 4 * H; ++i) vecs[l][i] += bh[i];
            ar.add(vecs[l].data(), vecs[l].size() * 4, reinterpret_cast<const void **>(&kp.b_lstm[l]));
        }
        if ((rc = tile_matrix(d->w_hh[l], 4 * H, H, &gmap, tiled[2 * l + 1], "predict.lstm.w_hh"))) return cleanup(rc);
        arena_tiled(ar, tiled[2 * l + 1], kp.w_hh[l]);
    }
    if ((rc = tile_matrix(d->joint_pred_w, J, H, nullptr, tiled[2 * L], "joint.pred.weight"))) return cleanup(rc);
    arena_tiled(ar, tiled[2 * L], kp.w_pred);
    if ((rc = tile_matrix(d->joint_out_w, Vo, J, nullptr, tiled[2 * L + 1], "joint.out.weight"))) return cleanup(rc);
    arena_tiled(ar, tiled[2 * L + 1], kp.w_out);
    // a phase multiplies one staged vector by two matrices in one pass: W_ih[l+1] (or
    // W_p) with W_hh[l]; the pair must share a storage type
    for (int l = 0; l < L; ++l) {
        const HostTiled &consumer = l + 1 < L ? tiled[2 * (l + 1)] : tiled[2 * L];
        if (consumer.type != tiled[2 * l + 1].type)
            return cleanup(fail(PK_ERR_UNSUPPORTED, "layer %d: w_hh type %d differs from its consumer's type %d", l,
                                tiled[2 * l + 1].type, consumer.type));
    }
    std::vector<float> b_pred, b_out, b_enc, w_enc;
    if ((rc = vec_f32(d->joint_pred_b, J, nullptr, b_pred, "joint.pred.bias"))) return cleanup(rc);
    if ((rc = vec_f32(d->joint_out_b, Vo, nullptr, b_out, "joint.out.bias"))) return cleanup(rc);
    if ((rc = vec_f32(d->joint_enc_b, J, nullptr, b_enc, "joint.enc.bias"))) return cleanup(rc);
    if ((rc = dense_f32(d->joint_enc_w, J, D, nullptr, w_enc, "joint.enc.weight"))) return cleanup(rc);
    // joint.out bias padded with zeros to whole 16-row tiles (read a float4 per lane)
    b_out.resize((size_t)(Vo + kTile - 1) / kTile * kTile, 0.0f);
    ar.add(b_pred.data(), b_pred.size() * 4, reinterpret_cast<const void **>(&kp.b_pred));
    ar.add(b_out.data(), b_out.size() * 4, reinterpret_cast<const void **>(&kp.b_out));
    ar.add(b_enc.data(), b_enc.size() * 4, reinterpret_cast<const void **>(&dec->b_enc));
    std::vector<_Float16> w_enc_hi(w_enc.size()), w_enc_lo(w_enc.size());
    for (size_t i = 0; i < w_enc.size(); ++i) {
        w_enc_hi[i] = (_Float16)w_enc[i];
        w_enc_lo[i] = (_Float16)(w_enc[i] - (float)w_enc_hi[i]);
    }
    ar.add(w_enc_hi.data(), w_enc_hi.size() * 2, reinterpret_cast<const void **>(&dec->w_enc_hi));
    ar.add(w_enc_lo.data(), w_enc_lo.size() * 2, reinterpret_cast<const void **>(&dec->w_enc_lo));
    if ((rc = ar.upload(dec->arena))) return cleanup(rc);
    // f32 matrices: the lo plane follows the hi plane in the same upload
    {
        auto lo_plane = [](pkdev::TMat &m) {
            m.a_lo = m.type == PK_TYPE_F32 ? static_cast<const uint8_t *>(m.a) + (size_t)m.tiles * m.KB * kWave * 16
                                           : nullptr;
        };
        for (int l = 0; l < L; ++l) {
            lo_plane(kp.w_ih[l]);
            lo_plane(kp.w_hh[l]);
        }
        lo_plane(kp.w_pred);
        lo_plane(kp.w_out);
    }

    // layer-0 input projection of every token: E'[v] = W_ih0 . embed[v] + b_ih0 + b_hh0 (f32)
    {
        std::vector<float> w0, emb, bi, bh;
        if ((rc = dense_f32(d->w_ih[0], 4 * H, H, &gmap, w0, "predict.lstm.0.w_ih"))) return cleanup(rc);
        if ((rc = dense_f32(d->embed, V1, H, nullptr, emb, "predict.embed.weight"))) return cleanup(rc);
        if ((rc = vec_f32(d->b_ih[0], 4 * H, &gmap, bi, "predict.lstm.0.b_ih"))) return cleanup(rc);
        if ((rc = vec_f32(d->b_hh[0], 4 * H, &gmap, bh, "predict.lstm.0.b_hh"))) return cleanup(rc);
        DevBuf tmp;
        const size_t nw = w0.size(), ne = emb.size();
        if ((rc = tmp.ensure((nw + ne + 8 * (size_t)H) * 4))) return cleanup(rc);
        float *dw = tmp.as<float>(), *de = dw + nw, *dbi = de + ne, *dbh = dbi + 4 * H;
        if (hipMemcpy(dw, w0.data(), nw * 4, hipMemcpyHostToDevice) != hipSuccess ||
            hipMemcpy(de, emb.data(), ne * 4, hipMemcpyHostToDevice) != hipSuccess ||
            hipMemcpy(dbi, bi.data(), 16 * (size_t)H, hipMemcpyHostToDevice) != hipSuccess ||
            hipMemcpy(dbh, bh.data(), 16 * (size_t)H, hipMemcpyHostToDevice) != hipSuccess)
            return cleanup(fail(PK_ERR_DEVICE, "embedding projection upload"));
        if ((size_t)V1 * 4 * H * 4 >= (1ull << 31))   // the loop reads E' rows with 32-bit buffer offsets
            return cleanup(fail(PK_ERR_UNSUPPORTED, "vocabulary x 4 x pred_hidden too large (%d x %d)", V1, H));
        if ((rc = dec->eproj.ensure((size_t)V1 * 4 * H * 4))) return cleanup(rc);
        dim3 grid((V1 + 15) / 16, (4 * H + 63) / 64);
        pkdev::embed_proj_kernel<<<grid, 256>>>(dw, de, 4 * H, V1, H, dbi, dbh, dec->eproj.as<float>());
        if (hipGetLastError() != hipSuccess || hipDeviceSynchronize() != hipSuccess)
            return cleanup(fail(PK_ERR_DEVICE, "embedding projection kernel failed"));
        kp.eproj = dec->eproj.as<float>();
    }

    kp.special = nullptr;
    kp.n_special = 0;
    if (d->special && d->n_special > 0) {
        if ((rc = dec->special.ensure(d->n_special))) return cleanup(rc);
        if (hipMemcpy(dec->special.p, d->special, d->n_special, hipMemcpyHostToDevice) != hipSuccess)
            return cleanup(fail(PK_ERR_DEVICE, "special upload"));
        kp.special = dec->special.as<unsigned char>();
        kp.n_special = d->n_special;
    }

    // slots
    if ((rc = dec->slots_h.ensure((size_t)n_slots * L * H * 4))) return cleanup(rc);
    if ((rc = dec->slots_c.ensure((size_t)n_slots * L * H * 4))) return cleanup(rc);
    if ((rc = dec->slots_pp.ensure((size_t)n_slots * J * 4))) return cleanup(rc);
    if ((rc = dec->slots_r.ensure((size_t)n_slots * L * 4 * H * 4))) return cleanup(rc);
    if ((rc = dec->slots_ctrl.ensure((size_t)n_slots * PK_CTRL_N * 4))) return cleanup(rc);
    if (hipMemset(dec->slots_h.p, 0, dec->slots_h.n) != hipSuccess ||
        hipMemset(dec->slots_c.p, 0, dec->slots_c.n) != hipSuccess ||
        hipMemset(dec->slots_pp.p, 0, dec->slots_pp.n) != hipSuccess ||
        hipMemset(dec->slots_r.p, 0, dec->slots_r.n) != hipSuccess ||
        hipMemset(dec->slots_ctrl.p, 0, dec->slots_ctrl.n) != hipSuccess)
        return cleanup(fail(PK_ERR_DEVICE, "slot memset"));
    kp.slot_h = dec->slots_h.as<float>();
    kp.slot_c = dec->slots_c.as<float>();
    kp.slot_pp = dec->slots_pp.as<float>();
    kp.slot_r = dec->slots_r.as<float>();
    kp.slot_ctrl = dec->slots_ctrl.as<int>();

    // decode-loop launch shape: one workgroup per CU; LDS = one activation
    // block (16 utterance rows, hidden or h_l) + per-wave partials + the
    // optional weight cache
    const size_t act = (size_t)kTile * (std::max(J, H) + kKPad) * 2 * 2;   // shared by the joint and LSTM phases
    if (std::max(J, H) > 4096)
        return cleanup(fail(PK_ERR_UNSUPPORTED, "hidden sizes above 4096"));
    dec->lds_fixed = act;
    // dynamic LDS bound of any launch: the block's LDS less the kernel's static LDS
    // the loop instantiation for this decoder's weight storage (all q8_0; all f16 / f32; mixed)
    {
        bool all_q8 = true, all_half = true;
        auto see = [&](const pkdev::TMat &m) {
            all_q8 = all_q8 && m.type == PK_TYPE_Q8_0;
            all_half = all_half && m.type != PK_TYPE_Q8_0;
        };
        for (int l = 0; l < kp.L; ++l) see(kp.w_hh[l]);
        for (int l = 1; l < kp.L; ++l) see(kp.w_ih[l]);
        see(kp.w_pred);
        see(kp.w_out);
        using namespace pkdev;
        // PK_GEMV=1 (comparisons only): all-q8_0 decoders run the instantiation with the
        // wavefront-reduction GEMV form for column tiles of at most 4 live utterances
        const char *gv = std::getenv("PK_GEMV");
        if (all_q8 && gv && gv[0] == '1') {
            dec->loop_fn[0] = reinterpret_cast<const void *>(decode_loop_kernel<pkdev::kWcQ8Gemv, false>);
            dec->loop_fn[1] = reinterpret_cast<const void *>(decode_loop_kernel<pkdev::kWcQ8Gemv, true>);
        } else {
            dec->loop_fn[0] = all_q8 ? reinterpret_cast<const void *>(decode_loop_kernel<kWcQ8, false>)
                            : all_half ? reinterpret_cast<const void *>(decode_loop_kernel<kWcHalf, false>)
                                       : reinterpret_cast<const void *>(decode_loop_kernel<kWcAny, false>);
            dec->loop_fn[1] = all_q8 ? reinterpret_cast<const void *>(decode_loop_kernel<kWcQ8, true>)
                            : all_half ? reinterpret_cast<const void *>(decode_loop_kernel<kWcHalf, true>)
                                       : reinterpret_cast<const void *>(decode_loop_kernel<kWcAny, true>);
        }
    }
    size_t stat = 0;   // the larger static LDS of the two instantiations
    for (const void *fn : dec->loop_fn) {
        hipFuncAttributes fa{};
        if (hipFuncGetAttributes(&fa, fn) != hipSuccess) return cleanup(fail(PK_ERR_DEVICE, "hipFuncGetAttributes"));
        stat = std::max(stat, fa.sharedSizeBytes);
    }
    const size_t need = (size_t)dec->lds_block > stat ? (size_t)dec->lds_block - stat : 0;
    if (dec->lds_fixed + (size_t)2 * kWaves * kWave * 16 > need)
        return cleanup(fail(PK_ERR_UNSUPPORTED, "LDS %zu B needed, %d available", dec->lds_fixed + stat,
                            dec->lds_block));
    dec->lds_bytes = need;
    for (const void *fn : dec->loop_fn) {
        if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)need) != hipSuccess)
            return cleanup(fail(PK_ERR_DEVICE, "hipFuncSetAttribute"));
        int per_cu = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kBlock, need) != hipSuccess || per_cu < 1)
            return cleanup(fail(PK_ERR_DEVICE, "decode kernel does not fit on a CU"));
    }
    dec->nwg = std::min(dec->n_cu, kBlock);
    if ((rc = scratch_address(dec->device, &dec->scratch))) return cleanup(rc);
    dec->lock_fd = open_loop_lock(dec->device);
    {   // the largest descriptor block of a call (n_slots utterances; at most nwg domains of kDomCap)
        const size_t nwg = (size_t)dec->nwg;
        const size_t most = (size_t)n_slots * (2 * 8 + 5 * 4) + 4 * (nwg + nwg * kDomCap + 3 * nwg);
        dec->pin_cnt = (16 + most + 15) & ~(size_t)15;
        if ((rc = dec->h_pin.ensure(dec->pin_cnt + 12 * (size_t)n_slots))) return cleanup(rc);
    }
    if (hipStreamCreateWithFlags(&dec->stream, hipStreamNonBlocking) != hipSuccess)
        return cleanup(fail(PK_ERR_DEVICE, "stream"));
    for (auto &e : dec->ev)
        // timing only (pk_last_timing, after a stream synchronisation): no system-scope fences,
        // which cost each call several microseconds
        if (hipEventCreateWithFlags(&e, hipEventDisableSystemFence) != hipSuccess)
            return cleanup(fail(PK_ERR_DEVICE, "event"));
    *out = dec;
    return 0;
}

PK_API int pk_decoder_destroy(pk_decoder *dec) {
    if (!dec) return 0;
    if (g_exiting.load()) {
        // process exit (a static runtime's destructor, as the reference CLI keeps at
        // src/main.cpp:746, :761): no HIP call here, the driver reclaims the device memory
        // with the process.  Every call has completed (pk_decode returns after its stream).
        dec->forget_device();
        if (dec->lock_fd >= 0) close(dec->lock_fd);
        delete dec;
        return 0;
    }
    (void)hipSetDevice(dec->device);
    if (dec->stream) (void)hipStreamSynchronize(dec->stream);
    {   // its loops have completed: a later launch from another stream need not wait for them
        std::lock_guard<std::mutex> lk(g_loops.mu);
        auto it = g_loops.last_stream.find(dec->device);
        if (it != g_loops.last_stream.end() && it->second == dec->stream) it->second = nullptr;
    }
    for (auto &e : dec->ev) if (e) (void)hipEventDestroy(e);
    if (dec->stream) (void)hipStreamDestroy(dec->stream);
    if (dec->lock_fd >= 0) close(dec->lock_fd);
    delete dec;
    return 0;
}

PK_API int pk_slot_reset(pk_decoder *dec, int32_t slot) {
    g_err.clear();
    if (!dec || slot < 0 || slot >= dec->n_slots) return fail(PK_ERR_ARG, "pk_slot_reset: bad slot");
    HIP_TRY(hipSetDevice(dec->device));
    HIP_TRY(hipMemsetAsync(dec->kp.slot_ctrl + (size_t)slot * PK_CTRL_N, 0, PK_CTRL_N * 4, dec->stream));
    HIP_TRY(hipStreamSynchronize(dec->stream));
    return 0;
}

PK_API int pk_slot_init(pk_decoder *dec, int32_t slot) {
    if (int rc = pk_slot_reset(dec, slot)) return rc;
    // an empty window on a reset slot runs exactly the initial LSTM step
    const int32_t T = 0;
    const int64_t row = 0;
    int32_t tok = 0, ntok = 0, steps = 0, nseg = 0;
    pk_batch b{};
    b.n_utts = 1;
    b.mem = PK_MEM_HOST;
    b.d_enc = dec->desc.d_enc;
    b.max_symbols = 1;
    b.enc = nullptr;
    b.enc_row = &row;
    b.n_frames = &T;
    b.slot = &slot;
    b.tokens = &tok;
    b.token_cap = 1;
    b.n_tokens = &ntok;
    b.steps = &steps;
    b.n_segments = &nseg;
    return decode_impl(dec, &b, true);
}

PK_API int pk_slot_read(pk_decoder *dec, int32_t slot, float *h, float *c, float *pred, int32_t *ctrl) {
    g_err.clear();
    if (!dec || slot < 0 || slot >= dec->n_slots) return fail(PK_ERR_ARG, "pk_slot_read: bad slot");
    HIP_TRY(hipSetDevice(dec->device));
    const KParams &kp = dec->kp;
    const size_t hn = (size_t)kp.L * kp.H;
    if (ctrl) HIP_TRY(hipMemcpy(ctrl, kp.slot_ctrl + (size_t)slot * PK_CTRL_N, PK_CTRL_N * 4, hipMemcpyDeviceToHost));
    if (h) HIP_TRY(hipMemcpy(h, kp.slot_h + (size_t)slot * hn, hn * 4, hipMemcpyDeviceToHost));
    if (c) HIP_TRY(hipMemcpy(c, kp.slot_c + (size_t)slot * hn, hn * 4, hipMemcpyDeviceToHost));
    if (pred) HIP_TRY(hipMemcpy(pred, kp.slot_h + (size_t)slot * hn + (size_t)(kp.L - 1) * kp.H,
                                (size_t)kp.H * 4, hipMemcpyDeviceToHost));
    return 0;
}

PK_API int pk_slot_copy(pk_decoder *dec, int32_t src, int32_t dst) {
    g_err.clear();
    if (!dec || src < 0 || src >= dec->n_slots || dst < 0 || dst >= dec->n_slots)
        return fail(PK_ERR_ARG, "pk_slot_copy: bad slot");
    if (src == dst) return 0;
    HIP_TRY(hipSetDevice(dec->device));
    const KParams &kp = dec->kp;
    const size_t hn = (size_t)kp.L * kp.H, rn = (size_t)kp.L * 4 * kp.H;
    auto cp = [&](void *base, size_t per_slot) {
        char *b = static_cast<char *>(base);
        return hipMemcpyAsync(b + (size_t)dst * per_slot, b + (size_t)src * per_slot, per_slot,
                              hipMemcpyDeviceToDevice, dec->stream);
    };
    HIP_TRY(cp(kp.slot_h, hn * 4));
    HIP_TRY(cp(kp.slot_c, hn * 4));
    HIP_TRY(cp(kp.slot_pp, (size_t)kp.J * 4));
    HIP_TRY(cp(kp.slot_r, rn * 4));
    HIP_TRY(cp(kp.slot_ctrl, PK_CTRL_N * 4));
    HIP_TRY(hipStreamSynchronize(dec->stream));
    return 0;
}

PK_API int pk_decoder_set_timing(pk_decoder *dec, int32_t on) {
    if (!dec) return fail(PK_ERR_ARG, "pk_decoder_set_timing: null");
    dec->timing = on != 0;
    return 0;
}

PK_API int pk_last_timing(pk_decoder *dec, float *enc_proj_ms, float *loop_ms, int32_t *iterations) {
    if (!dec) return fail(PK_ERR_ARG, "pk_last_timing: null");
    if (!dec->timed) {
        if (enc_proj_ms) *enc_proj_ms = -1.f;
        if (loop_ms) *loop_ms = -1.f;
        if (iterations) *iterations = dec->chained ? dec->chain_iters : dec->last_iters;
        return 0;
    }
    if (dec->chained) {
        if (enc_proj_ms) *enc_proj_ms = dec->chain_ep_ms;
        if (loop_ms) *loop_ms = dec->chain_loop_ms;
        if (iterations) *iterations = dec->chain_iters;
        return 0;
    }
    float a = 0, b = 0;
    HIP_TRY(hipEventElapsedTime(&a, dec->ev[0], dec->ev[1]));
    HIP_TRY(hipEventElapsedTime(&b, dec->ev[1], dec->ev[2]));
    if (enc_proj_ms) *enc_proj_ms = a;
    if (loop_ms) *loop_ms = b;
    if (iterations) *iterations = dec->last_iters;
    return 0;
}

PK_API int pk_window_split(int32_t n_utts, const int32_t *n_frames, int32_t max_symbols, int32_t joint_hidden,
                           int32_t max_duration, int32_t *piece_frames, int32_t *launches) {
    if (n_utts < 0 || (n_utts > 0 && !n_frames) || joint_hidden <= 0 || !piece_frames)
        return fail(PK_ERR_ARG, "pk_window_split: bad arguments");
    const long long S = std::max(max_symbols, 1);
    // one launch: max_T * (S + 1) + 4 < 2^18 - 1 iterations, rows * J * 4 < 2^31 bytes of enc_proj rows
    const long long w_stamp = ((long long)kMaxStamp - 1 - 4) / (S + 1);
    const long long rows_limit = ((1ll << 31) - 1) / (4ll * joint_hidden);
    long long max_T = 0, rows = 0;
    for (int u = 0; u < n_utts; ++u) {
        if (n_frames[u] < 0) return fail(PK_ERR_ARG, "negative n_frames");
        max_T = std::max<long long>(max_T, n_frames[u]);
        rows += n_frames[u];
    }
    long long W = max_T;
    if (max_T > w_stamp || rows > rows_limit)
        W = std::min({w_stamp, rows_limit / std::max(n_utts, 1), (long long)kChainFrames});
    if (W < 1 && max_T > 0) return fail(PK_ERR_UNSUPPORTED, "no launch takes one frame of %d utterances", n_utts);
    const long long carry = std::max(max_duration, 1) - 1;   // largest TDT carry_frames a step can leave
    for (int u = 0; u < n_utts; ++u) {
        const long long T = n_frames[u], k = T > 0 ? (T + W - 1) / W : 0;
        if (k > 1 && T / k <= carry)
            return fail(PK_ERR_UNSUPPORTED, "window of %lld frames: pieces of %lld frames are not longer than the "
                        "largest duration carry (%lld)", T, T / k, carry);
        if (launches) launches[u] = (int32_t)k;
    }
    *piece_frames = (int32_t)W;
    return 0;
}

PK_API int pk_decode(pk_decoder *dec, const pk_batch *bt) {
    g_err.clear();
    if (!dec || !bt) return fail(PK_ERR_ARG, "pk_decode: null argument");
    if (bt->n_utts > 0 && bt->n_utts <= kMaxBatch && bt->n_frames) {
        // a window one launch cannot take is decoded in several launches (state carried)
        int32_t W = 0;
        std::vector<int32_t> k(bt->n_utts);
        int max_dur = 1;
        if (dec->kp.kind == PK_KIND_TDT)
            for (int i = 0; i < dec->kp.Dn; ++i)
                max_dur = std::max(max_dur, dec->kp.n_dur > 0 ? dec->kp.durations[i] : i);
        bool ok = true;
        for (int u = 0; u < bt->n_utts; ++u) ok = ok && bt->n_frames[u] >= 0;
        if (ok) {
            if (int rc = pk_window_split(bt->n_utts, bt->n_frames, bt->max_symbols, dec->kp.J, max_dur, &W, k.data()))
                return rc;
            if (*std::max_element(k.begin(), k.end()) > 1) return decode_chained(dec, bt, W, k);
        }
    }
    return decode_impl(dec, bt, false);
}

PK_API int pk_decode_noalloc(pk_decoder *dec, const pk_batch *bt) {
    g_err.clear();
    if (!dec || !bt) return fail(PK_ERR_ARG, "pk_decode_noalloc: null argument");
    if (bt->mem != PK_MEM_DEVICE)
        return fail(PK_ERR_ARG, "pk_decode_noalloc takes device frames and device outputs (PK_MEM_DEVICE)");
    if (!dec->scratch) return fail(PK_ERR_DEVICE, "fixed scratch not resolved for device %d", dec->device);
    CallScratch cs;
    cs.fixed = dec->scratch;
    cs.cap = kScratchBytes;
    return decode_impl(dec, bt, false, cs);
}

}  // extern "C"

namespace {

// The decode loop needs every CU of its GPU at once, so two processes must not
// run it on one GPU together: an exclusive flock on a per-GPU file
// (/tmp/parakeet_hip-<PCI bus id>.lock, opened once per decoder) is held from a
// call's loop launch to its last stream synchronisation.  Advisory and
// best-effort: without the file (no /tmp, no permission, something other than
// a regular file at the path) calls are not serialised across processes, and
// overlapping loops end with PK_ERR_TIMEOUT.  The wait for the lock is bounded
// (kLockWaitMs): a process that holds it longer makes the call return
// PK_ERR_TIMEOUT instead of blocking forever.
constexpr int kLockWaitMs = 30000;
struct DeviceLoopLock {
    int fd;
    bool held = false;
    explicit DeviceLoopLock(int f) : fd(f) {}
    int acquire() {
        if (fd < 0) return 0;
        for (int waited = 0;; ++waited) {
            if (flock(fd, LOCK_EX | LOCK_NB) == 0) {
                held = true;
                return 0;
            }
            if (errno != EWOULDBLOCK && errno != EINTR) return 0;   // no usable lock: not serialised
            if (waited >= kLockWaitMs) return fail(PK_ERR_TIMEOUT, "another process held this GPU's decode lock for %d ms", kLockWaitMs);
            usleep(1000);
        }
    }
    ~DeviceLoopLock() {
        if (held) (void)flock(fd, LOCK_UN);
    }
    DeviceLoopLock(const DeviceLoopLock &) = delete;
    DeviceLoopLock &operator=(const DeviceLoopLock &) = delete;
};

int open_loop_lock(int device) {
    char bus[64] = {0};
    if (hipDeviceGetPCIBusId(bus, sizeof bus, device) != hipSuccess) return -1;
    char path[128];
    snprintf(path, sizeof path, "/tmp/parakeet_hip-%s.lock", bus);
    // never follow a link planted at the path; make the file shared only when this process created it
    bool created = true;
    int fd = open(path, O_RDWR | O_CREAT | O_EXCL | O_NOFOLLOW | O_CLOEXEC, 0666);
    if (fd < 0 && errno == EEXIST) {
        created = false;
        fd = open(path, O_RDWR | O_NOFOLLOW | O_CLOEXEC);
        if (fd < 0) fd = open(path, O_RDONLY | O_NOFOLLOW | O_CLOEXEC);   // created by another user
    }
    if (fd < 0) return -1;
    struct stat st;
    if (fstat(fd, &st) != 0 || !S_ISREG(st.st_mode)) {
        close(fd);
        return -1;
    }
    if (created) (void)fchmod(fd, 0666);   // (the umask may have narrowed the mode)
    return fd;
}


// The loop's grid (at most one workgroup per CU, checked at create) must be
// resident at once.  A cooperative launch guarantees that; the runtime refuses
// it (hipErrorIllegalState) while another process holds the device's
// cooperative queue.  An ordinary dispatch checks it in the kernel
// (pkdev::coresident).  Loops of this process are kept apart by the ordering
// above, loops of other processes by the per-device lock (DeviceLoopLock); if
// one overlaps anyway, the barriers' 2 s limit ends the launch with
// PK_ERR_TIMEOUT.
//
// Arrival limit of an ordinary dispatch's co-residency check (a workgroup's start to the whole
// grid arrived): a grid that has not arrived by then is relaunched cooperatively, and the next
// kCoopAfterAbort launches on that device are cooperative.  (The first launch after the GPU has
// idled has been seen to take over 100 us to bring every workgroup up.)
constexpr unsigned kArriveLimitUs = 1000;
constexpr int kCoopAfterAbort = 256;

// The loop launch.  By default an ordinary dispatch whose workgroups first check that the
// whole grid is resident (pkdev::coresident): a cooperative launch costs about 14 us more per
// call, and under rocprofv3 (ROCm 7.2) any process that made one ends with SIGSEGV in the HIP
// runtime's exit-time teardown.  A grid found not resident ends at once with
// kStatusNotResident and the call is relaunched with coop = true (decode_impl); the device's
// next kCoopAfterAbort launches are cooperative.  Where the runtime refuses a cooperative launch
// (another process holds the device's cooperative queue), the loop runs as an ordinary
// dispatch without the check, and its barriers' 2 s limit is the last guard.
// PK_LOOP_DISPATCH=0 makes every launch cooperative, =1 every launch an ordinary dispatch (a
// relaunch then without the check), as under a profiler;
// PK_ARRIVE_US sets the arrival limit for tests of the relaunch: the first launch of a call is
// then an ordinary dispatch whatever the device's history, and nothing is remembered.
int launch_loop(pk_decoder *dec, int nwg, KParams &p, size_t lds, bool coop) {
    std::lock_guard<std::mutex> lk(g_loops.mu);
    hipStream_t &prev = g_loops.last_stream[dec->device];
    if (prev && prev != dec->stream) {
        hipEvent_t &last = g_loops.last[dec->device];
        if (!last) HIP_TRY(hipEventCreateWithFlags(&last, hipEventDisableTiming | hipEventDisableSystemFence));
        HIP_TRY(hipEventRecord(last, prev));
        HIP_TRY(hipStreamWaitEvent(dec->stream, last, 0));
    }
    prev = dec->stream;
    void *args[] = {&p};
    const void *fn = dec->loop_fn[p.slots ? 1 : 0];   // one domain: the argmax-slot instantiation
    bool &refused = g_loops.coop_refused[dec->device];
    // 0: cooperative, 1: ordinary dispatch, -1: the default above.  Under a profiler (its
    // ROCPROF* environment, or its tool library preloaded) always an ordinary dispatch.
    static const int mode = [] {
        const char *v = std::getenv("PK_LOOP_DISPATCH");
        if (v && v[0]) return v[0] == '1' ? 1 : 0;
        const char *pre = std::getenv("LD_PRELOAD");
        if (pre && strstr(pre, "rocprof")) return 1;
        for (char **e = environ; e && *e; ++e)
            if (strncmp(*e, "ROCPROF", 7) == 0) return 1;
        return -1;
    }();
    const char *lim = std::getenv("PK_ARRIVE_US");   // a test setting of the arrival limit
    int &left = g_loops.coop_left[dec->device];
    const bool after_abort = mode == -1 && !coop && !(lim && lim[0]) && left > 0;
    if (after_abort) --left;
    const bool cooperative = mode == 0 || (mode == -1 && (coop || after_abort));
    if (cooperative && !refused) {
        p.arrive_ticks = 0u;
        const hipError_t e = hipLaunchCooperativeKernel(fn, dim3(nwg), dim3(kBlock), args, lds, dec->stream);
        if (e != hipErrorIllegalState) {
            HIP_TRY(e);
            return 0;
        }
        (void)hipGetLastError();
        refused = true;
    }
    const unsigned limit_us = lim && lim[0] ? (unsigned)std::min(std::max(0, atoi(lim)), 1000000) : kArriveLimitUs;
    // 100 MHz clock; a relaunch that cannot be cooperative (refused, or ordinary dispatch
    // forced) runs without the check
    p.arrive_ticks = cooperative || coop ? 0u : std::max(1u, limit_us * 100u);
    HIP_TRY(hipLaunchKernel(fn, dim3(nwg), dim3(kBlock), args, lds, dec->stream));
    return 0;
}

// A launch found not co-resident (kStatusNotResident): clear its status words and, unless the
// arrival limit is a test setting, make the device's next kCoopAfterAbort launches cooperative.
int after_not_resident(pk_decoder *dec, int *d_status) {
    pkdev::fill_zero_kernel<<<1, 256, 0, dec->stream>>>(reinterpret_cast<unsigned *>(d_status), 16);
    HIP_TRY(hipGetLastError());
    if (!std::getenv("PK_ARRIVE_US")) {
        std::lock_guard<std::mutex> lk(g_loops.mu);
        g_loops.coop_left[dec->device] = kCoopAfterAbort;
    }
    static std::atomic<bool> noted{false};
    if (!noted.exchange(true) || std::getenv("PK_ARRIVE_US"))
        fprintf(stderr, "[parakeet_hip] decode loop grid not co-resident: relaunched cooperatively\n");
    return 0;
}

int decode_impl(pk_decoder *dec, const pk_batch *bt, bool keep_empty, CallScratch cs) {
    if (!dec || !bt) return fail(PK_ERR_ARG, "pk_decode: null argument");
    dec->chained = false;   // (decode_chained sets it again after its last launch)
    dec->timed = false;     // (set where the call records its first event)
    KParams &p = dec->kp;
    if (bt->d_enc != dec->desc.d_enc)
        return fail(PK_ERR_D_ENC, "encoder d_model mismatch (%d vs %d)", bt->d_enc, dec->desc.d_enc);
    const int n = bt->n_utts;
    if (n < 0 || n > kMaxBatch) return fail(PK_ERR_ARG, "n_utts %d outside [0,%d]", n, kMaxBatch);
    if (n == 0) return 0;
    if (!bt->enc_row || !bt->n_frames || !bt->slot || !bt->n_tokens || !bt->steps || !bt->tokens)
        return fail(PK_ERR_ARG, "pk_decode: missing batch array");
    if (bt->mem != PK_MEM_HOST && bt->mem != PK_MEM_DEVICE && bt->mem != PK_MEM_DEVICE_FRAMES)
        return fail(PK_ERR_ARG, "bad mem kind");
    HIP_TRY(hipSetDevice(dec->device));
    std::vector<char> seen(dec->n_slots, 0);
    for (int u = 0; u < n; ++u) {
        const int s = bt->slot[u];
        if (s < 0 || s >= dec->n_slots || seen[s]) return fail(PK_ERR_ARG, "slot %d invalid or repeated", s);
        seen[s] = 1;
        if (bt->n_frames[u] < 0) return fail(PK_ERR_ARG, "negative n_frames");
    }
    // TDT windows with no frames return before initialising (src/parakeet_tdt.cpp:879).
    std::vector<int> map;
    for (int u = 0; u < n; ++u)
        if (keep_empty || p.kind == PK_KIND_EOU || bt->n_frames[u] > 0) map.push_back(u);
    const int m = (int)map.size();
    const bool enc_host = bt->mem == PK_MEM_HOST, host = bt->mem != PK_MEM_DEVICE;   // host: outputs
    if (!host && m != n) return fail(PK_ERR_ARG, "device-memory batches must not contain empty TDT windows");
    if (host)
        for (int u = 0; u < n; ++u) {   // outputs of utterances that do not run
            bt->n_tokens[u] = 0;
            bt->steps[u] = 0;
            if (bt->n_segments) bt->n_segments[u] = 0;
        }
    if (host && bt->ctrl_out && m < n)   // utterances that do not run keep their slot's words (a reset one reads as fresh)
        for (int u = 0, i = 0; u < n; ++u) {
            if (i < m && map[i] == u) { ++i; continue; }
            int32_t *dst = bt->ctrl_out + (size_t)u * PK_CTRL_N;
            if (bt->reset && bt->reset[u]) memset(dst, 0, PK_CTRL_N * 4);
            else HIP_TRY(hipMemcpy(dst, p.slot_ctrl + (size_t)bt->slot[u] * PK_CTRL_N, PK_CTRL_N * 4,
                                   hipMemcpyDeviceToHost));
        }
    if (m == 0) return 0;
    long long rows = 0;
    int max_T = 0;
    std::vector<long long> src_row(m), dst_row(m);
    std::vector<int32_t> T(m), slots(m), base(m), reset(m);
    std::vector<float> bias(m);
    for (int i = 0; i < m; ++i) {
        const int u = map[i];
        T[i] = bt->n_frames[u];
        slots[i] = bt->slot[u];
        src_row[i] = bt->enc_row[u];
        dst_row[i] = rows;
        rows += T[i];
        max_T = std::max(max_T, T[i]);
        bias[i] = bt->blank_bias ? bt->blank_bias[u] : 0.0f;
        base[i] = bt->tokens_base ? bt->tokens_base[u] : 0;
        reset[i] = bt->reset ? (bt->reset[u] ? 1 : 0) : 0;
    }
    const long long max_iter = (long long)max_T * ((long long)std::max(bt->max_symbols, 1) + 1) + 4;
    // the loop addresses encp with 32-bit buffer offsets below 2^31 (pk_decode splits longer
    // windows into several launches before it gets here; see pk_window_split)
    if (rows * (long long)p.J * 4 >= (1ll << 31))
        return fail(PK_ERR_UNSUPPORTED, "%lld frames in one launch; at most %lld", rows, ((1ll << 31) - 1) / (p.J * 4ll));
    if (max_iter >= (long long)kMaxStamp)
        return fail(PK_ERR_UNSUPPORTED, "window too long for the iteration stamp of one launch");
    const int D = dec->desc.d_enc, J = p.J, L = p.L, H = p.H;
    int rc;
    // encoder frames: device pointer as given, or packed host rows uploaded
    const float *enc = bt->enc;
    if (enc_host && rows > 0) {
        if ((rc = dec->d_enc.ensure((size_t)rows * D * 4))) return rc;
        // up to kPinnedFrames bytes the rows are gathered into pinned memory and go up in one
        // asynchronous copy; beyond, one copy from the caller's (pageable) memory per run of
        // utterances whose source rows follow each other.  The device rows are packed in
        // utterance order.
        const size_t fbytes = (size_t)rows * D * 4;
        float *pin = nullptr;
        if (fbytes <= kPinnedFrames && dec->h_frames.ensure(fbytes) == 0) pin = dec->h_frames.as<float>();
        for (int i = 0; i < m;) {
            int j = i + 1;
            long long end = src_row[i] + T[i];
            while (j < m && (T[j] == 0 || src_row[j] == end)) {
                if (T[j] > 0) end = src_row[j] + T[j];
                ++j;
            }
            const long long n_rows = end - src_row[i];
            if (n_rows > 0 && pin)
                memcpy(pin + (size_t)dst_row[i] * D, bt->enc + (size_t)src_row[i] * D, (size_t)n_rows * D * 4);
            else if (n_rows > 0)
                HIP_TRY(hipMemcpyAsync(dec->d_enc.as<float>() + (size_t)dst_row[i] * D,
                                       bt->enc + (size_t)src_row[i] * D, (size_t)n_rows * D * 4,
                                       hipMemcpyHostToDevice, dec->stream));
            i = j;
        }
        if (pin) HIP_TRY(hipMemcpyAsync(dec->d_enc.p, pin, fbytes, hipMemcpyHostToDevice, dec->stream));
        enc = dec->d_enc.as<float>();
        src_row = dst_row;
    }
    if (rows > 0 && !enc) return fail(PK_ERR_ARG, "pk_decode: missing encoder frames");
    if (rows > 0 && reinterpret_cast<uintptr_t>(enc) % 16 != 0)
        return fail(PK_ERR_ARG, "encoder frames must be 16-byte aligned");
    const Plan pl = plan_domains(m, dec->nwg, T);
    const int nwg = pl.n_dom * pl.P;
    for (int d = 0; d < pl.n_dom; ++d)
        if (pl.dom_n[d] > kDomCap) return fail(PK_ERR_UNSUPPORTED, "batch of %d too large for %d compute units", m, dec->nwg);
    // descriptor block (device): int64 src_row, dst_row; int32 T, slot, base; f32 bias;
    // int32 reset, dom_n, dom_list, wg_dom, wg_rank, dom_wg
    const size_t n64 = 2 * (size_t)m, n32 = 5 * (size_t)m + pl.dom_n.size() + pl.dom_list.size() +
                                              pl.wg_dom.size() + pl.wg_rank.size() + pl.dom_wg.size();
    const size_t desc_bytes = n64 * 8 + n32 * 4;
    void *d_desc = nullptr;
    if ((rc = cs.get(dec->d_desc, desc_bytes, &d_desc))) return rc;
    uint8_t *hd;
    if (16 + desc_bytes <= dec->pin_cnt) {
        hd = dec->h_pin.as<uint8_t>() + 16;
    } else {
        dec->h_desc.resize(desc_bytes);
        hd = dec->h_desc.data();
    }
    size_t off = 0;
    auto put = [&](const void *src, size_t bytes) {
        memcpy(hd + off, src, bytes);
        const size_t at = off;
        off += bytes;
        return static_cast<uint8_t *>(d_desc) + at;
    };
    const long long *d_src = reinterpret_cast<const long long *>(put(src_row.data(), 8 * (size_t)m));
    const long long *d_dst = reinterpret_cast<const long long *>(put(dst_row.data(), 8 * (size_t)m));
    const int *d_T = reinterpret_cast<const int *>(put(T.data(), 4 * (size_t)m));
    const int *d_slot = reinterpret_cast<const int *>(put(slots.data(), 4 * (size_t)m));
    const int *d_base = reinterpret_cast<const int *>(put(base.data(), 4 * (size_t)m));
    const float *d_bias = reinterpret_cast<const float *>(put(bias.data(), 4 * (size_t)m));
    const int *d_reset = reinterpret_cast<const int *>(put(reset.data(), 4 * (size_t)m));
    const int *d_dom_n = reinterpret_cast<const int *>(put(pl.dom_n.data(), 4 * pl.dom_n.size()));
    const int *d_dom_list = reinterpret_cast<const int *>(put(pl.dom_list.data(), 4 * pl.dom_list.size()));
    const int *d_wg_dom = reinterpret_cast<const int *>(put(pl.wg_dom.data(), 4 * pl.wg_dom.size()));
    const int *d_wg_rank = reinterpret_cast<const int *>(put(pl.wg_rank.data(), 4 * pl.wg_rank.size()));
    const int *d_dom_wg = reinterpret_cast<const int *>(put(pl.dom_wg.data(), 4 * pl.dom_wg.size()));
    HIP_TRY(hipMemcpyAsync(d_desc, hd, desc_bytes, hipMemcpyHostToDevice, dec->stream));

    // argmax shards: about 8 ranks per shard
    p.shards = 1;
    while (p.shards < pkdev::kShards && p.shards * 8 < pl.P) p.shards *= 2;
    const size_t keys_bytes = (size_t)2 * pl.n_dom * pkdev::kColCap * p.shards * 2 * 8;
    // one-domain launches: per-workgroup argmax key slots (used while at most
    // kSlotCols joint columns are live); PK_ARGMAX_SLOTS=0 keeps the sharded
    // atomics and barrier instead (for comparisons)
    const char *slots_env = std::getenv("PK_ARGMAX_SLOTS");
    const bool use_slots = pl.n_dom == 1 && !(slots_env && slots_env[0] == '0');
    const size_t slots_bytes = use_slots ? (size_t)2 * pl.P * pkdev::kSlotCols * 2 * 8 : 0;
    // the words every launch starts from zero, in one allocation cleared by
    // one fill: 64 B of status, the barrier flags, the argmax keys and slots
    const size_t flags_bytes = (size_t)nwg * kFlagStride * 4,
                 clear_bytes = 256 + flags_bytes + keys_bytes + slots_bytes;
    void *d_clear = nullptr;
    if ((rc = cs.get(dec->d_clear, clear_bytes, &d_clear))) return rc;
    // (one fill kernel, never a memset, so that the call may run under graph capture)
    const size_t clear_words = clear_bytes / 4;   // clear_bytes is a multiple of 32

    dec->timed = dec->timing;
    if (dec->timed) HIP_TRY(hipEventRecord(dec->ev[0], dec->stream));
    float *d_encp = nullptr;
    if (rows > 0) {
        if ((rc = cs.get(dec->d_encp, (size_t)rows * J * 4, reinterpret_cast<void **>(&d_encp)))) return rc;
        // tiles over the packed rows of all utterances; the kernel also clears the loop's words.
        // Both kernels give bit-identical rows (PK_ENC_PROJ=tile / narrow forces one).
        const char *ep_env = std::getenv("PK_ENC_PROJ");
        const bool narrow = ep_env ? ep_env[0] == 'n' : rows <= kNarrowRows;
        if (narrow) {
            dim3 grid((unsigned)((rows + 15) / 16), 1, (J + 63) / 64);
            pkdev::enc_proj_narrow_kernel<<<grid, 256, 0, dec->stream>>>(dec->w_enc_hi, dec->w_enc_lo, J, dec->b_enc,
                                                                         enc, D, d_src, d_dst, m, rows, d_encp,
                                                                         static_cast<unsigned *>(d_clear),
                                                                         clear_words);
        } else {
            dim3 grid((unsigned)((rows + pkdev::kEpTile - 1) / pkdev::kEpTile), 1,
                      (J + pkdev::kEpTile - 1) / pkdev::kEpTile);
            pkdev::enc_proj_kernel<<<grid, 256, 0, dec->stream>>>(dec->w_enc_hi, dec->w_enc_lo, J, dec->b_enc, enc,
                                                                  D, d_src, d_dst, m, rows, d_encp,
                                                                  static_cast<unsigned *>(d_clear), clear_words);
        }
        HIP_TRY(hipGetLastError());
    } else {
        pkdev::fill_zero_kernel<<<(unsigned)std::min<size_t>((clear_words + 255) / 256, 1024), 256, 0, dec->stream>>>(
            static_cast<unsigned *>(d_clear), clear_words);
        HIP_TRY(hipGetLastError());
    }
    if (dec->timed) HIP_TRY(hipEventRecord(dec->ev[1], dec->stream));

    // outputs: device arrays as given, or a device staging area copied back
    const int tcap = bt->token_cap, scap = std::max(bt->seg_cap, 0), trcap = bt->trace ? bt->trace_cap : 0;
    const int lsteps = bt->logits ? std::max(bt->logit_steps, 0) : 0;
    const size_t lrow = (size_t)lsteps * p.Vo;   // tapped floats per utterance
    int *o_tok, *o_ntok, *o_steps, *o_seg = nullptr, *o_nseg = nullptr, *o_trace = nullptr, *o_ctrl = nullptr;
    float *o_logits = nullptr;
    if (host) {
        const size_t need = ((size_t)m * tcap + 3 * (size_t)m + (size_t)m * scap + (size_t)m * trcap * 2 +
                             (size_t)m * PK_CTRL_N + (size_t)m * lrow) * 4 + 64;
        if ((rc = dec->d_out.ensure(need))) return rc;
        int *o = dec->d_out.as<int>();
        o_tok = o; o += (size_t)m * tcap;
        o_ntok = o; o += m;
        o_steps = o; o += m;
        o_nseg = o; o += m;
        o_seg = scap > 0 ? o : nullptr; o += (size_t)m * scap;
        o_trace = trcap > 0 ? o : nullptr; o += (size_t)m * trcap * 2;
        o_ctrl = bt->ctrl_out ? o : nullptr; o += (size_t)m * PK_CTRL_N;
        o_logits = lrow > 0 ? reinterpret_cast<float *>(o) : nullptr;
    } else {
        o_tok = bt->tokens; o_ntok = bt->n_tokens; o_steps = bt->steps;
        o_seg = bt->segments; o_nseg = bt->n_segments; o_trace = bt->trace;
        o_ctrl = bt->ctrl_out;
        o_logits = lrow > 0 ? bt->logits : nullptr;
    }
    p.n_utts = m;
    p.encp = d_encp;
    p.encp_rows = rows;
    p.encp_row = d_dst;
    p.T = d_T;
    p.slot = d_slot;
    p.blank_bias = bt->blank_bias ? d_bias : nullptr;
    p.tokens_base = bt->tokens_base ? d_base : nullptr;
    p.tokens = o_tok; p.token_cap = tcap;
    p.n_tokens = o_ntok; p.steps = o_steps;
    p.segs = o_seg; p.seg_cap = scap; p.n_segs = o_nseg;
    p.trace = o_trace; p.trace_cap = trcap;
    p.logits = o_logits; p.logit_steps = lsteps;
    p.reset = bt->reset ? d_reset : nullptr;
    p.ctrl_out = o_ctrl;
    p.max_sym = bt->max_symbols;
    p.max_iter = (int)max_iter;
    p.n_dom = pl.n_dom;
    p.dom_size = pl.P;
    // blank runs over the joint tile's spare columns (PK_SPEC=0 turns them off for comparisons)
    {
        const char *v = std::getenv("PK_SPEC");
        p.spec = !(v && v[0] == '0') ? 1 : 0;
    }
    // logit tap staging: one row of Vo logits per joint column of each domain
    p.lcol = nullptr;
    if (lsteps > 0 &&
        (rc = cs.get(dec->d_lcol, (size_t)pl.n_dom * pkdev::kColCap * p.Vo * 4, reinterpret_cast<void **>(&p.lcol))))
        return rc;
    p.nt = pl.nt;
    p.dom_n = d_dom_n;
    p.dom_list = d_dom_list;
    p.wg_dom = d_wg_dom;
    p.wg_rank = d_wg_rank;
    p.dom_wg = d_dom_wg;
    void *d_xchg = nullptr;
    const size_t xh = 2 * (size_t)L * m * H, xp = (size_t)m * J, xr = 2 * (size_t)L * m * 4 * H;
    // the loop addresses the exchange buffers with 32-bit buffer offsets
    if ((2 * xh + xp + xr) * 4 >= (1ull << 31))
        return fail(PK_ERR_UNSUPPORTED, "exchange buffers of %d utterances exceed 2 GiB", m);
    if ((rc = cs.get(dec->d_xchg, (2 * xh + xp + xr) * 4, &d_xchg))) return rc;
    p.hx = static_cast<float *>(d_xchg);
    p.cx = p.hx + xh;
    p.ppx = p.cx + xh;
    p.rx = p.ppx + xp;
    p.xchg_bytes = (unsigned)((2 * xh + xp + xr) * 4);
    p.status = static_cast<int *>(d_clear) + 4;
    p.flags = reinterpret_cast<unsigned *>(static_cast<uint8_t *>(d_clear) + 256);
    p.keys = reinterpret_cast<unsigned long long *>(static_cast<uint8_t *>(d_clear) + 256 + flags_bytes);
    p.slots = slots_bytes ? reinterpret_cast<unsigned long long *>(static_cast<uint8_t *>(d_clear) + 256 +
                                                                 flags_bytes + keys_bytes)
                          : nullptr;
    // PK_PROFILE_PHASES=1: workgroup 0 accumulates per-phase wall-clock time (stderr summary)
    const bool prof = !cs.fixed && getenv("PK_PROFILE_PHASES") != nullptr;
    p.prof = nullptr;
    if (prof) {
        if ((rc = dec->d_prof.ensure((pkdev::kPrN + 9 * pkdev::kTl) * 8))) return rc;
        HIP_TRY(hipMemsetAsync(dec->d_prof.p, 0, (pkdev::kPrN + 9 * pkdev::kTl) * 8, dec->stream));
        p.prof = dec->d_prof.as<unsigned long long>();
    }
    // LDS state of layers >= 1 (R and c of each workgroup's unit tiles)
    p.st_n = *std::max_element(pl.dom_n.begin(), pl.dom_n.end());
    p.st_k = p.L > 1 ? (p.w_hh[1].tiles + pl.P - 1) / pl.P : 0;
    const size_t st_bytes = (size_t)(p.L - 1) * p.st_n * p.st_k * pkdev::kStFloats * 4;
    // LDS bias table: 16 rows per owned tile of W_ih_l (l >= 1), W_p and W_o
    {
        auto own = [&](const pkdev::TMat &m) { return (m.tiles + pl.P - 1) / pl.P; };
        int rows = own(p.w_pred) + own(p.w_out);
        for (int l = 1; l < p.L; ++l) rows += own(p.w_ih[l]);
        p.bias_floats = rows * kTile;
    }
    const size_t lds_base = dec->lds_fixed + st_bytes + (size_t)p.bias_floats * 4;
    // LDS partial slots: one per (item, K chunk) of a pass.  Every item of the
    // largest phase in one pass when that fits; otherwise every slot the LDS
    // holds, and the phase runs in several passes (at least one item each).
    {
        auto items = [&](const pkdev::TMat &m) { return (m.tiles + pl.P - 1) / pl.P; };
        auto units = [&](const pkdev::TMat &m) {
            const int kbe = m.type == PK_TYPE_F32 ? 2 * m.KB : m.KB;
            return (kbe + pkdev::unit_blocks(m.type) - 1) / pkdev::unit_blocks(m.type);
        };
        int kslots = items(p.w_out) * units(p.w_out), min_slots = units(p.w_out);
        for (int l = 0; l < p.L; ++l) {
            const pkdev::TMat &c = l + 1 < p.L ? p.w_ih[l + 1] : p.w_pred;
            kslots = std::max(kslots, (items(c) + items(p.w_hh[l])) * units(c));
            min_slots = std::max(min_slots, units(c));
        }
        const size_t fit = dec->lds_bytes > lds_base ? (dec->lds_bytes - lds_base) / (kWave * 16) : 0;
        if ((int)fit < min_slots)
            return fail(PK_ERR_UNSUPPORTED, "LDS %zu B needed for %d workgroups per domain, %zu available",
                        lds_base + (size_t)min_slots * kWave * 16, pl.P, dec->lds_bytes);
        p.red_slots = std::min<int>(kslots, (int)fit);
    }
    size_t lds = lds_base + (size_t)p.red_slots * kWave * 16;
    // LDS weight cache, phase by phase: the matrices of a phase (the two that
    // consume one layer's output, or W_o) are copied into LDS once per launch
    // when the workgroup's tiles of both fit; the LSTM phases are tried first
    // (smaller), then the joint.  A phase whose tiles do not fit reads them from L2.
    // Windows of fewer than kCacheMinFrames frames (streaming chunks: a few lockstep
    // iterations per launch) read every phase from L2: the fill would cost more than the
    // iterations it serves.
    const bool cache_ok = max_T >= kCacheMinFrames;
    {
        std::vector<std::vector<pkdev::TMat *>> phases;
        for (int lc = 0; lc < p.L; ++lc) phases.push_back({lc + 1 < p.L ? &p.w_ih[lc + 1] : &p.w_pred, &p.w_hh[lc]});
        phases.push_back({&p.w_out});
        auto bytes = [&](const pkdev::TMat *m) {
            return (size_t)((m->tiles + pl.P - 1) / pl.P) * pkdev::tile_bytes(m->type, m->KB);
        };
        size_t off = 0;
        for (auto &ph : phases) {
            size_t need = 0;
            for (auto *m : ph) need += bytes(m);
            const bool fits = cache_ok && lds + off + need <= dec->lds_bytes;
            for (auto *m : ph) {
                m->lds_off = fits ? (int)off : -1;
                if (fits) off += bytes(m);
            }
        }
        p.wcache_bytes = (int)off;
        lds += off;
    }
    // held until this call's last stream synchronisation (scope end): another
    // process's decode loop on this GPU waits here instead of sharing the CUs
    DeviceLoopLock cross_process(dec->lock_fd);
    if ((rc = cross_process.acquire())) return rc;
    bool coop_retry = false;   // set when an ordinary dispatch found its grid not co-resident
relaunch:
    if ((rc = launch_loop(dec, nwg, p, lds, coop_retry))) return rc;
    if (dec->timed) HIP_TRY(hipEventRecord(dec->ev[2], dec->stream));
    int *status = dec->h_pin.as<int>();   // read after the stream synchronisation below
    HIP_TRY(hipMemcpyAsync(status, p.status, 4 * sizeof(int), hipMemcpyDeviceToHost, dec->stream));
    if (host) {
        // The device staging is one block: tokens | n_tokens, steps, n_segments | segments |
        // trace | control words.  Up to kEagerCopyBytes of rows it comes back whole in one
        // copy, so the call waits for the stream once.  Larger outputs copy the counters and
        // control words first, then only each row's filled prefix.
        const size_t tb = (size_t)m * tcap * 4, sb_all = (size_t)m * scap * 4,
                     rb = o_trace ? (size_t)m * trcap * 8 : 0, cb = o_ctrl ? (size_t)m * PK_CTRL_N * 4 : 0;
        const bool eager = tb + sb_all + rb <= kEagerCopyBytes;
        std::vector<int> cnt_v;
        int *cnt, *e_tok, *e_seg, *e_tr;
        int32_t *s_ctrl;
        if (eager) {
            const size_t whole = tb + 12 * (size_t)m + sb_all + rb + cb;
            if ((rc = dec->h_out.ensure(std::max<size_t>(whole, 64)))) return rc;
            HIP_TRY(hipMemcpyAsync(dec->h_out.p, o_tok, whole, hipMemcpyDeviceToHost, dec->stream));
            e_tok = dec->h_out.as<int>();
            cnt = e_tok + tb / 4;
            e_seg = cnt + 3 * (size_t)m;
            e_tr = e_seg + sb_all / 4;
            s_ctrl = e_tr + rb / 4;
        } else {
            if (dec->pin_cnt + 12 * (size_t)m <= dec->h_pin.n) {   // (m <= n_slots: slots are distinct)
                cnt = reinterpret_cast<int *>(dec->h_pin.as<uint8_t>() + dec->pin_cnt);
            } else {
                cnt_v.resize(3 * (size_t)m);
                cnt = cnt_v.data();
            }
            HIP_TRY(hipMemcpyAsync(cnt, o_ntok, 12 * (size_t)m, hipMemcpyDeviceToHost, dec->stream));
            if ((rc = dec->h_out.ensure(std::max<size_t>(cb, 64)))) return rc;
            s_ctrl = dec->h_out.as<int32_t>();
            if (cb) HIP_TRY(hipMemcpyAsync(s_ctrl, o_ctrl, cb, hipMemcpyDeviceToHost, dec->stream));
            e_tok = e_seg = e_tr = nullptr;
        }
        HIP_TRY(hipStreamSynchronize(dec->stream));
        if (status[0] == pkdev::kStatusNotResident && !coop_retry) {   // nothing was decoded: again
            if ((rc = after_not_resident(dec, p.status))) return rc;
            coop_retry = true;
            goto relaunch;
        }
        const int *c_tok = cnt, *c_steps = c_tok + m, *c_seg = c_steps + m;
        // rows of width wt / ws / wr (prefix copies) or of the full capacities (eager)
        int wt = tcap, ws = bt->segments ? scap : 0, wr = o_trace ? trcap : 0;
        const int *s_tok = e_tok, *s_seg = e_seg, *s_tr = e_tr;
        std::vector<int> prefix;
        if (!eager) {
            wt = ws = wr = 0;
            for (int i = 0; i < m; ++i) {
                wt = std::max(wt, std::min(c_tok[i], tcap));
                ws = std::max(ws, std::min(c_seg[i], scap));
                wr = std::max(wr, std::min(c_steps[i], trcap));
            }
            if (!bt->segments) ws = 0;
            if (!o_trace) wr = 0;
            const size_t stage = (size_t)m * (wt + ws + 2 * (size_t)wr) * 4;
            if (stage > 0) {
                prefix.resize(stage / 4);
                int *p_tok = prefix.data(), *p_seg = p_tok + (size_t)m * wt, *p_tr = p_seg + (size_t)m * ws;
                if (wt)
                    HIP_TRY(hipMemcpy2DAsync(p_tok, 4 * (size_t)wt, o_tok, 4 * (size_t)tcap, 4 * (size_t)wt, m,
                                             hipMemcpyDeviceToHost, dec->stream));
                if (ws)
                    HIP_TRY(hipMemcpy2DAsync(p_seg, 4 * (size_t)ws, o_seg, 4 * (size_t)scap, 4 * (size_t)ws, m,
                                             hipMemcpyDeviceToHost, dec->stream));
                if (wr)
                    HIP_TRY(hipMemcpy2DAsync(p_tr, 8 * (size_t)wr, o_trace, 8 * (size_t)trcap, 8 * (size_t)wr, m,
                                             hipMemcpyDeviceToHost, dec->stream));
                HIP_TRY(hipStreamSynchronize(dec->stream));
                s_tok = p_tok;
                s_seg = p_seg;
                s_tr = p_tr;
            }
        }
        if (o_ctrl)
            for (int i = 0; i < m; ++i)
                memcpy(bt->ctrl_out + (size_t)map[i] * PK_CTRL_N, s_ctrl + (size_t)i * PK_CTRL_N, PK_CTRL_N * 4);
        if (o_logits)   // debug tap: straight into the caller's rows (utterance order may differ)
            for (int i = 0; i < m; ++i)
                HIP_TRY(hipMemcpy(bt->logits + (size_t)map[i] * lrow, o_logits + (size_t)i * lrow, lrow * 4,
                                  hipMemcpyDeviceToHost));
        for (int i = 0; i < m; ++i) {
            const int u = map[i];
            bt->n_tokens[u] = c_tok[i];
            bt->steps[u] = c_steps[i];
            const int nt = std::min(c_tok[i], tcap);
            if (nt > 0) memcpy(bt->tokens + (size_t)u * tcap, s_tok + (size_t)i * wt, 4 * (size_t)nt);
            if (bt->n_segments) bt->n_segments[u] = c_seg[i];
            if (ws) {
                const int ns = std::min(c_seg[i], scap);
                if (ns > 0) memcpy(bt->segments + (size_t)u * scap, s_seg + (size_t)i * ws, 4 * (size_t)ns);
            }
            if (wr) {
                const int ns = std::min(c_steps[i], trcap);
                if (ns > 0) memcpy(bt->trace + (size_t)u * trcap * 2, s_tr + (size_t)i * wr * 2, 8 * (size_t)ns);
            }
        }
    } else {
        HIP_TRY(hipStreamSynchronize(dec->stream));
        if (status[0] == pkdev::kStatusNotResident && !coop_retry) {   // nothing was decoded: again
            if ((rc = after_not_resident(dec, p.status))) return rc;
            coop_retry = true;
            goto relaunch;
        }
    }
    if (status[0] == pkdev::kStatusNotResident) return fail(PK_ERR_DEVICE, "decode loop grid not co-resident");
    dec->last_iters = status[1];
    if (prof) {
        unsigned long long t[pkdev::kPrN];
        HIP_TRY(hipMemcpy(t, dec->d_prof.p, sizeof t, hipMemcpyDeviceToHost));
        static const char *names[pkdev::kPrN] = {"L0", "sync0", "L1", "sync1", "pred", "sync2",
                                                 "J-stage", "J-compute", "J-sync", "decide", "stageLSTM"};
        double total = 0;
        for (double v : t) total += v;
        fprintf(stderr, "[pk phases] %d iterations, %d domains x %d wg, total %.3f ms:", status[1], pl.n_dom, pl.P,
                total * 1e-5);
        for (int i = 0; i < pkdev::kPrN; ++i)
            fprintf(stderr, " %s=%.2fus", names[i], status[1] ? t[i] * 1e-2 / status[1] : 0.0);
        fprintf(stderr, "\n");
        unsigned long long tl[9 * pkdev::kTl];
        HIP_TRY(hipMemcpy(tl, dec->d_prof.as<unsigned long long>() + pkdev::kPrN, sizeof tl, hipMemcpyDeviceToHost));
        for (int k = 0; k < pkdev::kTl; ++k) {
            const unsigned long long cnt = tl[8 * pkdev::kTl + k];
            if (!cnt) continue;
            fprintf(stderr, "[pk tl] %2d n=%4llu", k, cnt);
            for (int w = 0; w < 8; ++w) fprintf(stderr, " %6.2f", tl[w * pkdev::kTl + k] * 1e-2 / cnt);
            fprintf(stderr, "\n");
        }
    }
    if (status[0]) return fail(status[0], "device decode failed (status %d)", status[0]);
    if (status[2]) return fail(PK_ERR_OVERFLOW, "token or segment capacity exceeded");
    return 0;
}

}  // namespace

namespace {

// A batch whose windows one launch cannot take (pk_window_split): utterance u
// decodes its window as launches[u] consecutive pieces of nearly equal length,
// one launch per piece index, its slot carrying the state from piece to piece
// exactly as between two calls (TDT symbols and carry_frames, EOU last token and
// segment start).  Every piece is longer than the largest duration carry, so
// the result equals one launch over the whole window.  Each launch's outputs
// come back to host memory and are appended to the caller's arrays (uploaded at
// the end for device outputs); EOU pieces count segment boundaries from the
// tokens of the earlier pieces (tokens_base).
int decode_chained(pk_decoder *dec, const pk_batch *bt, int W, const std::vector<int32_t> &launches) {
    const int n = bt->n_utts;
    if (bt->logits && bt->logit_steps > 0)
        return fail(PK_ERR_UNSUPPORTED, "the logit tap takes windows of at most %d frames (one launch)", W);
    if (!bt->enc_row || !bt->slot || !bt->n_tokens || !bt->steps || !bt->tokens)
        return fail(PK_ERR_ARG, "pk_decode: missing batch array");
    const bool dev_out = bt->mem == PK_MEM_DEVICE;
    const int S = std::max(bt->max_symbols, 1);
    const int tcap = std::max(bt->token_cap, 0), scap = bt->segments ? std::max(bt->seg_cap, 0) : 0;
    const int rcap = bt->trace ? std::max(bt->trace_cap, 0) : 0;
    // caller's outputs, assembled on the host
    std::vector<int32_t> h_tok, h_seg, h_tr, h_ctrl;
    int32_t *o_tok = bt->tokens, *o_seg = bt->segments, *o_tr = bt->trace, *o_ctrl = bt->ctrl_out;
    if (dev_out) {
        h_tok.assign((size_t)n * tcap, 0);
        o_tok = h_tok.data();
        if (scap) { h_seg.assign((size_t)n * scap, 0); o_seg = h_seg.data(); }
        if (rcap) { h_tr.assign((size_t)n * rcap * 2, 0); o_tr = h_tr.data(); }
        if (bt->ctrl_out) { h_ctrl.assign((size_t)n * PK_CTRL_N, 0); o_ctrl = h_ctrl.data(); }
    }
    std::vector<long long> done(n, 0);                 // frames decoded so far
    std::vector<int32_t> ntok(n, 0), nseg(n, 0), nst(n, 0);
    float ep_ms = 0.f, loop_ms = 0.f;
    int iters = 0;
    const int n_launch = *std::max_element(launches.begin(), launches.end());
    for (int j = 0; j < n_launch; ++j) {
        // the utterances with a piece j (launch 0: all, so windows with no frames are handled as usual)
        std::vector<int> idx;
        for (int u = 0; u < n; ++u)
            if (j == 0 || launches[u] > j) idx.push_back(u);
        const int m = (int)idx.size();
        std::vector<int64_t> row(m);
        std::vector<int32_t> T(m), sl(m), base(m);
        std::vector<float> bias(m);
        std::vector<uint8_t> rst(m, 0);
        int cap = 1, sc = scap ? 1 : 0, rc_cap = rcap ? 1 : 0;
        for (int i = 0; i < m; ++i) {
            const int u = idx[i];
            const long long Tu = bt->n_frames[u], k = launches[u];
            const long long piece = k > 0 ? Tu / k + (j < Tu % k ? 1 : 0) : 0;
            row[i] = bt->enc_row[u] + done[u];
            T[i] = (int32_t)piece;
            sl[i] = bt->slot[u];
            base[i] = (bt->tokens_base ? bt->tokens_base[u] : 0) + ntok[u];
            bias[i] = bt->blank_bias ? bt->blank_bias[u] : 0.0f;
            if (j == 0 && bt->reset) rst[i] = bt->reset[u];
            // staging just large enough for what this piece can add below the caller's capacity
            cap = std::max<long long>(cap, std::min<long long>(std::max(tcap - ntok[u], 0), piece * S + 1));
            if (scap) sc = std::max<long long>(sc, std::min<long long>(std::max(scap - nseg[u], 0), piece + 1));
            if (rcap) rc_cap = std::max<long long>(rc_cap, std::min<long long>(std::max(rcap - nst[u], 0),
                                                                               piece * (S + 1) + 1));
        }
        std::vector<int32_t> tok((size_t)m * cap), cnt(m), st(m), seg((size_t)m * std::max(sc, 1)), cs(m),
            tr((size_t)m * std::max(rc_cap, 1) * 2), ctrl((size_t)m * PK_CTRL_N);
        pk_batch b{};
        b.n_utts = m;
        b.mem = dev_out ? PK_MEM_DEVICE_FRAMES : bt->mem;
        b.d_enc = bt->d_enc;
        b.max_symbols = bt->max_symbols;
        b.enc = bt->enc;
        b.enc_row = row.data();
        b.n_frames = T.data();
        b.slot = sl.data();
        b.blank_bias = bt->blank_bias ? bias.data() : nullptr;
        b.tokens_base = base.data();
        b.tokens = tok.data();
        b.token_cap = cap;
        b.n_tokens = cnt.data();
        b.steps = st.data();
        b.segments = scap ? seg.data() : nullptr;
        b.seg_cap = sc;
        b.n_segments = cs.data();
        b.trace = rcap ? tr.data() : nullptr;
        b.trace_cap = rc_cap;
        b.reset = bt->reset ? rst.data() : nullptr;
        b.ctrl_out = ctrl.data();
        const int rc = decode_impl(dec, &b, false);
        if (rc != 0 && rc != PK_ERR_OVERFLOW) return rc;   // capacity is judged on the totals below
        float a = 0.f, c = 0.f;
        if (dec->timed && hipEventElapsedTime(&a, dec->ev[0], dec->ev[1]) == hipSuccess) ep_ms += a;
        if (dec->timed && hipEventElapsedTime(&c, dec->ev[1], dec->ev[2]) == hipSuccess) loop_ms += c;
        iters += dec->last_iters;
        for (int i = 0; i < m; ++i) {
            const int u = idx[i];
            const int nt = std::min(cnt[i], cap), keep_t = std::max(0, std::min(nt, tcap - ntok[u]));
            if (keep_t > 0)
                memcpy(o_tok + (size_t)u * tcap + ntok[u], tok.data() + (size_t)i * cap, 4 * (size_t)keep_t);
            if (scap) {
                const int ns = std::min(cs[i], sc), keep_s = std::max(0, std::min(ns, scap - nseg[u]));
                if (keep_s > 0)
                    memcpy(o_seg + (size_t)u * scap + nseg[u], seg.data() + (size_t)i * sc, 4 * (size_t)keep_s);
            }
            if (rcap) {
                const int nr = std::min(st[i], rc_cap), keep_r = std::max(0, std::min(nr, rcap - nst[u]));
                if (keep_r > 0)
                    memcpy(o_tr + ((size_t)u * rcap + nst[u]) * 2, tr.data() + (size_t)i * rc_cap * 2,
                           8 * (size_t)keep_r);
            }
            if (o_ctrl) memcpy(o_ctrl + (size_t)u * PK_CTRL_N, ctrl.data() + (size_t)i * PK_CTRL_N, 4 * PK_CTRL_N);
            ntok[u] += cnt[i];
            nseg[u] += cs[i];
            nst[u] += st[i];
            done[u] += T[i];
        }
    }
    bool over = false;
    for (int u = 0; u < n; ++u) over = over || ntok[u] > tcap || (bt->segments && nseg[u] > scap);
    if (dev_out) {
        HIP_TRY(hipMemcpy(bt->tokens, h_tok.data(), h_tok.size() * 4, hipMemcpyHostToDevice));
        HIP_TRY(hipMemcpy(bt->n_tokens, ntok.data(), 4 * (size_t)n, hipMemcpyHostToDevice));
        HIP_TRY(hipMemcpy(bt->steps, nst.data(), 4 * (size_t)n, hipMemcpyHostToDevice));
        if (bt->n_segments) HIP_TRY(hipMemcpy(bt->n_segments, nseg.data(), 4 * (size_t)n, hipMemcpyHostToDevice));
        if (scap) HIP_TRY(hipMemcpy(bt->segments, h_seg.data(), h_seg.size() * 4, hipMemcpyHostToDevice));
        if (rcap) HIP_TRY(hipMemcpy(bt->trace, h_tr.data(), h_tr.size() * 4, hipMemcpyHostToDevice));
        if (bt->ctrl_out) HIP_TRY(hipMemcpy(bt->ctrl_out, h_ctrl.data(), h_ctrl.size() * 4, hipMemcpyHostToDevice));
    } else {
        memcpy(bt->n_tokens, ntok.data(), 4 * (size_t)n);
        memcpy(bt->steps, nst.data(), 4 * (size_t)n);
        if (bt->n_segments) memcpy(bt->n_segments, nseg.data(), 4 * (size_t)n);
    }
    dec->chained = true;
    dec->chain_ep_ms = ep_ms;
    dec->chain_loop_ms = loop_ms;
    dec->chain_iters = iters;
    if (over) return fail(PK_ERR_OVERFLOW, "token or segment capacity exceeded");
    return 0;
}

}  // namespace
