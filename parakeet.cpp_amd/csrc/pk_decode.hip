// pk_decode.hip -- MI355X (gfx950) transducer greedy decode: kernels + C ABI.
//
// Replaces the decode loop of parakeet.cpp (tdt_decode_window,
// src/parakeet_tdt.cpp:865-981; eou_decode_window, src/parakeet_eou.cpp:232-336)
// with one persistent, batch-over-utterances kernel:
//
//   enc_proj_kernel     b_e + W_e . enc[t] for every frame of every utterance,
//                       once per window (src/parakeet_tdt.cpp:433-483 computes
//                       the same projection as a ggml graph; the CPU path
//                       recomputes it per step at :167-168).
//   decode_loop_kernel  all lockstep iterations of all utterances in one
//                       cooperative launch.  One iteration is
//                         LSTM layer 0..L-1   (utterances that emitted a token)
//                         pred projection     pp = b_p + W_p . h[L-1]
//                         joint + argmax      logits = b_o + W_o . relu(encp[t] + pp)
//                         decisions           token / duration / frame advance,
//                                             symbol cap, EOU reset, compaction
//                       separated by grid barriers.  The token and duration
//                       argmaxes are reduced with 64-bit atomic max on a key
//                       (iteration stamp | order-preserving value | inverted
//                       index), which reproduces the reference's first-index
//                       tie rule (src/parakeet_tdt.cpp:25-32) independently of
//                       reduction order.  Every workgroup applies the same
//                       decisions to its own copy of the control state, so no
//                       state is broadcast and no host round trip happens
//                       inside the loop.
//
// Weights stay at their stored precision: q8_0 is re-laid out as an int8
// plane [rows][cols] plus an f32 plane of block scales [rows][cols/32]
// (d converted exactly from f16); value = d * q as ggml's to_float.  LSTM
// gate rows are reordered unit-major (row 4j+g = gate g of unit j) so a wave
// owning unit j holds its four gates for the cell update.
//
// Arithmetic is f32 FMA throughout; summation order differs from the
// reference's sequential row sums, so logits differ by f32 rounding only.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "parakeet_hip.h"
#include "pk_device.h"

namespace {

using pkdev::DMat;
using pkdev::KParams;
using pkdev::kBlock;
using pkdev::kMaxBatch;
using pkdev::kIdxBits;
using pkdev::kMaxStamp;
using pkdev::kUC;
using pkdev::kSmallB;
using pkdev::kFlagStride;

// ---------------------------------------------------------------- host side

thread_local std::string g_err;

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

// Host copy of a repacked matrix, uploaded into one arena.
struct HostMat {
    int type, rows, cols;
    std::vector<uint8_t> w;       // plane bytes
    std::vector<float> d;         // q8 scales
};

int bytes_per_elem(int type) { return type == PK_TYPE_F32 ? 4 : type == PK_TYPE_F16 ? 2 : 1; }

// Repack a stored GGUF matrix [rows][cols]; row_map[r] = stored row placed at r (nullable).
int repack(const pk_tensor &t, int rows, int cols, const std::vector<int> *row_map, HostMat &out, const char *name) {
    if (!t.data) return fail(PK_ERR_TENSOR, "missing tensor %s", name);
    if (t.ne0 != cols || t.ne1 != rows)
        return fail(PK_ERR_TENSOR, "%s: ne=[%lld,%lld], expected [%d,%d]", name, (long long)t.ne0,
                    (long long)t.ne1, cols, rows);
    if (t.type != PK_TYPE_F32 && t.type != PK_TYPE_F16 && t.type != PK_TYPE_Q8_0)
        return fail(PK_ERR_UNSUPPORTED, "%s: ggml type %d not supported", name, t.type);
    if (cols % 4) return fail(PK_ERR_UNSUPPORTED, "%s: row length %d not a multiple of 4", name, cols);
    if (t.type == PK_TYPE_Q8_0 && cols % 32) return fail(PK_ERR_TENSOR, "%s: q8_0 row length %d", name, cols);
    out.type = t.type;
    out.rows = rows;
    out.cols = cols;
    const int bpe = bytes_per_elem(t.type);
    out.w.resize((size_t)rows * cols * bpe);
    if (t.type == PK_TYPE_Q8_0) out.d.resize((size_t)rows * (cols / 32));
    const uint8_t *src = static_cast<const uint8_t *>(t.data);
    const size_t row_bytes = t.type == PK_TYPE_Q8_0 ? (size_t)(cols / 32) * 34 : (size_t)cols * bpe;
    for (int r = 0; r < rows; ++r) {
        const int sr = row_map ? (*row_map)[r] : r;
        const uint8_t *row = src + (size_t)sr * row_bytes;
        if (t.type == PK_TYPE_Q8_0) {
            for (int b = 0; b < cols / 32; ++b) {
                uint16_t dh;
                memcpy(&dh, row + 34 * b, 2);
                out.d[(size_t)r * (cols / 32) + b] = f16_to_f32(dh);
                memcpy(&out.w[(size_t)r * cols + 32 * b], row + 34 * b + 2, 32);
            }
        } else {
            memcpy(&out.w[(size_t)r * cols * bpe], row, row_bytes);
        }
    }
    return 0;
}

int vec_f32(const pk_tensor &t, int n, const std::vector<int> *map, std::vector<float> &out, const char *name) {
    if (!t.data) return fail(PK_ERR_TENSOR, "missing tensor %s", name);
    if (t.ne0 * t.ne1 != n) return fail(PK_ERR_TENSOR, "%s: %lld elements, expected %d", name,
                                        (long long)(t.ne0 * t.ne1), n);
    std::vector<float> tmp(n);
    if (t.type == PK_TYPE_F32) memcpy(tmp.data(), t.data, 4 * (size_t)n);
    else if (t.type == PK_TYPE_F16) {
        const uint16_t *s = static_cast<const uint16_t *>(t.data);
        for (int i = 0; i < n; ++i) tmp[i] = f16_to_f32(s[i]);
    } else return fail(PK_ERR_UNSUPPORTED, "%s: bias type %d", name, t.type);
    out.resize(n);
    for (int i = 0; i < n; ++i) out[i] = tmp[map ? (*map)[i] : i];
    return 0;
}

}  // namespace

struct pk_decoder {
    KParams kp{};              // weights + dims (batch fields filled per call)
    pk_decoder_desc desc{};    // host copy of the description (tensor pointers not kept)
    DMat w_enc{};              // joint.enc.weight on the device
    const float *b_enc = nullptr;
    int n_slots = 0;
    int device = 0;
    int n_cu = 0, lds_block = 0;
    int nwg = 0;               // decode-loop workgroups
    size_t stage_bytes = 0;
    hipStream_t stream = nullptr;
    hipEvent_t ev[3] = {};
    DevBuf arena;              // weights
    DevBuf eproj;              // [V1][4H] layer-0 input projection of every token
    DevBuf slots_h, slots_c, slots_pp, slots_ctrl;
    DevBuf special;
    // per-call scratch
    DevBuf d_desc, d_encp, d_keys, d_sync, d_enc, d_out, d_xchg, d_flags;
    std::vector<uint8_t> h_desc;
    int last_iters = 0;
};

namespace {

int upload_weights(pk_decoder *dec, std::vector<HostMat> &mats, std::vector<std::vector<float>> &vecs,
                   std::vector<DMat *> &mat_dst, std::vector<const float **> &vec_dst) {
    size_t total = 0;
    auto align = [](size_t x) { return (x + 255) & ~(size_t)255; };
    for (auto &m : mats) total += align(m.w.size()) + align(m.d.size() * 4);
    for (auto &v : vecs) total += align(v.size() * 4);
    if (int rc = dec->arena.ensure(total)) return rc;
    uint8_t *base = dec->arena.as<uint8_t>();
    size_t off = 0;
    for (size_t i = 0; i < mats.size(); ++i) {
        DMat &dm = *mat_dst[i];
        dm.type = mats[i].type;
        dm.rows = mats[i].rows;
        dm.cols = mats[i].cols;
        HIP_TRY(hipMemcpy(base + off, mats[i].w.data(), mats[i].w.size(), hipMemcpyHostToDevice));
        dm.w = base + off;
        off += align(mats[i].w.size());
        dm.d = nullptr;
        if (!mats[i].d.empty()) {
            HIP_TRY(hipMemcpy(base + off, mats[i].d.data(), mats[i].d.size() * 4, hipMemcpyHostToDevice));
            dm.d = reinterpret_cast<const float *>(base + off);
            off += align(mats[i].d.size() * 4);
        }
    }
    for (size_t i = 0; i < vecs.size(); ++i) {
        HIP_TRY(hipMemcpy(base + off, vecs[i].data(), vecs[i].size() * 4, hipMemcpyHostToDevice));
        *vec_dst[i] = reinterpret_cast<const float *>(base + off);
        off += align(vecs[i].size() * 4);
    }
    return 0;
}

int decode_impl(pk_decoder *dec, const pk_batch *bt, bool keep_empty);

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
    if (!d || !out || n_slots <= 0) return fail(PK_ERR_ARG, "pk_decoder_create: bad arguments");
    *out = nullptr;
    const int H = d->pred_hidden, L = d->pred_rnn_layers, J = d->joint_hidden, D = d->d_enc;
    const int V1 = d->vocab_size + 1;
    const int Dn = d->kind == PK_KIND_TDT ? d->num_durations : 0;
    const int Vo = V1 + Dn;
    if (d->kind != PK_KIND_TDT && d->kind != PK_KIND_EOU) return fail(PK_ERR_ARG, "unknown decoder kind %d", d->kind);
    if (H <= 0 || J <= 0 || D <= 0 || L <= 0 || L > PK_MAX_LAYERS || d->vocab_size <= 0)
        return fail(PK_ERR_ARG, "bad dims H=%d L=%d J=%d D=%d V=%d", H, L, J, D, d->vocab_size);
    if (d->kind == PK_KIND_TDT && (Dn <= 0 || Dn > PK_MAX_DURATIONS))
        return fail(PK_ERR_UNSUPPORTED, "TDT num_durations %d", Dn);
    if (d->kind == PK_KIND_TDT && d->n_duration_values > 0 && d->n_duration_values < Dn)
        return fail(PK_ERR_ARG, "durations table (%d) shorter than num_durations (%d)", d->n_duration_values, Dn);
    if (V1 > (1 << kIdxBits) - 1 || Dn > (1 << kIdxBits) - 1)
        return fail(PK_ERR_UNSUPPORTED, "vocab %d exceeds the argmax key index field", V1);
    if (d->blank_id < 0 || d->blank_id >= V1) return fail(PK_ERR_ARG, "blank_id %d outside [0,%d)", d->blank_id, V1);

    auto *dec = new pk_decoder();
    dec->desc = *d;
    dec->n_slots = n_slots;
    KParams &kp = dec->kp;
    kp.kind = d->kind; kp.H = H; kp.L = L; kp.J = J; kp.V1 = V1; kp.Dn = Dn; kp.Vo = Vo;
    kp.blank = d->blank_id;
    kp.eou = d->eou_id >= 0 ? d->eou_id : d->vocab_size - 2;
    kp.eob = d->eob_id >= 0 ? d->eob_id : d->vocab_size - 1;
    kp.n_dur = d->kind == PK_KIND_TDT ? d->n_duration_values : 0;
    for (int i = 0; i < PK_MAX_DURATIONS; ++i) kp.durations[i] = d->durations[i];

    auto cleanup = [&](int rc) { delete dec; return rc; };
    if (hipGetDevice(&dec->device) != hipSuccess) return cleanup(fail(PK_ERR_DEVICE, "no HIP device"));
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dec->device) != hipSuccess) return cleanup(fail(PK_ERR_DEVICE, "device props"));
    dec->n_cu = prop.multiProcessorCount;
    dec->lds_block = (int)prop.sharedMemPerBlock;

    // unit-major gate rows: row 4j+g <- stored row g*H + j
    std::vector<int> gmap(4 * H);
    for (int j = 0; j < H; ++j)
        for (int g = 0; g < 4; ++g) gmap[4 * j + g] = g * H + j;

    std::vector<HostMat> mats;
    std::vector<DMat *> mat_dst;
    std::vector<std::vector<float>> vecs;
    std::vector<const float **> vec_dst;
    mats.reserve(4 + 2 * L);
    int rc;
    auto add_mat = [&](const pk_tensor &t, int rows, int cols, const std::vector<int> *map, DMat *dst,
                       const char *name) {
        mats.emplace_back();
        mat_dst.push_back(dst);
        return repack(t, rows, cols, map, mats.back(), name);
    };
    auto add_vec = [&](const pk_tensor &t, int n, const std::vector<int> *map, const float **dst, const char *name) {
        vecs.emplace_back();
        vec_dst.push_back(dst);
        return vec_f32(t, n, map, vecs.back(), name);
    };
    DMat embed{};
    const float *b_ih0 = nullptr, *b_hh0 = nullptr;
    if ((rc = add_mat(d->embed, V1, H, nullptr, &embed, "predict.embed.weight"))) return cleanup(rc);
    for (int l = 0; l < L; ++l) {
        if ((rc = add_mat(d->w_ih[l], 4 * H, H, &gmap, &kp.w_ih[l], "predict.lstm.w_ih"))) return cleanup(rc);
        if ((rc = add_mat(d->w_hh[l], 4 * H, H, &gmap, &kp.w_hh[l], "predict.lstm.w_hh"))) return cleanup(rc);
        std::vector<float> bi, bh;
        if ((rc = vec_f32(d->b_ih[l], 4 * H, &gmap, bi, "predict.lstm.b_ih"))) return cleanup(rc);
        if ((rc = vec_f32(d->b_hh[l], 4 * H, &gmap, bh, "predict.lstm.b_hh"))) return cleanup(rc);
        if (l == 0) {
            vecs.push_back(bi);
            vec_dst.push_back(&b_ih0);
            vecs.push_back(bh);
            vec_dst.push_back(&b_hh0);
        } else {
            for (int i = 0; i < 4 * H; ++i) bi[i] += bh[i];
            vecs.push_back(bi);
            vec_dst.push_back(&kp.b_lstm[l]);
        }
    }
    if ((rc = add_mat(d->joint_enc_w, J, D, nullptr, &dec->w_enc, "joint.enc.weight"))) return cleanup(rc);
    if ((rc = add_vec(d->joint_enc_b, J, nullptr, &dec->b_enc, "joint.enc.bias"))) return cleanup(rc);
    if ((rc = add_mat(d->joint_pred_w, J, H, nullptr, &kp.w_pred, "joint.pred.weight"))) return cleanup(rc);
    if ((rc = add_vec(d->joint_pred_b, J, nullptr, &kp.b_pred, "joint.pred.bias"))) return cleanup(rc);
    if ((rc = add_mat(d->joint_out_w, Vo, J, nullptr, &kp.w_out, "joint.out.weight"))) return cleanup(rc);
    if ((rc = add_vec(d->joint_out_b, Vo, nullptr, &kp.b_out, "joint.out.bias"))) return cleanup(rc);
    if (H % 4 || J % 4) return cleanup(fail(PK_ERR_UNSUPPORTED, "pred_hidden and joint_hidden must be multiples of 4"));
    if ((rc = upload_weights(dec, mats, vecs, mat_dst, vec_dst))) return cleanup(rc);
    // layer-0 input projection of every token: E'[v] = W_ih0 . embed[v] + b_ih0 + b_hh0
    if ((rc = dec->eproj.ensure((size_t)V1 * 4 * H * 4))) return cleanup(rc);
    {
        dim3 grid((V1 + 15) / 16, (4 * H + 63) / 64);
        pkdev::embed_proj_kernel<<<grid, 256>>>(kp.w_ih[0], embed, b_ih0, b_hh0, dec->eproj.as<float>());
        if (hipGetLastError() != hipSuccess || hipDeviceSynchronize() != hipSuccess)
            return cleanup(fail(PK_ERR_DEVICE, "embedding projection kernel failed"));
    }
    kp.eproj = dec->eproj.as<float>();
    dec->desc.special = nullptr;
    dec->kp.special = nullptr;
    dec->kp.n_special = 0;
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
    if ((rc = dec->slots_ctrl.ensure((size_t)n_slots * PK_CTRL_N * 4))) return cleanup(rc);
    if (hipMemset(dec->slots_h.p, 0, dec->slots_h.n) != hipSuccess ||
        hipMemset(dec->slots_c.p, 0, dec->slots_c.n) != hipSuccess ||
        hipMemset(dec->slots_pp.p, 0, dec->slots_pp.n) != hipSuccess ||
        hipMemset(dec->slots_ctrl.p, 0, dec->slots_ctrl.n) != hipSuccess)
        return cleanup(fail(PK_ERR_DEVICE, "slot memset"));
    kp.slot_h = dec->slots_h.as<float>();
    kp.slot_c = dec->slots_c.as<float>();
    kp.slot_pp = dec->slots_pp.as<float>();
    kp.slot_ctrl = dec->slots_ctrl.as<int>();

    // decode-loop launch shape: one workgroup per CU, LDS stage for kUC utterances
    const size_t need = std::max((size_t)kUC * (J + L * H), (size_t)kSmallB * H) * 4;
    if (need + sizeof(pkdev::Ctl) > (size_t)dec->lds_block)
        return cleanup(fail(PK_ERR_UNSUPPORTED, "LDS %zu B needed, %d available", need + sizeof(pkdev::Ctl),
                            dec->lds_block));
    dec->stage_bytes = need;
    if (hipFuncSetAttribute(reinterpret_cast<const void *>(pkdev::decode_loop_kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)need) != hipSuccess)
        return cleanup(fail(PK_ERR_DEVICE, "hipFuncSetAttribute"));
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void *>(pkdev::decode_loop_kernel),
                                                     kBlock, need) != hipSuccess || per_cu < 1)
        return cleanup(fail(PK_ERR_DEVICE, "decode kernel does not fit on a CU"));
    dec->nwg = std::min(dec->n_cu, kBlock);
    if (hipStreamCreateWithFlags(&dec->stream, hipStreamNonBlocking) != hipSuccess)
        return cleanup(fail(PK_ERR_DEVICE, "stream"));
    for (auto &e : dec->ev)
        if (hipEventCreate(&e) != hipSuccess) return cleanup(fail(PK_ERR_DEVICE, "event"));
    *out = dec;
    return 0;
}

PK_API int pk_decoder_destroy(pk_decoder *dec) {
    if (!dec) return 0;
    (void)hipSetDevice(dec->device);
    if (dec->stream) (void)hipStreamSynchronize(dec->stream);
    for (auto &e : dec->ev) if (e) (void)hipEventDestroy(e);
    if (dec->stream) (void)hipStreamDestroy(dec->stream);
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
    int32_t cw[PK_CTRL_N];
    HIP_TRY(hipMemcpy(cw, kp.slot_ctrl + (size_t)slot * PK_CTRL_N, sizeof cw, hipMemcpyDeviceToHost));
    const size_t hn = (size_t)kp.L * kp.H;
    if (h) HIP_TRY(hipMemcpy(h, kp.slot_h + (size_t)slot * hn, hn * 4, hipMemcpyDeviceToHost));
    if (c) HIP_TRY(hipMemcpy(c, kp.slot_c + (size_t)slot * hn, hn * 4, hipMemcpyDeviceToHost));
    if (pred) HIP_TRY(hipMemcpy(pred, kp.slot_h + (size_t)slot * hn + (size_t)(kp.L - 1) * kp.H,
                                (size_t)kp.H * 4, hipMemcpyDeviceToHost));
    if (ctrl) memcpy(ctrl, cw, sizeof cw);
    return 0;
}

PK_API int pk_last_timing(pk_decoder *dec, float *enc_proj_ms, float *loop_ms, int32_t *iterations) {
    if (!dec) return fail(PK_ERR_ARG, "pk_last_timing: null");
    float a = 0, b = 0;
    HIP_TRY(hipEventElapsedTime(&a, dec->ev[0], dec->ev[1]));
    HIP_TRY(hipEventElapsedTime(&b, dec->ev[1], dec->ev[2]));
    if (enc_proj_ms) *enc_proj_ms = a;
    if (loop_ms) *loop_ms = b;
    if (iterations) *iterations = dec->last_iters;
    return 0;
}

PK_API int pk_decode(pk_decoder *dec, const pk_batch *bt) {
    g_err.clear();
    return decode_impl(dec, bt, false);
}

}  // extern "C"

namespace {

int decode_impl(pk_decoder *dec, const pk_batch *bt, bool keep_empty) {
    if (!dec || !bt) return fail(PK_ERR_ARG, "pk_decode: null argument");
    const KParams &kp = dec->kp;
    if (bt->d_enc != dec->desc.d_enc) return fail(PK_ERR_D_ENC, "encoder d_model mismatch (%d vs %d)", bt->d_enc, dec->desc.d_enc);
    const int n = bt->n_utts;
    if (n < 0 || n > kMaxBatch) return fail(PK_ERR_ARG, "n_utts %d outside [0,%d]", n, kMaxBatch);
    if (n == 0) return 0;
    if (!bt->enc_row || !bt->n_frames || !bt->slot || !bt->n_tokens || !bt->steps || !bt->tokens)
        return fail(PK_ERR_ARG, "pk_decode: missing batch array");
    if (bt->mem != PK_MEM_HOST && bt->mem != PK_MEM_DEVICE) return fail(PK_ERR_ARG, "bad mem kind");
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
        if (keep_empty || kp.kind == PK_KIND_EOU || bt->n_frames[u] > 0) map.push_back(u);
    const int m = (int)map.size();
    long long rows = 0;
    int max_T = 0;
    std::vector<long long> src_row(m), dst_row(m);
    std::vector<int32_t> T(m), slots(m), base(m);
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
    }
    const bool host = bt->mem == PK_MEM_HOST;
    const int D = dec->desc.d_enc, J = kp.J;
    int rc;
    // encoder frames: device pointer as given, or packed host rows uploaded
    const float *enc = bt->enc;
    if (host && rows > 0) {
        if ((rc = dec->d_enc.ensure((size_t)rows * D * 4))) return rc;
        for (int i = 0; i < m; ++i)
            HIP_TRY(hipMemcpyAsync(dec->d_enc.as<float>() + (size_t)dst_row[i] * D, bt->enc + (size_t)src_row[i] * D,
                                   (size_t)T[i] * D * 4, hipMemcpyHostToDevice, dec->stream));
        enc = dec->d_enc.as<float>();
        src_row = dst_row;
    }
    // descriptor block: src_row, dst_row (int64), T, slot, base (int32), bias (f32)
    const size_t desc_bytes = (size_t)m * (8 + 8 + 4 + 4 + 4 + 4);
    if ((rc = dec->d_desc.ensure(std::max<size_t>(desc_bytes, 64)))) return rc;
    dec->h_desc.resize(desc_bytes);
    uint8_t *hd = dec->h_desc.data();
    memcpy(hd, src_row.data(), 8 * (size_t)m);
    memcpy(hd + 8 * (size_t)m, dst_row.data(), 8 * (size_t)m);
    memcpy(hd + 16 * (size_t)m, T.data(), 4 * (size_t)m);
    memcpy(hd + 20 * (size_t)m, slots.data(), 4 * (size_t)m);
    memcpy(hd + 24 * (size_t)m, base.data(), 4 * (size_t)m);
    memcpy(hd + 28 * (size_t)m, bias.data(), 4 * (size_t)m);
    if (m > 0) HIP_TRY(hipMemcpyAsync(dec->d_desc.p, hd, desc_bytes, hipMemcpyHostToDevice, dec->stream));
    uint8_t *dd = dec->d_desc.as<uint8_t>();
    const long long *d_src = reinterpret_cast<const long long *>(dd);
    const long long *d_dst = reinterpret_cast<const long long *>(dd + 8 * (size_t)m);
    const int *d_T = reinterpret_cast<const int *>(dd + 16 * (size_t)m);
    const int *d_slot = reinterpret_cast<const int *>(dd + 20 * (size_t)m);
    const int *d_base = reinterpret_cast<const int *>(dd + 24 * (size_t)m);
    const float *d_bias = reinterpret_cast<const float *>(dd + 28 * (size_t)m);

    HIP_TRY(hipEventRecord(dec->ev[0], dec->stream));
    if (rows > 0) {
        if ((rc = dec->d_encp.ensure((size_t)rows * J * 4))) return rc;
        dim3 grid((max_T + 63) / 64, m, (J + 63) / 64);
        pkdev::enc_proj_kernel<<<grid, 256, 0, dec->stream>>>(dec->w_enc, dec->b_enc, enc, D,
                                                       d_src, d_dst, d_T, dec->d_encp.as<float>());
        HIP_TRY(hipGetLastError());
    }
    HIP_TRY(hipEventRecord(dec->ev[1], dec->stream));

    // outputs: device arrays as given, or a device staging area copied back
    const int tcap = bt->token_cap, scap = bt->seg_cap, trcap = bt->trace ? bt->trace_cap : 0;
    int *o_tok, *o_ntok, *o_steps, *o_seg = nullptr, *o_nseg = nullptr, *o_trace = nullptr;
    std::vector<int> idx_map = map;
    if (host) {
        const size_t need = ((size_t)m * tcap + 3 * (size_t)m + (size_t)m * std::max(scap, 0) +
                             (size_t)m * trcap * 2) * 4 + 64;
        if ((rc = dec->d_out.ensure(need))) return rc;
        int *o = dec->d_out.as<int>();
        o_tok = o; o += (size_t)m * tcap;
        o_ntok = o; o += m;
        o_steps = o; o += m;
        o_nseg = o; o += m;
        o_seg = scap > 0 ? o : nullptr; o += (size_t)m * std::max(scap, 0);
        o_trace = trcap > 0 ? o : nullptr;
    } else {
        if (m != n) return fail(PK_ERR_ARG, "device-memory batches must not contain empty TDT windows");
        o_tok = bt->tokens; o_ntok = bt->n_tokens; o_steps = bt->steps;
        o_seg = bt->segments; o_nseg = bt->n_segments; o_trace = bt->trace;
    }
    // launch with the device descriptor arrays
    KParams &p = dec->kp;
    (void)d_base;
    rc = 0;
    {
        p.n_utts = m;
        p.encp = dec->d_encp.as<float>();
        p.encp_row = d_dst;
        p.T = d_T;
        p.slot = d_slot;
        p.blank_bias = bt->blank_bias ? d_bias : nullptr;
        p.tokens_base = bt->tokens_base ? d_base : nullptr;
        p.tokens = o_tok; p.token_cap = tcap;
        p.n_tokens = o_ntok; p.steps = o_steps;
        p.segs = o_seg; p.seg_cap = scap; p.n_segs = o_nseg;
        p.trace = o_trace; p.trace_cap = trcap;
        p.max_sym = bt->max_symbols;
        p.max_iter = max_T * (std::max(bt->max_symbols, 1) + 1) + 4;
        if ((unsigned)p.max_iter >= kMaxStamp) return fail(PK_ERR_UNSUPPORTED, "window too long for the iteration stamp");
        if ((rc = dec->d_keys.ensure((size_t)2 * std::max(m, 1) * 2 * 8))) return rc;
        if ((rc = dec->d_sync.ensure(64))) return rc;
        if ((rc = dec->d_flags.ensure((size_t)dec->nwg * kFlagStride * 4))) return rc;
        const int L = kp.L, H = kp.H;
        const size_t mm = std::max(m, 1);
        const size_t xh = 2 * (size_t)L * mm * H, xp = mm * J, xr = (size_t)L * mm * 4 * H;
        if ((rc = dec->d_xchg.ensure((2 * xh + xp + xr) * 4))) return rc;
        p.hx = dec->d_xchg.as<float>();
        p.cx = p.hx + xh;
        p.ppx = p.cx + xh;
        p.rx = p.ppx + xp;
        p.keys = dec->d_keys.as<unsigned long long>();
        p.flags = dec->d_flags.as<unsigned>();
        p.status = dec->d_sync.as<int>() + 4;
        HIP_TRY(hipMemsetAsync(dec->d_keys.p, 0, (size_t)2 * std::max(m, 1) * 2 * 8, dec->stream));
        HIP_TRY(hipMemsetAsync(dec->d_sync.p, 0, 64, dec->stream));
        HIP_TRY(hipMemsetAsync(dec->d_flags.p, 0, (size_t)dec->nwg * kFlagStride * 4, dec->stream));
        void *args[] = {&p};
        if (m > 0) {
            HIP_TRY(hipLaunchCooperativeKernel(reinterpret_cast<const void *>(pkdev::decode_loop_kernel), dim3(dec->nwg),
                                               dim3(kBlock), args, dec->stage_bytes, dec->stream));
        }
    }
    HIP_TRY(hipEventRecord(dec->ev[2], dec->stream));
    int status[4] = {0, 0, 0, 0};
    HIP_TRY(hipMemcpyAsync(status, p.status, sizeof status, hipMemcpyDeviceToHost, dec->stream));
    if (host) {
        std::vector<int> tmp_ntok(m), tmp_steps(m), tmp_nseg(m);
        HIP_TRY(hipMemcpyAsync(tmp_ntok.data(), o_ntok, 4 * (size_t)m, hipMemcpyDeviceToHost, dec->stream));
        HIP_TRY(hipMemcpyAsync(tmp_steps.data(), o_steps, 4 * (size_t)m, hipMemcpyDeviceToHost, dec->stream));
        HIP_TRY(hipMemcpyAsync(tmp_nseg.data(), o_nseg, 4 * (size_t)m, hipMemcpyDeviceToHost, dec->stream));
        HIP_TRY(hipStreamSynchronize(dec->stream));
        for (int u = 0; u < n; ++u) { bt->n_tokens[u] = 0; bt->steps[u] = 0; if (bt->n_segments) bt->n_segments[u] = 0; }
        for (int i = 0; i < m; ++i) {
            const int u = map[i];
            bt->n_tokens[u] = tmp_ntok[i];
            bt->steps[u] = tmp_steps[i];
            const int nt = std::min(tmp_ntok[i], tcap);
            if (nt > 0)
                HIP_TRY(hipMemcpy(bt->tokens + (size_t)u * tcap, o_tok + (size_t)i * tcap, 4 * (size_t)nt, hipMemcpyDeviceToHost));
            if (bt->n_segments) bt->n_segments[u] = tmp_nseg[i];
            if (bt->segments && scap > 0) {
                const int ns = std::min(tmp_nseg[i], scap);
                if (ns > 0)
                    HIP_TRY(hipMemcpy(bt->segments + (size_t)u * scap, o_seg + (size_t)i * scap, 4 * (size_t)ns, hipMemcpyDeviceToHost));
            }
            if (o_trace) {
                const int ns = std::min(tmp_steps[i], trcap);
                if (ns > 0)
                    HIP_TRY(hipMemcpy(bt->trace + (size_t)u * trcap * 2, o_trace + (size_t)i * trcap * 2, 8 * (size_t)ns, hipMemcpyDeviceToHost));
            }
        }
    } else {
        HIP_TRY(hipStreamSynchronize(dec->stream));
    }
    dec->last_iters = status[1];
    if (status[0]) return fail(status[0], "device decode failed (status %d)", status[0]);
    if (status[2]) return fail(PK_ERR_OVERFLOW, "token or segment capacity exceeded");
    return 0;
}

}  // namespace
