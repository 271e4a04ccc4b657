// decoder_core.cpp -- see decoder_core.h.
#include "decoder_core.h"

#include <algorithm>
#include <climits>
#include <cstdio>
#include <cstring>
#include <stdexcept>

namespace parakeet_hip {

SlotPool::~SlotPool() {
    if (dec) pk_decoder_destroy(dec);
}

int SlotPool::acquire() {
    std::lock_guard<std::mutex> lk(mu);
    if (free_slots.empty()) return -1;
    const int s = free_slots.back();
    free_slots.pop_back();
    return s;
}

void SlotPool::release(int s) {
    std::lock_guard<std::mutex> lk(mu);
    free_slots.push_back(s);
}

// ------------------------------------------------------------------ SlotHandle

void SlotHandle::release() {
    if (pool_ && slot_ >= 0) pool_->release(slot_);
    pool_.reset();
    slot_ = -1;
    pending_ = false;
}

SlotHandle::~SlotHandle() { release(); }

SlotHandle::SlotHandle(const SlotHandle &other) { *this = other; }

SlotHandle &SlotHandle::operator=(const SlotHandle &other) {
    if (this == &other) return *this;
    release();
    if (!other.valid()) return *this;
    const int s = other.pool_->acquire();
    if (s < 0) throw std::runtime_error("parakeet: no free decoder state slot for a state copy");
    pool_ = other.pool_;
    slot_ = s;
    pending_ = other.pending_;
    if (!pending_ && pk_slot_copy(pool_->dec, other.slot_, slot_) != 0)
        throw std::runtime_error(std::string("parakeet: state copy failed: ") + pk_last_error());
    return *this;
}

SlotHandle::SlotHandle(SlotHandle &&other) noexcept
    : pool_(std::move(other.pool_)), slot_(other.slot_), pending_(other.pending_) {
    other.slot_ = -1;
    other.pending_ = false;
}

SlotHandle &SlotHandle::operator=(SlotHandle &&other) noexcept {
    if (this == &other) return *this;
    release();
    pool_ = std::move(other.pool_);
    slot_ = other.slot_;
    pending_ = other.pending_;
    other.slot_ = -1;
    other.pending_ = false;
    return *this;
}

void SlotHandle::reset(const std::shared_ptr<SlotPool> &pool) {
    if (!pool) throw std::runtime_error("parakeet: decoder runtime not prepared");
    if (pool_ != pool) {
        release();
        const int s = pool->acquire();
        if (s < 0) throw std::runtime_error("parakeet: no free decoder state slot");
        pool_ = pool;
        slot_ = s;
    }
    pending_ = true;
}

namespace core {

int make_pool(const pk_decoder_desc &d, int n_slots, std::shared_ptr<SlotPool> &out) {
    auto pool = std::make_shared<SlotPool>();
    if (int rc = pk_decoder_create(&d, n_slots, &pool->dec)) {
        std::fprintf(stderr, "prepare_runtime: %s\n", pk_last_error());
        return rc;
    }
    // these runtimes never read pk_last_timing: leave its per-call event records out
    (void)pk_decoder_set_timing(pool->dec, 0);
    for (int s = n_slots - 1; s >= 0; --s) pool->free_slots.push_back(s);
    out = std::move(pool);
    return 0;
}

Frames Frames::pick(const std::vector<int> &idx, size_t i, size_t j) const {
    Frames f;
    f.device = device;
    f.dev = dev;
    for (size_t k = i; k < j; ++k) {
        if (device) f.dev_row.push_back(dev_row[idx[k]]);
        else f.host.push_back(host[idx[k]]);
    }
    return f;
}

int device_frames(const float *data, int64_t n_rows, int d_model, const std::vector<int64_t> &row_offset,
                  const std::vector<int> &n_frames, int D_expected, const char *who, Frames &fr) {
    if (d_model != D_expected) {
        std::fprintf(stderr, "%s: encoder d_model mismatch (%d vs %d)\n", who, d_model, D_expected);
        return 1;
    }
    if (row_offset.size() != n_frames.size()) return 3;
    for (size_t u = 0; u < n_frames.size(); ++u) {
        if (n_frames[u] <= 0) continue;
        if (!data || row_offset[u] < 0 || row_offset[u] + n_frames[u] > n_rows) {
            std::fprintf(stderr, "%s: utterance %zu rows [%lld, %lld) outside the encoder output (%lld rows)\n", who,
                         u, (long long)row_offset[u], (long long)(row_offset[u] + n_frames[u]), (long long)n_rows);
            return 3;
        }
    }
    fr.device = true;
    fr.dev = data;
    fr.dev_row = row_offset;
    return 0;
}

namespace {

// Host output staging of one batched call: at most 2^28 token slots (1 GiB).
constexpr long long kMaxOutputInts = 1ll << 28;

// One launch over utterances [i, j) of the batch.
int decode_launch(SlotPool &pool, int D_enc, int max_symbols, const Frames &fr, const std::vector<int> &n_frames,
                  const std::vector<SlotHandle *> &slots, const std::vector<int> &tokens_base, bool tdt, size_t i,
                  size_t j, BatchOut &out) {
    const int n = (int)(j - i);
    int64_t rows = 0;
    int max_T = 0;
    std::vector<int64_t> row(n);
    std::vector<int32_t> T(n), sl(n), base(n, 0);
    std::vector<uint8_t> reset(n);
    for (int u = 0; u < n; ++u) {
        T[u] = std::max(0, n_frames[i + u]);
        row[u] = fr.device ? fr.dev_row[i + u] : rows;
        rows += T[u];
        max_T = std::max(max_T, T[u]);
        sl[u] = slots[i + u]->slot();
        reset[u] = slots[i + u]->pending_init() ? 1 : 0;
        if (!tokens_base.empty()) base[u] = tokens_base[i + u];
    }
    // host windows: read in place when they follow one another in memory (always at
    // B=1: the caller's pointer is the batch's frames); otherwise packed in order
    std::vector<float> packed;
    const float *host_base = nullptr;
    if (!fr.device) {
        bool contiguous = true;
        const float *at = nullptr;
        for (int u = 0; u < n && contiguous; ++u) {
            if (T[u] <= 0) continue;
            if (!at) host_base = fr.host[i + u];
            else contiguous = fr.host[i + u] == at;
            at = fr.host[i + u] + (size_t)T[u] * D_enc;
        }
        if (!contiguous) {
            host_base = nullptr;
            packed.resize((size_t)std::max<int64_t>(rows, 1) * D_enc);
            for (int u = 0; u < n; ++u)
                if (T[u] > 0)
                    memcpy(packed.data() + (size_t)row[u] * D_enc, fr.host[i + u],
                           sizeof(float) * (size_t)T[u] * D_enc);
            host_base = packed.data();
        }
    }
    // every emission of a window fits (at most max_symbols per frame); an EOU boundary ends
    // its frame, so a window records at most max_T + 1 of them.  Sized in 64 bits and
    // bounded before anything is allocated.
    const long long cap64 = (long long)max_T * std::max(1, max_symbols) + 1;
    if (cap64 > INT32_MAX || (long long)n * cap64 > kMaxOutputInts) {
        std::fprintf(stderr, "decode: %d windows of up to %d frames at max_symbols %d need %lld output tokens "
                     "(at most %lld)\n", n, max_T, max_symbols, (long long)n * cap64, (long long)kMaxOutputInts);
        return PK_ERR_UNSUPPORTED;
    }
    const int cap = (int)cap64, scap = tdt ? 0 : max_T + 1;
    std::vector<int32_t> tok((size_t)n * cap), ntok(n), st(n), seg((size_t)n * std::max(scap, 1)), nseg(n);
    std::vector<int32_t> ctrl((size_t)n * PK_CTRL_N);
    pk_batch b{};
    b.n_utts = n;
    b.mem = fr.device ? PK_MEM_DEVICE_FRAMES : PK_MEM_HOST;
    b.d_enc = D_enc;
    b.max_symbols = max_symbols;
    b.enc = fr.device ? fr.dev : host_base;
    b.enc_row = row.data();
    b.n_frames = T.data();
    b.slot = sl.data();
    b.tokens_base = tokens_base.empty() ? nullptr : base.data();
    b.tokens = tok.data();
    b.token_cap = cap;
    b.n_tokens = ntok.data();
    b.steps = st.data();
    b.segments = scap ? seg.data() : nullptr;
    b.seg_cap = scap;
    b.n_segments = nseg.data();
    b.reset = reset.data();
    b.ctrl_out = ctrl.data();
    if (int rc = pk_decode(pool.dec, &b)) {
        std::fprintf(stderr, "decode: %s\n", pk_last_error());
        return rc;
    }
    for (int u = 0; u < n; ++u) {
        const size_t k = i + u;
        out.tokens[k].assign(tok.begin() + (size_t)u * cap, tok.begin() + (size_t)u * cap + ntok[u]);
        if (scap) out.segments[k].assign(seg.begin() + (size_t)u * scap, seg.begin() + (size_t)u * scap + nseg[u]);
        out.steps[k] = st[u];
        std::copy(ctrl.begin() + (size_t)u * PK_CTRL_N, ctrl.begin() + (size_t)(u + 1) * PK_CTRL_N,
                  out.ctrl[k].begin());
        if (!tdt || T[u] > 0) slots[k]->mark_initialised();
    }
    return 0;
}

}  // namespace

int decode(SlotPool &pool, int D_enc, int max_symbols, const Frames &fr, const std::vector<int> &n_frames,
           const std::vector<SlotHandle *> &slots, const std::vector<int> &tokens_base, bool tdt, BatchOut &out) {
    const size_t n = n_frames.size();
    out.tokens.assign(n, {});
    out.segments.assign(n, {});
    out.steps.assign(n, 0);
    out.ctrl.assign(n, {});
    for (size_t i = 0; i < n; i += PK_MAX_BATCH)
        if (int rc = decode_launch(pool, D_enc, max_symbols, fr, n_frames, slots, tokens_base, tdt, i,
                                   std::min(n, i + PK_MAX_BATCH), out))
            return rc;
    return 0;
}

std::string detokenize(const std::vector<std::string> &pieces, int32_t blank_id, int32_t bos_id, int32_t eos_id,
                       int32_t pad_id, const std::vector<int32_t> &ids) {
    std::string out;
    out.reserve(ids.size() * 3);
    for (int32_t id : ids) {
        if (id < 0 || id >= (int32_t)pieces.size()) continue;
        if (id == blank_id || id == bos_id || id == eos_id || id == pad_id) continue;
        const std::string &piece = pieces[id];
        for (size_t i = 0; i < piece.size();) {
            if ((unsigned char)piece[i] == 0xE2 && i + 2 < piece.size() && (unsigned char)piece[i + 1] == 0x96 &&
                (unsigned char)piece[i + 2] == 0x81) {
                out.push_back(' ');
                i += 3;
            } else {
                out.push_back(piece[i++]);
            }
        }
    }
    size_t start = 0;
    while (start < out.size() && out[start] == ' ') ++start;
    out.erase(0, start);
    return out;
}

namespace {
std::string trim_spaces(const std::string &s) {
    const size_t a = s.find_first_not_of(" \t\r\n");
    if (a == std::string::npos) return std::string();
    const size_t b = s.find_last_not_of(" \t\r\n");
    return s.substr(a, b - a + 1);
}
}  // namespace

std::string eou_text(const std::vector<std::string> &pieces, int32_t blank_id, int32_t bos_id, int32_t eos_id,
                     int32_t pad_id, const std::vector<int32_t> &ids, const std::vector<int32_t> &boundaries) {
    int seg_start = 0;
    std::string text;
    for (size_t i = 0; i <= boundaries.size(); ++i) {
        const int seg_end = i < boundaries.size() ? std::min(boundaries[i], (int32_t)ids.size()) : (int)ids.size();
        if (seg_end <= seg_start) {
            seg_start = seg_end;
            continue;
        }
        std::vector<int32_t> seg(ids.begin() + seg_start, ids.begin() + seg_end);
        const std::string s = trim_spaces(detokenize(pieces, blank_id, bos_id, eos_id, pad_id, seg));
        if (!s.empty()) {
            if (!text.empty()) text += "\n";
            text += s;
        }
        seg_start = seg_end;
    }
    return text;
}

std::vector<uint8_t> special_pieces(const std::vector<std::string> &pieces) {
    std::vector<uint8_t> special(pieces.size());
    for (size_t i = 0; i < pieces.size(); ++i)
        special[i] = (!pieces[i].empty() && pieces[i].front() == '<' && pieces[i].back() == '>') ? 1 : 0;
    return special;
}

}  // namespace core
}  // namespace parakeet_hip
