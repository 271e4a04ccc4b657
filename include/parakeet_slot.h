// parakeet_slot.h -- the device state slot held by a decode state.
//
// A decode state (TdtDecodeState / EouDecodeState) keeps its h, c, pred and
// control words in one numbered slot of its decoder on the device.  The
// handle behaves as a value, like the reference's state structs
// (src/parakeet_tdt.h:175-183, src/parakeet_eou.h:53-66): copying a state
// leases a new slot and copies the device state into it, so the copy decodes
// independently of the original; moving transfers the slot; destroying the
// state returns the slot to its decoder.
#pragma once

#include <memory>

namespace parakeet_hip {

struct SlotPool;   // the decoder of one runtime and its free slots (decoder_core)

class SlotHandle {
public:
    SlotHandle() = default;
    SlotHandle(const SlotHandle &other);
    SlotHandle &operator=(const SlotHandle &other);
    SlotHandle(SlotHandle &&other) noexcept;
    SlotHandle &operator=(SlotHandle &&other) noexcept;
    ~SlotHandle();

    bool valid() const { return slot_ >= 0; }
    int slot() const { return slot_; }
    const std::shared_ptr<SlotPool> &pool() const { return pool_; }
    // The state is fresh: its next decode starts from zero h, c and one LSTM
    // step on embed[blank], inside that decode's launch.  Leases a slot of
    // `pool` first when the handle holds none (or one of another decoder).
    // Throws std::runtime_error when every slot is in use.
    void reset(const std::shared_ptr<SlotPool> &pool);
    bool pending_init() const { return pending_; }
    void mark_initialised() { pending_ = false; }

private:
    void release();
    std::shared_ptr<SlotPool> pool_;
    int slot_ = -1;
    bool pending_ = false;
};

}  // namespace parakeet_hip
