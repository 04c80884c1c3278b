// Internal: the slice timer's ring as bookkeeping with no GPU in it. Which
// slot a frame's events use, when a slot's events may be read, and in what
// order; the C API in beatlm_schedule.h (bls_ring_*) wraps it for tests and
// hosts. The counterpart of crates/beatlm/src/gpu/ring.rs.
//
// A slot's life: FREE -> RECORDING (claimed by a frame) -> ENCODED (the
// frame's closing event is recorded; the host holds a ticket) -> SUBMITTED
// (the ticket came back: the host says the frame's work reached the stream)
// or HELD (came back held: read only once the host's verdict accepts it) ->
// back to FREE once collected. INVALID: submitted or held, and since marked
// untrustworthy by the host; freed unread once its work has completed.
//
// Rules, as the reference's ring states them:
//  1. a frame takes a slot only if the slot at the cursor is free; a busy
//     slot is not waited for, and the cursor stays on it (the oldest);
//  2. a slot is read only after its ticket came back; a ticket dropped
//     instead (bls_ticket_drop) frees the slot unread at the next claim;
//  3. an invalidated slot is never read, but is freed only once its work
//     has completed;
//  4. a held slot is collected only once its verdict has come and the ring
//     has settled it; a verdict that arrives after its slot moved on
//     reaches nothing;
//  5. slots are read in the order their tickets came back: a readable slot
//     waits while one submitted before it may still be read (held, or
//     submitted with its work not completed); slots that will not be read
//     (invalid, or whose work failed) hold back nothing.
//
// Tickets and holds are 64-bit values naming the ring, the slot and the lap
// (a serial number), so a ticket from an earlier lap or another ring is
// refused. A ticket or verdict may be dropped or given from any thread; the
// ring itself is used from one thread at a time.
#pragma once

#include <atomic>
#include <cstdint>
#include <memory>

namespace bl {

enum class Phase : uint8_t { FREE = 0, RECORDING, ENCODED, SUBMITTED, HELD, INVALID };

// Where a slot's work stands: its closing event's hipEventQuery.
enum class Done : uint8_t { PENDING = 0, OK, FAILED };

// What collecting a slot does now.
enum class Action : uint8_t { WAIT = 0, READ, DROP };

// ring.rs:98-111 (collect): only a submitted slot whose work completed is
// read; an invalid one is dropped once its work completed or failed; a held
// slot, and one in no collectable phase, waits.
Action collect_action(Phase phase, Done done);

constexpr uint32_t RING_MAX_DEPTH = 64;

class Ring {
  public:
    // A ring of `depth` free slots (0 is raised to 1; at most RING_MAX_DEPTH).
    explicit Ring(uint32_t depth);
    ~Ring();
    Ring(const Ring &) = delete;
    Ring &operator=(const Ring &) = delete;

    uint32_t depth() const { return depth_; }
    // Frees the slots whose tickets were dropped, then takes the slot at the
    // cursor if it is free and moves the cursor on. -1: busy.
    int claim();
    // The recording slot's frame is closed: its ticket (0 if the slot is not
    // recording).
    uint64_t encode(uint32_t slot);
    // The ticket comes back: its slot moves to SUBMITTED and is returned. -1
    // for a ticket this ring did not hand out for a slot now ENCODED (another
    // ring's is dropped in its own ring, an earlier lap's reaches nothing).
    int submit(uint64_t ticket);
    // submit, but the slot moves to HELD; *hold names it for its verdict.
    int submit_held(uint64_t ticket, uint64_t *hold);
    // HELD slots whose verdict came: accepted -> SUBMITTED, rejected -> INVALID.
    void settle();
    // Every SUBMITTED or HELD slot -> INVALID; how many moved.
    uint32_t invalidate();
    // The slots to collect now, oldest submission first, given where each
    // slot's work stands (`done(slot)`, asked only for slots past submission).
    // Returns how many were written to `slots`/`actions` (RING_MAX_DEPTH each).
    template <class F>
    uint32_t ready(F done, uint32_t *slots, Action *actions) const;
    // The slot back to FREE, whatever its phase.
    void release(uint32_t slot);
    // Slots neither free nor waiting on a dropped ticket.
    uint32_t in_flight() const;
    // The slot's phase; FREE for a slot the ring does not have.
    Phase phase(uint32_t slot) const { return slot < depth_ ? phase_[slot] : Phase::FREE; }
    // Slots freed so far because their ticket was dropped.
    uint64_t reclaimed() const { return reclaimed_; }

    // Ticket and hold handling that needs no ring borrowed (any thread).
    bool abandon(uint64_t ticket);
    bool give_verdict(uint64_t hold, bool accepted);

  private:
    bool abandoned(uint32_t slot) const;
    uint64_t make_id(uint32_t slot);

    uint32_t depth_;
    uint32_t id_;                // this ring's number in the process's table of live rings
    uint32_t cursor_ = 0;
    uint64_t serial_ = 0;        // laps handed out (tickets and holds)
    uint64_t submissions_ = 0;
    uint64_t reclaimed_ = 0;
    Phase phase_[RING_MAX_DEPTH];
    uint64_t order_[RING_MAX_DEPTH];  // when each slot's ticket came back
    // The slot's live ticket (ENCODED), with ABANDONED set once dropped; 0 otherwise.
    std::unique_ptr<std::atomic<uint64_t>[]> ticket_;
    // The slot's hold (HELD) with its verdict in the top two bits; 0 otherwise.
    std::unique_ptr<std::atomic<uint64_t>[]> verdict_;
};

// A ticket given up without being handed back (its frame's work was never
// submitted, or the host cannot tell): its slot is freed unread.
void drop_ticket(uint64_t ticket);
// The host's word on a held submission; false when it reached no held slot.
bool give_verdict(uint64_t hold, bool accepted);

template <class F>
uint32_t Ring::ready(F done, uint32_t *slots, Action *actions) const {
    uint32_t n = 0;
    uint64_t barrier = UINT64_MAX;  // the oldest submission that may still be read and cannot be yet
    for (uint32_t i = 0; i < depth_; i++) {
        const Phase p = phase_[i];
        if (p != Phase::SUBMITTED && p != Phase::HELD && p != Phase::INVALID) continue;
        const Action a = collect_action(p, done(i));
        if (a == Action::WAIT) {
            if (p != Phase::INVALID && order_[i] < barrier) barrier = order_[i];
            continue;
        }
        slots[n] = i;
        actions[n] = a;
        n++;
    }
    // Reads behind the barrier wait; drops never do. Then submission order
    // (insertion sort: at most RING_MAX_DEPTH entries).
    uint32_t kept = 0;
    for (uint32_t j = 0; j < n; j++) {
        if (actions[j] == Action::READ && order_[slots[j]] >= barrier) continue;
        uint32_t s = slots[j];
        Action a = actions[j];
        uint32_t k = kept++;
        while (k > 0 && order_[slots[k - 1]] > order_[s]) {
            slots[k] = slots[k - 1];
            actions[k] = actions[k - 1];
            k--;
        }
        slots[k] = s;
        actions[k] = a;
    }
    return kept;
}

}  // namespace bl
