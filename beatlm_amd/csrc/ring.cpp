// The slice timer's ring: which slot a frame's events use and when they may be
// read, with no GPU in it (crates/beatlm/src/gpu/ring.rs). The HIP timer
// (timer.cpp) drives one ring per timer; the bls_ring_* C API exposes the same
// rules to hosts and to CPU tests.
#include "ring.hpp"

#include <mutex>
#include <unordered_map>

#include "../../include/beatlm_schedule.h"

namespace bl {

namespace {

// Ticket and hold layout: bits 0-7 slot, 8-39 lap serial, 40-61 ring number.
// Bit 63 of a slot's ticket word marks it dropped; bits 62-63 of a slot's
// verdict word hold its verdict.
constexpr uint64_t ABANDONED = 1ull << 63;
constexpr int VERDICT_SHIFT = 62;
constexpr uint64_t ID_MASK = (1ull << VERDICT_SHIFT) - 1;
constexpr uint64_t VERDICT_PENDING = 0, VERDICT_ACCEPTED = 1, VERDICT_REJECTED = 2;
constexpr uint32_t RING_BITS = 22;

uint32_t slot_of(uint64_t id) { return (uint32_t)(id & 0xff); }
uint32_t ring_of(uint64_t id) { return (uint32_t)((id >> 40) & ((1u << RING_BITS) - 1)); }

// The process's live rings by number, so a ticket or verdict reaches the ring
// that made it from anywhere, and one whose ring is gone reaches nothing.
std::mutex table_lock;
std::unordered_map<uint32_t, Ring *> &table() {
    static std::unordered_map<uint32_t, Ring *> t;
    return t;
}
uint32_t next_number = 1;

}  // namespace

Action collect_action(Phase phase, Done done) {
    switch (phase) {
    case Phase::SUBMITTED:
        return done == Done::OK ? Action::READ : done == Done::FAILED ? Action::DROP : Action::WAIT;
    case Phase::INVALID:
        return done == Done::PENDING ? Action::WAIT : Action::DROP;
    default:  // FREE, RECORDING, ENCODED, HELD
        return Action::WAIT;
    }
}

Ring::Ring(uint32_t depth)
    : depth_(depth == 0 ? 1 : depth > RING_MAX_DEPTH ? RING_MAX_DEPTH : depth),
      ticket_(new std::atomic<uint64_t>[RING_MAX_DEPTH]),
      verdict_(new std::atomic<uint64_t>[RING_MAX_DEPTH]) {
    for (uint32_t i = 0; i < RING_MAX_DEPTH; i++) {
        phase_[i] = Phase::FREE;
        order_[i] = 0;
        ticket_[i].store(0, std::memory_order_relaxed);
        verdict_[i].store(0, std::memory_order_relaxed);
    }
    std::lock_guard<std::mutex> g(table_lock);
    auto &t = table();
    // Numbers wrap after 2^22 - 1 rings; skip any still live.
    do {
        id_ = next_number;
        next_number = next_number + 1 == (1u << RING_BITS) ? 1 : next_number + 1;
    } while (t.count(id_));
    t[id_] = this;
}

Ring::~Ring() {
    std::lock_guard<std::mutex> g(table_lock);
    table().erase(id_);
}

uint64_t Ring::make_id(uint32_t slot) {
    serial_++;
    return ((uint64_t)id_ << 40) | ((serial_ & 0xffffffffull) << 8) | slot;
}

bool Ring::abandoned(uint32_t slot) const {
    return phase_[slot] == Phase::ENCODED && (ticket_[slot].load(std::memory_order_acquire) & ABANDONED);
}

int Ring::claim() {
    for (uint32_t i = 0; i < depth_; i++) {
        if (abandoned(i)) {
            release(i);
            reclaimed_++;
        }
    }
    const uint32_t slot = cursor_;
    if (phase_[slot] != Phase::FREE) return -1;
    phase_[slot] = Phase::RECORDING;
    cursor_ = (slot + 1) % depth_;
    return (int)slot;
}

uint64_t Ring::encode(uint32_t slot) {
    if (slot >= depth_ || phase_[slot] != Phase::RECORDING) return 0;
    const uint64_t t = make_id(slot);
    ticket_[slot].store(t, std::memory_order_release);
    phase_[slot] = Phase::ENCODED;
    return t;
}

int Ring::submit(uint64_t ticket) {
    if (ticket == 0 || (ticket & ABANDONED)) return -1;
    if (ring_of(ticket) != id_) {
        // Spent here all the same: its own ring frees the slot unread.
        drop_ticket(ticket);
        return -1;
    }
    const uint32_t slot = slot_of(ticket);
    if (slot >= depth_ || phase_[slot] != Phase::ENCODED) return -1;
    uint64_t expect = ticket;
    // Fails for an earlier lap's ticket and for one dropped meanwhile.
    if (!ticket_[slot].compare_exchange_strong(expect, 0, std::memory_order_acq_rel)) return -1;
    phase_[slot] = Phase::SUBMITTED;
    order_[slot] = ++submissions_;
    return (int)slot;
}

int Ring::submit_held(uint64_t ticket, uint64_t *hold) {
    if (hold) *hold = 0;
    const int slot = submit(ticket);
    if (slot < 0) return -1;
    const uint64_t h = make_id((uint32_t)slot);
    verdict_[slot].store(h | (VERDICT_PENDING << VERDICT_SHIFT), std::memory_order_release);
    phase_[slot] = Phase::HELD;
    if (hold) *hold = h;
    return slot;
}

bool Ring::abandon(uint64_t ticket) {
    const uint32_t slot = slot_of(ticket);
    if (ticket == 0 || (ticket & ABANDONED) || ring_of(ticket) != id_ || slot >= depth_) return false;
    uint64_t expect = ticket;
    return ticket_[slot].compare_exchange_strong(expect, ticket | ABANDONED, std::memory_order_acq_rel);
}

bool Ring::give_verdict(uint64_t hold, bool accepted) {
    const uint32_t slot = slot_of(hold);
    if (hold == 0 || (hold & ~ID_MASK) || ring_of(hold) != id_ || slot >= depth_) return false;
    uint64_t expect = hold | (VERDICT_PENDING << VERDICT_SHIFT);
    const uint64_t v = hold | ((accepted ? VERDICT_ACCEPTED : VERDICT_REJECTED) << VERDICT_SHIFT);
    return verdict_[slot].compare_exchange_strong(expect, v, std::memory_order_acq_rel);
}

void Ring::settle() {
    for (uint32_t i = 0; i < depth_; i++) {
        if (phase_[i] != Phase::HELD) continue;
        const uint64_t v = verdict_[i].load(std::memory_order_acquire) >> VERDICT_SHIFT;
        if (v == VERDICT_PENDING) continue;
        phase_[i] = v == VERDICT_ACCEPTED ? Phase::SUBMITTED : Phase::INVALID;
        verdict_[i].store(0, std::memory_order_release);
    }
}

uint32_t Ring::invalidate() {
    uint32_t moved = 0;
    for (uint32_t i = 0; i < depth_; i++) {
        if (phase_[i] != Phase::SUBMITTED && phase_[i] != Phase::HELD) continue;
        phase_[i] = Phase::INVALID;
        verdict_[i].store(0, std::memory_order_release);  // a late verdict reaches nothing
        moved++;
    }
    return moved;
}

void Ring::release(uint32_t slot) {
    if (slot >= depth_) return;
    phase_[slot] = Phase::FREE;
    ticket_[slot].store(0, std::memory_order_release);
    verdict_[slot].store(0, std::memory_order_release);
}

uint32_t Ring::in_flight() const {
    uint32_t n = 0;
    for (uint32_t i = 0; i < depth_; i++)
        if (phase_[i] != Phase::FREE && !abandoned(i)) n++;
    return n;
}

void drop_ticket(uint64_t ticket) {
    std::lock_guard<std::mutex> g(table_lock);
    auto it = table().find(ring_of(ticket));
    if (it != table().end()) it->second->abandon(ticket);
}

bool give_verdict(uint64_t hold, bool accepted) {
    std::lock_guard<std::mutex> g(table_lock);
    auto it = table().find(ring_of(hold));
    return it != table().end() && it->second->give_verdict(hold, accepted);
}

}  // namespace bl

// ---- C API ----

struct bls_ring {
    bl::Ring ring;
    explicit bls_ring(uint32_t depth) : ring(depth) {}
};

extern "C" {

int bls_ring_new(uint32_t depth, bls_ring **out) {
    if (!out) return BLS_ERR_INVALID;
    *out = nullptr;
    if (depth > bl::RING_MAX_DEPTH) return BLS_ERR_INVALID;
    *out = new bls_ring(depth);
    return BLS_OK;
}

void bls_ring_free(bls_ring *r) { delete r; }
uint32_t bls_ring_depth(const bls_ring *r) { return r ? r->ring.depth() : 0; }
int32_t bls_ring_claim(bls_ring *r) { return r ? r->ring.claim() : -1; }
uint64_t bls_ring_encode(bls_ring *r, uint32_t slot) { return r ? r->ring.encode(slot) : 0; }
int32_t bls_ring_submit(bls_ring *r, uint64_t ticket) { return r ? r->ring.submit(ticket) : -1; }
int32_t bls_ring_submit_held(bls_ring *r, uint64_t ticket, uint64_t *hold) {
    if (hold) *hold = 0;
    return r ? r->ring.submit_held(ticket, hold) : -1;
}
void bls_ticket_drop(uint64_t ticket) { bl::drop_ticket(ticket); }
int bls_hold_verdict(uint64_t hold, uint32_t accepted) { return bl::give_verdict(hold, accepted != 0) ? 1 : 0; }
void bls_ring_settle(bls_ring *r) {
    if (r) r->ring.settle();
}
uint32_t bls_ring_invalidate(bls_ring *r) { return r ? r->ring.invalidate() : 0; }

uint32_t bls_ring_ready(const bls_ring *r, const uint8_t *done, uint32_t *slots, uint8_t *actions) {
    if (!r || !done || !slots || !actions) return 0;
    bl::Action a[bl::RING_MAX_DEPTH];
    const uint32_t n = r->ring.ready(
        [done](uint32_t i) { return done[i] > (uint8_t)bl::Done::FAILED ? bl::Done::PENDING : (bl::Done)done[i]; }, slots, a);
    for (uint32_t i = 0; i < n; i++) actions[i] = (uint8_t)a[i];
    return n;
}

void bls_ring_release(bls_ring *r, uint32_t slot) {
    if (r) r->ring.release(slot);
}
uint32_t bls_ring_in_flight(const bls_ring *r) { return r ? r->ring.in_flight() : 0; }
int32_t bls_ring_phase(const bls_ring *r, uint32_t slot) {
    if (!r || slot >= r->ring.depth()) return -1;
    return (int32_t)r->ring.phase(slot);
}
uint64_t bls_ring_reclaimed(const bls_ring *r) { return r ? r->ring.reclaimed() : 0; }

uint32_t bls_collect_action(uint32_t phase, uint32_t done) {
    if (phase > (uint32_t)bl::Phase::INVALID || done > (uint32_t)bl::Done::FAILED) return BLS_COLLECT_WAIT;
    return (uint32_t)bl::collect_action((bl::Phase)phase, (bl::Done)done);
}

}  // extern "C"
