// Failure paths of the VMM host logic (csrc/vmm_core.h), driven through the
// ev_* C ABI over the fault-injecting driver of vmm_fault_driver.cpp.
// Test infrastructure: built with g++ and AddressSanitizer + UBSan by
// tests/test_vmm_fault_injection.py; exits 0 when every case passes.
//
// The contract under test is the reference's native/elastic_vmm.cpp:
//   :97-153  a failed batch rolls back the chunks it created, after the zero
//            fills it started have finished; a rollback that fails poisons;
//   :166-184 a decommit that fails part-way poisons;
//   :186-215 close releases everything (this library keeps the object alive
//            when that fails, so the close can be retried);
//   :235-256 ids outside the reservation and NULL id arrays fail before any
//            driver call; duplicates are ignored.
#include "../../include/elastic_vmm.h"

#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

extern "C" {
void fake_reset(void);
void fake_fail(int op, long nth, int after);
void fake_set_chunk(uint64_t bytes);
long fake_calls(int op);
long fake_live_handles(void);
long fake_live_maps(void);
long fake_live_ranges(void);
long fake_zero_in_flight(void);
long fake_violations(void);
const char* fake_last_violation(void);
}

namespace {

enum Op { kReserve, kFree, kOpenStream, kCloseStream, kCreate, kMap, kSetAccess, kUnmap, kRelease, kZero,
          kWaitZero, kSync };

constexpr uint64_t kChunk = 2 << 20;
int failures = 0;
const char* current = "";

#define CHECK(cond)                                                                              \
    do {                                                                                         \
        if (!(cond)) {                                                                           \
            std::fprintf(stderr, "FAIL [%s] %s:%d: %s (ev_error: %s)\n", current, __FILE__,   \
                         __LINE__, #cond, ev_error());                                           \
            ++failures;                                                                          \
        }                                                                                        \
    } while (0)

bool error_has(const char* text) { return std::strstr(ev_error(), text) != nullptr; }

int ensure(void* h, std::vector<uint64_t> ids) { return ev_ensure(h, ids.data(), ids.size()); }
int precommit(void* h, std::vector<uint64_t> ids) { return ev_precommit(h, ids.data(), ids.size()); }
int drop(void* h, std::vector<uint64_t> ids) { return ev_drop(h, ids.data(), ids.size()); }

void* open_backing(uint64_t chunks) {
    fake_reset();
    void* h = ev_create(0, chunks * kChunk, kChunk);
    CHECK(h != nullptr);
    return h;
}

// Every resource is gone and the driver saw no contract breach.
void expect_clean() {
    CHECK(fake_live_handles() == 0);
    CHECK(fake_live_maps() == 0);
    CHECK(fake_live_ranges() == 0);
    CHECK(fake_violations() == 0);
}

void basic_bookkeeping() {
    current = "basic";
    void* h = open_backing(8);
    CHECK(ev_reserved(h) == 8 * kChunk && ev_granularity(h) == 4096 && ev_base(h) % kChunk == 0);
    CHECK(ensure(h, {0, 1, 2, 2, 1}) == 0);                      // duplicates ignored
    CHECK(fake_calls(kCreate) == 3 && ev_backed(h) == 3 * kChunk);
    CHECK(fake_calls(kZero) == 1);                                // one fill for the run 0..2
    CHECK(ensure(h, {1, 2}) == 0 && fake_calls(kCreate) == 3);   // already mapped: no-op
    CHECK(precommit(h, {3, 5}) == 0 && fake_zero_in_flight() == 2);
    CHECK(ensure(h, {}) == 0 && fake_zero_in_flight() == 0);     // the readiness barrier
    CHECK(drop(h, {1, 7}) == 0 && ev_backed(h) == 4 * kChunk);   // 7 was never mapped
    CHECK(ev_poisoned(h) == 0);
    CHECK(ev_close(h) == 0);
    expect_clean();
}

void rejects_bad_ids_before_any_call() {
    current = "bad ids";
    void* h = open_backing(4);
    const long creates = fake_calls(kCreate);
    CHECK(ensure(h, {0, 4}) == -1 && error_has("outside reserved range"));
    CHECK(ev_ensure(h, nullptr, 2) == -1 && error_has("null"));
    CHECK(ev_drop(h, nullptr, 0) == 0);
    CHECK(fake_calls(kCreate) == creates && ev_backed(h) == 0 && ev_poisoned(h) == 0);
    CHECK(ev_ensure(nullptr, nullptr, 0) == -1 && error_has("null backing handle"));
    CHECK(ev_base(nullptr) == UINT64_MAX && ev_poisoned(nullptr) == -1);
    CHECK(ev_close(nullptr) == 0);
    CHECK(ev_close(h) == 0);
    expect_clean();
}

// A failure at the `nth` call of `op` while committing chunks 0, 1, 2 rolls
// the batch back cleanly; the object stays usable.
void clean_rollback(Op op, long nth, const char* what) {
    current = what;
    void* h = open_backing(4);
    CHECK(ensure(h, {3}) == 0);                                   // an earlier batch survives
    fake_fail(op, nth, 0);
    CHECK(ensure(h, {0, 1, 2}) == -1);
    CHECK(error_has("injected"));
    CHECK(ev_poisoned(h) == 0);
    CHECK(ev_backed(h) == kChunk);
    CHECK(fake_live_handles() == 1 && fake_live_maps() == 1);
    CHECK(fake_violations() == 0);
    fake_reset();
    CHECK(ensure(h, {0, 1, 2}) == 0 && ev_backed(h) == 4 * kChunk);   // retry works
    CHECK(ev_close(h) == 0);
    expect_clean();
}

void rollback_waits_for_started_fills() {
    current = "rollback after a started fill";
    void* h = open_backing(4);
    fake_fail(kZero, 2, 0);                 // runs {0} and {2}: the second launch fails
    CHECK(ensure(h, {0, 2}) == -1 && error_has("launch zero fill"));
    CHECK(ev_poisoned(h) == 0 && ev_backed(h) == 0);
    CHECK(fake_calls(kWaitZero) == 1);     // the first fill was waited for before unmapping
    CHECK(fake_violations() == 0);
    CHECK(ev_close(h) == 0);
    expect_clean();
}

void precommitted_chunks_survive_a_later_failure() {
    current = "precommit then failure";
    void* h = open_backing(4);
    CHECK(precommit(h, {0}) == 0 && fake_zero_in_flight() == 1);
    fake_fail(kCreate, 1, 0);
    CHECK(ensure(h, {1}) == -1 && error_has("hipMemCreate"));
    CHECK(ev_poisoned(h) == 0 && ev_backed(h) == kChunk);        // chunk 0 belongs to an earlier batch
    CHECK(fake_violations() == 0);
    CHECK(drop(h, {0}) == 0 && fake_violations() == 0);          // drop waits for the fill first
    CHECK(ev_close(h) == 0);
    expect_clean();
}

void drop_waits_for_a_precommit_fill() {
    current = "drop after precommit";
    void* h = open_backing(4);
    CHECK(precommit(h, {0, 1}) == 0 && fake_zero_in_flight() == 1);
    CHECK(drop(h, {1}) == 0 && fake_zero_in_flight() == 0);
    CHECK(fake_calls(kWaitZero) == 1 && fake_violations() == 0);
    CHECK(ev_close(h) == 0);
    expect_clean();
}

void failed_rollback_poisons() {
    current = "failed rollback";
    void* h = open_backing(4);
    fake_fail(kMap, 3, 0);
    fake_fail(kUnmap, 1, 0);               // rollback of chunk 1 fails; chunk 0 still rolls back
    CHECK(ensure(h, {0, 1, 2}) == -1 && error_has("hipMemMap"));
    CHECK(ev_poisoned(h) == 1);
    CHECK(ev_backed(h) == kChunk);         // chunk 1 keeps its mapping
    CHECK(ensure(h, {3}) == -1 && error_has("poisoned"));
    CHECK(precommit(h, {3}) == -1 && drop(h, {1}) == -1 && error_has("poisoned"));
    CHECK(fake_violations() == 0);
    CHECK(ev_close(h) == 0);               // teardown still releases everything
    expect_clean();
}

void unwaitable_fill_poisons_without_releasing() {
    current = "unwaitable fill";
    void* h = open_backing(4);
    fake_fail(kWaitZero, 1, 1);            // every wait fails from now on
    CHECK(ensure(h, {0, 1}) == -1 && error_has("wait for backing initialization"));
    CHECK(ev_poisoned(h) == 1);
    CHECK(ev_backed(h) == 2 * kChunk);     // never released under a fill that may still run
    CHECK(fake_violations() == 0);
    CHECK(ev_close(h) == 0);               // the device synchronize completes the fills
    expect_clean();
}

void partial_decommit_poisons(Op op, const char* what) {
    current = what;
    void* h = open_backing(4);
    CHECK(ensure(h, {0, 1, 2, 3}) == 0);
    fake_fail(op, 2, 0);
    CHECK(drop(h, {0, 1, 2, 3}) == -1 && error_has("decommit chunk"));
    CHECK(ev_poisoned(h) == 1);
    CHECK(ev_backed(h) == 3 * kChunk);     // chunk 0 is gone, 1 failed, 2 and 3 were not reached
    CHECK(ensure(h, {0}) == -1 && error_has("poisoned"));
    CHECK(fake_violations() == 0);
    CHECK(ev_close(h) == 0);
    expect_clean();
}

void failed_close_can_be_retried(Op op, const char* what) {
    current = what;
    void* h = open_backing(4);
    CHECK(ensure(h, {0, 1}) == 0);
    fake_fail(op, 1, 0);
    CHECK(ev_close(h) == -1 && error_has("close backing") && error_has("injected"));
    CHECK(ev_backed(h) != UINT64_MAX);     // the object is still alive
    CHECK(ev_poisoned(h) == 1);
    fake_reset();
    CHECK(ev_close(h) == 0);
    expect_clean();
}

// The spare pool: dropped chunks up to the limit keep their physical memory,
// later commits map it instead of creating (and zero it like new chunks),
// lowering the limit and close release it, and a commit that fails after
// taking a spare chunk releases it with the rest of its batch.
void spare_pool() {
    current = "spare pool";
    void* h = open_backing(8);
    CHECK(ev_spare(h) == 0);
    CHECK(ev_set_spare(h, 9) == -1 && error_has("chunk count"));
    CHECK(ev_set_spare(h, 3) == 0);
    CHECK(ensure(h, {0, 1, 2, 3, 4}) == 0);
    CHECK(fake_calls(kCreate) == 5);
    CHECK(drop(h, {1, 2, 3, 4}) == 0);                       // three kept, one released
    CHECK(ev_spare(h) == 3 * kChunk && ev_backed(h) == kChunk);
    CHECK(fake_calls(kRelease) == 1 && fake_live_handles() == 4 && fake_live_maps() == 1);
    const long zeros = fake_calls(kZero);
    CHECK(ensure(h, {5, 6}) == 0);                           // both from the pool
    CHECK(fake_calls(kCreate) == 5 && ev_spare(h) == kChunk && ev_backed(h) == 3 * kChunk);
    CHECK(fake_calls(kZero) == zeros + 1);                   // one run, zero-filled like new chunks
    CHECK(ensure(h, {7}) == 0 && ev_spare(h) == 0);           // the last spare
    CHECK(ensure(h, {2}) == 0 && fake_calls(kCreate) == 6);   // pool empty: created
    // a failed batch releases the spare chunk it had taken
    CHECK(drop(h, {5, 6}) == 0 && ev_spare(h) == 2 * kChunk);
    const long released = fake_calls(kRelease);
    fake_fail(kMap, 2, 0);                                    // the batch's second map fails
    CHECK(ensure(h, {3, 4}) == -1 && error_has("hipMemMap"));
    CHECK(ev_poisoned(h) == 0 && ev_spare(h) == 0 && ev_backed(h) == 3 * kChunk);
    CHECK(fake_calls(kRelease) == released + 2);
    CHECK(fake_violations() == 0);
    // lowering the limit releases what is held above it
    CHECK(drop(h, {0, 2}) == 0 && ev_spare(h) == 2 * kChunk);
    CHECK(ev_set_spare(h, 1) == 0 && ev_spare(h) == kChunk);
    CHECK(ev_set_spare(h, 0) == 0 && ev_spare(h) == 0);
    const long before = fake_calls(kRelease);
    CHECK(ensure(h, {1}) == 0 && drop(h, {1}) == 0);          // limit 0: released at once
    CHECK(ev_spare(h) == 0 && fake_calls(kRelease) == before + 1);
    // close releases the pool
    CHECK(ev_set_spare(h, 4) == 0 && drop(h, {7}) == 0 && ev_spare(h) == kChunk);
    CHECK(ev_close(h) == 0);
    expect_clean();
    // a release that fails while lowering the limit poisons the object
    h = open_backing(4);
    CHECK(ev_set_spare(h, 2) == 0 && ensure(h, {0, 1}) == 0 && drop(h, {0, 1}) == 0);
    fake_fail(kRelease, 1, 0);
    CHECK(ev_set_spare(h, 0) == -1 && error_has("release spare chunk"));
    CHECK(ev_poisoned(h) == 1 && ensure(h, {2}) == -1);
    fake_reset();
    CHECK(ev_close(h) == 0);
    expect_clean();
    CHECK(ev_set_spare(nullptr, 1) == -1 && ev_spare(nullptr) == UINT64_MAX);
}

void create_failures() {
    current = "create";
    fake_reset();
    fake_fail(kReserve, 1, 0);
    CHECK(ev_create(0, 4 * kChunk, kChunk) == nullptr && error_has("hipMemAddressReserve"));
    fake_fail(kOpenStream, 1, 0);
    CHECK(ev_create(0, 4 * kChunk, kChunk) == nullptr && error_has("hipStreamCreateWithFlags"));
    CHECK(fake_live_ranges() == 0);        // the reservation was given back
    CHECK(ev_create(1, 4 * kChunk, kChunk) == nullptr && error_has("device ordinal"));
    CHECK(ev_create(0, 4 * kChunk, 4096 + 16) == nullptr && error_has("granularity"));
    CHECK(ev_create(0, 0, kChunk) == nullptr && error_has("positive"));
    CHECK(ev_create(0, 4 * kChunk, 8) == nullptr && error_has("multiple of 16"));
    void* h = ev_create(0, 3 * kChunk + 1, kChunk);     // rounded up to whole chunks
    CHECK(h != nullptr && ev_reserved(h) == 4 * kChunk);
    CHECK(ev_close(h) == 0);
    expect_clean();
}

}  // namespace

int main() {
    fake_set_chunk(kChunk);
    basic_bookkeeping();
    rejects_bad_ids_before_any_call();
    clean_rollback(kCreate, 2, "create fails");
    clean_rollback(kMap, 3, "map fails");
    clean_rollback(kSetAccess, 2, "set access fails");
    clean_rollback(kZero, 1, "zero launch fails");
    clean_rollback(kWaitZero, 1, "first wait fails");
    rollback_waits_for_started_fills();
    precommitted_chunks_survive_a_later_failure();
    drop_waits_for_a_precommit_fill();
    failed_rollback_poisons();
    unwaitable_fill_poisons_without_releasing();
    partial_decommit_poisons(kUnmap, "drop: unmap fails");
    partial_decommit_poisons(kRelease, "drop: release fails");
    failed_close_can_be_retried(kUnmap, "close: unmap fails");
    failed_close_can_be_retried(kSync, "close: synchronize fails");
    failed_close_can_be_retried(kFree, "close: free fails");
    failed_close_can_be_retried(kCloseStream, "close: stream fails");
    create_failures();
    spare_pool();
    if (failures != 0) {
        std::fprintf(stderr, "%d check(s) failed; last contract violation: %s\n", failures, fake_last_violation());
        return 1;
    }
    std::printf("all VMM fault cases passed\n");
    return 0;
}
