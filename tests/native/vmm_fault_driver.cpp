// A fault-injecting VMM driver for the host logic of csrc/vmm_core.h (test
// infrastructure, host only: built with g++, never with hipcc).
//
// It stands in for HIP's virtual memory calls with bookkeeping of its own -
// reservations, physical handles, mappings, access grants and zero fills in
// flight - and can fail the k-th call of any operation. It also checks the
// contract the core must keep with a real driver and counts every breach:
// mapping a live address twice, releasing a handle that is still mapped,
// unmapping or releasing memory whose zero fill might still run, zero-filling
// memory without access, freeing a reservation that still has mappings.
// The ev_* C ABI of include/elastic_vmm.h is defined over it, plus fake_*
// controls for the tests.
#include "vmm_core.h"

#include <cstdio>
#include <map>
#include <set>
#include <string>

namespace fake {

enum Op {
    kReserve, kFree, kOpenStream, kCloseStream, kCreate, kMap, kSetAccess, kUnmap, kRelease,
    kZero, kWaitZero, kSync, kOps
};
const char* const kOpNames[kOps] = {"reserve", "free", "open_stream", "close_stream", "create", "map",
                                    "set_access", "unmap", "release", "zero", "wait_zero", "sync"};
constexpr uint64_t kGranularity = 4096;
constexpr int kFailureBase = 100;   // status of an injected failure of op o: kFailureBase + o

struct World {
    long calls[kOps] = {};
    long fail_at[kOps] = {};     // call number (1-based) that fails; 0 = none
    bool fail_after[kOps] = {};  // ... and every later call too
    std::map<uintptr_t, uint64_t> ranges;      // reservation base -> bytes
    std::set<uint64_t> handles;                // live physical handles
    std::map<uintptr_t, uint64_t> maps;        // mapped chunk address -> handle
    std::set<uintptr_t> granted;               // mapped chunk addresses with access
    std::map<uintptr_t, uint64_t> zeroing;     // zero fills in flight: address -> bytes
    long violations = 0;
    std::string last_violation;
    uint64_t next_handle = 1;
    uintptr_t next_base = uintptr_t{1} << 40;
};

World& world() {
    static World w;
    return w;
}

void violate(const std::string& what) {
    ++world().violations;
    world().last_violation = what;
    std::fprintf(stderr, "contract violation: %s\n", what.c_str());
}

int inject(Op op) {
    World& w = world();
    const long n = ++w.calls[op];
    if (w.fail_at[op] != 0 && (n == w.fail_at[op] || (w.fail_after[op] && n > w.fail_at[op]))) {
        return kFailureBase + op;
    }
    return 0;
}

bool overlaps_zeroing(uintptr_t address, uint64_t bytes) {
    for (const auto& fill : world().zeroing) {
        if (address < fill.first + fill.second && fill.first < address + bytes) {
            return true;
        }
    }
    return false;
}

class FakeDriver {
public:
    class Scope {
    public:
        explicit Scope(FakeDriver&) {}
        int status() const { return 0; }
    };

    int init(int device, uint64_t* granularity) {
        if (device != 0) {
            throw std::invalid_argument("device ordinal " + std::to_string(device) + " out of range (1 devices)");
        }
        *granularity = kGranularity;
        return 0;
    }
    int reserve(uint64_t bytes, uint64_t alignment, uintptr_t* base) {
        if (const int s = inject(kReserve)) {
            return s;
        }
        World& w = world();
        const uintptr_t start = (w.next_base + alignment - 1) / alignment * alignment;
        w.next_base = start + bytes + alignment;
        w.ranges[start] = bytes;
        *base = start;
        return 0;
    }
    int free_range(uintptr_t base, uint64_t bytes) {
        if (const int s = inject(kFree)) {
            return s;
        }
        World& w = world();
        auto it = w.ranges.find(base);
        if (it == w.ranges.end() || it->second != bytes) {
            violate("free of an unknown reservation");
            return 0;
        }
        for (const auto& m : w.maps) {
            if (m.first >= base && m.first < base + bytes) {
                violate("reservation freed while a chunk is mapped");
                break;
            }
        }
        w.ranges.erase(it);
        return 0;
    }
    int open_stream() {
        if (const int s = inject(kOpenStream)) {
            return s;
        }
        ++streams_;
        return 0;
    }
    int close_stream() {
        if (const int s = inject(kCloseStream)) {
            return s;
        }
        if (streams_-- <= 0) {
            violate("stream closed twice");
        }
        world().zeroing.clear();
        return 0;
    }
    int create(uint64_t bytes, uint64_t* handle) {
        if (const int s = inject(kCreate)) {
            return s;
        }
        if (bytes % kGranularity != 0) {
            violate("create of a size that is not a multiple of the granularity");
        }
        *handle = world().next_handle++;
        world().handles.insert(*handle);
        return 0;
    }
    int map(uintptr_t address, uint64_t, uint64_t handle) {
        if (const int s = inject(kMap)) {
            return s;
        }
        World& w = world();
        if (!w.handles.count(handle)) {
            violate("map of a released handle");
        }
        if (!w.maps.emplace(address, handle).second) {
            violate("map of an address that is already mapped");
        }
        return 0;
    }
    int set_access(uintptr_t address, uint64_t) {
        if (const int s = inject(kSetAccess)) {
            return s;
        }
        if (!world().maps.count(address)) {
            violate("access granted to an unmapped address");
        }
        world().granted.insert(address);
        return 0;
    }
    int unmap(uintptr_t address, uint64_t bytes) {
        if (const int s = inject(kUnmap)) {
            return s;
        }
        World& w = world();
        if (overlaps_zeroing(address, bytes)) {
            violate("unmap while a zero fill of the chunk may still run");
        }
        if (w.maps.erase(address) == 0) {
            violate("unmap of an address that is not mapped");
        }
        w.granted.erase(address);
        return 0;
    }
    int release(uint64_t handle) {
        if (const int s = inject(kRelease)) {
            return s;
        }
        World& w = world();
        for (const auto& m : w.maps) {
            if (m.second == handle) {
                violate("release of a handle that is still mapped");
            }
        }
        if (w.handles.erase(handle) == 0) {
            violate("release of an unknown handle");
        }
        return 0;
    }
    int zero_async(uintptr_t address, uint64_t bytes) {
        if (const int s = inject(kZero)) {
            return s;
        }
        World& w = world();
        for (uint64_t offset = 0; offset < bytes; offset += chunk_hint_) {
            if (!w.granted.count(address + offset)) {
                violate("zero fill of memory without access");
                break;
            }
        }
        w.zeroing[address] = bytes;
        return 0;
    }
    int wait_zero() {
        if (const int s = inject(kWaitZero)) {
            return s;
        }
        world().zeroing.clear();
        return 0;
    }
    int synchronize_device() {
        if (const int s = inject(kSync)) {
            return s;
        }
        world().zeroing.clear();
        return 0;
    }
    std::string describe(int status) const {
        const int op = status - kFailureBase;
        if (op < 0 || op >= kOps) {
            return "fakeErrorUnknown (status " + std::to_string(status) + ")";
        }
        return std::string("fakeError_") + kOpNames[op] + " (injected " + kOpNames[op] + " failure)";
    }

    static uint64_t chunk_hint_;   // chunk size of the test's objects: the access check's step

private:
    int streams_ = 0;
};

uint64_t FakeDriver::chunk_hint_ = kGranularity;

}  // namespace fake

EKV_DEFINE_VMM_ABI(fake::FakeDriver)

extern "C" {

// Clears call counts and planned failures (live resources are kept).
void fake_reset(void) {
    fake::World& w = fake::world();
    for (int op = 0; op < fake::kOps; ++op) {
        w.calls[op] = 0;
        w.fail_at[op] = 0;
        w.fail_after[op] = false;
    }
}

// The `nth` next call of `op` fails (1 = the next one); with `after`, every later one too.
void fake_fail(int op, long nth, int after) {
    fake::World& w = fake::world();
    w.fail_at[op] = w.calls[op] + nth;
    w.fail_after[op] = after != 0;
}

// Chunk size of the objects under test (the step of the zero-fill access check).
void fake_set_chunk(uint64_t bytes) { fake::FakeDriver::chunk_hint_ = bytes; }

long fake_calls(int op) { return fake::world().calls[op]; }
long fake_live_handles(void) { return static_cast<long>(fake::world().handles.size()); }
long fake_live_maps(void) { return static_cast<long>(fake::world().maps.size()); }
long fake_live_ranges(void) { return static_cast<long>(fake::world().ranges.size()); }
long fake_zero_in_flight(void) { return static_cast<long>(fake::world().zeroing.size()); }
long fake_violations(void) { return fake::world().violations; }
const char* fake_last_violation(void) { return fake::world().last_violation.c_str(); }

}  // extern "C"
