// Host logic of the demand-backed virtual KV range, independent of the driver
// it runs on.
//
// Behaviour follows the reference's native/elastic_vmm.cpp (semantics of
// Backing::initialize :50-86, ensure_impl :97-153, drop :166-184, close
// :186-215, normalize :235-256, release :258-274 and the ABI :316-369):
//   * ids are checked against the reservation, sorted and de-duplicated, and
//     only those not yet in the wanted state are touched;
//   * a commit creates + maps + grants access chunk by chunk, then starts the
//     zero fill of each contiguous run of new chunks on the object's private
//     stream; a failure rolls back every chunk of the batch (after the zero
//     fills it started have finished), and when a rollback step fails, or the
//     zero fills cannot be waited for, the object is poisoned;
//   * a decommit that fails part-way poisons the object (the chunks released
//     before the failure cannot be restored);
//   * a failed close keeps the object alive so the close can be retried (the
//     one deliberate difference from the reference);
//   * an optional spare pool (off by default; no reference counterpart): up
//     to `spare limit` physical chunks that a decommit unmapped are kept
//     instead of released, and the next commits map them instead of creating
//     new ones (zero-filled like any committed chunk). It saves a create and
//     a release per recycled chunk, whose cost grows with the number of live
//     allocations, and holds that memory until a commit takes it, the limit
//     is lowered, or the object closes.
//
// The driver is a template parameter: HipDriver (vmm_backing.hip) on the GPU,
// a fault-injecting driver in the native tests. A driver provides, with int
// statuses (0 = success):
//   int init(int device, uint64_t* granularity)  device, VMM support, granularity
//   int reserve(uint64_t bytes, uint64_t alignment, uintptr_t* base)
//   int free_range(uintptr_t base, uint64_t bytes)
//   int open_stream(), int close_stream()        the private zero-fill stream
//   int create(uint64_t bytes, uint64_t* handle)
//   int map(uintptr_t address, uint64_t bytes, uint64_t handle)
//   int set_access(uintptr_t address, uint64_t bytes)
//   int unmap(uintptr_t address, uint64_t bytes)
//   int release(uint64_t handle)
//   int zero_async(uintptr_t address, uint64_t bytes)   on the private stream
//   int wait_zero()                              synchronize the private stream
//   int synchronize_device()
//   std::string describe(int status)             name of a failure status
//   Driver::Scope(Driver&)                       makes the device current for its
//                                                lifetime (RAII, never throws;
//                                                int status() reports a failure)
#pragma once

#include "ekv_errors.h"

#include <algorithm>
#include <cstdint>
#include <limits>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace ekv {
namespace vmm {

template <typename Driver>
class Backing {
public:
    Backing(int device, uint64_t capacity_bytes, uint64_t chunk_bytes) {
        if (capacity_bytes == 0 || chunk_bytes == 0) {
            throw std::invalid_argument("capacity and chunk size must be positive");
        }
        if (chunk_bytes % 16 != 0) {
            throw std::invalid_argument("chunk size must be a multiple of 16 bytes");
        }
        const uint64_t chunks = capacity_bytes / chunk_bytes + (capacity_bytes % chunk_bytes != 0);
        if (chunks > std::numeric_limits<uint64_t>::max() / chunk_bytes) {
            throw std::invalid_argument("aligned capacity overflows 64 bits");
        }
        chunk_bytes_ = chunk_bytes;
        reserved_bytes_ = chunks * chunk_bytes;
        check(driver_.init(device, &granularity_), "initialize the device");
        if (granularity_ == 0 || chunk_bytes_ % granularity_ != 0) {
            throw std::invalid_argument("chunk_bytes must be a multiple of VMM granularity " +
                                        std::to_string(granularity_));
        }
        typename Driver::Scope scope(driver_);
        check(scope.status(), "select the device");
        // A power-of-two chunk size aligns the reservation to it, so every
        // chunk can use the largest page that fits it.
        const bool power_of_two = (chunk_bytes_ & (chunk_bytes_ - 1)) == 0;
        check(driver_.reserve(reserved_bytes_, power_of_two ? chunk_bytes_ : granularity_, &base_),
              "hipMemAddressReserve");
        const int stream = driver_.open_stream();
        if (stream != 0) {
            (void)driver_.free_range(base_, reserved_bytes_);
            base_ = 0;
            check(stream, "hipStreamCreateWithFlags");
        }
        stream_open_ = true;
        open_ = true;
    }

    ~Backing() { (void)close(); }

    Backing(const Backing&) = delete;
    Backing& operator=(const Backing&) = delete;

    // ensure (wait = true) and precommit (wait = false).
    void commit(const uint64_t* ids, size_t count, bool wait) {
        const std::vector<uint64_t> fresh = pending(ids, count, /*want_mapped=*/false);
        typename Driver::Scope scope(driver_);
        check(scope.status(), "select the device");
        if (fresh.empty()) {
            if (wait) {
                wait_for_zero();
            }
            return;
        }
        size_t touched = 0;  // chunks of this batch that may own resources
        try {
            for (const uint64_t id : fresh) {
                Chunk& chunk = chunks_[id];
                ++touched;
                if (!spare_.empty()) {
                    chunk.handle = spare_.back();   // a rollback releases it like a created one
                    spare_.pop_back();
                } else {
                    check(driver_.create(chunk_bytes_, &chunk.handle), "hipMemCreate");
                }
                chunk.created = true;
                check(driver_.map(address(id), chunk_bytes_, chunk.handle), "hipMemMap");
                chunk.mapped = true;
                check(driver_.set_access(address(id), chunk_bytes_), "hipMemSetAccess");
            }
            // Zero each contiguous run of new chunks with one fill.
            for (size_t begin = 0; begin < fresh.size();) {
                size_t end = begin + 1;
                while (end < fresh.size() && fresh[end] == fresh[end - 1] + 1) {
                    ++end;
                }
                check(driver_.zero_async(address(fresh[begin]), (end - begin) * chunk_bytes_), "launch zero fill");
                zero_pending_ = true;
                begin = end;
            }
            if (wait) {
                wait_for_zero();
            }
        } catch (...) {
            // Never release memory whose zero fill might still be running.
            if (zero_pending_) {
                if (driver_.wait_zero() != 0) {
                    poisoned_ = true;
                    throw;
                }
                zero_pending_ = false;
            }
            while (touched > 0) {
                const uint64_t id = fresh[--touched];
                auto it = chunks_.find(id);
                if (release(id, it->second) == 0) {
                    chunks_.erase(it);
                } else {
                    poisoned_ = true;
                }
            }
            throw;
        }
    }

    void decommit(const uint64_t* ids, size_t count) {
        const std::vector<uint64_t> mapped = pending(ids, count, /*want_mapped=*/true);
        if (mapped.empty()) {
            return;
        }
        typename Driver::Scope scope(driver_);
        check(scope.status(), "select the device");
        wait_for_zero();
        for (const uint64_t id : mapped) {
            auto it = chunks_.find(id);
            const int status = release(id, it->second, /*keep_spare=*/true);
            if (status != 0) {
                // Earlier chunks of this call are gone already; the caller
                // must tear the object down.
                poisoned_ = true;
                check(status, "decommit chunk");
            }
            chunks_.erase(it);
        }
    }

    // Releases everything; returns the first failure (0 if none). Safe to call again.
    int close() noexcept {
        if (!open_) {
            return 0;
        }
        int first = 0;
        auto record = [&first](int status) {
            if (first == 0 && status != 0) {
                first = status;
            }
        };
        {
            typename Driver::Scope scope(driver_);
            record(scope.status());
            if (first == 0) {
                record(driver_.synchronize_device());
            }
            if (first == 0) {
                zero_pending_ = false;
                for (auto it = chunks_.begin(); it != chunks_.end();) {
                    const int status = release(it->first, it->second);
                    record(status);
                    it = status == 0 ? chunks_.erase(it) : std::next(it);
                }
                spare_limit_ = 0;
                record(release_spares(0));
                if (chunks_.empty() && spare_.empty() && base_) {
                    const int status = driver_.free_range(base_, reserved_bytes_);
                    record(status);
                    if (status == 0) {
                        base_ = 0;
                    }
                }
                if (base_ == 0 && stream_open_) {
                    const int status = driver_.close_stream();
                    record(status);
                    stream_open_ = status != 0;
                }
                if (base_ == 0 && !stream_open_) {
                    open_ = false;
                }
            }
        }
        if (first != 0) {
            poisoned_ = true;
        }
        return first;
    }

    // A close failure as an exception carrying the driver's name for it.
    void close_or_throw() {
        const int status = close();
        if (status != 0) {
            check(status, "close backing");
        }
    }

    // Keep up to `chunks` decommitted physical chunks for reuse (0 = release
    // every decommitted chunk at once, the reference's behaviour). Lowering
    // the limit releases the chunks held above it.
    void set_spare_limit(uint64_t chunks) {
        if (!open_) {
            throw std::runtime_error("backing is closed");
        }
        if (poisoned_) {
            throw std::runtime_error("backing is poisoned after a partial HIP failure");
        }
        if (chunks > reserved_bytes_ / chunk_bytes_) {
            throw std::invalid_argument("spare limit exceeds the reservation's chunk count");
        }
        typename Driver::Scope scope(driver_);
        check(scope.status(), "select the device");
        spare_.reserve(static_cast<size_t>(chunks));   // a decommit then never allocates to keep one
        spare_limit_ = chunks;
        const int status = release_spares(static_cast<size_t>(chunks));
        if (status != 0) {
            poisoned_ = true;
            check(status, "release spare chunk");
        }
    }

    uint64_t spare() const { return static_cast<uint64_t>(spare_.size()) * chunk_bytes_; }

    uint64_t base() const { return base_; }
    uint64_t granularity() const { return granularity_; }
    uint64_t reserved() const { return reserved_bytes_; }
    bool poisoned() const { return poisoned_; }

    uint64_t backed() const {
        uint64_t committed = 0;
        for (const auto& entry : chunks_) {
            committed += entry.second.created || entry.second.mapped;
        }
        return committed * chunk_bytes_;
    }

private:
    struct Chunk {
        uint64_t handle = 0;
        bool created = false;
        bool mapped = false;
    };

    uintptr_t address(uint64_t id) const { return base_ + id * chunk_bytes_; }

    void check(int status, const char* what) {
        if (status != 0) {
            throw std::runtime_error(std::string(what) + ": " + driver_.describe(status));
        }
    }

    void wait_for_zero() {
        if (!zero_pending_) {
            return;
        }
        check(driver_.wait_zero(), "wait for backing initialization");
        zero_pending_ = false;
    }

    // Sorted, de-duplicated ids whose mapped state equals `want_mapped`.
    std::vector<uint64_t> pending(const uint64_t* ids, size_t count, bool want_mapped) const {
        if (!open_) {
            throw std::runtime_error("backing is closed");
        }
        if (poisoned_) {
            throw std::runtime_error("backing is poisoned after a partial HIP failure");
        }
        if (count != 0 && ids == nullptr) {
            throw std::invalid_argument("chunk index array is null");
        }
        const uint64_t limit = reserved_bytes_ / chunk_bytes_;
        std::vector<uint64_t> result;
        result.reserve(count);
        for (size_t i = 0; i < count; ++i) {
            if (ids[i] >= limit) {
                throw std::out_of_range("chunk index outside reserved range");
            }
            if ((chunks_.count(ids[i]) != 0) == want_mapped) {
                result.push_back(ids[i]);
            }
        }
        std::sort(result.begin(), result.end());
        result.erase(std::unique(result.begin(), result.end()), result.end());
        return result;
    }

    // Unmaps and releases a chunk; with keep_spare, a created chunk goes to
    // the spare pool instead while it holds fewer than the limit.
    int release(uint64_t id, Chunk& chunk, bool keep_spare = false) noexcept {
        if (chunk.mapped) {
            const int status = driver_.unmap(address(id), chunk_bytes_);
            if (status != 0) {
                return status;
            }
            chunk.mapped = false;
        }
        if (chunk.created && keep_spare && spare_.size() < spare_limit_) {
            spare_.push_back(chunk.handle);   // capacity reserved by set_spare_limit
            chunk.created = false;
            return 0;
        }
        if (chunk.created) {
            const int status = driver_.release(chunk.handle);
            if (status != 0) {
                return status;
            }
            chunk.created = false;
        }
        return 0;
    }

    // Releases spare chunks until at most `keep` remain; the first failure (0 if none).
    int release_spares(size_t keep) noexcept {
        while (spare_.size() > keep) {
            const int status = driver_.release(spare_.back());
            if (status != 0) {
                return status;
            }
            spare_.pop_back();
        }
        return 0;
    }

    Driver driver_;
    uintptr_t base_ = 0;
    uint64_t reserved_bytes_ = 0;
    uint64_t chunk_bytes_ = 0;
    uint64_t granularity_ = 0;
    bool zero_pending_ = false;
    bool poisoned_ = false;
    bool stream_open_ = false;
    bool open_ = false;
    std::map<uint64_t, Chunk> chunks_;
    std::vector<uint64_t> spare_;   // unmapped physical chunks kept for reuse
    uint64_t spare_limit_ = 0;
};

constexpr uint64_t kInvalid = std::numeric_limits<uint64_t>::max();

// The ev_* C ABI over Backing<Driver> (native/elastic_vmm.cpp:316-369): no
// exception crosses it; failures return NULL, -1 or UINT64_MAX and leave a
// message for ev_error().
template <typename Driver>
struct Abi {
    using Object = Backing<Driver>;

    static Object& require(void* handle) {
        if (handle == nullptr) {
            throw std::invalid_argument("null backing handle");
        }
        return *static_cast<Object*>(handle);
    }

    static void* create(int device, uint64_t capacity_bytes, uint64_t chunk_bytes) {
        return guarded(static_cast<void*>(nullptr), [&] {
            auto backing = std::make_unique<Object>(device, capacity_bytes, chunk_bytes);
            return static_cast<void*>(backing.release());
        });
    }
    static int ensure(void* handle, const uint64_t* ids, size_t count) {
        return guarded(-1, [&] {
            require(handle).commit(ids, count, true);
            return 0;
        });
    }
    static int precommit(void* handle, const uint64_t* ids, size_t count) {
        return guarded(-1, [&] {
            require(handle).commit(ids, count, false);
            return 0;
        });
    }
    static int drop(void* handle, const uint64_t* ids, size_t count) {
        return guarded(-1, [&] {
            require(handle).decommit(ids, count);
            return 0;
        });
    }
    static uint64_t base(void* handle) {
        return guarded(kInvalid, [&] { return require(handle).base(); });
    }
    static uint64_t backed(void* handle) {
        return guarded(kInvalid, [&] { return require(handle).backed(); });
    }
    static uint64_t reserved(void* handle) {
        return guarded(kInvalid, [&] { return require(handle).reserved(); });
    }
    static uint64_t granularity(void* handle) {
        return guarded(kInvalid, [&] { return require(handle).granularity(); });
    }
    static int poisoned(void* handle) {
        return guarded(-1, [&] { return require(handle).poisoned() ? 1 : 0; });
    }
    static int set_spare(void* handle, uint64_t chunks) {
        return guarded(-1, [&] {
            require(handle).set_spare_limit(chunks);
            return 0;
        });
    }
    static uint64_t spare(void* handle) {
        return guarded(kInvalid, [&] { return require(handle).spare(); });
    }
    static int close(void* handle) {
        return guarded(-1, [&] {
            if (handle == nullptr) {
                return 0;
            }
            auto* backing = static_cast<Object*>(handle);
            backing->close_or_throw();   // on failure the object stays alive for a retry
            delete backing;
            return 0;
        });
    }
};

}  // namespace vmm
}  // namespace ekv

// Defines the extern "C" ev_* entry points of include/elastic_vmm.h over
// Backing<DRIVER>, and the thread-local error message they share.
#define EKV_DEFINE_VMM_ABI(DRIVER)                                                                            \
    namespace ekv {                                                                                           \
    std::string& last_error() {                                                                               \
        thread_local std::string message;                                                                     \
        return message;                                                                                       \
    }                                                                                                         \
    }                                                                                                         \
    extern "C" {                                                                                              \
    void* ev_create(int device, uint64_t capacity_bytes, uint64_t chunk_bytes) {                              \
        return ::ekv::vmm::Abi<DRIVER>::create(device, capacity_bytes, chunk_bytes);                          \
    }                                                                                                         \
    int ev_ensure(void* handle, const uint64_t* indices, size_t count) {                                      \
        return ::ekv::vmm::Abi<DRIVER>::ensure(handle, indices, count);                                       \
    }                                                                                                         \
    int ev_precommit(void* handle, const uint64_t* indices, size_t count) {                                   \
        return ::ekv::vmm::Abi<DRIVER>::precommit(handle, indices, count);                                    \
    }                                                                                                         \
    int ev_drop(void* handle, const uint64_t* indices, size_t count) {                                        \
        return ::ekv::vmm::Abi<DRIVER>::drop(handle, indices, count);                                         \
    }                                                                                                         \
    uint64_t ev_base(void* handle) { return ::ekv::vmm::Abi<DRIVER>::base(handle); }                          \
    uint64_t ev_backed(void* handle) { return ::ekv::vmm::Abi<DRIVER>::backed(handle); }                      \
    uint64_t ev_reserved(void* handle) { return ::ekv::vmm::Abi<DRIVER>::reserved(handle); }                  \
    uint64_t ev_granularity(void* handle) { return ::ekv::vmm::Abi<DRIVER>::granularity(handle); }            \
    int ev_poisoned(void* handle) { return ::ekv::vmm::Abi<DRIVER>::poisoned(handle); }                       \
    int ev_set_spare(void* handle, uint64_t chunks) { return ::ekv::vmm::Abi<DRIVER>::set_spare(handle, chunks); } \
    uint64_t ev_spare(void* handle) { return ::ekv::vmm::Abi<DRIVER>::spare(handle); }                        \
    const char* ev_error(void) { return ::ekv::last_error().c_str(); }                                        \
    int ev_close(void* handle) { return ::ekv::vmm::Abi<DRIVER>::close(handle); }                             \
    }
