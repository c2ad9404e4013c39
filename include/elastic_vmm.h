/*
 * elastic_vmm.h - demand-backed virtual KV range on HIP virtual memory.
 *
 * One object owns one stable virtual address reservation on one GPU. Physical
 * chunks of `chunk_bytes` are created, mapped, made accessible and zero-filled
 * on demand (hipMemCreate / hipMemMap / hipMemSetAccess), and unmapped and
 * released on request (hipMemUnmap / hipMemRelease). The reservation itself
 * (hipMemAddressReserve) never moves, so device pointers into it stay valid
 * across decommit and recommit.
 *
 * The entry points keep the names, argument meanings, return conventions and
 * error behaviour of the reference's C ABI (native/elastic_vmm.cpp:316-369),
 * which elastic_kv/backing.py:30-51 binds through ctypes:
 *   - no C++ exception crosses the ABI; a failing call returns its error value
 *     and leaves a message in a thread-local string read by ev_error();
 *   - chunk ids outside the reservation, or a NULL id array with count > 0,
 *     fail the whole call before anything is mapped;
 *   - duplicate ids are ignored; ensure/precommit of mapped ids and drop of
 *     unmapped ids are no-ops;
 *   - a failed batch rolls back the chunks it created when it can (the object
 *     stays usable); when rollback itself fails the object is "poisoned" and
 *     every later mutation fails.
 * One deliberate difference: when close fails, the object is NOT freed, so a
 * retry of ev_close on the same handle is well defined.
 *
 * Threading: one owner thread per object (no internal locks). Zero-filling of
 * new chunks runs on a private non-blocking stream and is fenced by the next
 * ev_ensure on that object. Callers must fence every device user of a chunk
 * before ev_drop.
 */
#ifndef ELASTIC_VMM_H
#define ELASTIC_VMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Reserve ceil(capacity_bytes / chunk_bytes) chunks of virtual address space
 * on `device`. chunk_bytes must be a multiple of the device's minimum VMM
 * granularity. Returns NULL on error.
 * Replaces: native/elastic_vmm.cpp:318-324 (ev_create). */
void* ev_create(int device, uint64_t capacity_bytes, uint64_t chunk_bytes);

/* Commit the listed chunks: create + map + set read/write access, zero-fill on
 * the object's private stream, then wait for every zero-fill still pending on
 * this object (including earlier ev_precommit calls). 0 on success, -1 on error.
 * Replaces: native/elastic_vmm.cpp:326-331 (ev_ensure). */
int ev_ensure(void* handle, const uint64_t* indices, size_t count);

/* Like ev_ensure but does not wait for zero-fill; a later ev_ensure (any ids)
 * is the readiness barrier. 0 on success, -1 on error.
 * Replaces: native/elastic_vmm.cpp:333-338 (ev_precommit). */
int ev_precommit(void* handle, const uint64_t* indices, size_t count);

/* Unmap and release the listed chunks. The caller guarantees no in-flight
 * device work can touch them. 0 on success, -1 on error.
 * Replaces: native/elastic_vmm.cpp:340-345 (ev_drop). */
int ev_drop(void* handle, const uint64_t* indices, size_t count);

/* Base device address of the reservation; UINT64_MAX on error.
 * Replaces: native/elastic_vmm.cpp:347 (ev_base). */
uint64_t ev_base(void* handle);

/* Bytes currently backed by physical chunks; UINT64_MAX on error.
 * Replaces: native/elastic_vmm.cpp:348 (ev_backed). */
uint64_t ev_backed(void* handle);

/* Reserved bytes (capacity rounded up to whole chunks); UINT64_MAX on error.
 * Replaces: native/elastic_vmm.cpp:349 (ev_reserved). */
uint64_t ev_reserved(void* handle);

/* Minimum VMM allocation granularity of the device; UINT64_MAX on error.
 * Replaces: native/elastic_vmm.cpp:350-352 (ev_granularity). */
uint64_t ev_granularity(void* handle);

/* 1 if a failed rollback left the object unusable, 0 if not, -1 on error.
 * Replaces: native/elastic_vmm.cpp:353-355 (ev_poisoned). */
int ev_poisoned(void* handle);

/* Keep up to `chunks` physical chunks that ev_drop unmaps, instead of
 * releasing them, for the next ev_ensure / ev_precommit to map (they are
 * zero-filled like new chunks); 0, the default, releases every dropped chunk
 * at once. Lowering the limit releases the chunks held above it; ev_close
 * releases them all. Saves a create and a release per recycled chunk, and
 * holds that memory (ev_spare) until a commit takes it. Returns 0, or -1 on
 * error (a limit above the reservation's chunk count, a closed or poisoned
 * object; a failed release poisons it).
 * No reference counterpart: for callers that decommit and recommit chunks
 * every step (remapping, migration) and can keep that memory. */
int ev_set_spare(void* handle, uint64_t chunks);

/* Bytes held by the spare pool; UINT64_MAX on error. No reference counterpart. */
uint64_t ev_spare(void* handle);

/* Message of the last failed call on this thread ("" after a success).
 * Shared by every entry point of this library, ekv_* included.
 * Replaces: native/elastic_vmm.cpp:357 (ev_error). */
const char* ev_error(void);

/* Synchronize the device, release every chunk, free the reservation and the
 * private stream, then free the object. NULL is a no-op. On failure returns -1
 * and keeps the object alive so the call can be retried.
 * Replaces: native/elastic_vmm.cpp:359-367 (ev_close). */
int ev_close(void* handle);

#ifdef __cplusplus
}
#endif

#endif /* ELASTIC_VMM_H */
