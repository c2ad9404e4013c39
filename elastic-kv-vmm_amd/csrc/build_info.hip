// Build fingerprint of libelastic_vmm: the hash of the sources it was built
// from (computed by build_native.py, checked by the Python loader).
#ifndef EKV_SOURCE_HASH
#error "build with -DEKV_SOURCE_HASH=<hash of the native sources> (build_native.py does)"
#endif

#define EKV_STRINGIFY_(x) #x
#define EKV_STRINGIFY(x) EKV_STRINGIFY_(x)

extern "C" const char* ekv_source_hash(void) { return EKV_STRINGIFY(EKV_SOURCE_HASH); }
