// q8_internal.h -- declarations shared by the host sources of libq8mi.so.
// Nothing here is part of the C-ABI (hidden, C++ linkage).
#ifndef Q8_INTERNAL_H
#define Q8_INTERNAL_H

struct q8_ctx;

namespace q8i {
// One kernel's metadata as the code object's AMDGPU note records it
// (llm_amd/build.py writes the table into q8_manifest.h): the bytes of its
// explicit arguments, the whole kernarg segment, VGPRs, AGPRs, SGPRs, static
// LDS, the largest workgroup it was compiled for and its private bytes per lane.
struct KernelMeta {
    const char *name;
    unsigned args, kernarg, vgpr, agpr, sgpr, lds, max_wg, priv;
};
// Record `fmt` as the calling thread's q8_last_error() message; returns code.
__attribute__((visibility("hidden"), format(printf, 2, 3))) int set_error(int code, const char *fmt, ...);
// Changes whenever the context reallocates a workspace; a graph captured
// before the change holds freed pointers.
__attribute__((visibility("hidden"))) unsigned long long workspace_generation(const q8_ctx *c);
// Positions one chunk of the split decode attention kernel covers: a split of
// about this many positions is one pass over its keys.
__attribute__((visibility("hidden"))) int attention_split_rows();
// The device address of q8_matmul_noalloc's static scratch on `device`, which
// must be the current device (q8_noalloc.hip); status code.
__attribute__((visibility("hidden"))) int noalloc_scratch(int device, void **out);
// Whether context `ctx` holds `device`'s no-allocation scratch: the first
// context to ask takes it and keeps it until noalloc_release (q8_close);
// another context on the same device is refused (q8_noalloc_owner.h).
__attribute__((visibility("hidden"))) bool noalloc_claim(int device, const q8_ctx *ctx);
__attribute__((visibility("hidden"))) void noalloc_release(const q8_ctx *ctx);
// q8_weight_synthetic, with slice_copy = false for a weight that only runs in
// groups or GEMMs: no slice-major copy of its quants is built.
__attribute__((visibility("hidden"))) int weight_synthetic(q8_ctx *c, int k, int out, uint64_t seed, float scale_std,
                                                            bool slice_copy, const q8_weight **weight);
}  // namespace q8i

#endif
