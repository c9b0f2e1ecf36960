// q8_internal.h -- declarations shared by the host sources of libq8mi.so.
// Nothing here is part of the C-ABI (hidden, C++ linkage).
#ifndef Q8_INTERNAL_H
#define Q8_INTERNAL_H

struct q8_ctx;

namespace q8i {
constexpr int kGroupPairSlices = -16;
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
// `count` synthetic matrices of one k (rows outs[i], seeds[i]) as a
// contiguous group: one allocation, each member's tiles after the previous
// member's, and with slice_rows 8 or 16 a slice-major copy of all of them;
// slice_rows = kGroupPairSlices builds a gate/up pair's paired copy instead
// (Q8SliceArgs::pair_tiles), which the pair's launches read.
// Members are weights of their own (released one by one; the allocation goes
// with the last); a group launch over them in order runs the contiguous-group
// row-slice GEMVs.
__attribute__((visibility("hidden"))) int weight_synthetic_group(q8_ctx *c, int k, int count, const int *outs,
                                                                  const uint64_t *seeds, float scale_std,
                                                                  int slice_rows, const q8_weight **weights);
// The slice height a contiguous group's launch at this k runs in (0: it
// keeps the tile kernel), for a plain group with a folded norm (silu = 0) or
// the gate/up pair (silu = 1); group_slice_rows is 0 too when the context
// builds no slice-major copies.
__attribute__((visibility("hidden"))) int group_rows(q8_ctx *c, int k, int silu);
__attribute__((visibility("hidden"))) int group_slice_rows(q8_ctx *c, int k, int silu);
// weight_synthetic_group's slice_rows for a gate/up pair at this k:
// kGroupPairSlices where the paired kernels run, else 0.
__attribute__((visibility("hidden"))) int group_pair_slices(q8_ctx *c, int k);
}  // namespace q8i

#endif
