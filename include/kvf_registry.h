/* kvf_registry.h - maps a variant id to the launcher of that instantiation.
 *
 * Replaces the reference's runtime/kvf_registry.h:15-29 with hipError_t /
 * hipStream_t: the generated dispatch sources (kvf emit-dispatch) define
 * kvf_register_<bucket> and kvf_register_all, which fill this table, so the
 * sweep harness runs kernels that code generation produced.
 *
 * LaunchFn takes `const Args &`, a C++ reference: this is an intra-C++
 * interface, exactly as in the reference. The C-ABI face is kvf_abi.h.
 *
 * Beside the reference's add(id, fn) a variant may also register its
 * extended launcher (variable lengths, binary16 q/out, fused merge, split
 * kernel only, kernel-bound timing events); the C-ABI entry points other than
 * kvf_launch_variant go through it.
 */
#ifndef KVF_REGISTRY_H
#define KVF_REGISTRY_H

#include "kvf_abi.h"

#include <string>
#include <unordered_map>

namespace kvf {
namespace gfx950 {
struct Ext;
struct Launch;
} /* namespace gfx950 */

using LaunchFn = hipError_t (*)(const Args &, hipStream_t);
using LaunchXFn = hipError_t (*)(const Args &, const gfx950::Ext &, const gfx950::Launch &,
                                 hipStream_t);

struct Registry {
  struct Entry {
    LaunchFn fn = nullptr;
    LaunchXFn xfn = nullptr;
  };
  std::unordered_map<std::string, Entry> fn;
  void add(const char *id, LaunchFn f) { fn[id].fn = f; }
  void add(const char *id, LaunchFn f, LaunchXFn x) { fn[id] = Entry{f, x}; }
  LaunchFn find(const std::string &id) const {
    const auto it = fn.find(id);
    return it == fn.end() ? nullptr : it->second.fn;
  }
  LaunchXFn findx(const std::string &id) const {
    const auto it = fn.find(id);
    return it == fn.end() ? nullptr : it->second.xfn;
  }
};

/* The launch template every dispatch source instantiates
 * (runtime/kvf_kernels.cuh:309-320 has the same signature). */
template <int FMT, int D, int G, int U, int ORD, bool PAGED>
hipError_t launch(const Args &a, hipStream_t st);

} /* namespace kvf */

/* Defined in the generated kvf_dispatch.hip. */
void kvf_register_all(kvf::Registry &r);

#endif /* KVF_REGISTRY_H */
