/* kvf_registry.h - maps a variant id to the launcher of that instantiation.
 *
 * Replaces the reference's runtime/kvf_registry.h:15-29 with hipError_t /
 * hipStream_t: the generated dispatch sources (kvf emit-dispatch) define
 * kvf_register_<bucket> and kvf_register_all, which fill this table, so the
 * sweep harness runs kernels that code generation produced.
 *
 * LaunchFn takes `const Args &`, a C++ reference: this is an intra-C++
 * interface, exactly as in the reference. The C-ABI face is kvf_abi.h.
 */
#ifndef KVF_REGISTRY_H
#define KVF_REGISTRY_H

#include "kvf_abi.h"

#include <string>
#include <unordered_map>

namespace kvf {

using LaunchFn = hipError_t (*)(const Args &, hipStream_t);

struct Registry {
  std::unordered_map<std::string, LaunchFn> fn;
  void add(const char *id, LaunchFn f) { fn[id] = f; }
  LaunchFn find(const std::string &id) const {
    const auto it = fn.find(id);
    return it == fn.end() ? nullptr : it->second;
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
