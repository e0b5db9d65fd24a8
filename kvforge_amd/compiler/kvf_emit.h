// kvf_emit.h - what `kvf plan` and `kvf emit-dispatch` write.
//
// For a planned module (kvf plan):
//   report.txt        the chosen plan, its predicted cost and the ranking
//   plans.csv         every candidate, in the reference's column layout
//                     (src/emit.cpp:77-97), so existing tools read it
//   ir.txt            the module before and after planning
//   decode_<name>.hip one translation unit exporting
//                       extern "C" hipError_t kvf_launch_<name>(const kvf::Args *, hipStream_t)
//                       extern "C" const char *kvf_plan_<name>()
//                     (the reference emits the same pair for CUDA,
//                     src/codegen.cpp:67-93)
//   plan_info.h       the shape and plan as KVF_* macros (src/codegen.cpp:95-116)
//
// For the library (kvf emit-dispatch): one registration source per
// format x order x residency bucket, one explicit-instantiation source per
// bucket and head dimension, and kvf_register_all.
#pragma once

#include "kvf_front.h"

#include <filesystem>
#include <string>
#include <utility>
#include <vector>

namespace kvfc {

// "{fmt}_{hm|tm}_{c|p}_g{G}_u{U}_d{D}" (src/codegen.cpp:59-65), G = 1 unless packed.
std::string variantId(const Plan &p, int g, int d);

std::string plansCsv(const Module &m);
std::string rooflineText(const Module &m);
std::string reportText(const Module &m, const std::string &ir_before, int top_n);
std::string kernelSource(const Module &m);
std::string planHeader(const Module &m);

struct Written {
  std::filesystem::path report, plans_csv, ir_txt, kernel;
};
Written writePlanOutputs(const Module &m, const std::filesystem::path &dir, const std::string &ir_before,
                         int top_n);

// (file name, contents) of the dispatch sources for the given head
// dimensions and pack sizes (pack 1 is always included).
std::vector<std::pair<std::string, std::string>> dispatchSources(const std::vector<int> &dims,
                                                                 const std::vector<int> &packs,
                                                                 bool include_quantized);

} // namespace kvfc
