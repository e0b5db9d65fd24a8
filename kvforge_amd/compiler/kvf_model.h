// kvf_model.h - plan space, machine description and cost model of the kvf
// compiler (host C++20, no GPU).
//
// What the reference's src/{format,layout,plan,machine,calib,cost,passes}.cpp
// compute is restated here so that a plan chosen for a reference machine file
// is the same plan, with the same predicted numbers:
//   formats and candidates     src/format.cpp:8-102
//   layouts and candidates     src/layout.cpp:52-78
//   plan enumeration           src/plan.cpp:25-86
//   machine file               src/machine.cpp:16-130
//   calibration file           src/calib.cpp:7-97
//   cost model                 src/cost.cpp:9-256
// On top of that, a machine file that declares `wave_size = 64` selects the
// CDNA form of the model (cdnaEvaluate), re-derived for compute units,
// 64-lane wavefronts and the gfx950 kernels' own tile geometry.
#pragma once

#include <filesystem>
#include <map>
#include <string>
#include <vector>

namespace kvfc {

// ---------------------------------------------------------------- shape
struct DecodeSpec {
  std::string name = "decode";
  int H = 32;      // query heads
  int H_kv = 32;   // key/value heads
  int d = 128;     // head dimension
  int n = 4096;    // cached tokens (the longest sequence when lens is set)
  int batch = 1;   // sequences decoded together
  float scale = 0; // 0: 1/sqrt(d)
  // per-sequence lengths (this build's extension): empty when every sequence
  // holds n tokens; lens_spec names their distribution ("uniform:LO:HI:SEED"
  // or "loguniform:LO:HI:SEED"), from which lens is drawn
  std::vector<int> lens;
  std::string lens_spec;
  int g() const { return H_kv > 0 ? H / H_kv : 1; }
  long long tokens() const; // sum of the sequence lengths (n * batch when uniform)
  int maxLen() const;       // the longest sequence
};

// Lengths of `batch` sequences from a distribution spec, drawn exactly as the
// harness draws them (libkvf_hostdata.so: kvfh_varlen_lengths,
// kvfh_lengths_loguniform):
//   uniform:LO:HI:SEED    LO + std::uniform_int_distribution<int>(0, HI-LO)
//                         on mt19937_64(SEED)
//   loguniform:LO:HI:SEED clamp(lround(exp(u)), LO, HI), u from
//                         std::uniform_real_distribution<double>(ln LO, ln HI)
// Throws on a malformed spec.
std::vector<int> drawLengths(const std::string &spec, int batch);

// ---------------------------------------------------------------- storage
enum class Format { F16, INT8, INT4, Unset };

struct KvFormat {
  Format fmt = Format::F16;
  int group = 0;         // elements per (scale, zero) group, 0 for f16
  int metadata_bits = 0; // 32 for quantized formats
  int rawBits() const;
  double effectiveBits() const;
  double effectiveBytes() const { return effectiveBits() / 8.0; }
  bool isQuantized() const { return fmt == Format::INT8 || fmt == Format::INT4; }
  int dataRowBytes(int d) const { return d * rawBits() / 8; }
  int metaRowBytes(int d) const { return isQuantized() ? (d / group) * 4 : 0; }
  double dequantFlopsPerElem() const;
  std::string str() const; // "int8:64"
  std::string key() const; // "int8_64"
};

Format parseFormat(const std::string &s);
const char *formatName(Format f);
std::vector<KvFormat> candidateFormats(int d, bool include_quantized);

enum class Order { HeadMajor, TokenMajor, Unset };
enum class Residency { Contiguous, Paged, Unset };

struct KvLayout {
  Order order = Order::HeadMajor;
  Residency residency = Residency::Contiguous;
  int block_tokens = 0;
  bool paged() const { return residency == Residency::Paged; }
  std::string str() const; // "head_major/paged:64"
};

Order parseOrder(const std::string &s);
Residency parseResidency(const std::string &s);
const char *orderName(Order o);
const char *residencyName(Residency r);
std::vector<KvLayout> candidateLayouts();

// ---------------------------------------------------------------- plans
struct Partition {
  int splits = 1;
  bool gqa_pack = false;
  int warps = 4;  // wavefronts per workgroup on CDNA, warps per block on NVIDIA
  int unroll = 2;
  std::string str() const; // "splits=8 pack w4 u2"
};

struct Plan {
  KvFormat fmt;
  KvLayout layout;
  Partition part;
  std::string str() const; // "int8:64 | head_major/contiguous | splits=8 pack w4 u2"
};

struct SearchSpace {
  bool format_free = true, layout_free = true, splits_free = true, pack_free = true;
  bool include_quantized = false;
  int max_splits = 0; // 0: 64
  KvFormat pinned_fmt;
  KvLayout pinned_layout;
  int pinned_splits = 1;
  bool pinned_pack = false;
  std::vector<int> warps_cand{4, 8};
  std::vector<int> unroll_cand{2, 4};
  double max_rel_err = 0.0;
};

std::vector<int> candidateSplits(const DecodeSpec &s, int max_splits);

// ---------------------------------------------------------------- machine
struct Machine {
  std::string name = "generic-gpu";
  double compute_capability = 0;
  double dram_gb = 0;
  int sms = 24; // streaming multiprocessors (NVIDIA) or compute units (CDNA)
  double bw_peak_gbs = 250.0;
  double bw_sm_gbs = 15.0;
  double lat_ns = 600.0;
  double bw_l2_gbs = 1000.0;
  long long l2_bytes = 32LL * 1024 * 1024;
  int sector_bytes = 32;
  int line_bytes = 128;
  double f32_gflops = 10000.0;
  double launch_us = 3.0;
  int max_warps_per_sm = 48;
  int max_blocks_per_sm = 24;
  int regs_per_sm = 0;
  std::string resources_file;
  std::map<std::string, int> kernel_regs;
  // gfx950 resource table (machines/resources_gfx950.csv, written by
  // kvforge_amd/tools/dump_resources.py): per split-kernel instantiation,
  // keyed "fmt_d_group_g_u_ord_paged_waves".
  struct KernelRes {
    int vgpr = 0, agpr = 0, scratch = 0, occupancy = 0;
    // instructions per 32-token tile of the kernel's main loop, counted in its
    // gfx950 assembly (0 when the table predates these columns)
    double valu = 0, mfma = 0, lds = 0, salu = 0;
  };
  std::map<std::string, KernelRes> kernel_res;
  // CDNA keys (written by kvforge_amd/tools/bw_probe); wave_size = 64 selects
  // the CDNA form of the cost model.
  int wave_size = 32;
  long long mall_bytes = 0;
  double bw_mall_gbs = 0;
  double lat_mall_ns = 0;
  double bw_copy_gbs = 0;
  double kernel_floor_us = 0;

  bool cdna() const { return wave_size == 64; }
  double fSmGflops() const { return sms > 0 ? f32_gflops / sms : 0; }
  double ridgeFlopPerByte() const { return bw_peak_gbs > 0 ? f32_gflops / bw_peak_gbs : 0; }
  double bwSmGbs(double bif_sm_bytes, double lat_scale = 1.0) const;
  double bwDeviceGbs(int active_sms, double bif_sm_bytes, double lat_scale = 1.0) const;
  int regsFor(const std::string &key) const {
    const auto it = kernel_regs.find(key);
    return it == kernel_regs.end() ? 0 : it->second;
  }
};

Machine loadMachine(const std::filesystem::path &p);
void applyMachineKey(Machine &m, const std::string &key, double value, const std::string &raw);
std::string dumpMachine(const Machine &m);

// ---------------------------------------------------------------- calibration
struct Calib {
  double r0_bytes = 64.0;
  double c_page_ns = 60.0;
  double unpack_l2_hit = 0.8;
  double lat_scale = 4.0;
  double issue_eff = 0.35;
  double wave_model = 0.0;
  double warp_w0 = 8.0;
  double overlap_p = 4.0;
  double launch_frac = 0.5;
  double merge_frac = 0.3;
  double meta_waste = 1.0;
  // CDNA form only: per-CU stream rate of the split kernel as a fraction of
  // the machine's bw_sm_gbs, and the issue cost of register spills. They are
  // written to and read from calibration files only when `cdna` is set, so a
  // file for a 32-lane-warp machine keeps the reference's keys exactly.
  double cu_frac = 0.6;
  double spill_cost = 0.5;
  // CDNA form only: one memory round trip of the merge kernel, in units of
  // the machine's lat_ns (the merge runs after the stream, on a quiet memory)
  double merge_trip = 1.5;
  // CDNA form only: issue slots a scalar instruction of the main loop takes
  // from its wave (address and page-table arithmetic, loop control)
  double salu_w = 0.0;
  bool cdna = false;
  std::map<std::string, double> rel_err;
  static Calib defaults();
};

Calib loadCalib(const std::filesystem::path &p);
void saveCalib(const Calib &c, const std::filesystem::path &p);
std::string dumpCalib(const Calib &c);
const std::vector<const char *> &calibScalarKeys();
double &calibScalar(Calib &c, const std::string &key);

// ---------------------------------------------------------------- cost
struct Cost {
  double kv_bytes = 0, meta_bytes = 0, qo_bytes = 0, partial_bytes = 0, total_bytes = 0;
  double attn_flops = 0, dequant_flops = 0, total_flops = 0;
  double intensity = 0;
  double eta = 1.0;
  long long blocks = 0;
  int active_sms = 0;
  int resident_blocks = 0;
  double bif_sm_bytes = 0;
  double imbalance = 1.0;
  double bw_eff_gbs = 0;
  double t_mem_us = 0, t_cmp_us = 0, t_merge_us = 0, t_page_us = 0, t_launch_us = 0;
  double t_total_us = 0;
  double achieved_gbs = 0;
  double frac_of_peak = 0;
  bool memory_bound = true;
  double rel_err = 0;
  bool rejected = false;
  std::string note;
};

Cost evaluate(const DecodeSpec &s, const Machine &m, const Calib &c, const Plan &p,
              double max_rel_err = 0.0);

struct Ranked {
  Plan plan;
  Cost cost;
};

std::vector<Ranked> rankPlans(const DecodeSpec &s, const Machine &m, const Calib &c,
                              const std::vector<Plan> &plans, double max_rel_err = 0.0);
std::vector<Plan> enumeratePlans(const DecodeSpec &s, const Machine &m, const SearchSpace &sp);
double idealIntensity(const DecodeSpec &s, const KvFormat &f);

} // namespace kvfc
