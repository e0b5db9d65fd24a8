// kvf_model.cpp - plan space, machine/calibration files and the cost model.
//
// The formulas of the reference's cost model (src/cost.cpp:81-243) are kept
// term for term in `evaluate` for machines with 32-lane warps, so plans.csv
// for a reference machine file reproduces the reference's. `cdnaEvaluate`
// is the MI355X form: the same decomposition (bytes, Little's law, waves,
// issue time, p-norm overlap, merge, paging, launch) with every
// warp/SM-specific term re-derived for the gfx950 kernels in
// kvforge_amd/csrc/kvf_kernels.hpp.
#include "kvf_model.h"

#include <random>

#include <algorithm>
#include <cmath>
#include <fstream>
#include <iomanip>
#include <sstream>
#include <stdexcept>

namespace kvfc {

long long DecodeSpec::tokens() const {
  if (lens.empty()) return 1LL * n * batch;
  long long t = 0;
  for (int l : lens) t += l;
  return t;
}

int DecodeSpec::maxLen() const {
  if (lens.empty()) return n;
  int m = 0;
  for (int l : lens) m = std::max(m, l);
  return m;
}

std::vector<int> drawLengths(const std::string &spec, int batch) {
  std::vector<std::string> f;
  {
    std::string cur;
    for (char ch : spec) {
      if (ch == ':') {
        f.push_back(cur);
        cur.clear();
      } else {
        cur.push_back(ch);
      }
    }
    f.push_back(cur);
  }
  if (f.size() != 4 || (f[0] != "uniform" && f[0] != "loguniform"))
    throw std::runtime_error("length distribution '" + spec + "': expected uniform:LO:HI:SEED or loguniform:LO:HI:SEED");
  const int lo = std::stoi(f[1]), hi = std::stoi(f[2]);
  const unsigned long long seed = std::stoull(f[3]);
  if (lo < 0 || hi < lo || (f[0] == "loguniform" && lo < 1))
    throw std::runtime_error("length distribution '" + spec + "': bad bounds");
  std::vector<int> out(static_cast<std::size_t>(std::max(batch, 0)));
  std::mt19937_64 rng(seed);
  if (f[0] == "uniform") {
    std::uniform_int_distribution<int> u(0, hi - lo);
    for (auto &l : out) l = lo + u(rng);
  } else {
    std::uniform_real_distribution<double> u(std::log(static_cast<double>(lo)), std::log(static_cast<double>(hi)));
    for (auto &l : out) {
      const long v = std::lround(std::exp(u(rng)));
      l = static_cast<int>(std::min<long>(hi, std::max<long>(lo, v)));
    }
  }
  return out;
}

// ======================================================================= formats
int KvFormat::rawBits() const {
  switch (fmt) {
  case Format::F16: return 16;
  case Format::INT8: return 8;
  case Format::INT4: return 4;
  case Format::Unset: break;
  }
  throw std::runtime_error("format not resolved");
}

double KvFormat::effectiveBits() const {
  if (!isQuantized()) return rawBits();
  if (group <= 0) throw std::runtime_error("quantized format needs a group size");
  return rawBits() + static_cast<double>(metadata_bits) / group;
}

// Issue-slot estimate per loaded element (src/format.cpp:36-51).
double KvFormat::dequantFlopsPerElem() const {
  switch (fmt) {
  case Format::F16: return 0.5;
  case Format::INT8: return 1.5;
  case Format::INT4: return 2.5;
  case Format::Unset: break;
  }
  return 0;
}

std::string KvFormat::str() const {
  std::string s = formatName(fmt);
  if (isQuantized()) s += ":" + std::to_string(group);
  return s;
}

std::string KvFormat::key() const {
  std::string s = formatName(fmt);
  if (isQuantized()) s += "_" + std::to_string(group);
  return s;
}

const char *formatName(Format f) {
  switch (f) {
  case Format::F16: return "f16";
  case Format::INT8: return "int8";
  case Format::INT4: return "int4";
  case Format::Unset: return "?";
  }
  return "?";
}

Format parseFormat(const std::string &s) {
  if (s == "f16") return Format::F16;
  if (s == "int8") return Format::INT8;
  if (s == "int4") return Format::INT4;
  if (s == "?") return Format::Unset;
  throw std::runtime_error("unknown KV format '" + s + "' (f16, int8, int4, ?)");
}

// f16 first, then int8 groups, then int4 groups; groups must divide d
// (src/format.cpp:90-102).
std::vector<KvFormat> candidateFormats(int d, bool include_quantized) {
  std::vector<KvFormat> out{KvFormat{Format::F16, 0, 0}};
  if (!include_quantized) return out;
  auto add = [&](Format f, std::initializer_list<int> groups) {
    for (int g : groups)
      if (g <= d && d % g == 0) out.push_back(KvFormat{f, g, 32});
  };
  add(Format::INT8, {64, 128});
  add(Format::INT4, {32, 64, 128});
  return out;
}

// ======================================================================= layouts
const char *orderName(Order o) {
  switch (o) {
  case Order::HeadMajor: return "head_major";
  case Order::TokenMajor: return "token_major";
  case Order::Unset: return "?";
  }
  return "?";
}

const char *residencyName(Residency r) {
  switch (r) {
  case Residency::Contiguous: return "contiguous";
  case Residency::Paged: return "paged";
  case Residency::Unset: return "?";
  }
  return "?";
}

Order parseOrder(const std::string &s) {
  if (s == "head_major") return Order::HeadMajor;
  if (s == "token_major") return Order::TokenMajor;
  if (s == "?") return Order::Unset;
  throw std::runtime_error("unknown KV order '" + s + "' (head_major, token_major, ?)");
}

Residency parseResidency(const std::string &s) {
  if (s == "contiguous") return Residency::Contiguous;
  if (s == "paged") return Residency::Paged;
  if (s == "?") return Residency::Unset;
  throw std::runtime_error("unknown KV residency '" + s + "' (contiguous, paged, ?)");
}

std::string KvLayout::str() const {
  std::string s = std::string(orderName(order)) + "/" + residencyName(residency);
  if (residency == Residency::Paged && block_tokens > 0) s += ":" + std::to_string(block_tokens);
  return s;
}

// src/layout.cpp:62-78: both contiguous orders, head-major pages of
// 16..128 tokens, token-major pages of 16 and 64.
std::vector<KvLayout> candidateLayouts() {
  std::vector<KvLayout> out;
  out.push_back({Order::HeadMajor, Residency::Contiguous, 0});
  out.push_back({Order::TokenMajor, Residency::Contiguous, 0});
  for (int b : {16, 32, 64, 128}) out.push_back({Order::HeadMajor, Residency::Paged, b});
  for (int b : {16, 64}) out.push_back({Order::TokenMajor, Residency::Paged, b});
  return out;
}

// ======================================================================= plans
std::string Partition::str() const {
  return "splits=" + std::to_string(splits) + (gqa_pack ? " pack" : "") + " w" +
         std::to_string(warps) + " u" + std::to_string(unroll);
}

std::string Plan::str() const { return fmt.str() + " | " + layout.str() + " | " + part.str(); }

// Powers of two up to the cap, keeping a split only while each chunk still
// holds at least 128 tokens (src/plan.cpp:25-33).
std::vector<int> candidateSplits(const DecodeSpec &s, int max_splits) {
  const int cap = max_splits > 0 ? max_splits : 64;
  std::vector<int> out;
  for (int v = 1; v <= cap; v *= 2)
    if (v == 1 || s.n / v >= 128) out.push_back(v);
  return out;
}

// Cartesian product in the order format, layout, pack, splits, warps,
// unroll (src/plan.cpp:37-86); the order fixes the ranking of tied plans.
std::vector<Plan> enumeratePlans(const DecodeSpec &s, const Machine &, const SearchSpace &sp) {
  const std::vector<KvFormat> formats =
      sp.format_free ? candidateFormats(s.d, sp.include_quantized) : std::vector<KvFormat>{sp.pinned_fmt};
  const std::vector<KvLayout> layouts =
      sp.layout_free ? candidateLayouts() : std::vector<KvLayout>{sp.pinned_layout};
  std::vector<bool> packs;
  if (sp.pack_free) {
    packs.push_back(false);
    const int g = s.g();
    if (g == 2 || g == 4 || g == 8) packs.push_back(true);
  } else {
    packs.push_back(sp.pinned_pack);
  }
  const std::vector<int> splits =
      sp.splits_free ? candidateSplits(s, sp.max_splits) : std::vector<int>{sp.pinned_splits};
  std::vector<Plan> out;
  for (const auto &f : formats)
    for (const auto &l : layouts)
      for (bool pk : packs)
        for (int sv : splits)
          for (int w : sp.warps_cand)
            for (int u : sp.unroll_cand) {
              Plan p;
              p.fmt = f;
              p.layout = l;
              p.part = Partition{sv, pk, w, u};
              out.push_back(p);
            }
  return out;
}

// ======================================================================= machine
double Machine::bwSmGbs(double bif_sm_bytes, double lat_scale) const {
  if (lat_ns <= 0) return bw_sm_gbs;
  return std::min(bw_sm_gbs, bif_sm_bytes / (lat_ns * std::max(1.0, lat_scale)));
}

double Machine::bwDeviceGbs(int active_sms, double bif_sm_bytes, double lat_scale) const {
  active_sms = std::clamp(active_sms, 1, std::max(1, sms));
  return std::min(bw_peak_gbs, active_sms * bwSmGbs(bif_sm_bytes, lat_scale));
}

void applyMachineKey(Machine &m, const std::string &key, double value, const std::string &raw) {
  auto i = [&](int &f) { f = static_cast<int>(value); };
  if (key == "name") m.name = raw;
  else if (key == "compute_capability") m.compute_capability = value;
  else if (key == "dram_gb") m.dram_gb = value;
  else if (key == "sms") i(m.sms);
  else if (key == "bw_peak_gbs") m.bw_peak_gbs = value;
  else if (key == "bw_sm_gbs") m.bw_sm_gbs = value;
  else if (key == "lat_ns") m.lat_ns = value;
  else if (key == "bw_l2_gbs") m.bw_l2_gbs = value;
  else if (key == "l2_bytes") m.l2_bytes = static_cast<long long>(value);
  else if (key == "sector_bytes") i(m.sector_bytes);
  else if (key == "line_bytes") i(m.line_bytes);
  else if (key == "f32_gflops") m.f32_gflops = value;
  else if (key == "launch_us") m.launch_us = value;
  else if (key == "max_warps_per_sm") i(m.max_warps_per_sm);
  else if (key == "max_blocks_per_sm") i(m.max_blocks_per_sm);
  else if (key == "regs_per_sm") i(m.regs_per_sm);
  else if (key == "resources") m.resources_file = raw;
  else if (key == "wave_size") i(m.wave_size);
  else if (key == "mall_bytes") m.mall_bytes = static_cast<long long>(value);
  else if (key == "bw_mall_gbs") m.bw_mall_gbs = value;
  else if (key == "lat_mall_ns") m.lat_mall_ns = value;
  else if (key == "bw_copy_gbs") m.bw_copy_gbs = value;
  else if (key == "kernel_floor_us") m.kernel_floor_us = value;
  else throw std::runtime_error("unknown machine key '" + key + "'");
}

namespace {

std::string trim(const std::string &s, const char *ws) {
  const auto a = s.find_first_not_of(ws);
  const auto b = s.find_last_not_of(ws);
  return a == std::string::npos ? std::string() : s.substr(a, b - a + 1);
}

// Strict `key = value` reader shared by machine and calibration files: `#`
// starts a comment, a non-blank line without `=` is an error.
template <class F>
void readKeyValues(const std::filesystem::path &p, const char *what, const char *ws, F &&apply) {
  std::ifstream in(p);
  if (!in) throw std::runtime_error(std::string("cannot read ") + what + " " + p.string());
  std::string line;
  int lineno = 0;
  while (std::getline(in, line)) {
    ++lineno;
    const auto hash = line.find('#');
    if (hash != std::string::npos) line.resize(hash);
    const auto eq = line.find('=');
    if (eq == std::string::npos) {
      if (line.find_first_not_of(" \t\r\n") != std::string::npos)
        throw std::runtime_error(p.string() + ":" + std::to_string(lineno) + ": expected key = value");
      continue;
    }
    apply(trim(line.substr(0, eq), ws), trim(line.substr(eq + 1), ws));
  }
}

} // namespace

// src/machine.cpp:70-130: unknown keys are errors; `resources` names a
// register table keyed by kernel variant, relative to the machine file.
Machine loadMachine(const std::filesystem::path &p) {
  Machine m;
  readKeyValues(p, "machine file", " \t\r\n\"", [&](const std::string &k, const std::string &raw) {
    double v = 0;
    try {
      v = std::stod(raw);
    } catch (const std::exception &) {
      v = 0;
    }
    applyMachineKey(m, k, v, raw);
  });
  if (!m.resources_file.empty()) {
    std::filesystem::path rp(m.resources_file);
    if (!std::filesystem::exists(rp) && rp.is_relative()) rp = p.parent_path() / rp;
    std::ifstream rin(rp);
    if (!rin) throw std::runtime_error("cannot read resource table " + rp.string());
    std::string rl;
    std::getline(rin, rl); // header
    if (rl.find("waves") != std::string::npos) {
      // gfx950 layout: fmt,d,group,g,u,ord,paged,waves,vgpr,agpr,sgpr,scratch,occupancy
      // and, optionally, the main loop's instructions per tile: valu,mfma,lds,salu
      while (std::getline(rin, rl)) {
        std::vector<double> f;
        std::stringstream ss(rl);
        std::string tok;
        while (std::getline(ss, tok, ',')) f.push_back(std::stod(tok));
        if (f.size() < 13) continue;
        std::string key;
        for (int i = 0; i < 8; ++i) key += (i ? "_" : "") + std::to_string(static_cast<int>(f[i]));
        Machine::KernelRes r{static_cast<int>(f[8]), static_cast<int>(f[9]), static_cast<int>(f[11]),
                             static_cast<int>(f[12])};
        if (f.size() >= 17) {
          r.valu = f[13];
          r.mfma = f[14];
          r.lds = f[15];
          r.salu = f[16];
        }
        m.kernel_res[key] = r;
      }
      return m;
    }
    while (std::getline(rin, rl)) {
      std::vector<int> f;
      std::stringstream ss(rl);
      std::string tok;
      while (std::getline(ss, tok, ',')) f.push_back(std::stoi(tok));
      if (f.size() < 8) continue;
      std::string key;
      for (int i = 0; i < 7; ++i) key += (i ? "_" : "") + std::to_string(f[i]);
      m.kernel_regs[key] = f[7];
    }
  }
  return m;
}

std::string dumpMachine(const Machine &m) {
  std::ostringstream o;
  o << "name = " << m.name << "\n"
    << "compute_capability = " << m.compute_capability << "\n"
    << "dram_gb = " << m.dram_gb << "\n"
    << "sms = " << m.sms << "\n"
    << "bw_peak_gbs = " << m.bw_peak_gbs << "\n"
    << "bw_sm_gbs = " << m.bw_sm_gbs << "\n"
    << "lat_ns = " << m.lat_ns << "\n"
    << "bw_l2_gbs = " << m.bw_l2_gbs << "\n"
    << "l2_bytes = " << m.l2_bytes << "\n"
    << "sector_bytes = " << m.sector_bytes << "\n"
    << "line_bytes = " << m.line_bytes << "\n"
    << "f32_gflops = " << m.f32_gflops << "\n"
    << "launch_us = " << m.launch_us << "\n"
    << "max_warps_per_sm = " << m.max_warps_per_sm << "\n"
    << "max_blocks_per_sm = " << m.max_blocks_per_sm << "\n"
    << "regs_per_sm = " << m.regs_per_sm << "\n";
  if (!m.resources_file.empty()) o << "resources = " << m.resources_file << "\n";
  if (m.cdna()) {
    o << "wave_size = " << m.wave_size << "\n"
      << "mall_bytes = " << m.mall_bytes << "\n"
      << "bw_mall_gbs = " << m.bw_mall_gbs << "\n"
      << "lat_mall_ns = " << m.lat_mall_ns << "\n"
      << "bw_copy_gbs = " << m.bw_copy_gbs << "\n"
      << "kernel_floor_us = " << m.kernel_floor_us << "\n";
  }
  return o.str();
}

// ======================================================================= calibration
// Placeholder accuracy figures until a sweep measures them
// (src/calib.cpp:7-18).
Calib Calib::defaults() {
  Calib c;
  c.rel_err["int8_64"] = 0.004;
  c.rel_err["int8_128"] = 0.005;
  c.rel_err["int4_32"] = 0.06;
  c.rel_err["int4_64"] = 0.07;
  c.rel_err["int4_128"] = 0.08;
  return c;
}

const std::vector<const char *> &calibScalarKeys() {
  static const std::vector<const char *> keys{"r0_bytes",  "c_page_ns",   "unpack_l2_hit", "issue_eff",
                                              "meta_waste", "overlap_p",  "launch_frac",   "merge_frac",
                                              "lat_scale", "warp_w0",     "wave_model"};
  return keys;
}

double &calibScalar(Calib &c, const std::string &k) {
  if (k == "r0_bytes") return c.r0_bytes;
  if (k == "c_page_ns") return c.c_page_ns;
  if (k == "unpack_l2_hit") return c.unpack_l2_hit;
  if (k == "issue_eff") return c.issue_eff;
  if (k == "meta_waste") return c.meta_waste;
  if (k == "overlap_p") return c.overlap_p;
  if (k == "launch_frac") return c.launch_frac;
  if (k == "merge_frac") return c.merge_frac;
  if (k == "lat_scale") return c.lat_scale;
  if (k == "warp_w0") return c.warp_w0;
  if (k == "wave_model") return c.wave_model;
  throw std::runtime_error("unknown calibration key '" + k + "'");
}

Calib loadCalib(const std::filesystem::path &p) {
  Calib c = Calib::defaults();
  readKeyValues(p, "calibration file", " \t\r\n", [&](const std::string &k, const std::string &raw) {
    const double v = std::stod(raw);
    if (k.rfind("rel_err.", 0) == 0) {
      c.rel_err[k.substr(8)] = v;
    } else if (k == "cu_frac" || k == "spill_cost" || k == "merge_trip" || k == "salu_w") {
      (k == "cu_frac" ? c.cu_frac : k == "spill_cost" ? c.spill_cost : k == "merge_trip" ? c.merge_trip : c.salu_w) = v;
      c.cdna = true;
    } else {
      calibScalar(c, k) = v;
    }
  });
  return c;
}

std::string dumpCalib(const Calib &c) {
  std::ostringstream o;
  o << std::setprecision(8);
  Calib t = c;
  for (const char *k : calibScalarKeys()) o << k << " = " << calibScalar(t, k) << "\n";
  if (c.cdna)
    o << "cu_frac = " << c.cu_frac << "\nspill_cost = " << c.spill_cost << "\nmerge_trip = " << c.merge_trip
      << "\nsalu_w = " << c.salu_w << "\n";
  for (const auto &kv : c.rel_err) o << "rel_err." << kv.first << " = " << kv.second << "\n";
  return o.str();
}

void saveCalib(const Calib &c, const std::filesystem::path &p) {
  std::ofstream o(p);
  if (!o) throw std::runtime_error("cannot write " + p.string());
  o << "# KVForge cost-model constants. Fitted once on one GPU, then frozen.\n" << dumpCalib(c);
}

// ======================================================================= cost model
double idealIntensity(const DecodeSpec &s, const KvFormat &f) {
  // 4nd FLOPs per query head over 2nd*b_eff bytes per KV head
  return 2.0 * s.g() / f.effectiveBytes();
}

namespace {

// eta_run = run / (run + r0), normalised so an unbounded run scores 1
// (src/cost.cpp:64-69).
double runEfficiency(double run, double r0) {
  const double big = 1 << 22;
  const double ref = big / (big + r0);
  return std::min(1.0, (run / (run + r0)) / ref);
}

// Contiguous bytes one block reads before it jumps (src/cost.cpp:51-60);
// the gfx950 kernels read the same runs (a workgroup scans one KV head).
double runBytes(const DecodeSpec &s, const KvFormat &f, const KvLayout &l, double chunk) {
  const double row = f.dataRowBytes(s.d);
  if (l.order == Order::TokenMajor) return row;
  if (l.paged()) return std::min<double>(l.block_tokens, chunk) * row;
  return chunk * row;
}

// Accuracy gate shared by both forms of the model.
void gate(Cost &k, const Calib &c, const Plan &p, double max_rel_err) {
  if (p.fmt.isQuantized()) {
    const auto it = c.rel_err.find(p.fmt.key());
    k.rel_err = it == c.rel_err.end() ? 1.0 : it->second;
  }
  if (max_rel_err > 0 && k.rel_err > max_rel_err) {
    k.rejected = true;
    k.note = "rejected: error above accuracy limit";
  }
}

// Common byte and FLOP accounting (src/cost.cpp:88-137).
void countBytes(Cost &k, const DecodeSpec &s, const Machine &m, const Calib &c, const Plan &p,
                double reread, double &main_bytes) {
  const double rows = 1.0 * s.tokens() * s.H_kv;
  const double data_row = p.fmt.dataRowBytes(s.d);
  const double meta_row = p.fmt.metaRowBytes(s.d);
  k.kv_bytes = 2.0 * rows * data_row * reread;
  double meta_eff = 1.0;
  if (meta_row > 0 && p.layout.order == Order::TokenMajor)
    meta_eff = std::min(1.0, meta_row / m.sector_bytes);
  k.meta_bytes = 2.0 * rows * meta_row * reread / std::pow(meta_eff, c.meta_waste);
  k.qo_bytes = 2.0 * s.H * s.d * 4.0 * s.batch;
  if (p.part.splits > 1) k.partial_bytes = 2.0 * s.H * p.part.splits * (s.d + 2) * 4.0 * s.batch;
  main_bytes = k.kv_bytes + k.meta_bytes + k.qo_bytes;
  k.total_bytes = main_bytes + k.partial_bytes;
  const int loading_heads = p.part.gqa_pack ? s.H_kv : s.H;
  k.attn_flops = 4.0 * s.tokens() * s.d * s.H;
  const double elems = 2.0 * s.tokens() * s.d * loading_heads;
  k.dequant_flops = elems * p.fmt.dequantFlopsPerElem();
  k.total_flops = k.attn_flops + k.dequant_flops;
  k.intensity = k.total_bytes > 0 ? k.total_flops / k.total_bytes : 0;
}

// Memory time over the launch's waves of resident blocks
// (src/cost.cpp:161-195).
template <class Agg>
void memoryTime(Cost &k, const Calib &c, long long capacity, int sms, long long per_sm,
                double main_bytes, Agg &&aggregate) {
  k.bw_eff_gbs = aggregate(std::min(k.blocks, capacity));
  const double per_block_bytes = main_bytes / static_cast<double>(k.blocks);
  const long long full = k.blocks / capacity;
  const long long tail = k.blocks - full * capacity;
  double t = 0;
  if (full > 0) t += full * (capacity * per_block_bytes) / (aggregate(capacity) * 1000.0);
  if (tail > 0) t += (tail * per_block_bytes) / (aggregate(tail) * 1000.0);
  const double ideal = main_bytes / (k.bw_eff_gbs * 1000.0);
  if (c.wave_model < 0.5) {
    if (k.blocks > capacity) {
      const long long waves = (k.blocks + capacity - 1) / capacity;
      k.imbalance = static_cast<double>(waves * capacity) / static_cast<double>(k.blocks);
    } else if (k.blocks > sms) {
      k.imbalance = static_cast<double>(per_sm * sms) / static_cast<double>(k.blocks);
    } else {
      k.imbalance = 1.0;
    }
    k.t_mem_us = ideal * k.imbalance;
  } else {
    k.t_mem_us = t;
    k.imbalance = ideal > 0 ? t / ideal : 1.0;
  }
}

// ------------------------------------------------------------ 32-lane warps
// Registers per thread of the plan's kernel from the machine's resource
// table, else the reference's estimate (src/cost.cpp:40-49).
int warpKernelRegs(const Machine &m, const DecodeSpec &s, const Plan &p) {
  const int fmt = p.fmt.fmt == Format::F16 ? 0 : p.fmt.fmt == Format::INT8 ? 1 : 2;
  const int g = p.part.gqa_pack ? s.g() : 1;
  const int ord = p.layout.order == Order::HeadMajor ? 0 : 1;
  const int fin = p.part.splits == 1 ? 1 : 0;
  const std::string key = std::to_string(fmt) + "_" + std::to_string(s.d) + "_" + std::to_string(g) + "_" +
                          std::to_string(p.part.unroll) + "_" + std::to_string(ord) + "_" +
                          std::to_string(p.layout.paged() ? 1 : 0) + "_" + std::to_string(fin);
  const int r = m.regsFor(key);
  return r > 0 ? r : 64 + 22 * g + 8 * p.part.unroll;
}

Cost warpEvaluate(const DecodeSpec &s, const Machine &m, const Calib &c, const Plan &p,
                  double max_rel_err) {
  Cost k;
  const int g = s.g();
  const bool pack = p.part.gqa_pack;
  const int loading_heads = pack ? s.H_kv : s.H;

  int resident_cap = std::max(1, std::min(m.max_blocks_per_sm, m.max_warps_per_sm / p.part.warps));
  if (m.regs_per_sm > 0) {
    const int regs = (warpKernelRegs(m, s, p) + 7) / 8 * 8;
    const int warp_regs = (regs * 32 + 255) / 256 * 256;
    resident_cap = std::max(1, std::min(resident_cap, m.regs_per_sm / (warp_regs * p.part.warps)));
  }
  const double resident_total = 1.0 * m.sms * resident_cap;
  const double window = std::clamp(resident_total / (1.0 * g * p.part.splits), 0.0, 1.0);
  const double reread = pack ? 1.0 : 1.0 + (g - 1) * (1.0 - c.unpack_l2_hit * window);
  double main_bytes = 0;
  countBytes(k, s, m, c, p, reread, main_bytes);

  k.blocks = 1LL * p.part.splits * loading_heads * s.batch;
  k.active_sms = static_cast<int>(std::min<long long>(k.blocks, m.sms));
  const long long per_sm = (k.blocks + m.sms - 1) / m.sms;
  k.resident_blocks = static_cast<int>(std::clamp<long long>(per_sm, 1, resident_cap));

  // every lane keeps `unroll` 8-element vectors of K and V in flight
  const int lane_vec = 8 * p.fmt.rawBits() / 8;
  const double bif_block = 1.0 * p.part.warps * 32 * lane_vec * p.part.unroll * 2.0;
  k.bif_sm_bytes = k.resident_blocks * bif_block;

  const double chunk = std::ceil(static_cast<double>(s.n) / p.part.splits);
  k.eta = runEfficiency(runBytes(s, p.fmt, p.layout, chunk), c.r0_bytes);

  const long long capacity = static_cast<long long>(resident_total);
  auto aggregate = [&](long long nb) {
    const long long act = std::min<long long>(nb, m.sms);
    const long long per = std::clamp<long long>((nb + m.sms - 1) / m.sms, 1, resident_cap);
    return k.eta * m.bwDeviceGbs(static_cast<int>(act), per * bif_block, c.lat_scale);
  };
  memoryTime(k, c, capacity, m.sms, per_sm, main_bytes, aggregate);

  // issue time: warp instructions of the reference kernel's inner loop
  // (src/cost.cpp:17-38, 196-211)
  {
    const int lanes = s.d / 8;
    const double tokens_per_warp_step = 32.0 / lanes;
    const int pack_g = pack ? g : 1;
    const bool q = p.fmt.isQuantized();
    const double unpack = p.fmt.fmt == Format::F16 ? 8.0 : 32.0;
    const double per_token = 10.0 + unpack;
    const double reduce = 2.0 * std::log2(static_cast<double>(lanes));
    const double per_token_head = 8.0 + (q ? 2.0 : 0.0) + reduce + 12.0 + (q ? 16.0 : 8.0);
    const double visits = 1.0 * s.batch * loading_heads * s.n;
    const double warp_instr = visits * (per_token + pack_g * per_token_head) / tokens_per_warp_step;
    const double rate_per_sm = m.fSmGflops() / 64.0;
    const double warps_per_sm = 1.0 * k.resident_blocks * p.part.warps;
    const double occupancy = 1.0 - std::exp(-warps_per_sm / c.warp_w0);
    k.t_cmp_us = warp_instr / (std::max(1, k.active_sms) * rate_per_sm * c.issue_eff * occupancy) / 1000.0;
  }
  k.memory_bound = k.t_mem_us >= k.t_cmp_us;
  const double t_par =
      std::pow(std::pow(k.t_mem_us, c.overlap_p) + std::pow(k.t_cmp_us, c.overlap_p), 1.0 / c.overlap_p);
  if (p.part.splits > 1) k.t_merge_us = c.merge_frac * m.launch_us + k.partial_bytes / (m.bw_l2_gbs * 1000.0);
  if (p.layout.paged() && p.layout.block_tokens > 0) {
    const double pages = std::ceil(chunk / p.layout.block_tokens) * k.blocks * p.part.warps;
    const double parallel = std::max(1.0, 1.0 * k.active_sms * k.resident_blocks * p.part.warps);
    k.t_page_us = pages * c.c_page_ns / parallel / 1000.0;
  }
  k.t_launch_us = c.launch_frac * m.launch_us;
  k.t_total_us = t_par + k.t_merge_us + k.t_page_us + k.t_launch_us;
  k.achieved_gbs = k.t_total_us > 0 ? (k.kv_bytes + k.meta_bytes) / (k.t_total_us * 1000.0) : 0;
  k.frac_of_peak = m.bw_peak_gbs > 0 ? k.achieved_gbs / m.bw_peak_gbs : 0;
  gate(k, c, p, max_rel_err);
  return k;
}

// ------------------------------------------------------------ CDNA (wave64)
// The gfx950 split kernel (kvforge_amd/csrc/kvf_kernels.hpp) works in
// 32-token tiles: a wave keeps depth(U) - 1 tiles in flight ahead of the one
// it computes, tiles are dealt round-robin to the W waves of a workgroup, and
// one workgroup covers one (split, KV head or query head, sequence). Terms:
//
//   residency  workgroups per CU = min(blocks per CU, waves/SIMD * 4 / W) from
//              the compiler's occupancy for that instantiation (resource
//              table), else from a register estimate; blocks beyond
//              CUs x residency run in further rounds
//   stream     per workgroup min(cu_frac * bw_sm / workgroups on its CU,
//              bytes in flight / (lat * lat_scale)) (Little's law), the device
//              capped at bw_peak * eta (run-length efficiency)
//   fill       bytes in flight at the start, drained at peak bandwidth before
//              the stream is steady: deeper rings and more waves cost queueing
//   GQA        unpacked query heads re-read their KV head; the re-reads hit L2
//              with probability unpack_l2_hit * window and go at bw_l2, the
//              rest come from HBM again
//   issue      VALU wave-instructions and MFMA issue slots (cycles / 4) per
//              tile at one per SIMD slot, waves per SIMD sharing it: their sum
//              for a wave alone on its SIMD, the larger of the two once two or
//              more waves share it (one's MFMAs run under another's VALU);
//              spills (scratch bytes per lane) costing spill_cost per 64 B.
//              The counts are the compiled loop's own (resource table
//              columns valu, mfma, lds, and salu weighted salu_w) where the
//              table has them, else the estimate of cdnaTile
//   fixed      launch_frac of launch_us, plus warp_w0 loaded latencies per
//              round of workgroups (query load, first tile, wave combine and
//              partial write)
//   merge      the second kernel: merge_frac of launch_us, then one
//              workgroup per (sequence, query head) folding its S partial
//              rows in chunks of 32, 1, 2, 4 or 8 chunks side by side
//              (kvf_merge.hip), so ceil(chunks / slices) round trips of
//              merge_trip * lat_ns, and the rows streamed at one
//              workgroup's rate (cu_frac * bw_sm)
//   paging     c_page_ns per page a workgroup walks, per round
struct CdnaTile {
  int depth = 2;     // ring of tiles per wave
  double bytes = 0;  // K + V + meta bytes of one tile
  double valu = 0;   // VALU wave-instructions per tile
  double mfma = 0;   // MFMA issue slots per tile (cycles / 4)
};

CdnaTile cdnaTile(const DecodeSpec &s, const Plan &p, int G) {
  CdnaTile t;
  t.depth = p.part.unroll == 2 ? 2 : 3;
  t.bytes = 32.0 * 2.0 * (p.fmt.dataRowBytes(s.d) + p.fmt.metaRowBytes(s.d));
  const int ng = p.fmt.isQuantized() ? s.d / p.fmt.group : 1;
  const int cols = G * ng;
  const bool hl = cols <= 8; // hi/lo share one MFMA
  const int passes = cols > 16 ? 2 : 1;
  const int nq = hl ? 1 : 2;
  // QK: 2 sub-tiles x D/32 k-steps x (hi, lo) x passes; PV: D/16 per (hi, lo, pass)
  const double mfma = 2.0 * (s.d / 32) * nq * passes + 1.0 * (s.d / 16) * nq * passes;
  // code -> binary16 conversions per element of K and V, softmax per token slot
  const double k_conv = p.fmt.fmt == Format::F16 ? 0.0 : p.fmt.fmt == Format::INT8 ? 0.5 : 0.75;
  const double v_conv = p.fmt.fmt == Format::INT4 ? 0.8 : 0.5;
  const double softmax = 8.0 * (p.fmt.isQuantized() ? 9.0 : 6.0) * passes;
  t.valu = (k_conv + v_conv) * 32.0 * s.d / 64.0 + softmax + 24.0;
  t.mfma = 16.0 * mfma / 4.0;
  return t;
}

std::string cdnaKernelKey(const DecodeSpec &s, const Plan &p, int G) {
  const int fmt = p.fmt.fmt == Format::F16 ? 0 : p.fmt.fmt == Format::INT8 ? 1 : 2;
  const int group = p.fmt.isQuantized() ? p.fmt.group : 0;
  return std::to_string(fmt) + "_" + std::to_string(s.d) + "_" + std::to_string(group) + "_" + std::to_string(G) +
         "_" + std::to_string(p.part.unroll) + "_" + std::to_string(p.layout.order == Order::HeadMajor ? 0 : 1) +
         "_" + std::to_string(p.layout.paged() ? 1 : 0) + "_" + std::to_string(p.part.warps);
}

Machine::KernelRes cdnaResources(const Machine &m, const DecodeSpec &s, const Plan &p, int G, const CdnaTile &t) {
  const auto it = m.kernel_res.find(cdnaKernelKey(s, p, G));
  if (it != m.kernel_res.end()) return it->second;
  // estimate: query operands, accumulators and the ring in VGPRs; 512
  // registers per lane and SIMD, granule 8
  Machine::KernelRes r;
  r.vgpr = static_cast<int>(std::min(512.0, 96.0 + t.bytes / 64.0 / 4.0 * t.depth));
  const int alloc = (r.vgpr + 7) / 8 * 8;
  r.occupancy = std::max(1, std::min(8, 512 / alloc));
  return r;
}

Cost cdnaEvaluate(const DecodeSpec &s, const Machine &m, const Calib &c, const Plan &p,
                  double max_rel_err) {
  Cost k;
  const int g = s.g();
  const bool pack = p.part.gqa_pack;
  const int G = pack ? g : 1;
  const int loading_heads = pack ? s.H_kv : s.H;
  const int waves = p.part.warps;
  CdnaTile t = cdnaTile(s, p, G);
  const Machine::KernelRes kr = cdnaResources(m, s, p, G, t);
  if (kr.mfma > 0) {
    // the compiled loop's own counts replace the estimate; a cross-row
    // shuffle through LDS occupies an issue slot like a VALU instruction, a
    // scalar instruction salu_w of one
    t.valu = kr.valu + kr.lds + c.salu_w * kr.salu;
    t.mfma = 16.0 * kr.mfma / 4.0;
  }

  // residency and rounds
  const int resident_cap =
      std::max(1, std::min({m.max_blocks_per_sm, m.max_warps_per_sm / waves, kr.occupancy * 4 / waves}));
  const long long capacity = 1LL * m.sms * resident_cap;
  k.blocks = 1LL * p.part.splits * loading_heads * s.batch;
  const long long conc = std::min(k.blocks, capacity);
  const long long rounds = (k.blocks + capacity - 1) / capacity;
  const long long per_cu = (conc + m.sms - 1) / m.sms;
  k.active_sms = static_cast<int>(std::min<long long>(conc, m.sms));
  k.resident_blocks = static_cast<int>(per_cu);
  k.imbalance = static_cast<double>(rounds * capacity) / static_cast<double>(k.blocks);

  // unpacked GQA: the g query heads of a KV head share its rows through L2
  // while they are resident together
  const double window = std::clamp(static_cast<double>(capacity) / (1.0 * g * p.part.splits), 0.0, 1.0);
  const double hit = pack ? 0.0 : c.unpack_l2_hit * window;
  const double reread_hbm = pack ? 1.0 : 1.0 + (g - 1) * (1.0 - hit);
  double main_bytes = 0;
  countBytes(k, s, m, c, p, reread_hbm, main_bytes);

  // chunk of an average workgroup and of the longest sequence's workgroups
  // (split s of sequence b covers ceil(len_b / splits) tokens); they are equal
  // when every sequence holds n tokens
  const double chunk = std::ceil(static_cast<double>(s.tokens()) / s.batch / p.part.splits);
  const double chunk_max = std::ceil(static_cast<double>(s.maxLen()) / p.part.splits);
  k.eta = runEfficiency(runBytes(s, p.fmt, p.layout, chunk), c.r0_bytes);
  const double lat_us = m.lat_ns * std::max(1.0, c.lat_scale) / 1000.0;

  // stream: bytes per workgroup from HBM and (re-reads) from L2
  const double wg_kv = (k.kv_bytes + k.meta_bytes) / static_cast<double>(k.blocks);
  const double wg_l2 = pack ? 0.0 : wg_kv / reread_hbm * (g - 1) * hit;
  const double bif_wg = 1.0 * waves * (t.depth - 1) * t.bytes;
  k.bif_sm_bytes = per_cu * bif_wg;
  const double r_wg = std::min(c.cu_frac * m.bw_sm_gbs / per_cu, bif_wg / 1000.0 / lat_us); // GB/s
  const double peak = m.bw_peak_gbs * k.eta;
  k.bw_eff_gbs = std::min(peak, conc * r_wg);
  const double l2 = m.bw_l2_gbs > 0 ? m.bw_l2_gbs : m.bw_peak_gbs;
  k.t_mem_us = rounds * (conc * wg_kv / (k.bw_eff_gbs * 1000.0) + conc * wg_l2 / (l2 * 1000.0));

  // issue: tiles per wave, waves per SIMD sharing its slots. A wave alone on
  // its SIMD waits on its own MFMA chain between VALU sections; with two or
  // more, the matrix core runs one wave's MFMAs while another issues VALU, so
  // a tile costs the SIMD the larger of the two rather than their sum
  const double tiles_wave = std::ceil((std::ceil(chunk / 32.0) + 1.0) / waves);
  const double simd_waves = std::max(1.0, waves * per_cu / 4.0);
  const double simd_rate = m.fSmGflops() / 4.0 / 128.0; // wave-instructions per ns per SIMD
  const double per_tile = simd_waves >= 2.0 ? std::max(t.valu, t.mfma) : t.valu + t.mfma;
  k.t_cmp_us = rounds * tiles_wave * per_tile * simd_waves * (1.0 + c.spill_cost * kr.scratch / 64.0) /
               (simd_rate * std::max(1e-6, c.issue_eff)) / 1000.0;
  k.memory_bound = k.t_mem_us >= k.t_cmp_us;
  // critical path: the step cannot end before the longest sequence's
  // workgroups, which stream their chunk at no more than one workgroup's rate
  // on an otherwise idle CU and issue their tiles with only their own waves on
  // the SIMDs. With equal lengths this never exceeds the throughput terms.
  const double r_alone = std::min(c.cu_frac * m.bw_sm_gbs, bif_wg / 1000.0 / lat_us);
  const double t_crit_mem = wg_kv * (chunk_max / std::max(1.0, chunk)) / (r_alone * 1000.0);
  const double tiles_max = std::ceil((std::ceil(chunk_max / 32.0) + 1.0) / waves);
  const double own = std::max(1.0, waves / 4.0);
  const double t_crit_cmp = tiles_max * (own >= 2.0 ? std::max(t.valu, t.mfma) : t.valu + t.mfma) * own *
                            (1.0 + c.spill_cost * kr.scratch / 64.0) /
                            (simd_rate * std::max(1e-6, c.issue_eff)) / 1000.0;
  const double t_par = std::max(
      std::pow(std::pow(k.t_mem_us, c.overlap_p) + std::pow(k.t_cmp_us, c.overlap_p), 1.0 / c.overlap_p),
      std::pow(std::pow(t_crit_mem, c.overlap_p) + std::pow(t_crit_cmp, c.overlap_p), 1.0 / c.overlap_p));

  // fill: the bytes requested at the start queue at peak bandwidth
  const double t_fill = conc * bif_wg / (peak * 1000.0);
  if (p.part.splits > 1) {
    const int chunks = (p.part.splits + 31) / 32;
    const int slices = chunks <= 1 ? 1 : chunks == 2 ? 2 : chunks <= 4 ? 4 : 8;
    const double trips = std::ceil(static_cast<double>(chunks) / slices);
    const double wg_rows = 4.0 * p.part.splits * (s.d + 2);
    k.t_merge_us = c.merge_frac * m.launch_us + trips * c.merge_trip * m.lat_ns / 1000.0 +
                   wg_rows / (c.cu_frac * m.bw_sm_gbs * 1000.0);
  }
  if (p.layout.paged() && p.layout.block_tokens > 0)
    k.t_page_us = rounds * std::ceil(chunk_max / p.layout.block_tokens) * c.c_page_ns / 1000.0;
  k.t_launch_us = c.launch_frac * m.launch_us + c.warp_w0 * lat_us * rounds + t_fill;
  k.t_total_us = t_par + k.t_merge_us + k.t_page_us + k.t_launch_us;
  k.achieved_gbs = k.t_total_us > 0 ? (k.kv_bytes + k.meta_bytes) / (k.t_total_us * 1000.0) : 0;
  k.frac_of_peak = m.bw_peak_gbs > 0 ? k.achieved_gbs / m.bw_peak_gbs : 0;
  gate(k, c, p, max_rel_err);
  return k;
}

} // namespace

Cost evaluate(const DecodeSpec &s, const Machine &m, const Calib &c, const Plan &p, double max_rel_err) {
  return m.cdna() ? cdnaEvaluate(s, m, c, p, max_rel_err) : warpEvaluate(s, m, c, p, max_rel_err);
}

std::vector<Ranked> rankPlans(const DecodeSpec &s, const Machine &m, const Calib &c,
                              const std::vector<Plan> &plans, double max_rel_err) {
  std::vector<Ranked> out;
  out.reserve(plans.size());
  for (const auto &p : plans) out.push_back(Ranked{p, evaluate(s, m, c, p, max_rel_err)});
  std::stable_sort(out.begin(), out.end(),
                   [](const Ranked &a, const Ranked &b) { return a.cost.t_total_us < b.cost.t_total_us; });
  return out;
}

} // namespace kvfc
