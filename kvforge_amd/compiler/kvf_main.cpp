// kvf_main.cpp - the kvf command line (same commands and options as the
// reference's src/main.cpp:38-333, so scripts written for it keep working).
#include "kvf_emit.h"
#include "kvf_fit.h"
#include "kvf_front.h"

#include <filesystem>
#include <algorithm>
#include <fstream>
#include <iomanip>
#include <iostream>
#include <map>
#include <set>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

using namespace kvfc;

namespace {

std::string slurp(const std::filesystem::path &p) {
  std::ifstream in(p, std::ios::binary);
  if (!in) throw std::runtime_error("cannot read " + p.string());
  std::ostringstream s;
  s << in.rdbuf();
  return s.str();
}

void spill(const std::filesystem::path &p, const std::string &text) {
  if (!p.parent_path().empty()) std::filesystem::create_directories(p.parent_path());
  std::ofstream o(p, std::ios::binary);
  if (!o) throw std::runtime_error("cannot write " + p.string());
  o << text;
}

int usage() {
  std::cerr << "kvf - plans and generates split-KV decode attention for a measured GPU\n\n"
               "  kvf plan <file.kv> [--out DIR] [--top N] [--all] [--quant]\n"
               "                     [--machine FILE] [--calib FILE] [--max-err X]\n"
               "  kvf roofline <file.kv> [--machine FILE]\n"
               "  kvf machine <file.gpu>\n"
               "  kvf emit-dispatch [--out DIR] [--d 128,64] [--g 1,2,4,8]\n"
               "  kvf calibrate --sweep A.csv[,B.csv] --machine FILE [--out FILE] [--holdout-every N]\n"
               "  kvf predict   --sweep A.csv --machine FILE [--calib FILE] [--out FILE]\n"
               "  kvf evaluate  --sweep A.csv[,B.csv] --machine FILE [--calib FILE]\n"
               "                [--holdout-every N] [--which fit|heldout|all] [--only int8:64,...]\n\n"
               "  --quant        search lossy formats (int8, int4) too\n"
               "  --max-err X    accuracy limit for lossy formats (implies --quant)\n"
               "  --machine FILE machine description (overrides `target machine`)\n"
               "  --calib FILE   fitted cost-model constants (overrides `target calib`)\n"
               "  --top N        rows of the ranking in the report (default 12); --all for every row\n"
               "A machine file with `wave_size = 64` (kvforge_amd/bin/bw_probe writes one) selects the\n"
               "CDNA cost model.\n";
  return 2;
}

struct Cli {
  std::string cmd;
  std::vector<std::string> positional;
  std::map<std::string, std::string> opts;
  std::set<std::string> flags;
  bool has(const std::string &k) const { return opts.count(k) || flags.count(k); }
  std::string opt(const std::string &k, const std::string &dflt = "") const {
    const auto it = opts.find(k);
    return it == opts.end() ? dflt : it->second;
  }
};

Cli parseCli(int argc, char **argv) {
  Cli c;
  c.cmd = argv[1];
  for (int i = 2; i < argc; ++i) {
    const std::string a = argv[i];
    if (a.rfind("--", 0) != 0) {
      c.positional.push_back(a);
      continue;
    }
    const std::string k = a.substr(2);
    if (k == "all" || k == "quant") c.flags.insert(k);
    else if (i + 1 < argc) c.opts[k] = argv[++i];
    else throw std::runtime_error("option --" + k + " needs a value");
  }
  return c;
}

std::vector<int> ints(const std::string &s) {
  std::vector<int> v;
  std::stringstream ss(s);
  std::string t;
  while (std::getline(ss, t, ','))
    if (!t.empty()) v.push_back(std::stoi(t));
  return v;
}

Module compileFront(const Cli &c) {
  if (c.positional.empty()) throw std::runtime_error("missing input file");
  Module m = lowerSource(parseSource(slurp(c.positional[0])));
  if (c.has("machine")) {
    m.machine = loadMachine(c.opt("machine"));
    m.machine_file = c.opt("machine");
  }
  if (c.has("calib")) {
    m.calib = loadCalib(c.opt("calib"));
    m.calib_file = c.opt("calib");
  }
  if (c.flags.count("quant")) m.space.include_quantized = true;
  if (c.has("max-err")) {
    m.space.max_rel_err = std::stod(c.opt("max-err"));
    m.space.include_quantized = true;
  }
  return m;
}

std::vector<SweepRow> sweeps(const std::string &list) {
  std::vector<SweepRow> rows;
  std::stringstream ss(list);
  std::string p;
  while (std::getline(ss, p, ',')) {
    auto part = loadSweep(p);
    rows.insert(rows.end(), part.begin(), part.end());
  }
  return rows;
}

int run(const Cli &c) {
  if (c.cmd == "machine") {
    if (c.positional.empty()) return usage();
    const Machine m = loadMachine(c.positional[0]);
    std::cout << dumpMachine(m) << "# derived\n"
              << "# ridge          = " << m.ridgeFlopPerByte() << " FLOP/byte\n"
              << "# f_sm_gflops    = " << m.fSmGflops() << "\n"
              << "# bw_device(all, full flight) = " << m.bwDeviceGbs(m.sms, 1e9) << " GB/s\n"
              << "# cost model     = " << (m.cdna() ? "cdna" : "warp") << "\n";
    return 0;
  }
  if (c.cmd == "emit-dispatch") {
    const std::filesystem::path out = c.opt("out", "gen");
    const auto files = dispatchSources(ints(c.opt("d", "128,64")), ints(c.opt("g", "1,2,4,8")), true);
    std::filesystem::create_directories(out);
    for (const auto &[name, text] : files) spill(out / name, text);
    std::cout << "wrote " << files.size() << " dispatch sources to " << out.string() << "\n";
    for (const auto &f : files) std::cout << f.first << "\n";
    return 0;
  }
  if (c.cmd == "predict") {
    if (!c.has("sweep") || !c.has("machine")) return usage();
    const auto rows = loadSweep(c.opt("sweep"));
    const Machine m = loadMachine(c.opt("machine"));
    const Calib k = c.has("calib") ? loadCalib(c.opt("calib")) : Calib::defaults();
    std::ostringstream o;
    o << "shape,fmt,group,order,residency,block_tokens,splits,gqa_pack,warps,unroll,"
         "t_us,pred_us,pred_mem_us,pred_merge_us,pred_page_us,eta,verified,err_exact\n";
    o << std::setprecision(10);
    for (const auto &r : rows) {
      const Cost e = evaluate(r.spec, m, k, r.plan);
      o << shapeKey(r.spec) << ',' << formatName(r.plan.fmt.fmt) << ',' << r.plan.fmt.group << ','
        << orderName(r.plan.layout.order) << ',' << residencyName(r.plan.layout.residency) << ','
        << r.plan.layout.block_tokens << ',' << r.plan.part.splits << ',' << (r.plan.part.gqa_pack ? 1 : 0) << ','
        << r.plan.part.warps << ',' << r.plan.part.unroll << ',' << r.t_us << ',' << e.t_total_us << ','
        << e.t_mem_us << ',' << e.t_merge_us << ',' << e.t_page_us << ',' << e.eta << ',' << (r.verified ? 1 : 0)
        << ',' << r.err_exact << "\n";
    }
    const std::string out = c.opt("out", "predicted.csv");
    spill(out, o.str());
    std::cout << "wrote " << out << " (" << rows.size() << " rows)\n";
    return 0;
  }
  if (c.cmd == "calibrate" || c.cmd == "evaluate") {
    if (!c.has("sweep") || !c.has("machine")) return usage();
    const auto rows = sweeps(c.opt("sweep"));
    const Machine m = loadMachine(c.opt("machine"));
    const auto held_list = heldOutShapes(rows, std::stoi(c.opt("holdout-every", "3")));
    const std::set<std::string> held(held_list.begin(), held_list.end());
    const ShapeFilter fitted = [&](const std::string &k) { return !held.count(k); };
    const ShapeFilter heldout = [&](const std::string &k) { return held.count(k) > 0; };
    const ShapeFilter every = [](const std::string &) { return true; };
    if (c.cmd == "calibrate") {
      Calib start = Calib::defaults();
      if (c.has("wave-model")) start.wave_model = std::stod(c.opt("wave-model"));
      const Calib k = calibrate(rows, m, start, fitted);
      if (c.has("out")) saveCalib(k, c.opt("out"));
      std::cout << "fitted constants (machine " << m.name << ", " << rows.size() << " rows, " << held.size()
                << " held-out shapes)\n"
                << dumpCalib(k) << "\n"
                << evaluationReport(rows, m, k, fitted);
      if (!held.empty())
        std::cout << "=== HELD-OUT shapes (not used in the fit) ===\n" << evaluationReport(rows, m, k, heldout);
      return 0;
    }
    const Calib k = c.has("calib") ? loadCalib(c.opt("calib")) : Calib::defaults();
    const std::string which = c.opt("which", "all");
    const ShapeFilter &pick = which == "fit" ? fitted : which == "heldout" ? heldout : every;
    std::cout << "machine " << m.name << ", constants " << (c.has("calib") ? c.opt("calib") : "defaults")
              << ", shapes: " << which << "\n\n";
    if (c.has("only")) {
      // e.g. --only int8:64,int8:128 : the plans of those formats alone
      std::vector<std::string> keys;
      std::stringstream ss(c.opt("only"));
      std::string f;
      while (std::getline(ss, f, ',')) {
        std::replace(f.begin(), f.end(), ':', '_');
        keys.push_back(f);
      }
      std::cout << evaluationReport(rows, m, k, pick, keys);
    } else {
      std::cout << evaluationReport(rows, m, k, pick);
    }
    return 0;
  }
  if (c.positional.empty()) return usage();
  Module mod = compileFront(c);
  if (c.cmd == "roofline") {
    std::cout << rooflineText(mod);
    return 0;
  }
  if (c.cmd != "plan") return usage();
  const std::string before = printModule(mod);
  planModule(mod);
  const int top = c.flags.count("all") ? 0 : std::stoi(c.opt("top", "12"));
  const Written w = writePlanOutputs(mod, c.opt("out", "out"), before, top);
  std::cout << slurp(w.report) << "\nwrote " << w.report.string() << "\nwrote " << w.plans_csv.string()
            << "\nwrote " << w.ir_txt.string() << "\nwrote " << w.kernel.string() << "\n";
  return 0;
}

} // namespace

int main(int argc, char **argv) {
  if (argc < 2) return usage();
  try {
    return run(parseCli(argc, argv));
  } catch (const std::exception &e) {
    std::cerr << "kvf: " << e.what() << "\n";
    return 1;
  }
}
