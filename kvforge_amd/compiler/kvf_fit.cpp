// kvf_fit.cpp - sweep scoring and calibration of the cost model.
#include "kvf_fit.h"

#include <algorithm>
#include <cmath>
#include <fstream>
#include <iomanip>
#include <map>
#include <numeric>
#include <set>
#include <sstream>
#include <stdexcept>

namespace kvfc {

namespace {

std::vector<std::string> cells(const std::string &line) {
  std::vector<std::string> out(1);
  for (char ch : line) {
    if (ch == ',') out.emplace_back();
    else if (ch != '\r') out.back().push_back(ch);
  }
  return out;
}

// Ranks with ties sharing their average rank (1-based).
std::vector<double> tiedRanks(const std::vector<double> &v) {
  std::vector<std::size_t> order(v.size());
  std::iota(order.begin(), order.end(), 0);
  std::sort(order.begin(), order.end(), [&](std::size_t a, std::size_t b) { return v[a] < v[b]; });
  std::vector<double> r(v.size());
  std::size_t i = 0;
  while (i < order.size()) {
    std::size_t j = i;
    while (j + 1 < order.size() && v[order[j + 1]] == v[order[i]]) ++j;
    const double shared = 0.5 * static_cast<double>(i + j) + 1.0;
    for (std::size_t k = i; k <= j; ++k) r[order[k]] = shared;
    i = j + 1;
  }
  return r;
}

double correlation(const std::vector<double> &a, const std::vector<double> &b) {
  const double n = static_cast<double>(a.size());
  const double ma = std::accumulate(a.begin(), a.end(), 0.0) / n;
  const double mb = std::accumulate(b.begin(), b.end(), 0.0) / n;
  double sab = 0, saa = 0, sbb = 0;
  for (std::size_t i = 0; i < a.size(); ++i) {
    sab += (a[i] - ma) * (b[i] - mb);
    saa += (a[i] - ma) * (a[i] - ma);
    sbb += (b[i] - mb) * (b[i] - mb);
  }
  return saa > 0 && sbb > 0 ? sab / std::sqrt(saa * sbb) : 0.0;
}

// Kendall's tau-a over concordant and discordant pairs (ties count as neither).
double kendall(const std::vector<double> &a, const std::vector<double> &b) {
  long long agree = 0, disagree = 0;
  for (std::size_t i = 0; i < a.size(); ++i)
    for (std::size_t j = i + 1; j < a.size(); ++j) {
      const double s = (a[i] - a[j]) * (b[i] - b[j]);
      agree += s > 0;
      disagree += s < 0;
    }
  const long long pairs = agree + disagree;
  return pairs ? static_cast<double>(agree - disagree) / static_cast<double>(pairs) : 0.0;
}

bool eligible(const SweepRow &r, const Calib &c, const Eligibility &e) {
  if (!e.keys.empty() && std::find(e.keys.begin(), e.keys.end(), r.plan.fmt.key()) == e.keys.end()) return false;
  if (!e.formats.empty() &&
      std::find(e.formats.begin(), e.formats.end(), std::string(formatName(r.plan.fmt.fmt))) == e.formats.end())
    return false;
  if (e.max_rel_err > 0 && r.plan.fmt.isQuantized()) {
    const auto it = c.rel_err.find(r.plan.fmt.key());
    if ((it == c.rel_err.end() ? 1.0 : it->second) > e.max_rel_err) return false;
  }
  return true;
}

} // namespace

std::string shapeKey(const DecodeSpec &s) {
  std::string k = "H" + std::to_string(s.H) + "_Hkv" + std::to_string(s.H_kv) + "_d" + std::to_string(s.d) + "_n" +
                  std::to_string(s.n) + "_b" + std::to_string(s.batch);
  if (!s.lens_spec.empty()) {
    k += "_";
    for (char ch : s.lens_spec) k += ch == ':' ? '-' : ch;
  }
  return k;
}

std::vector<SweepRow> loadSweep(const std::filesystem::path &p) {
  std::ifstream in(p);
  if (!in) throw std::runtime_error("cannot read sweep file " + p.string());
  std::string line;
  if (!std::getline(in, line)) throw std::runtime_error("empty sweep file " + p.string());
  std::map<std::string, std::size_t> at;
  {
    const auto head = cells(line);
    for (std::size_t i = 0; i < head.size(); ++i) at[head[i]] = i;
  }
  for (const char *need : {"H", "H_kv", "d", "n", "batch", "fmt", "group", "order", "residency", "block_tokens",
                           "splits", "gqa_pack", "warps", "unroll", "t_us"})
    if (!at.count(need)) throw std::runtime_error(p.string() + ": missing column " + need);
  std::vector<SweepRow> rows;
  while (std::getline(in, line)) {
    if (line.empty()) continue;
    const auto f = cells(line);
    auto s = [&](const char *k) -> const std::string & { return f.at(at.at(k)); };
    auto i = [&](const char *k) { return std::stoi(s(k)); };
    auto x = [&](const char *k, double dflt) { return at.count(k) ? std::stod(f.at(at.at(k))) : dflt; };
    SweepRow r;
    r.spec.H = i("H");
    r.spec.H_kv = i("H_kv");
    r.spec.d = i("d");
    r.spec.n = i("n");
    r.spec.batch = i("batch");
    // per-sequence lengths (this build's extension): a distribution spec,
    // empty or absent when every sequence holds n tokens
    if (at.count("seq_lens") && !s("seq_lens").empty()) {
      r.spec.lens_spec = s("seq_lens");
      r.spec.lens = drawLengths(r.spec.lens_spec, r.spec.batch);
    }
    r.plan.fmt.fmt = parseFormat(s("fmt"));
    r.plan.fmt.group = i("group");
    r.plan.fmt.metadata_bits = r.plan.fmt.isQuantized() ? 32 : 0;
    r.plan.layout.order = parseOrder(s("order"));
    r.plan.layout.residency = parseResidency(s("residency"));
    r.plan.layout.block_tokens = i("block_tokens");
    r.plan.part.splits = i("splits");
    r.plan.part.gqa_pack = i("gqa_pack") != 0;
    r.plan.part.warps = i("warps");
    r.plan.part.unroll = i("unroll");
    r.t_us = x("t_us", 0);
    r.t_p25 = x("t_p25", 0);
    r.t_p75 = x("t_p75", 0);
    r.err_exact = x("err_exact", 0);
    r.verified = x("verified", 1.0) != 0;
    if (r.t_us > 0) rows.push_back(std::move(r));
  }
  return rows;
}

Metrics evaluateSweep(const std::vector<SweepRow> &rows, const Machine &m, const Calib &c, const Eligibility &e,
                      const ShapeFilter &use) {
  std::map<std::string, std::vector<const SweepRow *>> shapes;
  for (const auto &r : rows)
    if (r.verified && eligible(r, c, e) && use(shapeKey(r.spec))) shapes[shapeKey(r.spec)].push_back(&r);
  Metrics out;
  std::ostringstream lines;
  double ape = 0;
  long long n_ape = 0;
  for (const auto &[key, v] : shapes) {
    if (v.size() < 2) continue;
    std::vector<double> pred, meas;
    for (const SweepRow *r : v) {
      pred.push_back(evaluate(r->spec, m, c, r->plan).t_total_us);
      meas.push_back(r->t_us);
      ape += std::abs(pred.back() - r->t_us) / r->t_us;
      ++n_ape;
    }
    const double rho = correlation(tiedRanks(pred), tiedRanks(meas));
    const double tau = kendall(pred, meas);
    const std::size_t chosen = static_cast<std::size_t>(std::min_element(pred.begin(), pred.end()) - pred.begin());
    const double best = *std::min_element(meas.begin(), meas.end());
    const double regret = meas[chosen] / best - 1.0;
    out.spearman += rho;
    out.kendall += tau;
    out.regret_mean += regret;
    out.regret_max = std::max(out.regret_max, regret);
    out.top1 += regret <= 1e-9 ? 1.0 : 0.0;
    ++out.shapes;
    out.rows += static_cast<int>(v.size());
    lines << "  " << key << "  rows=" << v.size() << "  rho=" << rho << "  tau=" << tau
          << "  regret=" << 100.0 * regret << "%  chosen=" << v[chosen]->plan.str() << " (" << meas[chosen]
          << " us vs best " << best << " us)\n";
  }
  if (out.shapes) {
    out.spearman /= out.shapes;
    out.kendall /= out.shapes;
    out.regret_mean /= out.shapes;
    out.top1 /= out.shapes;
  }
  out.mape = n_ape ? ape / static_cast<double>(n_ape) : 0;
  out.per_shape = lines.str();
  return out;
}

Calib calibrate(const std::vector<SweepRow> &rows, const Machine &m, const Calib &start, const ShapeFilter &use) {
  std::vector<const SweepRow *> fit;
  for (const auto &r : rows)
    if (r.verified && use(shapeKey(r.spec))) fit.push_back(&r);
  if (fit.empty()) throw std::runtime_error("calibrate: no rows selected");

  std::map<std::string, std::vector<std::size_t>> shapes;
  for (std::size_t i = 0; i < fit.size(); ++i) shapes[shapeKey(fit[i]->spec)].push_back(i);
  // eligibility classes: 0 lossless, 1 up to int8, 2 everything
  auto inClass = [](const SweepRow &r, int cls) {
    return cls == 2 || (cls == 1 ? r.plan.fmt.fmt != Format::INT4 : r.plan.fmt.fmt == Format::F16);
  };
  std::vector<double> pred(fit.size());
  // loss = mean |log(pred/meas)| + w x mean selection regret over (shape,
  // class); w = 1 in the reference's form (src/fit.cpp:226-260), 3 in the CDNA
  // form: the planner acts on the ranking, so a wrong top-1 weighs more than
  // the same error spread over the other plans
  const double regret_w = m.cdna() ? 3.0 : 1.0;
  auto loss = [&](const Calib &c) {
    double log_err = 0;
    for (std::size_t i = 0; i < fit.size(); ++i) {
      pred[i] = evaluate(fit[i]->spec, m, c, fit[i]->plan).t_total_us;
      log_err += std::abs(std::log(std::max(pred[i], 1e-6) / fit[i]->t_us));
    }
    log_err /= static_cast<double>(fit.size());
    double regret = 0;
    int cases = 0;
    for (const auto &[key, idx] : shapes) {
      (void)key;
      for (int cls = 0; cls < 3; ++cls) {
        double best = 1e300, lowest_pred = 1e300, picked = 0;
        for (std::size_t i : idx) {
          if (!inClass(*fit[i], cls)) continue;
          best = std::min(best, fit[i]->t_us);
          if (pred[i] < lowest_pred) {
            lowest_pred = pred[i];
            picked = fit[i]->t_us;
          }
        }
        if (best < 1e299) {
          regret += picked / best - 1.0;
          ++cases;
        }
      }
    }
    return log_err + regret_w * (cases ? regret / cases : 0.0);
  };

  // Ten constants, each searched on a 41-point grid (log-spaced where the
  // range spans decades) that halves around the incumbent every round.
  struct Knob {
    double Calib::*field;
    double lo, hi;
    bool log;
  };
  std::vector<Knob> knobs = {
      {&Calib::r0_bytes, 2.0, 8192.0, true},     {&Calib::c_page_ns, 0.5, 4000.0, true},
      {&Calib::unpack_l2_hit, 0.0, 1.0, false},  {&Calib::issue_eff, 0.02, 1.0, true},
      {&Calib::meta_waste, 0.0, 2.0, false},     {&Calib::overlap_p, 1.0, 24.0, true},
      {&Calib::launch_frac, 0.0, 1.5, false},    {&Calib::merge_frac, 0.0, 1.5, false},
      {&Calib::lat_scale, 1.0, 40.0, true},      {&Calib::warp_w0, 0.5, 40.0, true},
  };
  Calib best = start;
  if (m.cdna()) {
    // the CDNA form's own constants (per-CU stream rate, spill cost, merge round trip,
    // scalar issue weight)
    knobs.push_back({&Calib::cu_frac, 0.1, 1.5, false});
    knobs.push_back({&Calib::spill_cost, 0.0, 4.0, false});
    knobs.push_back({&Calib::merge_trip, 0.0, 32.0, false});
    knobs.push_back({&Calib::salu_w, 0.0, 1.0, false});
    best.cdna = true;
  }
  double best_loss = loss(best);
  for (int round = 0; round < 6; ++round) {
    const double span = round == 0 ? 1.0 : std::pow(0.5, round);
    for (const Knob &k : knobs) {
      const double cur = best.*k.field;
      double lo, hi;
      if (k.log) {
        const double a = std::log(k.lo), b = std::log(k.hi), x = std::log(std::max(cur, k.lo));
        lo = round == 0 ? a : std::max(a, x - span * (b - a) / 2);
        hi = round == 0 ? b : std::min(b, x + span * (b - a) / 2);
      } else {
        lo = round == 0 ? k.lo : std::max(k.lo, cur - span * (k.hi - k.lo) / 2);
        hi = round == 0 ? k.hi : std::min(k.hi, cur + span * (k.hi - k.lo) / 2);
      }
      for (int i = 0; i <= 40; ++i) {
        const double t = i / 40.0;
        Calib trial = best;
        trial.*k.field = k.log ? std::exp(lo + t * (hi - lo)) : lo + t * (hi - lo);
        const double l = loss(trial);
        if (l < best_loss) {
          best_loss = l;
          best = trial;
        }
      }
    }
  }
  // accuracy of each lossy format: median measured error of its rows
  std::map<std::string, std::vector<double>> errs;
  for (const SweepRow *r : fit)
    if (r->plan.fmt.isQuantized() && r->err_exact > 0) errs[r->plan.fmt.key()].push_back(r->err_exact);
  for (auto &[key, v] : errs) {
    std::sort(v.begin(), v.end());
    best.rel_err[key] = v[v.size() / 2];
  }
  return best;
}

std::vector<std::string> heldOutShapes(const std::vector<SweepRow> &rows, int every) {
  std::set<std::string> keys;
  for (const auto &r : rows) keys.insert(shapeKey(r.spec));
  std::vector<std::string> held;
  int i = 0;
  for (const auto &k : keys) {
    if (every > 0 && i % every == every - 1) held.push_back(k);
    ++i;
  }
  return held;
}

namespace {

struct Class {
  std::string title;
  Eligibility e;
};

std::string report(const std::vector<SweepRow> &rows, const Machine &m, const Calib &c, const ShapeFilter &use,
                   const std::vector<Class> &classes) {
  std::ostringstream o;
  for (const auto &cl : classes) {
    const Metrics mt = evaluateSweep(rows, m, c, cl.e, use);
    o << std::fixed << std::setprecision(3) << cl.title << "\n"
      << "  shapes " << mt.shapes << ", rows " << mt.rows << "\n"
      << "  MAPE            " << 100.0 * mt.mape << " %\n"
      << "  Spearman rho    " << mt.spearman << "\n"
      << "  Kendall tau     " << mt.kendall << "\n"
      << "  regret mean     " << 100.0 * mt.regret_mean << " %\n"
      << "  regret max      " << 100.0 * mt.regret_max << " %\n"
      << "  top-1 hit       " << 100.0 * mt.top1 << " %\n";
    o.unsetf(std::ios::floatfield);
    o << std::setprecision(6) << mt.per_shape << "\n";
  }
  return o.str();
}

} // namespace

std::string evaluationReport(const std::vector<SweepRow> &rows, const Machine &m, const Calib &c,
                             const ShapeFilter &use) {
  std::vector<Class> classes(3);
  classes[0].title = "lossless only (f16)";
  classes[0].e.formats = {"f16"};
  classes[1].title = "accuracy limit 0.02 (f16 + int8)";
  classes[1].e.max_rel_err = 0.02;
  classes[2].title = "no accuracy limit (f16 + int8 + int4)";
  return report(rows, m, c, use, classes);
}

std::string evaluationReport(const std::vector<SweepRow> &rows, const Machine &m, const Calib &c,
                             const ShapeFilter &use, const std::vector<std::string> &keys) {
  std::vector<Class> classes(1);
  for (const auto &k : keys) classes[0].title += (classes[0].title.empty() ? "" : " + ") + k;
  classes[0].title = "format " + classes[0].title + " only";
  classes[0].e.keys = keys;
  return report(rows, m, c, use, classes);
}

} // namespace kvfc
