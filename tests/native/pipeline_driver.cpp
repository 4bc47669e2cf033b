// pipeline_driver.cpp - runs librelx's C ABI over the CPU stand-in of the
// HIP runtime (tests/native/hip_fake.cpp), built under ThreadSanitizer by
// tests/native/Makefile and driven by tests/test_fake_backend.py.
//
// stdin: one scenario per line, `<scenario> <case dir> key=value ...`.
// stdout: one JSON object per scenario: the C-ABI calls' results, the
// ordering checker's violations, and whether every result matched the
// case's expected bytes.
//
// A case directory holds plan.bin, bind.txt (`sym NAME VALUE`,
// `param NAME KIND BITS RANK LENGTH FILE`, `index KIND BITS RANK E... FILE`),
// src.bin (the dense source, or an indexed plan's table) and, optionally,
// want.bin (the oracle's result for that source).
//
// Scenarios:
//   h2d      relx_execute_h2d, `repeat` calls (no_wait: then
//            relx_ctx_synchronize or the caller stream)
//   group    relx_execute_group_h2d of `members` copies of the case
//   submit   relx_submit_group_h2d, polled with relx_completion_query, then
//            waited (`twice=1`: two submissions in flight)
//   d2h      relx_execute_d2h from a device source written on the caller
//            stream just before
//   device   relx_relayout_device (an indexed plan: relx_index_select_device)
//            on the caller stream after the wire (table) was
//            written on it
//   static   relx_execute_h2d_static from a page-locked source
//   static_pair  no_wait static calls alternating between two contexts on
//            one device, then both synchronized
//   threads  several host threads uploading at once, through one context
//            (`shared=1`) or one context each
// Options: pinned, chunk, nbuf, threads, hs (host stages), caller (none,
// null, stream), nowait, streams (copy streams), repeat, members, twice, check, the fault knobs and
// delays of fake_knobs, and devices / device (device count, context device).
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iostream>
#include <map>
#include <memory>
#include <sstream>
#include <string>
#include <thread>
#include <vector>

#include "../../include/relx.h"
#include "hip_fake.h"

namespace {

std::string read_file(const std::string &path) {
  std::ifstream f(path, std::ios::binary);
  if (!f)
    return std::string();
  std::ostringstream ss;
  ss << f.rdbuf();
  return ss.str();
}

bool file_exists(const std::string &path) { return static_cast<bool>(std::ifstream(path)); }

std::string jstr(const std::string &s) {
  std::string o = "\"";
  for (char c : s) {
    if (c == '"' || c == '\\')
      o += '\\', o += c;
    else if (static_cast<unsigned char>(c) < 0x20)
      o += ' ';
    else
      o += c;
  }
  return o + "\"";
}

struct Case {
  std::string dir;
  relx_plan *plan = nullptr;
  relx_bound *bound = nullptr;
  relx_bound_info info{};
  std::string src, want;
  std::string error; // load or bind failure
  std::vector<std::string> keep; // parameter and index bytes
  // what the bound was made from, for a fresh binding per call (layout and
  // typed plans)
  std::vector<std::string> sym_names, param_names;
  std::vector<int64_t> sym_values;
  std::vector<relx_param> params;
  bool indexed = false;
};

// A new binding of the case's plan with its symbols and parameters.
relx_bound *bind_again(const Case &c) {
  std::vector<const char *> np;
  for (const std::string &n : c.sym_names)
    np.push_back(n.c_str());
  relx_bound *b = nullptr;
  relx_err err{};
  if (relx_bind(c.plan, np.data(), c.sym_values.data(), static_cast<int>(np.size()), c.params.data(),
                static_cast<int>(c.params.size()), &b, &err) != RELX_OK)
    return nullptr;
  return b;
}

bool load_case(const std::string &dir, Case &c) {
  c.dir = dir;
  const std::string plan = read_file(dir + "/plan.bin");
  relx_err err{};
  if (relx_plan_load(reinterpret_cast<const uint8_t *>(plan.data()), plan.size(), &c.plan, &err) != RELX_OK) {
    c.error = std::string("plan: ") + err.code + ": " + err.message;
    return false;
  }
  std::vector<std::string> names;
  std::vector<int64_t> values;
  std::vector<relx_param> params;
  std::vector<std::string> pnames;
  bool indexed = false;
  int ikind = 0, ibits = 0, irank = 0;
  std::vector<int64_t> iext;
  std::string idata;
  std::istringstream bt(read_file(dir + "/bind.txt"));
  std::string line;
  pnames.reserve(64);
  c.keep.reserve(64);
  while (std::getline(bt, line)) {
    std::istringstream ls(line);
    std::string kw;
    ls >> kw;
    if (kw == "sym") {
      std::string n;
      int64_t v;
      ls >> n >> v;
      names.push_back(n);
      values.push_back(v);
    } else if (kw == "param") {
      relx_param p{};
      std::string n, file;
      ls >> n >> p.kind >> p.bits >> p.rank >> p.length >> file;
      pnames.push_back(n);
      c.keep.push_back(read_file(dir + "/" + file));
      p.name = pnames.back().c_str();
      p.data = c.keep.back().data();
      p.nbytes = c.keep.back().size();
      params.push_back(p);
    } else if (kw == "index") {
      indexed = true;
      ls >> ikind >> ibits >> irank;
      iext.resize(static_cast<size_t>(irank));
      for (int i = 0; i < irank; ++i)
        ls >> iext[static_cast<size_t>(i)];
      std::string file;
      ls >> file;
      idata = read_file(dir + "/" + file);
    }
  }
  std::vector<const char *> np;
  for (const std::string &n : names)
    np.push_back(n.c_str());
  int rc;
  if (indexed)
    rc = relx_bind_indexed(c.plan, np.data(), values.data(), static_cast<int>(np.size()), ikind, ibits,
                           iext.data(), irank, idata.data(), idata.size(), &c.bound, &err);
  else
    rc = relx_bind(c.plan, np.data(), values.data(), static_cast<int>(np.size()), params.data(),
                   static_cast<int>(params.size()), &c.bound, &err);
  if (rc != RELX_OK) {
    c.error = std::string("bind: ") + err.code + ": " + err.message;
    return false;
  }
  relx_bound_query(c.bound, &c.info);
  c.sym_names = std::move(names);
  c.sym_values = std::move(values);
  c.param_names = std::move(pnames); // the params' name pointers move with the buffer
  c.params = std::move(params);
  c.indexed = indexed;
  c.src = read_file(dir + "/src.bin");
  if (file_exists(dir + "/want.bin"))
    c.want = read_file(dir + "/want.bin");
  return true;
}

struct Opts {
  std::map<std::string, std::string> kv;
  int64_t get(const std::string &k, int64_t dflt) const {
    auto it = kv.find(k);
    return it == kv.end() ? dflt : std::strtoll(it->second.c_str(), nullptr, 10);
  }
  std::string str(const std::string &k, const std::string &dflt) const {
    auto it = kv.find(k);
    return it == kv.end() ? dflt : it->second;
  }
};

struct Call {
  int rc;
  std::string code, message;
  int completion;
};

struct Result {
  std::vector<Call> calls;
  int64_t mismatches = 0, checked = 0;
  std::vector<std::string> notes;
  int quarantined = 0;
  int64_t pinned_bytes = 0, device_bytes = 0; // the context's scratch after the scenario
  Call close{RELX_OK, "", "", 0};
  relx_report report{};
};

Call call_of(int rc, const relx_err &e) {
  return Call{rc, rc == RELX_OK ? "" : e.code, rc == RELX_OK ? "" : e.message,
              rc == RELX_OK ? 0 : e.completion};
}

// A device buffer: allocated through the HIP calls (the stand-in's device
// memory), filled with `fill`.
void *device_buffer(size_t n, int fill) {
  void *p = nullptr;
  if (hipMalloc(&p, n) != hipSuccess)
    return nullptr;
  if (hipMemset(p, fill, n) != hipSuccess)
    return nullptr;
  return p;
}

// Compare the host-visible bytes of a result with the expected ones. The
// host read is checked for ordering after the writes that produced it.
void check(Result &r, const Case &c, const void *p, size_t n, bool want_check) {
  fake_host_read(p, n, "host reads the result");
  if (!want_check || c.want.empty())
    return;
  ++r.checked;
  if (c.want.size() != n || std::memcmp(p, c.want.data(), n) != 0) {
    ++r.mismatches;
    size_t first = 0;
    const size_t m = std::min(n, c.want.size());
    while (first < m && static_cast<const uint8_t *>(p)[first] == static_cast<const uint8_t>(c.want[first]))
      ++first;
    r.notes.push_back("result differs from want.bin at byte " + std::to_string(first) + " of " +
                      std::to_string(n));
  }
}

relx_options options_of(const Opts &o) {
  relx_options opt{};
  opt.n_buffers = static_cast<int>(o.get("nbuf", 0));
  opt.chunk_bytes = o.get("chunk", 0);
  opt.host_stages = static_cast<int>(o.get("hs", -1));
  opt.gather_threads = static_cast<int>(o.get("threads", 0));
  opt.source_pinned = static_cast<int>(o.get("pinned", -1));
  opt.no_wait = static_cast<int>(o.get("nowait", 0));
  opt.n_streams = static_cast<int>(o.get("streams", 0));
  return opt;
}

// The caller's stream: none, the null stream, or a stream of its own.
struct Caller {
  std::string mode;
  hipStream_t s = nullptr;
  explicit Caller(const std::string &m) : mode(m) {
    if (mode == "stream" || mode == "stream_untold")
      (void)hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
  }
  ~Caller() {
    if (s)
      (void)hipStreamDestroy(s);
  }
  void apply(relx_options &opt) const {
    // "stream_untold": work is produced on a stream the call is not told of
    opt.has_caller_stream = mode == "none" || mode == "stream_untold" ? 0 : 1;
    opt.caller_stream = reinterpret_cast<uint64_t>(s);
  }
  // Work on the caller's stream just before the call: `dst` is written
  // (a producer the call must follow, or an earlier user of its output).
  void produce(void *dst, const void *src, size_t n) const {
    if (mode != "none")
      (void)hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, s);
    else
      (void)hipMemcpy(dst, src, n, hipMemcpyHostToDevice);
  }
};

// The scenario's fault knobs and delays, applied once the driver's own
// buffers are allocated (the knobs count the library's calls only).
fake_knobs g_armed{};
void arm() { fake_configure(&g_armed); }

bool quarantined(relx_ctx *ctx) {
  relx_ctx_stats st{};
  relx_ctx_stats_get(ctx, &st);
  return st.quarantined != 0;
}

void run_h2d(const Case &c, const Opts &o, Result &r, relx_ctx *ctx) {
  const size_t out = static_cast<size_t>(c.info.destination_bytes);
  const bool pinned = o.get("pinned", 0) == 1;
  const bool nowait = o.get("nowait", 0) == 1;
  Caller caller(o.str("caller", "none"));
  void *src = nullptr;
  std::vector<uint8_t> pageable;
  if (pinned) {
    relx_err e{};
    relx_host_alloc(c.src.size(), &src, &e);
    fake_mark_user_pinned(src);
    std::memcpy(src, c.src.data(), c.src.size());
  } else {
    pageable.assign(c.src.begin(), c.src.end());
    src = pageable.data();
    fake_register_host(src, pageable.size());
  }
  void *dst = device_buffer(out, 0xA5);
  std::vector<uint8_t> poison(out, 0x5A), host(out);
  const int repeat = static_cast<int>(o.get("repeat", 2));
  arm();
  // burst: no_wait calls back to back, each overwriting what the one before
  // may still be reading and writing; one synchronization at the end
  const bool burst = nowait && o.get("burst", 0) != 0;
  bool failed = false;
  // rebind: every call runs a fresh binding of the plan, freed after the call
  const bool rebind = o.get("rebind", 0) != 0 && !c.indexed;
  std::unique_ptr<relx_bound, void (*)(relx_bound *)> fresh(nullptr, relx_bound_free);
  for (int i = 0; i < repeat && !failed; ++i) {
    relx_options opt = options_of(o);
    caller.apply(opt);
    if (!burst || i == 0)
      caller.produce(dst, poison.data(), out); // an earlier writer of the destination
    relx_bound *bound = c.bound;
    if (rebind) {
      fresh.reset(bind_again(c));
      if (!fresh) {
        r.notes.push_back("rebind failed");
        return;
      }
      bound = fresh.get();
    }
    relx_err e{};
    fake_call_begin();
    const int rc = relx_execute_h2d(ctx, bound, src, c.src.size(), dst, out, &opt, &r.report, &e);
    r.calls.push_back(call_of(rc, e));
    if (rc != RELX_OK) {
      relx_ctx_stats st{};
      relx_ctx_stats_get(ctx, &st);
      failed = st.quarantined != 0; // a drained context takes the next call
      // persist: call a quarantined context again (it must refuse at once)
      if (failed && o.get("persist", 0)) {
        for (++i; i < repeat; ++i) {
          relx_err e3{};
          relx_options o3 = options_of(o);
          fake_call_begin();
          r.calls.push_back(call_of(
              relx_execute_h2d(ctx, c.bound, src, c.src.size(), dst, out, &o3, nullptr, &e3), e3));
        }
      }
      continue;
    }
    if (burst && i + 1 < repeat)
      continue;
    if (nowait) {
      if (caller.mode == "none") {
        relx_err e2{};
        const int rc2 = relx_ctx_synchronize(ctx, &e2);
        r.calls.push_back(call_of(rc2, e2));
      } else {
        (void)hipStreamSynchronize(caller.s); // the caller's stream waits for the call
      }
    }
    fake_host_read(dst, out, "host reads the result");
    (void)hipMemcpy(host.data(), dst, out, hipMemcpyDeviceToHost);
    check(r, c, host.data(), out, o.get("check", 1) != 0);
  }
  if (!failed) {
    (void)hipFree(dst);
    if (pinned)
      relx_host_free(src);
  }
  if (!pinned)
    fake_unregister_host(src);
  if (failed) // a failed call's context may still read the source: kept
    new std::vector<uint8_t>(std::move(pageable));
}

void run_group(const Case &c, const Opts &o, Result &r, relx_ctx *ctx, bool submit) {
  const int n = static_cast<int>(o.get("members", 3));
  const size_t out = static_cast<size_t>(c.info.destination_bytes);
  const int rounds = submit && o.get("twice", 0) ? 2 : 1;
  std::vector<std::vector<uint8_t>> srcs(static_cast<size_t>(n * rounds));
  std::vector<void *> dsts(static_cast<size_t>(n * rounds));
  for (size_t i = 0; i < srcs.size(); ++i) {
    srcs[i].assign(c.src.begin(), c.src.end());
    fake_register_host(srcs[i].data(), srcs[i].size());
    dsts[i] = device_buffer(out, 0xA5);
  }
  std::vector<const relx_bound *> bounds(static_cast<size_t>(n), c.bound);
  std::vector<size_t> sb(static_cast<size_t>(n), c.src.size()), db(static_cast<size_t>(n), out);
  std::vector<relx_report> reps(static_cast<size_t>(n));
  std::vector<relx_completion *> comps;
  bool ok = true;
  arm();
  for (int round = 0; round < rounds; ++round) {
    std::vector<const void *> sp;
    std::vector<void *> dp;
    for (int i = 0; i < n; ++i) {
      sp.push_back(srcs[static_cast<size_t>(round * n + i)].data());
      dp.push_back(dsts[static_cast<size_t>(round * n + i)]);
    }
    relx_options opt = options_of(o);
    relx_err e{};
    relx_report total{};
    int rc;
    fake_call_begin();
    if (submit) {
      relx_completion *comp = nullptr;
      rc = relx_submit_group_h2d(ctx, n, bounds.data(), sp.data(), sb.data(), dp.data(), db.data(), &opt,
                                 reps.data(), &total, &comp, &e);
      if (rc == RELX_OK)
        comps.push_back(comp);
    } else {
      rc = relx_execute_group_h2d(ctx, n, bounds.data(), sp.data(), sb.data(), dp.data(), db.data(),
                                  &opt, reps.data(), &total, &e);
    }
    r.calls.push_back(call_of(rc, e));
    ok = ok && rc == RELX_OK;
  }
  for (relx_completion *comp : comps) {
    int done = 0;
    for (int spin = 0; spin < 200000 && !done; ++spin) {
      relx_err e{};
      if (relx_completion_query(comp, &done, &e) != RELX_OK) {
        r.calls.push_back(call_of(RELX_ERROR, e));
        break;
      }
      if (!done)
        std::this_thread::sleep_for(std::chrono::microseconds(20));
    }
    relx_err e{};
    r.calls.push_back(call_of(relx_completion_wait(comp, &e), e));
    relx_completion_free(comp);
  }
  std::vector<uint8_t> host(out);
  if (ok) {
    for (size_t i = 0; i < dsts.size(); ++i) {
      fake_host_read(dsts[i], out, "host reads a member's result");
      (void)hipMemcpy(host.data(), dsts[i], out, hipMemcpyDeviceToHost);
      check(r, c, host.data(), out, o.get("check", 1) != 0);
    }
  }
  for (size_t i = 0; i < srcs.size(); ++i) {
    fake_unregister_host(srcs[i].data());
    if (ok)
      (void)hipFree(dsts[i]);
  }
  if (!ok)
    for (auto &s : srcs)
      new std::vector<uint8_t>(std::move(s)); // kept: a failed call may still read them
}

void run_d2h(const Case &c, const Opts &o, Result &r, relx_ctx *ctx) {
  const size_t out = static_cast<size_t>(c.info.destination_bytes);
  const bool pinned = o.get("pinned", 0) == 1;
  Caller caller(o.str("caller", "stream"));
  void *src = device_buffer(c.src.size(), 0xA5);
  void *dst = nullptr;
  std::vector<uint8_t> pageable;
  if (pinned) {
    relx_err e{};
    relx_host_alloc(out, &dst, &e);
    fake_mark_user_pinned(dst);
  } else {
    pageable.assign(out, 0);
    dst = pageable.data();
    fake_register_host(dst, out);
  }
  const int repeat = static_cast<int>(o.get("repeat", 2));
  arm();
  bool ok = true;
  for (int i = 0; i < repeat && ok; ++i) {
    relx_options opt = options_of(o);
    opt.source_pinned = pinned ? 1 : 0;
    opt.host_stages = 0;
    caller.apply(opt);
    caller.produce(src, c.src.data(), c.src.size()); // the device source's producer
    relx_err e{};
    fake_call_begin();
    const int rc = relx_execute_d2h(ctx, c.bound, src, c.src.size(), dst, out, &opt, &r.report, &e);
    r.calls.push_back(call_of(rc, e));
    if (rc == RELX_OK)
      check(r, c, dst, out, o.get("check", 1) != 0);
    else
      ok = !quarantined(ctx); // a drained context takes the next call
  }
  if (!pinned)
    fake_unregister_host(dst);
  if (ok) {
    (void)hipFree(src);
    if (pinned)
      relx_host_free(dst);
  } else if (!pinned) {
    new std::vector<uint8_t>(std::move(pageable));
  }
}

void run_device(const Case &c, const Opts &o, Result &r, relx_ctx *ctx) {
  const size_t out = static_cast<size_t>(c.info.destination_bytes);
  Caller caller(o.str("caller", "stream"));
  void *wire = device_buffer(c.src.size(), 0xA5);
  void *dst = device_buffer(out, 0xA5);
  std::vector<uint8_t> host(out);
  const int repeat = static_cast<int>(o.get("repeat", 2));
  arm();
  bool ok = true;
  for (int i = 0; i < repeat && ok; ++i) {
    caller.produce(wire, c.src.data(), c.src.size());
    relx_err e{};
    // an indexed plan gathers its rows from the device-resident table
    const int rc = c.info.indexed
                       ? relx_index_select_device(ctx, c.bound, wire, c.src.size(), dst, out,
                                                  reinterpret_cast<uint64_t>(caller.s), &e)
                       : relx_relayout_device(ctx, c.bound, static_cast<int>(o.get("hs", 0)), wire,
                                              dst, reinterpret_cast<uint64_t>(caller.s), &e);
    r.calls.push_back(call_of(rc, e));
    const hipError_t se = hipStreamSynchronize(caller.s);
    relx_err e2{};
    const int rc2 = relx_ctx_synchronize(ctx, &e2);
    r.calls.push_back(call_of(rc2, e2));
    if (rc != RELX_OK || rc2 != RELX_OK || se != hipSuccess) {
      ok = se == hipSuccess; // a device fault leaves the buffers to the device
      continue;
    }
    fake_host_read(dst, out, "host reads the result");
    (void)hipMemcpy(host.data(), dst, out, hipMemcpyDeviceToHost);
    check(r, c, host.data(), out, o.get("check", 1) != 0);
  }
  if (ok) {
    (void)hipFree(wire);
    (void)hipFree(dst);
  }
}

// Several host threads upload at once, each with its own buffers: through
// the one context (`shared=1`, whose calls the library serializes) or one
// context each, all sharing the bound plan and its device caches.
void run_threads(const Case &c, const Opts &o, Result &r, relx_ctx *ctx) {
  const int nt = static_cast<int>(o.get("threads_n", 4));
  const bool shared = o.get("shared", 1) != 0;
  const int repeat = static_cast<int>(o.get("repeat", 3));
  const size_t out = static_cast<size_t>(c.info.destination_bytes);
  std::vector<relx_ctx *> ctxs(static_cast<size_t>(nt), ctx);
  for (int t = 0; t < nt && !shared; ++t) {
    relx_err e{};
    if (relx_ctx_create(0, o.get("retained", -1), &ctxs[static_cast<size_t>(t)], &e) != RELX_OK) {
      r.notes.push_back(std::string("context: ") + e.code);
      return;
    }
  }
  std::vector<std::vector<uint8_t>> srcs(static_cast<size_t>(nt));
  std::vector<void *> dsts(static_cast<size_t>(nt));
  for (int t = 0; t < nt; ++t) {
    srcs[static_cast<size_t>(t)].assign(c.src.begin(), c.src.end());
    fake_register_host(srcs[static_cast<size_t>(t)].data(), c.src.size());
    dsts[static_cast<size_t>(t)] = device_buffer(out, 0xA5);
  }
  arm();
  std::vector<std::vector<Call>> calls(static_cast<size_t>(nt));
  std::vector<int64_t> bad(static_cast<size_t>(nt), 0), seen(static_cast<size_t>(nt), 0);
  std::vector<std::thread> pool;
  std::vector<int> done(static_cast<size_t>(nt), -1);
  const int start = fake_host_handoff(); // the threads follow the set-up
  for (int t = 0; t < nt; ++t)
    pool.emplace_back([&, t] {
      const size_t i = static_cast<size_t>(t);
      fake_host_adopt(start);
      std::vector<uint8_t> host(out);
      for (int k = 0; k < repeat; ++k) {
        relx_options opt = options_of(o);
        relx_err e{};
        fake_call_begin();
        const int rc = relx_execute_h2d(ctxs[i], c.bound, srcs[i].data(), c.src.size(), dsts[i], out,
                                        &opt, nullptr, &e);
        calls[i].push_back(call_of(rc, e));
        if (rc != RELX_OK)
          continue;
        fake_host_read(dsts[i], out, "a thread reads its result");
        (void)hipMemcpy(host.data(), dsts[i], out, hipMemcpyDeviceToHost);
        ++seen[i];
        if (!c.want.empty() && std::memcmp(host.data(), c.want.data(), out) != 0)
          ++bad[i];
      }
      done[i] = fake_host_handoff();
    });
  for (std::thread &th : pool)
    th.join();
  for (int token : done) // the main thread follows every thread's work
    fake_host_adopt(token);
  for (int t = 0; t < nt; ++t) {
    const size_t i = static_cast<size_t>(t);
    r.calls.insert(r.calls.end(), calls[i].begin(), calls[i].end());
    r.checked += c.want.empty() ? 0 : seen[i];
    r.mismatches += bad[i];
    fake_unregister_host(srcs[i].data());
    (void)hipFree(dsts[i]);
    if (!shared) {
      relx_err e{};
      if (relx_ctx_close(ctxs[i], &e) != RELX_OK)
        r.notes.push_back(std::string("close: ") + e.code);
    }
  }
}

void run_static(const Case &c, const Opts &o, Result &r, relx_ctx *ctx) {
  const size_t out = static_cast<size_t>(c.info.destination_bytes);
  void *src = nullptr;
  relx_err ea{};
  relx_host_alloc(c.src.size(), &src, &ea);
  fake_mark_user_pinned(src);
  std::memcpy(src, c.src.data(), c.src.size());
  void *dst = device_buffer(out, 0xA5);
  std::vector<uint8_t> host(out);
  const int repeat = static_cast<int>(o.get("repeat", 2));
  arm();
  bool ok = true;
  for (int i = 0; i < repeat && ok; ++i) {
    relx_options opt = options_of(o);
    opt.source_pinned = 1;
    relx_err e{};
    fake_call_begin();
    const int rc = relx_execute_h2d_static(ctx, c.bound, src, c.src.size(), dst, out, &opt, &r.report, &e);
    r.calls.push_back(call_of(rc, e));
    if (rc != RELX_OK) {
      ok = !quarantined(ctx); // a drained context takes the next call
      continue;
    }
    fake_host_read(dst, out, "host reads the result");
    (void)hipMemcpy(host.data(), dst, out, hipMemcpyDeviceToHost);
    check(r, c, host.data(), out, o.get("check", 1) != 0);
  }
  if (ok) {
    (void)hipFree(dst);
    relx_host_free(src);
  }
}

// Two contexts on one device alternate no_wait static calls (`repeat` in
// all), each call into a destination of its own, then both contexts
// synchronize: every call stages its wire in the device's one static
// scratch, so each must start writing it only after the previous call,
// from either context, has read it.
void run_static_pair(const Case &c, const Opts &o, Result &r, relx_ctx *ctx) {
  relx_ctx *other = nullptr;
  relx_err ec{};
  if (relx_ctx_create(0, -1, &other, &ec) != RELX_OK) {
    r.notes.push_back(std::string("context: ") + ec.code);
    return;
  }
  const size_t out = static_cast<size_t>(c.info.destination_bytes);
  void *src = nullptr;
  relx_err ea{};
  relx_host_alloc(c.src.size(), &src, &ea);
  fake_mark_user_pinned(src);
  std::memcpy(src, c.src.data(), c.src.size());
  const int repeat = static_cast<int>(o.get("repeat", 4));
  std::vector<void *> dsts(static_cast<size_t>(repeat));
  for (void *&d : dsts)
    d = device_buffer(out, 0xA5);
  std::vector<uint8_t> host(out);
  arm();
  bool ok = true;
  for (int i = 0; i < repeat; ++i) {
    relx_options opt = options_of(o);
    opt.source_pinned = 1;
    opt.no_wait = 1;
    relx_err e{};
    fake_call_begin();
    const int rc = relx_execute_h2d_static(i % 2 ? other : ctx, c.bound, src, c.src.size(),
                                           dsts[static_cast<size_t>(i)], out, &opt, &r.report, &e);
    r.calls.push_back(call_of(rc, e));
    ok = ok && rc == RELX_OK;
  }
  for (relx_ctx *x : {ctx, other}) {
    relx_err e{};
    const int rc = relx_ctx_synchronize(x, &e);
    r.calls.push_back(call_of(rc, e));
    ok = ok && rc == RELX_OK;
  }
  for (int i = 0; i < repeat && ok; ++i) {
    void *d = dsts[static_cast<size_t>(i)];
    fake_host_read(d, out, "host reads the result");
    (void)hipMemcpy(host.data(), d, out, hipMemcpyDeviceToHost);
    check(r, c, host.data(), out, o.get("check", 1) != 0);
  }
  relx_err e{};
  if (relx_ctx_close(other, &e) != RELX_OK)
    r.notes.push_back(std::string("close: ") + e.code);
  if (ok) {
    for (void *d : dsts)
      (void)hipFree(d);
    relx_host_free(src);
  }
}

fake_knobs knobs_of(const Opts &o) {
  fake_knobs k{};
  k.fail_malloc_at = static_cast<int>(o.get("fail_malloc_at", 0));
  k.fail_host_malloc_at = static_cast<int>(o.get("fail_host_malloc_at", 0));
  k.fail_copy_at = static_cast<int>(o.get("fail_copy_at", 0));
  k.fail_copy_async_at = static_cast<int>(o.get("fail_copy_async_at", 0));
  k.fail_launch_at = static_cast<int>(o.get("fail_launch_at", 0));
  k.fail_kernel_async_at = static_cast<int>(o.get("fail_kernel_async_at", 0));
  k.fail_record_at = static_cast<int>(o.get("fail_record_at", 0));
  k.fail_wait_at = static_cast<int>(o.get("fail_wait_at", 0));
  k.fail_sync_at = static_cast<int>(o.get("fail_sync_at", 0));
  k.sync_unknown = static_cast<int>(o.get("sync_unknown", 0));
  k.delay_copy_us = static_cast<int>(o.get("delay_copy", 0));
  k.delay_kernel_us = static_cast<int>(o.get("delay_kernel", 0));
  k.jitter = static_cast<int>(o.get("jitter", 0));
  k.seed = static_cast<uint32_t>(o.get("seed", 1));
  k.device_count = static_cast<int>(o.get("devices", 1));
  return k;
}

std::string call_json(const Call &c) {
  return "{\"rc\":" + std::to_string(c.rc) + ",\"code\":" + jstr(c.code) + ",\"message\":" + jstr(c.message) +
         ",\"completion\":" + std::to_string(c.completion) + "}";
}

} // namespace

int main() {
  std::string line;
  std::map<std::string, Case> cases;
  while (std::getline(std::cin, line)) {
    std::istringstream ls(line);
    std::string scenario, dir, kv;
    if (!(ls >> scenario >> dir))
      continue;
    Opts o;
    while (ls >> kv) {
      const size_t eq = kv.find('=');
      if (eq != std::string::npos)
        o.kv[kv.substr(0, eq)] = kv.substr(eq + 1);
    }
    Case &c = cases[dir];
    if (c.dir.empty())
      load_case(dir, c);
    Result r;
    std::string setup_error = c.error;
    // The context is made before the knobs apply (faults hit the calls),
    // unless the knob is about making it.
    fake_knobs k = knobs_of(o);
    const bool knobs_first = o.get("knobs_first", 0) != 0;
    if (knobs_first)
      fake_configure(&k);
    else
      fake_configure(nullptr);
    relx_ctx *ctx = nullptr;
    Call create{RELX_OK, "", "", 0};
    if (setup_error.empty()) {
      if (!knobs_first) {
        fake_knobs pre{};
        pre.device_count = k.device_count;
        fake_configure(&pre);
      }
      relx_err e{};
      const int rc =
          relx_ctx_create(static_cast<int>(o.get("device", 0)), o.get("retained", -1), &ctx, &e);
      create = call_of(rc, e);
      g_armed = k; // the scenario arms the knobs once its buffers exist
      if (rc == RELX_OK) {
        if (scenario == "h2d")
          run_h2d(c, o, r, ctx);
        else if (scenario == "group")
          run_group(c, o, r, ctx, false);
        else if (scenario == "submit")
          run_group(c, o, r, ctx, true);
        else if (scenario == "d2h")
          run_d2h(c, o, r, ctx);
        else if (scenario == "device")
          run_device(c, o, r, ctx);
        else if (scenario == "static")
          run_static(c, o, r, ctx);
        else if (scenario == "static_pair")
          run_static_pair(c, o, r, ctx);
        else if (scenario == "threads")
          run_threads(c, o, r, ctx);
        else
          setup_error = "unknown scenario " + scenario;
        relx_ctx_stats st{};
        relx_ctx_stats_get(ctx, &st);
        r.quarantined = st.quarantined;
        r.pinned_bytes = st.pinned_bytes;
        r.device_bytes = st.device_bytes;
        if (o.get("close", 1)) {
          relx_err e2{};
          r.close = call_of(relx_ctx_close(ctx, &e2), e2);
        }
      }
    }
    fake_counts counts{};
    fake_get_counts(&counts);
    std::ostringstream js;
    js << "{\"scenario\":" << jstr(scenario) << ",\"case\":" << jstr(dir) << ",\"setup_error\":" << jstr(setup_error)
       << ",\"create\":" << call_json(create) << ",\"calls\":[";
    for (size_t i = 0; i < r.calls.size(); ++i)
      js << (i ? "," : "") << call_json(r.calls[i]);
    js << "],\"close\":" << call_json(r.close) << ",\"quarantined\":" << r.quarantined
       << ",\"pinned_bytes\":" << r.pinned_bytes << ",\"device_bytes\":" << r.device_bytes
       << ",\"checked\":" << r.checked << ",\"mismatches\":" << r.mismatches << ",\"notes\":[";
    for (size_t i = 0; i < r.notes.size(); ++i)
      js << (i ? "," : "") << jstr(r.notes[i]);
    js << "],\"violations\":[";
    const int nv = fake_violation_count();
    for (int i = 0; i < nv; ++i)
      js << (i ? "," : "") << jstr(fake_violation(i));
    js << "],\"report\":{\"implementation\":" << jstr(r.report.implementation) << ",\"chunks\":" << r.report.chunks
       << ",\"kernel_launches\":" << r.report.kernel_launches << ",\"direct_dma\":" << r.report.direct_dma
       << ",\"wire_boundary\":" << r.report.wire_boundary << ",\"wire_bytes\":" << r.report.wire_bytes
       << ",\"host_chunk_bytes\":" << r.report.host_chunk_bytes
       << ",\"host_buffers\":" << r.report.host_buffers << ",\"staging_bytes\":" << r.report.staging_bytes
       << ",\"staging_slots\":" << r.report.staging_slots
       << ",\"staging_reused\":" << r.report.staging_reused
       << ",\"copy_streams\":" << r.report.copy_streams << "},\"counts\":{\"copies\":" << counts.copies
       << ",\"launches\":" << counts.launches << ",\"syncs\":" << counts.syncs
       << ",\"unemulated\":" << counts.unemulated << ",\"mallocs\":" << counts.mallocs
       << ",\"host_mallocs\":" << counts.host_mallocs << ",\"frees\":" << counts.frees
       << ",\"host_frees\":" << counts.host_frees << ",\"zero_copy\":" << counts.zero_copy << "}}";
    std::cout << js.str() << std::endl;
    fake_configure(nullptr);
    fake_reset();
  }
  fake_shutdown();
  return 0;
}
