// fusion.hip -- the pointwise fusion compiler: IR text -> HIP C++ -> hipRTC
// (gfx950) -> cached module -> launch through the shared pointwise engine.
//
// The reference has no fusion (torch.jit.strict_fusion is a warning-only
// no-op and torch.compile is unsupported, README.md:178); this component is
// new.  A program is a straight-line DAG of reference ops; the generated
// functor evaluates it per element with one IEEE rounding per op, exactly as
// the eager chain would, and is instantiated into the same kernel bodies the
// eager ops use (pw_core.h), so fused and eager runs differ only in that
// intermediates never touch HBM.
#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <map>
#include <thread>
#include <unordered_map>
#include <memory>
#include <mutex>
#include <sstream>
#include <string>
#include <vector>

#include "pw_host.h"
#include "trs_internal.h"

namespace trs {

namespace {

// pw_core.h as a string literal, generated at build time.
const char kPwCoreSource[] =
#include "pw_core_src.inc"
    ;

// A code object and its per-device modules and functions.
struct CodeObject {
    std::vector<char> code;
    hipModule_t module[16] = {};
    std::map<std::string, hipFunction_t> functions[16];
};

struct Program {
    std::string ir;
    std::string functor;  // the TrsFused struct
    std::string source;   // functor + the standard kernel wrappers
    int nin = 0;
    int nout = 1;
    unsigned u8mask = 0;
    double compile_ms = 0.0;
    bool from_disk = false;
    CodeObject base;
    // pw_xpose kernels specialised on operand roles, built on first launch
    // of each role signature (kernel name -> code object).  spec_mu guards
    // the maps and is held only for lookups and inserts; compile_mu is held
    // over a specialisation's hipRTC compile, so launches of kernels already
    // built never wait for one.
    std::mutex spec_mu;
    std::mutex compile_mu;
    std::map<std::string, std::unique_ptr<CodeObject>> specs;
    // Launch-plan signature -> function, per device: a repeated launch looks
    // its kernel up here without building names or sources.
    std::unordered_map<uint64_t, hipFunction_t> by_plan[16];
};

std::mutex g_mu;
std::vector<std::unique_ptr<Program>> g_programs;  // kernel_id = index + 1
std::map<std::string, uint64_t> g_by_ir;

struct Instr {
    std::string op;
    std::vector<int> args;
    uint32_t bits = 0;
};

int parse_value(const std::string &tok, int defined, int *out) {
    if (tok.size() < 2 || tok[0] != '%') return -1;
    char *end = nullptr;
    long v = std::strtol(tok.c_str() + 1, &end, 10);
    if (*end != '\0' || v < 0 || v >= defined) return -1;
    *out = (int)v;
    return 0;
}

// Parses the IR, emits the functor and the extern "C" kernel wrappers.
int generate(const std::string &ir, Program *prog) {
    std::istringstream in(ir);
    std::string line;
    std::vector<Instr> code;
    std::vector<int> results;
    int defined = 0, nin = 0, lineno = 0;
    unsigned u8mask = 0;
    while (std::getline(in, line)) {
        lineno++;
        const size_t hash = line.find('#');
        if (hash != std::string::npos) line.resize(hash);
        std::istringstream ls(line);
        std::string op;
        if (!(ls >> op)) continue;
        if (!results.empty() && op != "out")
            return set_error(TRS_E_FUSION, "line %d: instruction after 'out'", lineno);
        Instr ins;
        ins.op = op;
        std::vector<std::string> toks;
        std::string t;
        while (ls >> t) toks.push_back(t);
        if (op == "in") {
            if (toks.size() != 1 || (toks[0] != "f32" && toks[0] != "u8"))
                return set_error(TRS_E_FUSION, "line %d: expected 'in f32' or 'in u8'", lineno);
            if (nin >= kMaxIn) return set_error(TRS_E_FUSION, "line %d: more than %d inputs", lineno, kMaxIn);
            if (toks[0] == "u8") u8mask |= 1u << nin;
            ins.args.push_back(nin++);
            code.push_back(ins);
            defined++;
        } else if (op == "const") {
            if (toks.size() != 1) return set_error(TRS_E_FUSION, "line %d: expected 'const 0x<bits>'", lineno);
            char *end = nullptr;
            unsigned long v = std::strtoul(toks[0].c_str(), &end, 0);
            if (*end != '\0' || v > 0xffffffffUL)
                return set_error(TRS_E_FUSION, "line %d: bad constant '%s'", lineno, toks[0].c_str());
            ins.bits = (uint32_t)v;
            code.push_back(ins);
            defined++;
        } else if (op == "add" || op == "sub" || op == "mul" || op == "div" || op == "relub") {
            if (toks.size() != 2) return set_error(TRS_E_FUSION, "line %d: '%s' takes two values", lineno, op.c_str());
            for (auto &tk : toks) {
                int v;
                if (parse_value(tk, defined, &v))
                    return set_error(TRS_E_FUSION, "line %d: bad operand '%s'", lineno, tk.c_str());
                ins.args.push_back(v);
            }
            code.push_back(ins);
            defined++;
        } else if (op == "exp" || op == "relu" || op == "neg") {
            int v;
            if (toks.size() != 1 || parse_value(toks[0], defined, &v))
                return set_error(TRS_E_FUSION, "line %d: '%s' takes one value", lineno, op.c_str());
            ins.args.push_back(v);
            code.push_back(ins);
            defined++;
        } else if (op == "out") {
            int v;
            if (toks.size() != 1 || parse_value(toks[0], defined, &v))
                return set_error(TRS_E_FUSION, "line %d: 'out' takes one value", lineno);
            if ((int)results.size() >= kMaxOut)
                return set_error(TRS_E_FUSION, "line %d: more than %d outputs", lineno, kMaxOut);
            results.push_back(v);
        } else {
            return set_error(TRS_E_FUSION, "line %d: unknown instruction '%s'", lineno, op.c_str());
        }
    }
    if (results.empty()) return set_error(TRS_E_FUSION, "program has no 'out'");
    if (nin == 0) return set_error(TRS_E_FUSION, "program has no inputs");
    const int nout = (int)results.size();

    std::ostringstream s;
    s << "// generated by libtrs_hip fusion compiler\n";
    s << "struct TrsFused {\n  static constexpr int NIN = " << nin << ";\n";
    if (nout == 1) {
        s << "  __device__ __forceinline__ float operator()(const float *a) const {\n";
    } else {
        s << "  static constexpr int NOUT = " << nout << ";\n";
        s << "  __device__ __forceinline__ void operator()(const float *a, float *r) const {\n";
    }
    for (size_t i = 0; i < code.size(); i++) {
        const Instr &c = code[i];
        s << "    const float v" << i << " = ";
        if (c.op == "in") s << "a[" << c.args[0] << "]";
        else if (c.op == "const") {
            char buf[32];
            std::snprintf(buf, sizeof buf, "0x%08xu", c.bits);
            s << "__uint_as_float(" << buf << ")";
        } else if (c.op == "add") s << "v" << c.args[0] << " + v" << c.args[1];
        else if (c.op == "sub") s << "v" << c.args[0] << " - v" << c.args[1];
        else if (c.op == "mul") s << "v" << c.args[0] << " * v" << c.args[1];
        else if (c.op == "div") s << "v" << c.args[0] << " / v" << c.args[1];
        else if (c.op == "exp") s << "trs::exp_value(v" << c.args[0] << ")";
        else if (c.op == "relu") s << "trs::relu_value(v" << c.args[0] << ")";
        else if (c.op == "neg") s << "trs::negate_value(v" << c.args[0] << ")";
        else if (c.op == "relub") s << "trs::relu_backward_value(v" << c.args[0] << ", v" << c.args[1] << ")";
        s << ";\n";
    }
    if (nout == 1) {
        s << "    return v" << results[0] << ";\n";
    } else {
        for (int o = 0; o < nout; o++) s << "    r[" << o << "] = v" << results[o] << ";\n";
    }
    s << "  }\n};\n";
    prog->functor = s.str();
    const std::string mask = std::to_string(u8mask) + "u";
    auto wrap = [&](const char *name, const std::string &body, const char *lanes = "256") {
        s << "extern \"C\" __global__ void __launch_bounds__(" << lanes << ") " << name
          << "(trs::PwGeom, trs::PwPtrs p) { " << body << "(TrsFused{}, trs::kernarg_geom(), p); }\n";
    };
    // Compiled with the program: the variants that need no launch-time
    // specialisation.  Vector flat/rows kernels (specialised on the inputs
    // read once) and pw_xpose kernels (also on operand roles) are compiled on
    // their first launch: get_spec_function.
    wrap("trs_fused_flat_c", "trs::pw_flat_contig_body<TrsFused, " + mask + ">", "trs::kFlatBlock");
    wrap("trs_fused_flat_s", "trs::pw_flat_body<TrsFused, " + mask + ", false>", "trs::kFlatBlock");
    wrap("trs_fused_rows_s", "trs::pw_rows_body<TrsFused, " + mask + ", false>");
    wrap("trs_fused_generic", "trs::pw_generic_body<TrsFused, " + mask + ">", "trs::kGenericBlock");
    prog->nin = nin;
    prog->nout = nout;
    prog->u8mask = u8mask;
    prog->source = s.str();
    return TRS_OK;
}

const char *const kRtcOpts[] = {"--offload-arch=gfx950", "-O3", "-ffp-contract=off", "-std=c++20", "-DTRS_RTC",
                                "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-w"};

// ---- on-disk code-object cache ------------------------------------------------
// A compiled program is stored as <dir>/<fnv1a64(key)>.co holding a magic line,
// the full key (hipRTC version, options, complete source) and the code
// object; a hit requires the stored key to equal the current one, so a hash
// collision or a stale file is a miss.  Files are written to a temporary name
// and renamed, so concurrent processes never read a partial file.  Any I/O
// failure falls back to compiling.  The directory is TRS_FUSION_CACHE_DIR
// when set (empty disables the cache), else $XDG_CACHE_HOME/trs_hip/fusion
// or $HOME/.cache/trs_hip/fusion.

constexpr char kCacheMagic[] = "TRS-FUSION-CO-1\n";

std::string cache_dir() {
    if (const char *d = std::getenv("TRS_FUSION_CACHE_DIR")) return d;
    if (const char *x = std::getenv("XDG_CACHE_HOME"); x && *x) return std::string(x) + "/trs_hip/fusion";
    if (const char *h = std::getenv("HOME"); h && *h) return std::string(h) + "/.cache/trs_hip/fusion";
    return "";
}

bool make_dirs(const std::string &dir) {
    for (size_t i = 1; i <= dir.size(); i++) {
        if (i == dir.size() || dir[i] == '/') {
            const std::string part = dir.substr(0, i);
            if (mkdir(part.c_str(), 0755) != 0 && errno != EEXIST) return false;
        }
    }
    return true;
}

uint64_t fnv1a64(const std::string &s) {
    uint64_t h = 1469598103934665603ull;
    for (unsigned char c : s) {
        h ^= c;
        h *= 1099511628211ull;
    }
    return h;
}

std::string cache_key(const std::string &full_source) {
    int major = 0, minor = 0;
    hiprtcVersion(&major, &minor);
    std::string key = "hiprtc " + std::to_string(major) + "." + std::to_string(minor) + "\n";
    for (const char *o : kRtcOpts) key += std::string(o) + "\n";
    return key + full_source;
}

std::string cache_path(const std::string &dir, const std::string &key) {
    char name[32];
    std::snprintf(name, sizeof name, "%016llx.co", (unsigned long long)fnv1a64(key));
    return dir + "/" + name;
}

bool cache_load(const std::string &path, const std::string &key, std::vector<char> *code) {
    std::ifstream f(path, std::ios::binary);
    if (!f) return false;
    char magic[sizeof kCacheMagic - 1];
    uint64_t klen = 0, clen = 0;
    if (!f.read(magic, sizeof magic) || std::memcmp(magic, kCacheMagic, sizeof magic) != 0) return false;
    if (!f.read((char *)&klen, sizeof klen) || klen != key.size()) return false;
    std::string stored(klen, '\0');
    if (!f.read(&stored[0], (std::streamsize)klen) || stored != key) return false;
    if (!f.read((char *)&clen, sizeof clen) || clen == 0 || clen > (1ull << 30)) return false;
    code->resize(clen);
    return (bool)f.read(code->data(), (std::streamsize)clen);
}

void cache_store(const std::string &dir, const std::string &path, const std::string &key,
                 const std::vector<char> &code) {
    if (!make_dirs(dir)) return;
    std::ostringstream tmp_name;
    tmp_name << path << ".tmp." << getpid() << "." << std::this_thread::get_id();
    const std::string tmp = tmp_name.str();
    {
        std::ofstream f(tmp, std::ios::binary | std::ios::trunc);
        if (!f) return;
        const uint64_t klen = key.size(), clen = code.size();
        f.write(kCacheMagic, sizeof kCacheMagic - 1);
        f.write((const char *)&klen, sizeof klen);
        f.write(key.data(), (std::streamsize)klen);
        f.write((const char *)&clen, sizeof clen);
        f.write(code.data(), (std::streamsize)clen);
        if (!f) {
            f.close();
            std::remove(tmp.c_str());
            return;
        }
    }
    if (std::rename(tmp.c_str(), path.c_str()) != 0) std::remove(tmp.c_str());
}

// Compiles pw_core.h + `tail` into `co->code` (or loads it from the disk
// cache); `ms` receives the time taken and `from_disk` whether it was a hit.
int compile_source(const std::string &tail, CodeObject *co, double *ms, bool *from_disk) {
    std::string full = std::string(kPwCoreSource) + "\n" + tail;
    const auto t0 = std::chrono::steady_clock::now();
    const std::string dir = cache_dir();
    std::string key, path;
    if (!dir.empty()) {
        key = cache_key(full);
        path = cache_path(dir, key);
        if (cache_load(path, key, &co->code)) {
            if (from_disk) *from_disk = true;
            if (ms) *ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
            return TRS_OK;
        }
    }
    hiprtcProgram rp;
    hiprtcResult r = hiprtcCreateProgram(&rp, full.c_str(), "trs_fused.hip", 0, nullptr, nullptr);
    if (r != HIPRTC_SUCCESS) return set_error(TRS_E_FUSION, "hiprtcCreateProgram: %s", hiprtcGetErrorString(r));
    r = hiprtcCompileProgram(rp, (int)(sizeof kRtcOpts / sizeof kRtcOpts[0]), kRtcOpts);
    if (ms) *ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    if (r != HIPRTC_SUCCESS) {
        size_t n = 0;
        hiprtcGetProgramLogSize(rp, &n);
        std::string log(n + 1, '\0');
        hiprtcGetProgramLog(rp, &log[0]);
        hiprtcDestroyProgram(&rp);
        return set_error(TRS_E_FUSION, "hipRTC compile failed: %.900s", log.c_str());
    }
    size_t n = 0;
    hiprtcGetCodeSize(rp, &n);
    co->code.resize(n);
    hiprtcGetCode(rp, co->code.data());
    hiprtcDestroyProgram(&rp);
    if (from_disk) *from_disk = false;
    if (!dir.empty()) cache_store(dir, path, key, co->code);
    return TRS_OK;
}

int compile(Program *prog) { return compile_source(prog->source, &prog->base, &prog->compile_ms, &prog->from_disk); }

Program *lookup(uint64_t id) {
    std::lock_guard<std::mutex> lock(g_mu);
    if (id == 0 || id > g_programs.size()) return nullptr;
    return g_programs[id - 1].get();
}

int get_function(CodeObject *co, DeviceState *dev, const std::string &name, hipFunction_t *fn) {
    std::lock_guard<std::mutex> lock(g_mu);
    const int d = dev->index;
    if (!co->module[d]) TRS_HIP_CHECK(hipModuleLoadData(&co->module[d], co->code.data()), "hipModuleLoadData");
    auto it = co->functions[d].find(name);
    if (it != co->functions[d].end()) {
        *fn = it->second;
        return TRS_OK;
    }
    TRS_HIP_CHECK(hipModuleGetFunction(fn, co->module[d], name.c_str()), "hipModuleGetFunction");
    co->functions[d][name] = *fn;
    return TRS_OK;
}

// A kernel specialised for a launch (streamed-input mask, pw_xpose operand
// roles), compiled on the first launch that needs it and kept, like the
// program, in the process and in the disk cache.  `name` identifies the
// specialisation; `body` is the kernel body call.
int get_spec_function(Program *prog, DeviceState *dev, const std::string &name, const std::string &body,
                      int lanes, hipFunction_t *fn) {
    auto find = [&]() -> CodeObject * {
        std::lock_guard<std::mutex> lock(prog->spec_mu);
        auto it = prog->specs.find(name);
        return it == prog->specs.end() ? nullptr : it->second.get();
    };
    CodeObject *co = find();
    if (!co) {
        // One compile at a time per program; a thread that waited here finds
        // the specialisation another one built meanwhile.
        std::lock_guard<std::mutex> compile_lock(prog->compile_mu);
        co = find();
        if (!co) {
            std::ostringstream w;
            w << prog->functor << "extern \"C\" __global__ void __launch_bounds__(" << lanes << ") " << name
              << "(trs::PwGeom, trs::PwPtrs p) { " << body << "(TrsFused{}, trs::kernarg_geom(), p); }\n";
            auto spec = std::make_unique<CodeObject>();
            const int rc = compile_source(w.str(), spec.get(), nullptr, nullptr);
            if (rc) return rc;
            co = spec.get();
            std::lock_guard<std::mutex> lock(prog->spec_mu);
            prog->specs.emplace(name, std::move(spec));
        }
    }
    return get_function(co, dev, name, fn);
}

int resolve_plan_function(Program *prog, DeviceState *dev, const PwPlan &pl, hipFunction_t *fn) {
    const unsigned strm = pl.g.streamed & ((1u << prog->nin) - 1u);
    const std::string mask = std::to_string(prog->u8mask) + "u";
    char name[128];
    switch (pl.variant) {
    case PwVariant::Flat:
        if (pl.contig) return get_function(&prog->base, dev, "trs_fused_flat_c", fn);
        if (!pl.vec) return get_function(&prog->base, dev, "trs_fused_flat_s", fn);
        std::snprintf(name, sizeof name, "trs_fused_flat_v_%u", strm);
        return get_spec_function(prog, dev, name,
                                 "trs::pw_flat_body<TrsFused, " + mask + ", true, " + std::to_string(strm) + "u>",
                                 kFlatBlock, fn);
    case PwVariant::Rows:
        if (!pl.vec) return get_function(&prog->base, dev, "trs_fused_rows_s", fn);
    {
        const int rk = pl.rk;
        std::snprintf(name, sizeof name, "trs_fused_rows_v%d_%u", rk, strm);
        return get_spec_function(prog, dev, name,
                                 "trs::pw_rows_body<TrsFused, " + mask + ", true, " + std::to_string(strm) + "u, " +
                                     std::to_string(rk) + ">",
                                 kRowLanesMax, fn);
    }
    case PwVariant::Xpose: {
        // The scalar form reads every input plainly, so the streamed mask is
        // not part of its name (one kernel for every mask).
        // Rank 3 fixes the t dim (0 or 1) too; other ranks read it at run time.
        const int td = pl.rk == 3 ? (int)pl.g.tdim : -1;
        std::snprintf(name, sizeof name, "trs_fused_xpose_%c%d_%u_%u_%u_%u_%d_%u%s%s", pl.vec ? 'v' : 's', pl.rk,
                      pl.trans, pl.held, pl.once, pl.xbc, pl.walk, pl.vec ? strm : 0u,
                      td == 0 ? "_t0" : td == 1 ? "_t1" : "", pl.plain ? "_p" : "");
        std::ostringstream b;
        b << "trs::pw_xpose_body<TrsFused, " << mask << ", " << (pl.vec ? "true" : "false") << ", " << kXposeWT << ", "
          << kXposeWX << ", " << pl.trans << "u, " << pl.held << "u, " << pl.once << "u, " << pl.walk << ", "
          << (pl.vec ? strm : 0u) << "u, " << pl.xbc << "u, " << pl.rk << ", " << td << ", "
          << (pl.plain ? "true" : "false") << ">";
        return get_spec_function(prog, dev, name, b.str(), 64 * kXposeWT * kXposeWX, fn);
    }
    case PwVariant::Generic: return get_function(&prog->base, dev, "trs_fused_generic", fn);
    case PwVariant::Empty: break;
    }
    return set_error(TRS_E_INVALID_ARGUMENT, "no kernel for an empty launch");
}

// The kernel of a launch plan: looked up by the plan's signature (variant,
// vector access, role masks, walk, streamed inputs, fixed rank and, at rank
// 3, the transposing kernel's t dim and plain tiles), resolved on a miss.
int get_plan_function(Program *prog, DeviceState *dev, const PwPlan &pl, hipFunction_t *fn) {
    // The streamed mask selects among vector kernels only (the scalar
    // transposing kernel ignores it).
    const uint64_t strm =
        (pl.variant == PwVariant::Xpose && !pl.vec) ? 0 : pl.g.streamed & ((1u << prog->nin) - 1u);
    const uint64_t key = (uint64_t)pl.variant | (uint64_t)pl.vec << 3 | (uint64_t)pl.contig << 4 |
                         (uint64_t)pl.walk << 5 | strm << 9 | (uint64_t)pl.trans << 17 | (uint64_t)pl.held << 25 |
                         (uint64_t)pl.once << 33 | (uint64_t)pl.xbc << 41 | (uint64_t)pl.rk << 49 |
                         (uint64_t)(pl.rk == 3 ? pl.g.tdim : 0) << 52 | (uint64_t)pl.plain << 53;
    {
        std::lock_guard<std::mutex> lock(prog->spec_mu);
        auto it = prog->by_plan[dev->index].find(key);
        if (it != prog->by_plan[dev->index].end()) {
            *fn = it->second;
            return TRS_OK;
        }
    }
    const int rc = resolve_plan_function(prog, dev, pl, fn);
    if (rc) return rc;
    std::lock_guard<std::mutex> lock(prog->spec_mu);
    prog->by_plan[dev->index][key] = *fn;
    return TRS_OK;
}

}  // namespace

}  // namespace trs

using namespace trs;

extern "C" {

int trs_fusion_compile(const char *ir, size_t ir_len, uint64_t *kernel_id) {
    return abi_guard([&]() -> int {
        if (!ir || !kernel_id) return set_error(TRS_E_INVALID_ARGUMENT, "null IR or kernel id pointer");
        const std::string text(ir, ir_len);
        {
            std::lock_guard<std::mutex> lock(g_mu);
            auto it = g_by_ir.find(text);
            if (it != g_by_ir.end()) {
                *kernel_id = it->second;
                return TRS_OK;
            }
        }
        auto prog = std::make_unique<Program>();
        prog->ir = text;
        int rc = generate(text, prog.get());
        if (rc) return rc;
        rc = compile(prog.get());
        if (rc) return rc;
        std::lock_guard<std::mutex> lock(g_mu);
        auto it = g_by_ir.find(text);  // another thread may have won the race
        if (it != g_by_ir.end()) {
            *kernel_id = it->second;
            return TRS_OK;
        }
        g_programs.push_back(std::move(prog));
        *kernel_id = g_programs.size();
        g_by_ir[text] = *kernel_id;
        return TRS_OK;
    });
}

int trs_fusion_launch(uint64_t kernel_id, int n_inputs, const void *const *inputs, const trs_layout *in_layouts,
                      float *out, const trs_layout *lo) {
    return trs_fusion_launch_multi(kernel_id, n_inputs, inputs, in_layouts, 1, &out, lo);
}

int trs_fusion_launch_multi(uint64_t kernel_id, int n_inputs, const void *const *inputs,
                            const trs_layout *in_layouts, int n_outputs, float *const *outputs,
                            const trs_layout *lo) {
    return abi_guard([&]() -> int {
        Program *prog = lookup(kernel_id);
        if (!prog) return set_error(TRS_E_INVALID_ARGUMENT, "unknown fusion kernel id %llu", (unsigned long long)kernel_id);
        if (n_inputs != prog->nin)
            return set_error(TRS_E_INVALID_ARGUMENT, "program takes %d inputs, got %d", prog->nin, n_inputs);
        if (n_outputs != prog->nout)
            return set_error(TRS_E_INVALID_ARGUMENT, "program has %d outputs, got %d", prog->nout, n_outputs);
        if (!inputs || !in_layouts || !outputs) return set_error(TRS_E_INVALID_ARGUMENT, "null inputs or outputs");
        DeviceState *dev = device_state();
        if (!dev) return TRS_E_NO_DEVICE;
        const trs_layout *ls[kMaxIn];
        int eb[kMaxIn];
        for (int i = 0; i < n_inputs; i++) {
            ls[i] = &in_layouts[i];
            eb[i] = ((prog->u8mask >> i) & 1u) ? 1 : 4;
        }
        PwPlan pl;
        int rc = plan_pointwise(lo, outputs[0], n_inputs, inputs, ls, eb, dev->cu_count, &pl, n_outputs, outputs + 1,
                                /*roles=*/true);
        if (rc) return rc;
        if (pl.variant == PwVariant::Empty) return TRS_OK;
        hipFunction_t fn;
        rc = get_plan_function(prog, dev, pl, &fn);
        if (rc) return rc;
        return for_each_part(pl, [&](const PwGeom &g) -> int {
            PwGeom gp = g;
            PwPtrs pp = pl.p;
            void *args[] = {(void *)&gp, (void *)&pp};
            TRS_HIP_CHECK(hipModuleLaunchKernel(fn, (unsigned)pl.grid, 1, 1, (unsigned)pl.block, 1, 1, 0, dev->stream,
                                                args, nullptr),
                          "hipModuleLaunchKernel");
            return TRS_OK;
        });
    });
}

int trs_fusion_outputs(uint64_t kernel_id, int *n_outputs) {
    Program *prog = lookup(kernel_id);
    if (!prog || !n_outputs) return set_error(TRS_E_INVALID_ARGUMENT, "unknown fusion kernel id");
    *n_outputs = prog->nout;
    return TRS_OK;
}

int trs_fusion_source(uint64_t kernel_id, char *buf, size_t buf_len, size_t *needed) {
    Program *prog = lookup(kernel_id);
    if (!prog) return set_error(TRS_E_INVALID_ARGUMENT, "unknown fusion kernel id");
    if (needed) *needed = prog->source.size() + 1;
    if (buf && buf_len) {
        const size_t n = std::min(buf_len - 1, prog->source.size());
        std::memcpy(buf, prog->source.data(), n);
        buf[n] = '\0';
    }
    return TRS_OK;
}

int trs_fusion_compile_ms(uint64_t kernel_id, double *ms) {
    Program *prog = lookup(kernel_id);
    if (!prog || !ms) return set_error(TRS_E_INVALID_ARGUMENT, "unknown fusion kernel id");
    *ms = prog->compile_ms;
    return TRS_OK;
}

int trs_fusion_from_disk_cache(uint64_t kernel_id, int *hit) {
    Program *prog = lookup(kernel_id);
    if (!prog || !hit) return set_error(TRS_E_INVALID_ARGUMENT, "unknown fusion kernel id");
    *hit = prog->from_disk ? 1 : 0;
    return TRS_OK;
}

}  // extern "C"
