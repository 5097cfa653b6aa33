// mambo_loadtest: binds libmambo_hip.so through its runtime ABI manifests.
//
// A C++ consumer of the library (an inference runtime) needs to know, before it calls
// anything, that the shared object it loads has the ABI it was compiled against. The
// manifests (mambo_amd/abi.py, one schema-version-1 JSON document per extern "C" entry
// point) describe each entry point's ordered parameters and the constraints on its
// pointer arguments; this program validates a manifest, checks its parameter list
// against the declarations of include/mambo_hip.h it was compiled with (types from the
// declarations themselves via decltype, names from the table below), dlopens the
// library the manifest names and resolves the symbol. With --probe it then runs one
// projection (quantize -> prepare -> fused matmul) on device 0 through the resolved
// entry points and checks it against a golden fixture.
//
// Counterpart of the reference's tests/cpp/loadtest/loadtest.cpp: schema validation
// with "invalid ABI JSON: ..." errors and exit status 1 (loadtest.cpp:201-219,
// 416-426), exact key sets (:120-136), parameter-by-parameter comparison (:318-335)
// and an ABI-driven launch whose result is checked on the host (:347-412). The
// reference loads a cubin with the CUDA driver API because its kernels have no host
// launcher; this library exports host entry points that choose grids themselves, so
// the unit bound here is a C function in a shared object.
//
//   mambo_loadtest --validate-abi-json <manifest>
//   mambo_loadtest --abi-json <manifest>
//   mambo_loadtest --probe <fixture.npz> --abi-dir <dir>
//   mambo_loadtest --list
#include <dlfcn.h>
#include <hip/hip_runtime_api.h>
#include <zlib.h>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <fstream>
#include <iostream>
#include <map>
#include <memory>
#include <set>
#include <sstream>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "mambo_hip.h"

namespace {

// ------------------------------------------------------------------ JSON (RFC 8259 subset)
struct Json {
    enum Kind { Null, Bool, Int, Real, String, Array, Object } kind = Null;
    bool b = false;
    int64_t i = 0;
    double d = 0.0;
    std::string s;
    std::vector<Json> a;
    std::vector<std::pair<std::string, Json>> o;

    const Json *find(const std::string &key) const
    {
        for (const auto &kv : o)
            if (kv.first == key)
                return &kv.second;
        return nullptr;
    }
};

class JsonParser {
  public:
    explicit JsonParser(const std::string &text) : t_(text) {}

    Json parse()
    {
        Json v = value();
        ws();
        if (p_ != t_.size())
            fail("trailing characters");
        return v;
    }

  private:
    const std::string &t_;
    size_t p_ = 0;
    int depth_ = 0;

    [[noreturn]] void fail(const std::string &what) const
    {
        throw std::runtime_error(what + " at offset " + std::to_string(p_));
    }
    void ws()
    {
        while (p_ < t_.size() && (t_[p_] == ' ' || t_[p_] == '\t' || t_[p_] == '\n' || t_[p_] == '\r'))
            ++p_;
    }
    bool eat(const char *lit)
    {
        size_t n = std::strlen(lit);
        if (t_.compare(p_, n, lit) == 0) {
            p_ += n;
            return true;
        }
        return false;
    }
    Json value()
    {
        ws();
        if (p_ >= t_.size())
            fail("unexpected end of input");
        if (++depth_ > 64)
            fail("nesting too deep");
        Json v;
        const char c = t_[p_];
        if (c == '{') {
            v.kind = Json::Object;
            ++p_;
            ws();
            if (p_ < t_.size() && t_[p_] == '}') {
                ++p_;
            } else {
                for (;;) {
                    ws();
                    if (p_ >= t_.size() || t_[p_] != '"')
                        fail("expected a string key");
                    std::string key = string();
                    if (v.find(key))
                        fail("duplicate key \"" + key + "\"");
                    ws();
                    if (p_ >= t_.size() || t_[p_++] != ':')
                        fail("expected ':'");
                    v.o.emplace_back(key, value());
                    ws();
                    if (p_ < t_.size() && t_[p_] == ',') {
                        ++p_;
                        continue;
                    }
                    if (p_ < t_.size() && t_[p_] == '}') {
                        ++p_;
                        break;
                    }
                    fail("expected ',' or '}'");
                }
            }
        } else if (c == '[') {
            v.kind = Json::Array;
            ++p_;
            ws();
            if (p_ < t_.size() && t_[p_] == ']') {
                ++p_;
            } else {
                for (;;) {
                    v.a.push_back(value());
                    ws();
                    if (p_ < t_.size() && t_[p_] == ',') {
                        ++p_;
                        continue;
                    }
                    if (p_ < t_.size() && t_[p_] == ']') {
                        ++p_;
                        break;
                    }
                    fail("expected ',' or ']'");
                }
            }
        } else if (c == '"') {
            v.kind = Json::String;
            v.s = string();
        } else if (eat("true")) {
            v.kind = Json::Bool;
            v.b = true;
        } else if (eat("false")) {
            v.kind = Json::Bool;
        } else if (eat("null")) {
            v.kind = Json::Null;
        } else if (c == '-' || (c >= '0' && c <= '9')) {
            number(v);
        } else {
            fail("unexpected character");
        }
        --depth_;
        return v;
    }
    std::string string()
    {
        ++p_;  // opening quote
        std::string out;
        for (;;) {
            if (p_ >= t_.size())
                fail("unterminated string");
            char c = t_[p_++];
            if (c == '"')
                return out;
            if ((unsigned char)c < 0x20)
                fail("control character in string");
            if (c != '\\') {
                out += c;
                continue;
            }
            if (p_ >= t_.size())
                fail("unterminated escape");
            char e = t_[p_++];
            switch (e) {
            case '"': out += '"'; break;
            case '\\': out += '\\'; break;
            case '/': out += '/'; break;
            case 'b': out += '\b'; break;
            case 'f': out += '\f'; break;
            case 'n': out += '\n'; break;
            case 'r': out += '\r'; break;
            case 't': out += '\t'; break;
            case 'u': {
                if (p_ + 4 > t_.size())
                    fail("short \\u escape");
                unsigned cp = (unsigned)std::stoul(t_.substr(p_, 4), nullptr, 16);
                p_ += 4;
                if (cp >= 0xD800 && cp < 0xE000)
                    fail("surrogate escapes are not supported");
                if (cp < 0x80) {
                    out += (char)cp;
                } else if (cp < 0x800) {
                    out += (char)(0xC0 | (cp >> 6));
                    out += (char)(0x80 | (cp & 0x3F));
                } else {
                    out += (char)(0xE0 | (cp >> 12));
                    out += (char)(0x80 | ((cp >> 6) & 0x3F));
                    out += (char)(0x80 | (cp & 0x3F));
                }
                break;
            }
            default: fail("bad escape");
            }
        }
    }
    void number(Json &v)
    {
        const size_t start = p_;
        if (t_[p_] == '-')
            ++p_;
        bool real = false;
        while (p_ < t_.size()) {
            char c = t_[p_];
            if (c >= '0' && c <= '9') {
                ++p_;
            } else if (c == '.' || c == 'e' || c == 'E' || c == '+' || (c == '-' && p_ > start)) {
                real = true;
                ++p_;
            } else {
                break;
            }
        }
        const std::string text = t_.substr(start, p_ - start);
        size_t used = 0;
        try {
            if (real) {
                v.kind = Json::Real;
                v.d = std::stod(text, &used);
            } else {
                v.kind = Json::Int;
                v.i = std::stoll(text, &used, 10);
            }
        } catch (const std::out_of_range &) {
            fail("number outside the supported range");
        } catch (const std::exception &) {
            fail("malformed number");
        }
        if (used != text.size())
            fail("malformed number");
    }
};

// ------------------------------------------------------------------ compiled declarations
// ABI type names of the C types in mambo_hip.h (the vocabulary mambo_amd/abi.py writes).
template <class T> struct AbiName;
#define MAMBO_ABI_NAME(T, S)                                                                                          \
    template <> struct AbiName<T> {                                                                                   \
        static std::string get() { return S; }                                                                        \
    };
MAMBO_ABI_NAME(void, "void")
MAMBO_ABI_NAME(char, "char")
MAMBO_ABI_NAME(int32_t, "int32")
MAMBO_ABI_NAME(int64_t, "int64")
MAMBO_ABI_NAME(uint8_t, "uint8")
MAMBO_ABI_NAME(uint16_t, "uint16")
MAMBO_ABI_NAME(uint32_t, "uint32")
MAMBO_ABI_NAME(uint64_t, "uint64")
MAMBO_ABI_NAME(float, "float32")
MAMBO_ABI_NAME(double, "float64")
MAMBO_ABI_NAME(mambo_gemm_config, "mambo_gemm_config")
MAMBO_ABI_NAME(mambo_projection, "mambo_projection")
MAMBO_ABI_NAME(mambo_chain_launch, "mambo_chain_launch")
MAMBO_ABI_NAME(mambo_chain_config, "mambo_chain_config")
MAMBO_ABI_NAME(mambo_stream_t, "hipStream_t")
#undef MAMBO_ABI_NAME
template <class T> struct AbiName<T *> {
    static std::string get() { return AbiName<T>::get() + "*"; }
};
template <class T> struct AbiName<const T *> {
    static std::string get() { return "const " + AbiName<T>::get() + "*"; }
};

template <class F> struct Signature;
template <class R, class... A> struct Signature<R(A...)> {
    static constexpr size_t arity = sizeof...(A);
    static std::string returns() { return AbiName<R>::get(); }
    static std::vector<std::string> params() { return {AbiName<A>::get()...}; }
};

struct EntryDecl {
    std::string symbol;
    std::string returns;
    std::vector<std::string> types;
    std::vector<std::string> names;
};

template <class F, class... N> EntryDecl declare(const char *symbol, N... names)
{
    static_assert(sizeof...(N) == Signature<F>::arity, "parameter names must match the declaration's arity");
    return EntryDecl{symbol, Signature<F>::returns(), Signature<F>::params(), {names...}};
}

#define MAMBO_ENTRY(fn, ...) declare<decltype(fn)>(#fn, ##__VA_ARGS__)

const std::vector<EntryDecl> &compiled_entries()
{
    static const std::vector<EntryDecl> entries = {
        MAMBO_ENTRY(mambo_last_error),
        MAMBO_ENTRY(mambo_abi_version),
        MAMBO_ENTRY(mambo_build_arch),
        MAMBO_ENTRY(mambo_device_arch, "device", "buf", "buf_len"),
        MAMBO_ENTRY(mambo_iq3s_grid, "out"),
        MAMBO_ENTRY(mambo_iq3s_fp8_grid, "out"),
        MAMBO_ENTRY(mambo_iq3s_split_table, "out"),
        MAMBO_ENTRY(mambo_quantize_mxfp8, "x", "x_dtype", "m", "k", "ldx", "values", "ldv", "scales", "lds", "stream"),
        MAMBO_ENTRY(mambo_iq3s_packed_bytes, "n", "blocks"),
        MAMBO_ENTRY(mambo_iq3s_prepare, "raw", "n", "blocks", "stride_n", "stride_b", "stride_byte", "d", "qs", "qh",
                    "signs", "scales", "packed", "stream"),
        MAMBO_ENTRY(mambo_iq3s_pack, "d", "qs", "qh", "signs", "scales", "n", "blocks", "packed", "stream"),
        MAMBO_ENTRY(mambo_iq3s_dequant, "d", "qs", "qh", "signs", "scales", "n", "blocks", "values", "out_scales",
                    "stream"),
        MAMBO_ENTRY(mambo_iq3s_fp8_matmul, "xv", "ldxv", "xs", "ldxs", "m", "packed", "n", "blocks", "out", "ldo", "cfg",
                    "stream"),
        MAMBO_ENTRY(mambo_iq3s_fp8_matmul_grouped, "xv", "ldxv", "xs", "ldxs", "m", "proj", "count", "blocks", "cfg",
                    "stream"),
        MAMBO_ENTRY(mambo_iq3s_matmul_quantize_grouped, "x", "x_dtype", "ldx", "m", "proj", "count", "blocks", "cfg",
                    "xv", "ldxv", "xs", "ldxs", "stream"),
        MAMBO_ENTRY(mambo_iq3s_matmul_quantize_grouped_noalloc, "x", "x_dtype", "ldx", "m", "proj", "count", "blocks",
                    "cfg", "stream"),
        MAMBO_ENTRY(mambo_iq3s_fp8_matmul_chain, "m", "launches", "count", "cfg", "sync", "stream"),
        MAMBO_ENTRY(mambo_chain_status, "sync"),
        MAMBO_ENTRY(mambo_gemm_default_config, "m", "n", "blocks", "out"),
        MAMBO_ENTRY(mambo_gemm_check_config, "m", "n", "blocks", "cfg"),
        MAMBO_ENTRY(mambo_gemm_config_enumerate, "m", "n", "blocks", "out", "capacity"),
        MAMBO_ENTRY(mambo_synth_iq3s, "seed", "blocks", "row0", "nrows", "raw", "stream"),
        MAMBO_ENTRY(mambo_synth_bf16, "seed", "outlier_seed", "outlier_frac", "i0", "count", "out", "stream"),
        MAMBO_ENTRY(mambo_e4m3_convert, "in", "n", "out_sw", "out_hw", "stream"),
        MAMBO_ENTRY(mambo_fill_f32, "ptr", "n", "value", "stream"),
        MAMBO_ENTRY(mambo_copy_bytes, "src", "dst", "bytes", "stream"),
        MAMBO_ENTRY(mambo_read_bytes, "src", "bytes", "sink", "stream"),
        MAMBO_ENTRY(mambo_mfma_peak, "workgroups", "iters", "out", "stream"),
    };
    return entries;
}
#undef MAMBO_ENTRY

const EntryDecl *compiled_entry(const std::string &symbol)
{
    for (const auto &e : compiled_entries())
        if (e.symbol == symbol)
            return &e;
    return nullptr;
}

// ------------------------------------------------------------------ manifest validation
[[noreturn]] void invalid_abi(const std::string &message)
{
    throw std::invalid_argument("invalid ABI JSON: " + message);
}

void require_exact_keys(const Json &object, const std::set<std::string> &expected, const std::string &where)
{
    if (object.kind != Json::Object)
        invalid_abi(where + " must be an object");
    std::set<std::string> actual;
    for (const auto &kv : object.o)
        actual.insert(kv.first);
    if (actual == expected)
        return;
    std::string message = where + " has unsupported fields";
    for (const auto &k : actual)
        if (!expected.count(k)) {
            message += "; unknown=" + k;
            break;
        }
    for (const auto &k : expected)
        if (!actual.count(k)) {
            message += "; missing=" + k;
            break;
        }
    invalid_abi(message);
}

const std::string &string_field(const Json &object, const std::string &key, const std::string &message)
{
    const Json *v = object.find(key);
    if (!v || v->kind != Json::String || v->s.empty())
        invalid_abi(message);
    return v->s;
}

struct Parameter {
    std::string name;
    std::string type;
};

struct Manifest {
    std::string path;
    std::string symbol;
    std::string library_path;  // resolved against the manifest's directory
    int64_t abi_version = 0;
    std::string returns;
    std::vector<Parameter> parameters;
    size_t constraints = 0;
};

const std::set<std::string> kDtypes = {"uint8",  "uint16",  "uint32",           "int32",
                                       "float32", "char",   "float32|bfloat16", "mambo_gemm_config",
                                       "mambo_projection", "mambo_chain_launch", "mambo_chain_config"};

void validate_constraint(const Json &c, const std::map<std::string, std::string> &pointer_types)
{
    if (c.kind != Json::Object || !c.find("name") || c.find("name")->kind != Json::String)
        invalid_abi("each constraint must have a string name");
    const std::string name = c.find("name")->s;
    require_exact_keys(c,
                       {"name", "kind", "dtype", "ndim", "shape", "strides", "base_addr_divisible_by", "memory",
                        "nullable", "access"},
                       "constraint " + name);
    auto ptr = pointer_types.find(name);
    if (ptr == pointer_types.end())
        invalid_abi("constraint " + name + " does not name a pointer parameter");
    if (c.find("kind")->kind != Json::String || c.find("kind")->s != "array")
        invalid_abi("constraint " + name + ": only array constraints are supported");
    const Json &dtype = *c.find("dtype");
    if (dtype.kind != Json::String || !kDtypes.count(dtype.s))
        invalid_abi("constraint " + name + ": unsupported dtype");
    const Json &ndim = *c.find("ndim");
    if (ndim.kind != Json::Int || ndim.i < 1 || ndim.i > 4)
        invalid_abi("constraint " + name + ": ndim must be an integer in [1, 4]");
    for (const char *key : {"shape", "strides"}) {
        const Json &v = *c.find(key);
        if (v.kind != Json::Array || (int64_t)v.a.size() != ndim.i)
            invalid_abi("constraint " + name + ": " + key + " must list ndim extents");
        for (const Json &e : v.a)
            if (e.kind != Json::String || e.s.empty())
                invalid_abi("constraint " + name + ": " + key + " entries must be non-empty expressions");
    }
    const Json &align = *c.find("base_addr_divisible_by");
    if (align.kind != Json::Int || align.i < 1 || align.i > 256 || (align.i & (align.i - 1)))
        invalid_abi("constraint " + name + ": base_addr_divisible_by must be a power of two in [1, 256]");
    const Json &memory = *c.find("memory");
    if (memory.kind != Json::String || (memory.s != "device" && memory.s != "host"))
        invalid_abi("constraint " + name + ": memory must be \"device\" or \"host\"");
    if (c.find("nullable")->kind != Json::Bool)
        invalid_abi("constraint " + name + ": nullable must be a boolean");
    const Json &access = *c.find("access");
    if (access.kind != Json::String || (access.s != "read" && access.s != "write" && access.s != "readwrite"))
        invalid_abi("constraint " + name + ": access must be read, write or readwrite");
    if (ptr->second.rfind("const ", 0) == 0 && access.s != "read")
        invalid_abi("constraint " + name + ": a const pointer parameter cannot be written");
}

Manifest load_manifest(const std::string &path)
{
    Json doc;
    {
        std::ifstream in(path, std::ios::binary);
        if (!in)
            invalid_abi("cannot open " + path);
        std::stringstream buf;
        buf << in.rdbuf();
        try {
            doc = JsonParser(buf.str()).parse();
        } catch (const std::runtime_error &e) {
            invalid_abi(std::string("malformed JSON: ") + e.what());
        }
    }
    if (doc.kind != Json::Object)
        invalid_abi("root must be an object");
    const Json *schema = doc.find("schema_version");
    if (!schema || schema->kind != Json::Int || schema->i != 1)
        invalid_abi("schema_version 1 is required");
    if (doc.find("constants"))
        invalid_abi("compile-time constants must be omitted from runtime ABI JSON");
    const Json *cc = doc.find("calling_convention");
    if (!cc || cc->kind != Json::String || cc->s != "mambo_c_abi_v1")
        invalid_abi("unsupported calling convention");
    const Json *name = doc.find("name");
    const Json *symbol = doc.find("symbol");
    if (!name || !symbol || name->kind != Json::String || symbol->kind != Json::String || name->s != symbol->s ||
        symbol->s.empty())
        invalid_abi("name and symbol must be matching strings");
    require_exact_keys(doc,
                       {"schema_version", "name", "symbol", "library_path", "gpu_code", "calling_convention",
                        "abi_version", "returns", "parameters", "constraints", "toolchain"},
                       "root");
    Manifest m;
    m.path = path;
    m.symbol = symbol->s;
    m.library_path = string_field(doc, "library_path", "library_path must be a non-empty string");
    const std::string &gpu = string_field(doc, "gpu_code", "gpu_code must use the gfxNNN form");
    if (gpu.rfind("gfx", 0) != 0 || gpu.size() < 6 || gpu.find_first_not_of("0123456789abcdef", 3) != std::string::npos)
        invalid_abi("gpu_code must use the gfxNNN form");
    const Json *tc = doc.find("toolchain");
    if (tc->kind != Json::Object || !tc->find("python") || !tc->find("hipcc"))
        invalid_abi("toolchain metadata is missing");
    const Json *ver = doc.find("abi_version");
    if (ver->kind != Json::Int || ver->i <= 0)
        invalid_abi("abi_version must be a positive integer");
    m.abi_version = ver->i;
    m.returns = string_field(doc, "returns", "returns must be a type name");

    const Json &params = *doc.find("parameters");
    if (params.kind != Json::Array)
        invalid_abi("parameters must be an array");
    std::map<std::string, std::string> pointer_types;
    std::set<std::string> names;
    for (const Json &p : params.a) {
        require_exact_keys(p, {"name", "type"}, "parameter");
        if (p.find("name")->kind != Json::String || p.find("type")->kind != Json::String ||
            p.find("name")->s.empty() || p.find("type")->s.empty())
            invalid_abi("parameter name and type must be non-empty strings");
        Parameter q{p.find("name")->s, p.find("type")->s};
        if (!names.insert(q.name).second)
            invalid_abi("duplicate parameter name " + q.name);
        if (q.type.back() == '*')
            pointer_types[q.name] = q.type;
        m.parameters.push_back(q);
    }
    const Json &cons = *doc.find("constraints");
    if (cons.kind != Json::Array)
        invalid_abi("constraints must be an array");
    std::set<std::string> constrained;
    for (const Json &c : cons.a) {
        validate_constraint(c, pointer_types);
        if (!constrained.insert(c.find("name")->s).second)
            invalid_abi("duplicate constraint name " + c.find("name")->s);
    }
    for (const auto &kv : pointer_types)
        if (!constrained.count(kv.first))
            invalid_abi("pointer parameter " + kv.first + " has no constraint");
    m.constraints = cons.a.size();

    // The manifest against the declaration this program was compiled with.
    const EntryDecl *decl = compiled_entry(m.symbol);
    if (!decl)
        invalid_abi("entry point " + m.symbol + " is unknown to this loader");
    if (decl->returns != m.returns)
        invalid_abi("return type " + m.returns + " does not match the declaration (" + decl->returns + ")");
    if (decl->types.size() != m.parameters.size())
        invalid_abi("parameter count " + std::to_string(m.parameters.size()) + " does not match the declaration (" +
                    std::to_string(decl->types.size()) + ")");
    for (size_t i = 0; i < m.parameters.size(); ++i)
        if (m.parameters[i].type != decl->types[i] || m.parameters[i].name != decl->names[i])
            invalid_abi("unsupported or reordered ABI parameter at index " + std::to_string(i) + " (declared " +
                        decl->types[i] + " " + decl->names[i] + ", manifest has " + m.parameters[i].type + " " +
                        m.parameters[i].name + ")");

    if (m.library_path[0] != '/') {
        const size_t slash = path.find_last_of('/');
        const std::string dir = slash == std::string::npos ? "." : path.substr(0, slash);
        m.library_path = dir + "/" + m.library_path;
    }
    return m;
}

// ------------------------------------------------------------------ binding
struct Library {
    void *handle = nullptr;
    std::string path;
    ~Library()
    {
        if (handle)
            dlclose(handle);
    }
};

class Binder {
  public:
    // Validates the manifest, opens its library (once per path) and resolves the symbol.
    void *bind(const Manifest &m)
    {
        Library &lib = libs_[m.library_path];
        if (!lib.handle) {
            lib.path = m.library_path;
            lib.handle = dlopen(m.library_path.c_str(), RTLD_NOW | RTLD_LOCAL);
            if (!lib.handle)
                throw std::runtime_error("cannot load " + m.library_path + ": " + dlerror());
            auto version = reinterpret_cast<decltype(&mambo_abi_version)>(dlsym(lib.handle, "mambo_abi_version"));
            if (!version)
                throw std::runtime_error(m.library_path + " does not export mambo_abi_version");
            const int have = version();
            if (have != m.abi_version)
                throw std::runtime_error("library ABI version " + std::to_string(have) + " does not match the manifest's " +
                                         std::to_string(m.abi_version));
        }
        void *fn = dlsym(lib.handle, m.symbol.c_str());
        if (!fn)
            throw std::runtime_error("symbol " + m.symbol + " is not exported by " + m.library_path);
        return fn;
    }

    template <class F> F *bind_from(const std::string &dir, const char *symbol)
    {
        const Manifest m = load_manifest(dir + "/" + symbol + ".abi.json");
        if (m.symbol != symbol)
            invalid_abi("manifest for " + std::string(symbol) + " names " + m.symbol);
        return reinterpret_cast<F *>(bind(m));
    }

  private:
    std::map<std::string, Library> libs_;
};

// ------------------------------------------------------------------ .npz fixture reader
struct NpyArray {
    std::string descr;
    std::vector<int64_t> shape;
    std::vector<uint8_t> data;
    int64_t count() const
    {
        int64_t n = 1;
        for (int64_t s : shape)
            n *= s;
        return n;
    }
};

uint32_t le32(const uint8_t *p) { return p[0] | (p[1] << 8) | (p[2] << 16) | ((uint32_t)p[3] << 24); }
uint16_t le16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
uint64_t le64(const uint8_t *p) { return le32(p) | ((uint64_t)le32(p + 4) << 32); }

NpyArray parse_npy(const std::vector<uint8_t> &b, const std::string &what)
{
    if (b.size() < 10 || std::memcmp(b.data(), "\x93NUMPY", 6) != 0)
        throw std::runtime_error(what + ": not an NPY array");
    const int major = b[6];
    size_t hlen, off;
    if (major == 1) {
        hlen = le16(&b[8]);
        off = 10;
    } else {
        hlen = le32(&b[8]);
        off = 12;
    }
    if (off + hlen > b.size())
        throw std::runtime_error(what + ": truncated NPY header");
    const std::string h(reinterpret_cast<const char *>(&b[off]), hlen);
    NpyArray a;
    auto field = [&](const char *key) {
        size_t k = h.find(key);
        if (k == std::string::npos)
            throw std::runtime_error(what + ": NPY header lacks " + key);
        return h.find(':', k) + 1;
    };
    size_t d = h.find('\'', field("'descr'"));
    a.descr = h.substr(d + 1, h.find('\'', d + 1) - d - 1);
    const size_t order = h.find_first_not_of(' ', field("'fortran_order'"));
    if (order == std::string::npos || h.compare(order, 5, "False") != 0)
        throw std::runtime_error(what + ": only C-ordered arrays are supported");
    size_t s = h.find('(', field("'shape'")), e = h.find(')', s);
    std::stringstream dims(h.substr(s + 1, e - s - 1));
    std::string tok;
    while (std::getline(dims, tok, ','))
        if (tok.find_first_not_of(' ') != std::string::npos)
            a.shape.push_back(std::stoll(tok));
    const size_t body = off + hlen;
    a.data.assign(b.begin() + (long)body, b.end());
    return a;
}

std::map<std::string, NpyArray> read_npz(const std::string &path)
{
    std::ifstream in(path, std::ios::binary);
    if (!in)
        throw std::runtime_error("cannot open " + path);
    std::vector<uint8_t> z((std::istreambuf_iterator<char>(in)), std::istreambuf_iterator<char>());
    // end of central directory record
    if (z.size() < 22)
        throw std::runtime_error(path + ": not a zip archive");
    size_t eocd = std::string::npos;
    for (size_t i = z.size() - 22 + 1; i-- > 0;)
        if (le32(&z[i]) == 0x06054b50) {
            eocd = i;
            break;
        }
    if (eocd == std::string::npos)
        throw std::runtime_error(path + ": no end of central directory");
    uint64_t entries = le16(&z[eocd + 10]);
    uint64_t cd = le32(&z[eocd + 16]);
    if ((cd == 0xFFFFFFFFu || entries == 0xFFFF) && eocd >= 20 && le32(&z[eocd - 20]) == 0x07064b50) {
        const uint64_t rec = le64(&z[eocd - 20 + 8]);
        if (rec + 56 > z.size() || le32(&z[rec]) != 0x06064b50)
            throw std::runtime_error(path + ": bad zip64 end record");
        entries = le64(&z[rec + 32]);
        cd = le64(&z[rec + 48]);
    }
    std::map<std::string, NpyArray> out;
    size_t p = cd;
    for (uint64_t n = 0; n < entries; ++n) {
        if (p + 46 > z.size() || le32(&z[p]) != 0x02014b50)
            throw std::runtime_error(path + ": bad central directory entry");
        const uint16_t method = le16(&z[p + 10]);
        uint64_t csize = le32(&z[p + 20]), usize = le32(&z[p + 24]);
        const uint16_t nlen = le16(&z[p + 28]), xlen = le16(&z[p + 30]), clen = le16(&z[p + 32]);
        uint64_t local = le32(&z[p + 42]);
        std::string name(reinterpret_cast<const char *>(&z[p + 46]), nlen);
        // zip64 extended information: the fields that read 0xFFFFFFFF, in this order
        for (size_t x = p + 46 + nlen; x + 4 <= p + 46 + nlen + xlen;) {
            const uint16_t id = le16(&z[x]), len = le16(&z[x + 2]);
            if (id == 0x0001) {
                size_t q = x + 4;
                if (usize == 0xFFFFFFFFu) { usize = le64(&z[q]); q += 8; }
                if (csize == 0xFFFFFFFFu) { csize = le64(&z[q]); q += 8; }
                if (local == 0xFFFFFFFFu) { local = le64(&z[q]); }
            }
            x += 4 + len;
        }
        p += 46 + nlen + xlen + clen;
        if (local + 30 > z.size() || le32(&z[local]) != 0x04034b50)
            throw std::runtime_error(path + ": bad local header for " + name);
        const size_t data = local + 30 + le16(&z[local + 26]) + le16(&z[local + 28]);
        if (data + csize > z.size())
            throw std::runtime_error(path + ": truncated member " + name);
        std::vector<uint8_t> raw(usize);
        if (method == 0) {
            if (csize != usize)
                throw std::runtime_error(path + ": stored member size mismatch");
            std::memcpy(raw.data(), &z[data], usize);
        } else if (method == 8) {
            z_stream zs{};
            if (inflateInit2(&zs, -MAX_WBITS) != Z_OK)
                throw std::runtime_error("inflateInit2 failed");
            zs.next_in = &z[data];
            zs.avail_in = (uInt)csize;
            zs.next_out = raw.data();
            zs.avail_out = (uInt)usize;
            const int rc = inflate(&zs, Z_FINISH);
            inflateEnd(&zs);
            if (rc != Z_STREAM_END || zs.total_out != usize)
                throw std::runtime_error(path + ": cannot inflate " + name);
        } else {
            throw std::runtime_error(path + ": unsupported compression method for " + name);
        }
        if (name.size() > 4 && name.compare(name.size() - 4, 4, ".npy") == 0)
            name.resize(name.size() - 4);
        out[name] = parse_npy(raw, path + ":" + name);
    }
    return out;
}

const NpyArray &member(const std::map<std::string, NpyArray> &npz, const std::string &name, const std::string &descr,
                       size_t ndim)
{
    auto it = npz.find(name);
    if (it == npz.end())
        throw std::runtime_error("fixture lacks array " + name);
    if (it->second.descr != descr || it->second.shape.size() != ndim)
        throw std::runtime_error("fixture array " + name + " has dtype " + it->second.descr + " and " +
                                 std::to_string(it->second.shape.size()) + " dimensions, expected " + descr);
    if ((int64_t)it->second.data.size() < it->second.count() * (descr == "<f4" ? 4 : 1))
        throw std::runtime_error("fixture array " + name + " is truncated");
    return it->second;
}

// ------------------------------------------------------------------ probe
void hip_check(hipError_t err, const char *what)
{
    if (err != hipSuccess)
        throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(err));
}

struct DeviceBuffers {
    std::vector<void *> ptrs;
    void *alloc(size_t bytes)
    {
        void *p = nullptr;
        hip_check(hipMalloc(&p, bytes ? bytes : 1), "hipMalloc");
        ptrs.push_back(p);
        return p;
    }
    ~DeviceBuffers()
    {
        for (void *p : ptrs)
            (void)hipFree(p);
    }
};

int run_probe(const std::string &fixture, const std::string &abi_dir)
{
    Binder binder;
    auto last_error = binder.bind_from<decltype(mambo_last_error)>(abi_dir, "mambo_last_error");
    auto quantize = binder.bind_from<decltype(mambo_quantize_mxfp8)>(abi_dir, "mambo_quantize_mxfp8");
    auto packed_bytes = binder.bind_from<decltype(mambo_iq3s_packed_bytes)>(abi_dir, "mambo_iq3s_packed_bytes");
    auto prepare = binder.bind_from<decltype(mambo_iq3s_prepare)>(abi_dir, "mambo_iq3s_prepare");
    auto matmul = binder.bind_from<decltype(mambo_iq3s_fp8_matmul)>(abi_dir, "mambo_iq3s_fp8_matmul");
    auto call = [&](int rc, const char *what) {
        if (rc != MAMBO_OK)
            throw std::runtime_error(std::string(what) + " returned " + std::to_string(rc) + ": " + last_error());
    };

    const auto npz = read_npz(fixture);
    const NpyArray &raw = member(npz, "raw", "|u1", 3);
    const NpyArray &x = member(npz, "x", "<f4", 2);
    const NpyArray &xv_ref = member(npz, "x_values", "|u1", 2);
    const NpyArray &xs_ref = member(npz, "x_scales", "|u1", 2);
    const NpyArray &out_ref = member(npz, "out", "<f4", 2);
    const int64_t n = raw.shape[0], blocks = raw.shape[1], m = x.shape[0], k = x.shape[1];
    if (raw.shape[2] != 110 || k != blocks * 256 || xv_ref.shape != std::vector<int64_t>{m, k} ||
        xs_ref.shape != std::vector<int64_t>{m, k / 32} || out_ref.shape != std::vector<int64_t>{m, n})
        throw std::runtime_error("fixture shapes are inconsistent");

    hip_check(hipSetDevice(0), "hipSetDevice");
    DeviceBuffers dev;
    void *raw_d = dev.alloc(raw.data.size());
    void *x_d = dev.alloc((size_t)(m * k) * 4);
    auto *xv_d = static_cast<uint8_t *>(dev.alloc((size_t)(m * k)));
    auto *xs_d = static_cast<uint8_t *>(dev.alloc((size_t)(m * k / 32)));
    auto *out_d = static_cast<float *>(dev.alloc((size_t)(m * n) * 4));
    const int64_t pbytes = packed_bytes(n, blocks);
    if (pbytes <= 0)
        throw std::runtime_error("mambo_iq3s_packed_bytes returned " + std::to_string(pbytes));
    auto *packed_d = static_cast<uint8_t *>(dev.alloc((size_t)pbytes));
    hip_check(hipMemcpy(raw_d, raw.data.data(), raw.data.size(), hipMemcpyHostToDevice), "hipMemcpy raw");
    hip_check(hipMemcpy(x_d, x.data.data(), (size_t)(m * k) * 4, hipMemcpyHostToDevice), "hipMemcpy x");

    call(quantize(x_d, MAMBO_DTYPE_F32, m, k, k, xv_d, k, xs_d, k / 32, nullptr), "mambo_quantize_mxfp8");
    call(prepare(static_cast<const uint8_t *>(raw_d), n, blocks, blocks * 110, 110, 1, nullptr, nullptr, nullptr,
                 nullptr, nullptr, packed_d, nullptr),
         "mambo_iq3s_prepare");
    call(matmul(xv_d, k, xs_d, k / 32, m, packed_d, n, blocks, out_d, n, nullptr, nullptr), "mambo_iq3s_fp8_matmul");
    hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");

    std::vector<uint8_t> xv((size_t)(m * k)), xs((size_t)(m * k / 32));
    std::vector<float> out((size_t)(m * n));
    hip_check(hipMemcpy(xv.data(), xv_d, xv.size(), hipMemcpyDeviceToHost), "hipMemcpy values");
    hip_check(hipMemcpy(xs.data(), xs_d, xs.size(), hipMemcpyDeviceToHost), "hipMemcpy scales");
    hip_check(hipMemcpy(out.data(), out_d, out.size() * 4, hipMemcpyDeviceToHost), "hipMemcpy out");
    if (std::memcmp(xv.data(), xv_ref.data.data(), xv.size()) != 0 ||
        std::memcmp(xs.data(), xs_ref.data.data(), xs.size()) != 0) {
        std::cerr << "MXFP8 codes or scales differ from the fixture\n";
        return 1;
    }
    const float *expected = reinterpret_cast<const float *>(out_ref.data.data());
    double num = 0.0, den = 0.0;
    for (size_t i = 0; i < out.size(); ++i) {
        const double e = expected[i], g = out[i];
        num += (g - e) * (g - e);
        den += e * e;
        // the reference test's elementwise bound (test_iq3_s_fp8.py:201)
        if (!(std::fabs(g - e) <= 5e-3 + 5e-4 * std::fabs(e))) {
            std::cerr << "projection mismatch at (" << i / n << ", " << i % n << "): got " << g << ", expected " << e
                      << '\n';
            return 1;
        }
    }
    const double rel = den > 0 ? std::sqrt(num / den) : std::sqrt(num);
    if (!(rel <= 1e-3)) {
        std::cerr << "projection rel-L2 " << rel << " exceeds 1e-3\n";
        return 1;
    }
    std::cout << "ABI-driven projection passed for M=" << m << " N=" << n << " K=" << k
              << " (mambo_quantize_mxfp8, mambo_iq3s_prepare, mambo_iq3s_fp8_matmul bound through " << abi_dir
              << "), rel-L2 " << rel << ".\n";
    return 0;
}

void usage(const char *argv0)
{
    std::cerr << "Usage: " << argv0 << " --validate-abi-json <manifest>\n"
              << "       " << argv0 << " --abi-json <manifest>\n"
              << "       " << argv0 << " --probe <fixture.npz> --abi-dir <dir>\n"
              << "       " << argv0 << " --list\n"
              << "Validates libmambo_hip runtime ABI manifests (schema_version 1) against the declarations this "
                 "program was compiled with, binds the entry points they describe, and runs one projection "
                 "through them.\n";
}

}  // namespace

int main(int argc, char **argv)
{
    const std::string mode = argc >= 2 ? argv[1] : "";
    try {
        if (argc == 3 && mode == "--validate-abi-json") {
            const Manifest m = load_manifest(argv[2]);
            std::cout << "ABI JSON valid for entry point " << m.symbol << " (" << m.parameters.size() << " parameters, "
                      << m.constraints << " constraints).\n";
            return 0;
        }
        if (argc == 3 && mode == "--abi-json") {
            const Manifest m = load_manifest(argv[2]);
            Binder binder;
            binder.bind(m);
            std::cout << "bound " << m.symbol << " from " << m.library_path << " (ABI version " << m.abi_version
                      << ").\n";
            return 0;
        }
        if (argc == 5 && mode == "--probe" && std::string(argv[3]) == "--abi-dir")
            return run_probe(argv[2], argv[4]);
        if (argc == 2 && mode == "--list") {
            for (const auto &e : compiled_entries()) {
                std::cout << e.symbol << '\t' << e.returns;
                for (size_t i = 0; i < e.types.size(); ++i)
                    std::cout << '\t' << e.types[i] << ':' << e.names[i];
                std::cout << '\n';
            }
            return 0;
        }
    } catch (const std::exception &error) {
        std::cerr << "loadtest: " << error.what() << '\n';
        return 1;
    }
    usage(argv[0]);
    return 2;
}
