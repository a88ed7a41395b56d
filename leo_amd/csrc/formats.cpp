// Host-side persistent artifacts: PSCLS100 checkpoints, LEODATA1 prepared
// datasets and their SHA-256 identities (include/leo_formats.h). Byte layouts
// follow crates/leo-format/src/lib.rs and crates/leo-data/src/lib.rs; all
// integers are little-endian, as the reference writes them.

#include <dirent.h>
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "leo_formats.h"
#include "leo_host.h"

namespace leo {
namespace {

// ---------------------------------------------------------------------------
// SHA-256 (FIPS 180-4, section 6.2).
class Sha256 {
public:
    Sha256() { reset(); }
    void reset() {
        static const uint32_t init[8] = {0x6a09e667u, 0xbb67ae85u, 0x3c6ef372u, 0xa54ff53au,
                                         0x510e527fu, 0x9b05688cu, 0x1f83d9abu, 0x5be0cd19u};
        std::memcpy(h_, init, sizeof(h_));
        total_ = 0;
        fill_ = 0;
    }
    void update(const uint8_t* data, uint64_t length) {
        total_ += length;
        if (fill_) {
            const uint64_t take = std::min<uint64_t>(length, 64 - fill_);
            std::memcpy(block_ + fill_, data, take);
            fill_ += static_cast<uint32_t>(take);
            data += take;
            length -= take;
            if (fill_ < 64) return;
            compress(block_);
            fill_ = 0;
        }
        while (length >= 64) {
            compress(data);
            data += 64;
            length -= 64;
        }
        std::memcpy(block_, data, length);
        fill_ = static_cast<uint32_t>(length);
    }
    LeoDigest finish() {
        const uint64_t bits = total_ * 8;
        const uint8_t one = 0x80, zero = 0;
        update(&one, 1);
        while (fill_ != 56) update(&zero, 1);
        uint8_t length_be[8];
        for (int i = 0; i < 8; ++i) length_be[i] = static_cast<uint8_t>(bits >> (56 - 8 * i));
        update(length_be, 8);
        LeoDigest out;
        for (int i = 0; i < 8; ++i)
            for (int b = 0; b < 4; ++b) out.bytes[4 * i + b] = static_cast<uint8_t>(h_[i] >> (24 - 8 * b));
        return out;
    }

private:
    static uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }
    void compress(const uint8_t* p) {
        // round constants: the first 32 bits of the fractional parts of the
        // cube roots of the first 64 primes
        static const uint32_t k[64] = {
            0x428a2f98u, 0x71374491u, 0xb5c0fbcfu, 0xe9b5dba5u, 0x3956c25bu, 0x59f111f1u, 0x923f82a4u, 0xab1c5ed5u,
            0xd807aa98u, 0x12835b01u, 0x243185beu, 0x550c7dc3u, 0x72be5d74u, 0x80deb1feu, 0x9bdc06a7u, 0xc19bf174u,
            0xe49b69c1u, 0xefbe4786u, 0x0fc19dc6u, 0x240ca1ccu, 0x2de92c6fu, 0x4a7484aau, 0x5cb0a9dcu, 0x76f988dau,
            0x983e5152u, 0xa831c66du, 0xb00327c8u, 0xbf597fc7u, 0xc6e00bf3u, 0xd5a79147u, 0x06ca6351u, 0x14292967u,
            0x27b70a85u, 0x2e1b2138u, 0x4d2c6dfcu, 0x53380d13u, 0x650a7354u, 0x766a0abbu, 0x81c2c92eu, 0x92722c85u,
            0xa2bfe8a1u, 0xa81a664bu, 0xc24b8b70u, 0xc76c51a3u, 0xd192e819u, 0xd6990624u, 0xf40e3585u, 0x106aa070u,
            0x19a4c116u, 0x1e376c08u, 0x2748774cu, 0x34b0bcb5u, 0x391c0cb3u, 0x4ed8aa4au, 0x5b9cca4fu, 0x682e6ff3u,
            0x748f82eeu, 0x78a5636fu, 0x84c87814u, 0x8cc70208u, 0x90befffau, 0xa4506cebu, 0xbef9a3f7u, 0xc67178f2u};
        uint32_t w[64];
        for (int t = 0; t < 16; ++t)
            w[t] = (uint32_t(p[4 * t]) << 24) | (uint32_t(p[4 * t + 1]) << 16) | (uint32_t(p[4 * t + 2]) << 8) |
                   uint32_t(p[4 * t + 3]);
        for (int t = 16; t < 64; ++t) {
            const uint32_t s0 = rotr(w[t - 15], 7) ^ rotr(w[t - 15], 18) ^ (w[t - 15] >> 3);
            const uint32_t s1 = rotr(w[t - 2], 17) ^ rotr(w[t - 2], 19) ^ (w[t - 2] >> 10);
            w[t] = w[t - 16] + s0 + w[t - 7] + s1;
        }
        uint32_t a = h_[0], b = h_[1], c = h_[2], d = h_[3], e = h_[4], f = h_[5], g = h_[6], h = h_[7];
        for (int t = 0; t < 64; ++t) {
            const uint32_t t1 = h + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) + k[t] + w[t];
            const uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & b) ^ (a & c) ^ (b & c));
            h = g;
            g = f;
            f = e;
            e = d + t1;
            d = c;
            c = b;
            b = a;
            a = t1 + t2;
        }
        h_[0] += a;
        h_[1] += b;
        h_[2] += c;
        h_[3] += d;
        h_[4] += e;
        h_[5] += f;
        h_[6] += g;
        h_[7] += h;
    }
    uint32_t h_[8];
    uint8_t block_[64];
    uint64_t total_;
    uint32_t fill_;
};

LeoDigest digest(const uint8_t* data, uint64_t length) {
    Sha256 s;
    s.update(data, length);
    return s.finish();
}

bool same(const LeoDigest& a, const LeoDigest& b) { return std::memcmp(a.bytes, b.bytes, 32) == 0; }

Error corrupt(const std::string& m) { return Error(LEO_ERR_CORRUPT, m); }
Error incompatible(const std::string& m) { return Error(LEO_ERR_INCOMPATIBLE, m); }
Error io_error(const std::string& what, const std::string& path) {
    return Error(LEO_ERR_IO, what + " " + path + ": " + std::strerror(errno));
}

// ---------------------------------------------------------------------------
// Files.
struct Fd {
    int fd = -1;
    ~Fd() {
        if (fd >= 0) ::close(fd);
    }
};

LeoDigest digest_file(const std::string& path) {
    Fd f;
    f.fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (f.fd < 0) throw io_error("cannot open", path);
    Sha256 s;
    std::vector<uint8_t> buffer(size_t(1) << 20);
    for (;;) {
        const ssize_t n = ::read(f.fd, buffer.data(), buffer.size());
        if (n < 0) {
            if (errno == EINTR) continue;
            throw io_error("cannot read", path);
        }
        if (n == 0) break;
        s.update(buffer.data(), static_cast<uint64_t>(n));
    }
    return s.finish();
}

uint64_t file_length(const std::string& path) {
    struct stat st;
    if (::stat(path.c_str(), &st) != 0) throw io_error("cannot stat", path);
    return static_cast<uint64_t>(st.st_size);
}

bool file_exists(const std::string& path) {
    struct stat st;
    return ::stat(path.c_str(), &st) == 0;
}

std::vector<uint8_t> read_file(const std::string& path) {
    Fd f;
    f.fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (f.fd < 0) throw io_error("cannot open", path);
    std::vector<uint8_t> out;
    std::vector<uint8_t> buffer(size_t(1) << 20);
    for (;;) {
        const ssize_t n = ::read(f.fd, buffer.data(), buffer.size());
        if (n < 0) {
            if (errno == EINTR) continue;
            throw io_error("cannot read", path);
        }
        if (n == 0) break;
        out.insert(out.end(), buffer.begin(), buffer.begin() + n);
    }
    return out;
}

void write_all(int fd, const uint8_t* data, uint64_t length, const std::string& path) {
    while (length) {
        const ssize_t n = ::write(fd, data, static_cast<size_t>(std::min<uint64_t>(length, uint64_t(1) << 30)));
        if (n < 0) {
            if (errno == EINTR) continue;
            throw io_error("cannot write", path);
        }
        data += n;
        length -= static_cast<uint64_t>(n);
    }
}

void read_exact_at(int fd, uint8_t* out, uint64_t length, uint64_t offset, const std::string& path) {
    while (length) {
        const ssize_t n = ::pread(fd, out, static_cast<size_t>(std::min<uint64_t>(length, uint64_t(1) << 30)),
                                  static_cast<off_t>(offset));
        if (n < 0) {
            if (errno == EINTR) continue;
            throw io_error("cannot read", path);
        }
        if (n == 0) throw Error(LEO_ERR_IO, "unexpected end of file reading " + path);
        out += n;
        offset += static_cast<uint64_t>(n);
        length -= static_cast<uint64_t>(n);
    }
}

std::string parent_of(const std::string& path) {
    const size_t slash = path.find_last_of('/');
    if (slash == std::string::npos) return ".";
    return slash == 0 ? "/" : path.substr(0, slash);
}

std::string name_of(const std::string& path) {
    const size_t slash = path.find_last_of('/');
    return slash == std::string::npos ? path : path.substr(slash + 1);
}

void make_dirs(const std::string& dir) {
    if (dir.empty() || dir == "." || dir == "/" || file_exists(dir)) return;
    make_dirs(parent_of(dir));
    if (::mkdir(dir.c_str(), 0777) != 0 && errno != EEXIST) throw io_error("cannot create directory", dir);
}

void copy_file(const std::string& from, const std::string& to) {
    const std::vector<uint8_t> bytes = read_file(from);
    Fd f;
    f.fd = ::open(to.c_str(), O_WRONLY | O_CREAT | O_TRUNC | O_CLOEXEC, 0666);
    if (f.fd < 0) throw io_error("cannot create", to);
    write_all(f.fd, bytes.data(), bytes.size(), to);
}

// Strict UTF-8 (no overlong forms, no surrogates, nothing above U+10FFFF),
// the rule std::str::from_utf8 applies.
bool valid_utf8(const uint8_t* s, uint64_t n) {
    uint64_t i = 0;
    while (i < n) {
        const uint8_t c = s[i];
        if (c < 0x80) {
            ++i;
            continue;
        }
        uint32_t need, cp;
        if (c >= 0xc2 && c <= 0xdf) {
            need = 1;
            cp = c & 0x1f;
        } else if (c >= 0xe0 && c <= 0xef) {
            need = 2;
            cp = c & 0x0f;
        } else if (c >= 0xf0 && c <= 0xf4) {
            need = 3;
            cp = c & 0x07;
        } else {
            return false;
        }
        if (i + need >= n) return false;
        for (uint32_t k = 1; k <= need; ++k) {
            const uint8_t b = s[i + k];
            if ((b & 0xc0) != 0x80) return false;
            cp = (cp << 6) | (b & 0x3f);
        }
        if ((need == 2 && cp < 0x800) || (need == 3 && (cp < 0x10000 || cp > 0x10ffff)) ||
            (cp >= 0xd800 && cp <= 0xdfff))
            return false;
        i += need + 1;
    }
    return true;
}

// ---------------------------------------------------------------------------
// Little-endian byte streams (put_* / Reader, lib.rs:1044-1160).
struct Writer {
    std::vector<uint8_t> out;
    void u32(uint32_t v) {
        for (int i = 0; i < 4; ++i) out.push_back(static_cast<uint8_t>(v >> (8 * i)));
    }
    void u64(uint64_t v) {
        for (int i = 0; i < 8; ++i) out.push_back(static_cast<uint8_t>(v >> (8 * i)));
    }
    void f64(double v) {
        uint64_t bits;
        std::memcpy(&bits, &v, 8);
        u64(bits);
    }
    void raw(const void* p, uint64_t bytes) {
        const uint8_t* b = static_cast<const uint8_t*>(p);
        out.insert(out.end(), b, b + bytes);
    }
    // a length-prefixed vector of little-endian elements (the host is
    // little-endian: gfx950 hosts are x86-64)
    template <class T>
    void vec(const T* values, uint64_t count) {
        u64(count);
        raw(values, count * sizeof(T));
    }
};

struct Reader {
    const uint8_t* p;
    uint64_t n, at = 0;
    Reader(const uint8_t* data, uint64_t length) : p(data), n(length) {}
    const uint8_t* take(uint64_t length) {
        if (length > n - at) throw corrupt("truncated checkpoint tensor");
        const uint8_t* out = p + at;
        at += length;
        return out;
    }
    uint64_t u64() {
        uint64_t v;
        std::memcpy(&v, take(8), 8);
        return v;
    }
    double f64() {
        double v;
        std::memcpy(&v, take(8), 8);
        return v;
    }
    // a length-prefixed vector that must hold exactly `expected` elements
    template <class T>
    void vec(T* out, uint64_t expected, const char* what) {
        const uint64_t count = u64();
        if (count > (n - at) / sizeof(T)) throw corrupt("truncated checkpoint tensor");
        const uint8_t* bytes = take(count * sizeof(T));
        if (count != expected) throw corrupt(std::string("shape mismatch in ") + what);
        std::memcpy(out, bytes, count * sizeof(T));
    }
    uint64_t vec_length() {  // the prefix of a vector read later with vec_body
        return u64();
    }
    void finish() const {
        if (at != n) throw corrupt("unexpected trailing checkpoint data");
    }
};

uint32_t le32(const uint8_t* p) {
    uint32_t v;
    std::memcpy(&v, p, 4);
    return v;
}
uint64_t le64(const uint8_t* p) {
    uint64_t v;
    std::memcpy(&v, p, 8);
    return v;
}
void put32(uint8_t* p, uint32_t v) { std::memcpy(p, &v, 4); }
void put64(uint8_t* p, uint64_t v) { std::memcpy(p, &v, 8); }

// ---------------------------------------------------------------------------
// PSCLS100 (lib.rs:20-28 and the section table lib.rs:30-96).
constexpr uint8_t kMagic[8] = {'P', 'S', 'C', 'L', 'S', '1', '0', '0'};
constexpr uint32_t kFormatVersion = 1;  // CHECKPOINT_SCHEMA_VERSION (semantics.rs)
constexpr uint32_t kEndianMarker = 0x01020304u;
constexpr uint64_t kHeaderSize = 128, kDescriptorSize = 128, kAlignment = 64, kHeaderDigestOffset = 96;
constexpr uint64_t kMaxConfigBytes = 1024 * 1024;
constexpr uint32_t kSections = 12;
// SemanticsContract::CURRENT (semantics.rs:8-34): model schema, training
// policy, execution semantics, dataset schema, CUDA ABI versions
constexpr uint32_t kSemantics[5] = {1, 1, 1, 1, 1};
constexpr uint32_t kOutputClasses = 257, kSymbolCount = 258;

enum Kind : uint32_t {
    kConfig = 1,
    kNeurons,
    kRecTargets,
    kRecMetadata,
    kRecWeights,
    kInput,
    kOutputWeights,
    kOutputBias,
    kContext,
    kStatistics,
    kGeneration,
    kSemantic
};
enum DType : uint32_t { kBytes = 1, kF32 = 2, kU32 = 3, kU64 = 4 };

const char* kind_name(uint32_t k) {
    static const char* names[] = {"?",
                                  "Config",
                                  "NeuronParameters",
                                  "RecurrentTargets",
                                  "RecurrentMetadata",
                                  "RecurrentWeights",
                                  "InputProjection",
                                  "OutputWeights",
                                  "OutputBias",
                                  "ContextProjection",
                                  "TrainingStatistics",
                                  "GenerationMetadata",
                                  "SemanticsContract"};
    return k >= 1 && k <= kSections ? names[k] : names[0];
}

uint32_t expected_dtype(uint32_t k) {
    switch (k) {
        case kRecWeights:
        case kOutputWeights:
        case kOutputBias: return kF32;
        case kGeneration: return kU64;
        case kSemantic: return kU32;
        default: return kBytes;
    }
}

// rank_for_shape (lib.rs:866-880): leading nonzero dimensions; a nonzero
// dimension after a zero gives the invalid rank 5
uint32_t rank_for_shape(const uint64_t s[4]) {
    uint32_t rank = 0;
    bool zero = false;
    for (int i = 0; i < 4; ++i) {
        if (s[i] == 0) zero = true;
        else if (zero) return 5;
        else ++rank;
    }
    return rank;
}

uint64_t align_up(uint64_t v, uint64_t a) { return (v + a - 1) / a * a; }

struct Shapes {
    uint64_t n, s, f, slots, e;
};

Shapes shapes_of(const LeoHostConfig& c) {
    Shapes z;
    z.n = c.device.neuron_count;
    z.s = c.device.synapses_per_neuron;
    z.f = c.device.input_fanout;
    z.slots = static_cast<uint64_t>(c.device.context_max_order) * c.device.context_slots_per_order;
    z.e = c.device.context_embedding_dim;
    return z;
}

// The expected shape of each section (validate_shapes, lib.rs:718-800).
void expected_shape(uint32_t kind, const Shapes& z, uint64_t out[4]) {
    std::fill(out, out + 4, 0);
    switch (kind) {
        case kConfig: break;
        case kNeurons: out[0] = z.n; break;
        case kRecTargets:
        case kRecMetadata:
            out[0] = z.n;
            out[1] = z.s;
            break;
        case kRecWeights: out[0] = z.n * z.s; break;
        case kInput:
            out[0] = kSymbolCount;
            out[1] = z.f;
            break;
        case kOutputWeights:
            out[0] = kOutputClasses;
            out[1] = z.n;
            break;
        case kOutputBias: out[0] = kOutputClasses; break;
        case kContext:
            out[0] = z.slots;
            out[1] = z.e;
            out[2] = kOutputClasses;
            break;
        case kStatistics: out[0] = 9; break;
        case kGeneration: out[0] = 2; break;
        case kSemantic: out[0] = 5; break;
    }
}

// The payload of every section in kind order (encode_model, lib.rs:289-392).
std::vector<std::vector<uint8_t>> section_payloads(const LeoHostConfig& c, const LeoModelView& m, const char* toml,
                                                   uint64_t toml_length) {
    const Shapes z = shapes_of(c);
    std::vector<std::vector<uint8_t>> out(kSections);
    out[kConfig - 1].assign(toml, toml + toml_length);
    Writer w;
    w.vec(m.threshold, z.n);
    w.vec(m.excitability, z.n);
    w.vec(m.neuron_type, z.n);
    out[kNeurons - 1] = std::move(w.out);
    w = Writer{};
    w.u64(z.s);
    w.vec(m.rec_target, z.n * z.s);
    out[kRecTargets - 1] = std::move(w.out);
    w = Writer{};
    w.vec(m.rec_branch, z.n * z.s);
    w.vec(m.rec_delay, z.n * z.s);
    out[kRecMetadata - 1] = std::move(w.out);
    w = Writer{};
    w.vec(m.rec_weight, z.n * z.s);
    out[kRecWeights - 1] = std::move(w.out);
    w = Writer{};
    w.u64(z.f);
    w.vec(m.in_target, kSymbolCount * z.f);
    w.vec(m.in_branch, kSymbolCount * z.f);
    w.vec(m.in_weight, kSymbolCount * z.f);
    out[kInput - 1] = std::move(w.out);
    w = Writer{};
    w.vec(m.out_weight, kOutputClasses * z.n);
    out[kOutputWeights - 1] = std::move(w.out);
    w = Writer{};
    w.vec(m.bias, kOutputClasses);
    out[kOutputBias - 1] = std::move(w.out);
    w = Writer{};
    w.vec(m.ctx_keys, z.slots);
    w.vec(m.ctx_emb, z.slots * z.e);
    w.vec(m.ctx_obs, z.slots);
    w.vec(m.ctx_out, kOutputClasses * z.e);
    out[kContext - 1] = std::move(w.out);
    w = Writer{};
    const LeoStatistics& st = m.statistics;
    w.u64(st.processed_bytes);
    w.u64(st.processed_stories);
    w.f64(st.training_loss_sum);
    w.u64(st.training_targets);
    w.u64(st.active_neurons_sum);
    w.u64(st.active_neurons_peak);
    w.u64(st.synaptic_events);
    w.u64(st.numerical_rejections);
    w.u64(st.persistent_ticks);
    out[kStatistics - 1] = std::move(w.out);
    w = Writer{};
    w.u64(m.generation);
    w.u64(m.parameter_revision);
    out[kGeneration - 1] = std::move(w.out);
    w = Writer{};
    for (uint32_t v : kSemantics) w.u32(v);
    out[kSemantic - 1] = std::move(w.out);
    return out;
}

// Payload byte counts without building them (for leo_checkpoint_encoded_size).
uint64_t encoded_size(const LeoHostConfig& c, uint64_t toml_length) {
    const Shapes z = shapes_of(c);
    const uint64_t lengths[kSections] = {
        toml_length,
        8 + 4 * z.n + 8 + 4 * z.n + 8 + z.n,
        8 + 8 + 4 * z.n * z.s,
        8 + z.n * z.s + 8 + z.n * z.s,
        8 + 4 * z.n * z.s,
        8 + 8 + 4 * kSymbolCount * z.f + 8 + kSymbolCount * z.f + 8 + 4 * kSymbolCount * z.f,
        8 + 4 * kOutputClasses * z.n,
        8 + 4 * kOutputClasses,
        8 + 8 * z.slots + 8 + 4 * z.slots * z.e + 8 + 4 * z.slots + 8 + 4 * kOutputClasses * z.e,
        72,
        16,
        20};
    uint64_t cursor = align_up(kHeaderSize + kDescriptorSize * kSections, kAlignment);
    for (uint64_t l : lengths) cursor = align_up(cursor + l, kAlignment);
    return cursor;
}

void encode(const LeoHostConfig& c, const LeoModelView& m, const char* toml, uint64_t toml_length, uint8_t* out,
            uint64_t capacity) {
    const uint64_t total = encoded_size(c, toml_length);
    if (capacity < total) throw Error(LEO_ERR_INVALID_ARGUMENT, "checkpoint output buffer is too small");
    const Shapes z = shapes_of(c);
    const auto payloads = section_payloads(c, m, toml, toml_length);
    std::memset(out, 0, total);
    uint64_t cursor = align_up(kHeaderSize + kDescriptorSize * kSections, kAlignment);
    uint64_t config_offset = 0, config_length = 0;
    for (uint32_t i = 0; i < kSections; ++i) {
        const uint32_t kind = i + 1;
        const std::vector<uint8_t>& p = payloads[i];
        uint8_t* d = out + kHeaderSize + i * kDescriptorSize;  // encode_descriptor (lib.rs:810-827)
        uint64_t shape[4];
        expected_shape(kind, z, shape);
        put32(d + 0, kind);
        put32(d + 4, 1);  // section schema version
        put32(d + 8, expected_dtype(kind));
        put32(d + 12, rank_for_shape(shape));
        for (int k = 0; k < 4; ++k) put64(d + 16 + 8 * k, shape[k]);
        put64(d + 48, cursor);
        put64(d + 56, p.size());
        put32(d + 64, static_cast<uint32_t>(kAlignment));
        put32(d + 68, 0);  // no compression
        const LeoDigest dg = digest(p.data(), p.size());
        std::memcpy(d + 72, dg.bytes, 32);
        if (!p.empty()) std::memcpy(out + cursor, p.data(), p.size());
        if (kind == kConfig) {
            config_offset = cursor;
            config_length = p.size();
        }
        cursor = align_up(cursor + p.size(), kAlignment);
    }
    std::memcpy(out, kMagic, 8);
    put32(out + 8, kFormatVersion);
    put32(out + 12, kEndianMarker);
    put64(out + 16, m.generation);
    put32(out + 24, kSections);
    put32(out + 28, 0);  // header flags
    put64(out + 32, config_offset);
    put64(out + 40, config_length);
    const LeoDigest hd = digest(out, kHeaderSize);  // with the digest field still zero
    std::memcpy(out + kHeaderDigestOffset, hd.bytes, 32);
}

// validate_header (lib.rs:622-659)
void validate_header(const uint8_t* h) {
    if (std::memcmp(h, kMagic, 8) != 0)
        throw incompatible("unsupported checkpoint magic; the current Leo v1 runtime accepts only PSCLS100 artifacts");
    const uint32_t version = le32(h + 8);
    if (version != kFormatVersion)
        throw incompatible("unsupported checkpoint format version " + std::to_string(version) + "; expected 1");
    if (le32(h + 12) != kEndianMarker) throw incompatible("unsupported checkpoint endianness");
    for (uint64_t i = 48; i < kHeaderDigestOffset; ++i)
        if (h[i] != 0) throw corrupt("checkpoint header reserved bytes are nonzero");
    uint8_t normalized[kHeaderSize];
    std::memcpy(normalized, h, kHeaderSize);
    std::memset(normalized + kHeaderDigestOffset, 0, kHeaderSize - kHeaderDigestOffset);
    LeoDigest declared;
    std::memcpy(declared.bytes, h + kHeaderDigestOffset, 32);
    if (!same(digest(normalized, kHeaderSize), declared)) throw corrupt("checkpoint header SHA-256 mismatch");
}

struct Descriptor {
    uint32_t kind, schema, dtype, rank;
    uint64_t shape[4];
    uint64_t offset, length;
    uint32_t alignment, compression;
    LeoDigest digest;
};

struct Parsed {
    uint64_t generation;
    Descriptor by_kind[kSections];
};

// decode_model's structural checks (lib.rs:446-543, 661-716, 829-864)
Parsed parse(const uint8_t* bytes, uint64_t length) {
    if (length < kHeaderSize) throw corrupt("checkpoint is smaller than the v1 header");
    validate_header(bytes);
    Parsed out{};
    out.generation = le64(bytes + 16);
    const uint32_t count = le32(bytes + 24);
    if (count != kSections)
        throw corrupt("invalid checkpoint section count " + std::to_string(count) + "; expected 12");
    if (le32(bytes + 28) != 0) throw corrupt("unsupported checkpoint header flags");
    const uint64_t table_end = kHeaderSize + uint64_t(count) * kDescriptorSize;
    if (table_end > length) throw corrupt("truncated checkpoint descriptor table");
    const uint64_t region = align_up(table_end, kAlignment);
    std::vector<Descriptor> ds(count);
    for (uint32_t i = 0; i < count; ++i) {
        const uint8_t* d = bytes + kHeaderSize + i * kDescriptorSize;
        for (uint64_t k = 104; k < kDescriptorSize; ++k)
            if (d[k] != 0) throw corrupt("checkpoint descriptor reserved bytes are nonzero");
        Descriptor& x = ds[i];
        x.kind = le32(d);
        if (x.kind < 1 || x.kind > kSections) throw corrupt("unknown checkpoint section type: " + std::to_string(x.kind));
        x.schema = le32(d + 4);
        x.dtype = le32(d + 8);
        if (x.dtype < kBytes || x.dtype > kU64) throw corrupt("unknown checkpoint dtype: " + std::to_string(x.dtype));
        x.rank = le32(d + 12);
        for (int k = 0; k < 4; ++k) x.shape[k] = le64(d + 16 + 8 * k);
        x.offset = le64(d + 48);
        x.length = le64(d + 56);
        x.alignment = le32(d + 64);
        x.compression = le32(d + 68);
        std::memcpy(x.digest.bytes, d + 72, 32);
    }
    // validate_descriptor (lib.rs:661-716)
    std::vector<std::pair<uint64_t, uint64_t>> ranges;
    for (const Descriptor& x : ds) {
        const std::string name = kind_name(x.kind);
        if (x.schema != 1)
            throw incompatible("unsupported schema version " + std::to_string(x.schema) + " in " + name);
        if (x.dtype != expected_dtype(x.kind)) throw corrupt("invalid dtype in " + name + " section");
        if (x.rank != rank_for_shape(x.shape) || x.rank > 4) throw corrupt("invalid rank/shape in " + name + " section");
        if (x.alignment != kAlignment) throw corrupt("invalid alignment in " + name + " section");
        if (x.compression != 0) throw incompatible("compressed checkpoint sections are not supported in v1");
        if (x.length > length || x.offset > length - x.length || x.offset < region || x.offset % kAlignment != 0)
            throw corrupt("invalid byte range for " + name + " section");
        ranges.push_back({x.offset, x.offset + x.length});
    }
    std::sort(ranges.begin(), ranges.end());
    uint64_t previous = region;
    for (auto& r : ranges) {
        if (r.first < previous) throw corrupt("overlapping checkpoint section");
        previous = r.second;
    }
    bool seen[kSections] = {};
    for (const Descriptor& x : ds) {
        if (!same(digest(bytes + x.offset, x.length), x.digest))
            throw corrupt(std::string("SHA-256 mismatch in ") + kind_name(x.kind) + " section");
        if (seen[x.kind - 1]) throw corrupt(std::string("duplicate ") + kind_name(x.kind) + " checkpoint section");
        seen[x.kind - 1] = true;
        out.by_kind[x.kind - 1] = x;
    }
    for (uint32_t k = 0; k < kSections; ++k)
        if (!seen[k]) throw corrupt(std::string("missing ") + kind_name(k + 1) + " checkpoint section");
    const Descriptor& cfg = out.by_kind[kConfig - 1];
    if (cfg.length > kMaxConfigBytes) throw corrupt("CONFIG section exceeds 1 MiB");
    if (cfg.offset != le64(bytes + 32) || cfg.length != le64(bytes + 40))
        throw corrupt("CONFIG header pointer does not match descriptor");
    const Descriptor& sem = out.by_kind[kSemantic - 1];
    if (sem.length != 20) throw corrupt("invalid semantics contract length");
    for (int i = 0; i < 5; ++i)
        if (le32(bytes + sem.offset + 4 * i) != kSemantics[i])
            throw incompatible("checkpoint semantics do not match the current Leo v1 semantics");
    return out;
}

void inspect(const uint8_t* bytes, uint64_t length, LeoCheckpointInfo& info) {
    const Parsed p = parse(bytes, length);
    info = LeoCheckpointInfo{};
    info.generation = p.generation;
    const Descriptor& gen = p.by_kind[kGeneration - 1];
    if (gen.length == 16) info.parameter_revision = le64(bytes + gen.offset + 8);
    info.config_offset = p.by_kind[kConfig - 1].offset;
    info.config_length = p.by_kind[kConfig - 1].length;
    info.neuron_count = p.by_kind[kNeurons - 1].shape[0];
    info.synapses_per_neuron = p.by_kind[kRecTargets - 1].shape[1];
    info.input_fanout = p.by_kind[kInput - 1].shape[1];
    info.context_slots = p.by_kind[kContext - 1].shape[0];
    info.context_embedding_dim = p.by_kind[kContext - 1].shape[1];
}

void decode(const uint8_t* bytes, uint64_t length, const LeoHostConfig& c, LeoModelView& m) {
    const Parsed p = parse(bytes, length);
    const Shapes z = shapes_of(c);
    auto section = [&](uint32_t kind) {
        const Descriptor& d = p.by_kind[kind - 1];
        return Reader(bytes + d.offset, d.length);
    };
    // payloads (decode_neurons .. decode_generation, lib.rs:884-1043)
    {
        Reader r = section(kNeurons);
        r.vec(m.threshold, z.n, "NeuronParameters");
        r.vec(m.excitability, z.n, "NeuronParameters");
        r.vec(m.neuron_type, z.n, "NeuronParameters");
        r.finish();
    }
    {
        Reader r = section(kRecTargets);
        if (r.u64() != z.s) throw corrupt("shape mismatch in RecurrentTargets");
        r.vec(m.rec_target, z.n * z.s, "RecurrentTargets");
        r.finish();
    }
    {
        Reader r = section(kRecMetadata);
        r.vec(m.rec_branch, z.n * z.s, "RecurrentMetadata");
        r.vec(m.rec_delay, z.n * z.s, "RecurrentMetadata");
        r.finish();
    }
    {
        Reader r = section(kRecWeights);
        r.vec(m.rec_weight, z.n * z.s, "RecurrentWeights");
        r.finish();
    }
    {
        Reader r = section(kInput);
        if (r.u64() != z.f) throw corrupt("shape mismatch in InputProjection");
        r.vec(m.in_target, kSymbolCount * z.f, "InputProjection");
        r.vec(m.in_branch, kSymbolCount * z.f, "InputProjection");
        r.vec(m.in_weight, kSymbolCount * z.f, "InputProjection");
        r.finish();
    }
    {
        Reader r = section(kOutputWeights);
        r.vec(m.out_weight, kOutputClasses * z.n, "OutputWeights");
        r.finish();
    }
    {
        Reader r = section(kOutputBias);
        r.vec(m.bias, kOutputClasses, "OutputBias");
        r.finish();
    }
    {
        Reader r = section(kContext);
        r.vec(m.ctx_keys, z.slots, "ContextProjection");
        r.vec(m.ctx_emb, z.slots * z.e, "ContextProjection");
        r.vec(m.ctx_obs, z.slots, "ContextProjection");
        r.vec(m.ctx_out, kOutputClasses * z.e, "ContextProjection");
        r.finish();
    }
    {
        Reader r = section(kStatistics);
        if (p.by_kind[kStatistics - 1].length != 72)
            throw corrupt("invalid training statistics length: " + std::to_string(p.by_kind[kStatistics - 1].length));
        LeoStatistics& st = m.statistics;
        st.processed_bytes = r.u64();
        st.processed_stories = r.u64();
        st.training_loss_sum = r.f64();
        st.training_targets = r.u64();
        st.active_neurons_sum = r.u64();
        st.active_neurons_peak = r.u64();
        st.synaptic_events = r.u64();
        st.numerical_rejections = r.u64();
        st.persistent_ticks = r.u64();
        r.finish();
    }
    {
        Reader r = section(kGeneration);
        if (p.by_kind[kGeneration - 1].length != 16) throw corrupt("invalid generation metadata length");
        const uint64_t generation = r.u64();
        m.parameter_revision = r.u64();
        r.finish();
        if (generation != p.generation) throw corrupt("generation metadata does not match checkpoint header");
        m.generation = generation;
    }
    model_validate(c, m);
    for (uint32_t kind = 1; kind <= kSections; ++kind) {  // validate_shapes (lib.rs:718-800)
        uint64_t shape[4];
        expected_shape(kind, z, shape);
        if (std::memcmp(shape, p.by_kind[kind - 1].shape, sizeof(shape)) != 0)
            throw corrupt(std::string("shape mismatch in ") + kind_name(kind) + " section");
    }
}

std::string generation_path(const std::string& path, uint64_t generation) {
    char suffix[32];
    std::snprintf(suffix, sizeof(suffix), ".gen%06llu", static_cast<unsigned long long>(generation));
    return path + suffix;
}

uint64_t read_generation(const std::string& path) {
    Fd f;
    f.fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (f.fd < 0) throw io_error("cannot open", path);
    uint8_t header[kHeaderSize];
    read_exact_at(f.fd, header, kHeaderSize, 0, path);
    validate_header(header);
    return le64(header + 16);
}

// save_model_atomic (lib.rs:144-175)
void save_atomic(const std::string& path, const LeoHostConfig& c, const LeoModelView& m, const char* toml,
                 uint64_t toml_length, bool retain_previous) {
    model_validate(c, m);
    make_dirs(parent_of(path));
    if (retain_previous && file_exists(path)) {
        const std::string previous = generation_path(path, read_generation(path));
        if (!file_exists(previous)) copy_file(path, previous);
    }
    std::vector<uint8_t> bytes(encoded_size(c, toml_length));
    encode(c, m, toml, toml_length, bytes.data(), bytes.size());
    const std::string temporary = path + ".tmp";
    {
        Fd f;
        f.fd = ::open(temporary.c_str(), O_WRONLY | O_CREAT | O_TRUNC | O_CLOEXEC, 0666);
        if (f.fd < 0) throw io_error("cannot create", temporary);
        write_all(f.fd, bytes.data(), bytes.size(), temporary);
        if (::fsync(f.fd) != 0) throw io_error("cannot sync", temporary);
    }
    if (::rename(temporary.c_str(), path.c_str()) != 0) throw io_error("cannot rename onto", path);
    Fd dir;
    dir.fd = ::open(parent_of(path).c_str(), O_RDONLY | O_DIRECTORY | O_CLOEXEC);
    if (dir.fd >= 0) (void)::fsync(dir.fd);  // best effort, as the reference
}

// prune_generations (lib.rs:201-239)
void prune(const std::string& path, uint64_t keep) {
    const std::string dir = parent_of(path), prefix = name_of(path) + ".gen";
    std::vector<std::pair<uint64_t, std::string>> generations;
    std::vector<std::string> names;
    {
        DIR* d = ::opendir(dir.c_str());
        if (!d) throw io_error("cannot list", dir);
        while (const dirent* e = ::readdir(d)) names.emplace_back(e->d_name);
        ::closedir(d);
    }
    for (const std::string& name : names) {
        if (name.compare(0, prefix.size(), prefix) != 0) continue;
        const std::string suffix = name.substr(prefix.size());
        if (suffix.empty() || !std::all_of(suffix.begin(), suffix.end(), [](char ch) { return ch >= '0' && ch <= '9'; }))
            continue;
        if (suffix.size() > 20) continue;  // does not parse as u64
        errno = 0;
        char* end = nullptr;
        const unsigned long long g = std::strtoull(suffix.c_str(), &end, 10);
        if (errno == ERANGE) continue;
        const std::string full = dir + "/" + name;
        struct stat st;
        if (::lstat(full.c_str(), &st) != 0 || !S_ISREG(st.st_mode)) continue;
        generations.push_back({static_cast<uint64_t>(g), full});
    }
    std::sort(generations.begin(), generations.end());
    const size_t remove = generations.size() > keep ? generations.size() - static_cast<size_t>(keep) : 0;
    for (size_t i = 0; i < remove; ++i)
        if (::unlink(generations[i].second.c_str()) != 0) throw io_error("cannot remove", generations[i].second);
}

}  // namespace
}  // namespace leo

// ---------------------------------------------------------------------------
// LEODATA1 (crates/leo-data/src/lib.rs:18-20: magic, 192-byte header,
// 16-byte records).
namespace leo {
namespace {

constexpr uint8_t kIndexMagic[8] = {'L', 'E', 'O', 'D', 'A', 'T', 'A', '1'};
constexpr uint32_t kDatasetSchema = 1;  // DATASET_SCHEMA_VERSION (semantics.rs)
constexpr uint64_t kIndexHeader = 192, kIndexRecord = 16;

// compute_dataset_id (lib.rs:237-253): SHA-256 over a domain tag and the
// identity fields in order
LeoDigest dataset_id(uint32_t schema, uint64_t records, uint64_t length, const LeoDigest& bytes_digest,
                     const LeoDigest& records_digest, const LeoDigest& provenance) {
    static const char tag[] = "LEO-DATASET-ID";  // written with its terminating NUL
    Sha256 s;
    s.update(reinterpret_cast<const uint8_t*>(tag), sizeof(tag));
    uint8_t le[8];
    put32(le, schema);
    s.update(le, 4);
    put64(le, records);
    s.update(le, 8);
    put64(le, length);
    s.update(le, 8);
    s.update(bytes_digest.bytes, 32);
    s.update(records_digest.bytes, 32);
    s.update(provenance.bytes, 32);
    return s.finish();
}

// record ranges: nonzero, inside the bytes file, in order without overlap
// (lib.rs:149-178, 267-289)
void check_records(const LeoStoryIndex* e, uint64_t count, uint64_t bytes_length) {
    uint64_t previous_end = 0;
    for (uint64_t i = 0; i < count; ++i) {
        if (e[i].length == 0) throw corrupt("dataset story " + std::to_string(i) + " has zero length");
        const uint64_t end = e[i].offset + e[i].length;
        if (end < e[i].offset) throw corrupt("dataset story range overflow");
        if (end > bytes_length) throw corrupt("dataset story " + std::to_string(i) + " extends past the bytes file");
        if (e[i].offset < previous_end)
            throw corrupt("dataset story " + std::to_string(i) + " overlaps a previous story");
        previous_end = end;
    }
}

}  // namespace
}  // namespace leo

struct LeoDataset {
    std::string bytes_path;
    int fd = -1;
    std::vector<LeoStoryIndex> entries;
    LeoDatasetIdentity identity{};
    ~LeoDataset() {
        if (fd >= 0) ::close(fd);
    }
};

namespace leo {
namespace {

// PreparedDataset::open (lib.rs:46-185)
LeoDataset* open_dataset(const std::string& bytes_path, const std::string& index_path) {
    auto ds = std::make_unique<LeoDataset>();
    ds->bytes_path = bytes_path;
    ds->fd = ::open(bytes_path.c_str(), O_RDONLY | O_CLOEXEC);
    if (ds->fd < 0) throw io_error("cannot open", bytes_path);
    struct stat st;
    if (::fstat(ds->fd, &st) != 0) throw io_error("cannot stat", bytes_path);
    const uint64_t bytes_length = static_cast<uint64_t>(st.st_size);
    const LeoDigest bytes_digest = digest_file(bytes_path);
    const std::vector<uint8_t> raw = read_file(index_path);
    if (raw.size() < kIndexHeader) throw corrupt("dataset index is smaller than the v1 header");
    if (std::memcmp(raw.data(), kIndexMagic, 8) != 0)
        throw corrupt("invalid dataset index magic; regenerate data for the current Leo v1 runtime");
    const uint32_t schema = le32(raw.data() + 8);
    if (schema != kDatasetSchema)
        throw corrupt("unsupported dataset schema version " + std::to_string(schema) + "; expected 1");
    const uint32_t header_size = le32(raw.data() + 12);
    if (header_size != kIndexHeader) throw corrupt("invalid dataset index header size " + std::to_string(header_size));
    const uint64_t records = le64(raw.data() + 16), declared_length = le64(raw.data() + 24);
    LeoDigest declared_bytes, declared_records, provenance, declared_id, declared_header;
    std::memcpy(declared_bytes.bytes, raw.data() + 32, 32);
    std::memcpy(declared_records.bytes, raw.data() + 64, 32);
    std::memcpy(provenance.bytes, raw.data() + 96, 32);
    std::memcpy(declared_id.bytes, raw.data() + 128, 32);
    std::memcpy(declared_header.bytes, raw.data() + 160, 32);
    uint8_t header[kIndexHeader];
    std::memcpy(header, raw.data(), kIndexHeader);
    std::memset(header + 160, 0, 32);
    if (!same(digest(header, kIndexHeader), declared_header)) throw corrupt("dataset index header SHA-256 mismatch");
    if (declared_length != bytes_length)
        throw corrupt("dataset byte length mismatch: index declares " + std::to_string(declared_length) +
                      ", file has " + std::to_string(bytes_length));
    if (!same(declared_bytes, bytes_digest)) throw corrupt("dataset bytes SHA-256 mismatch");
    if (records > (UINT64_MAX - kIndexHeader) / kIndexRecord) throw corrupt("dataset record table overflow");
    const uint64_t expected = kIndexHeader + records * kIndexRecord;
    if (raw.size() != expected)
        throw corrupt("dataset index length mismatch: expected " + std::to_string(expected) + ", got " +
                      std::to_string(raw.size()));
    const uint8_t* table = raw.data() + kIndexHeader;
    if (!same(digest(table, records * kIndexRecord), declared_records))
        throw corrupt("dataset record-table SHA-256 mismatch");
    if (!same(dataset_id(schema, records, bytes_length, bytes_digest, declared_records, provenance), declared_id))
        throw corrupt("dataset ID does not match content and provenance");
    ds->entries.resize(records);
    for (uint64_t i = 0; i < records; ++i) {
        ds->entries[i].offset = le64(table + i * kIndexRecord);
        ds->entries[i].length = le32(table + i * kIndexRecord + 8);
        ds->entries[i].split_flags = le32(table + i * kIndexRecord + 12);
    }
    check_records(ds->entries.data(), records, bytes_length);
    LeoDatasetIdentity& id = ds->identity;
    id.schema_version = schema;
    id.record_count = records;
    id.bytes_length = bytes_length;
    id.bytes_digest = bytes_digest;
    id.records_digest = declared_records;
    id.provenance_digest = provenance;
    id.dataset_id = declared_id;
    return ds.release();
}

// write_index (lib.rs:255-323)
LeoDatasetIdentity write_index(const std::string& index_path, const std::string& bytes_path,
                               const LeoStoryIndex* entries, uint64_t count, const LeoDigest& provenance) {
    const uint64_t bytes_length = file_length(bytes_path);
    const LeoDigest bytes_digest = digest_file(bytes_path);
    check_records(entries, count, bytes_length);
    std::vector<uint8_t> records(count * kIndexRecord);
    for (uint64_t i = 0; i < count; ++i) {
        put64(records.data() + i * kIndexRecord, entries[i].offset);
        put32(records.data() + i * kIndexRecord + 8, entries[i].length);
        put32(records.data() + i * kIndexRecord + 12, entries[i].split_flags);
    }
    LeoDatasetIdentity id{};
    id.schema_version = kDatasetSchema;
    id.record_count = count;
    id.bytes_length = bytes_length;
    id.bytes_digest = bytes_digest;
    id.records_digest = digest(records.data(), records.size());
    id.provenance_digest = provenance;
    id.dataset_id = dataset_id(kDatasetSchema, count, bytes_length, bytes_digest, id.records_digest, provenance);
    uint8_t header[kIndexHeader] = {};
    std::memcpy(header, kIndexMagic, 8);
    put32(header + 8, kDatasetSchema);
    put32(header + 12, static_cast<uint32_t>(kIndexHeader));
    put64(header + 16, count);
    put64(header + 24, bytes_length);
    std::memcpy(header + 32, id.bytes_digest.bytes, 32);
    std::memcpy(header + 64, id.records_digest.bytes, 32);
    std::memcpy(header + 96, provenance.bytes, 32);
    std::memcpy(header + 128, id.dataset_id.bytes, 32);
    const LeoDigest hd = digest(header, kIndexHeader);
    std::memcpy(header + 160, hd.bytes, 32);
    Fd f;
    f.fd = ::open(index_path.c_str(), O_WRONLY | O_CREAT | O_TRUNC | O_CLOEXEC, 0666);
    if (f.fd < 0) throw io_error("cannot create", index_path);
    write_all(f.fd, header, kIndexHeader, index_path);
    write_all(f.fd, records.data(), records.size(), index_path);
    if (::fsync(f.fd) != 0) throw io_error("cannot sync", index_path);
    return id;
}

void read_story(LeoDataset* ds, uint64_t index, uint8_t* out) {
    const LeoStoryIndex& e = ds->entries[index];
    read_exact_at(ds->fd, out, e.length, e.offset, ds->bytes_path);
    if (!valid_utf8(out, e.length)) throw corrupt("story is not valid UTF-8");
}

const char* need_path(const char* p) {
    if (!p || !*p) throw Error(LEO_ERR_INVALID_ARGUMENT, "empty path");
    return p;
}

}  // namespace
}  // namespace leo

using leo::Error;
using leo::guarded;

extern "C" {

int32_t leo_sha256(const uint8_t* data, uint64_t length, LeoDigest* out) {
    return guarded([&] {
        if ((!data && length) || !out) throw Error(LEO_ERR_INVALID_ARGUMENT, "null argument");
        *out = leo::digest(data, length);
    });
}

int32_t leo_sha256_file(const char* path, LeoDigest* out) {
    return guarded([&] {
        if (!out) throw Error(LEO_ERR_INVALID_ARGUMENT, "null argument");
        *out = leo::digest_file(leo::need_path(path));
    });
}

int32_t leo_checkpoint_encoded_size(const LeoHostConfig* config, uint64_t config_length, uint64_t* bytes_out) {
    return guarded([&] {
        if (!config || !bytes_out) throw Error(LEO_ERR_INVALID_ARGUMENT, "null argument");
        leo::validate_config(*config);
        *bytes_out = leo::encoded_size(*config, config_length);
    });
}

int32_t leo_checkpoint_encode(const LeoHostConfig* config, const LeoModelView* model, const char* config_toml,
                              uint64_t config_length, uint8_t* out, uint64_t capacity) {
    return guarded([&] {
        if (!config || !model || !out || (!config_toml && config_length))
            throw Error(LEO_ERR_INVALID_ARGUMENT, "null argument");
        if (config_length > leo::kMaxConfigBytes) throw Error(LEO_ERR_INVALID_ARGUMENT, "CONFIG section exceeds 1 MiB");
        leo::model_validate(*config, *model);
        leo::encode(*config, *model, config_toml, config_length, out, capacity);
    });
}

int32_t leo_checkpoint_inspect(const uint8_t* bytes, uint64_t length, LeoCheckpointInfo* info) {
    return guarded([&] {
        if (!bytes || !info) throw Error(LEO_ERR_INVALID_ARGUMENT, "null argument");
        leo::inspect(bytes, length, *info);
    });
}

int32_t leo_checkpoint_decode(const uint8_t* bytes, uint64_t length, const LeoHostConfig* config,
                              LeoModelView* model) {
    return guarded([&] {
        if (!bytes || !config || !model) throw Error(LEO_ERR_INVALID_ARGUMENT, "null argument");
        leo::validate_config(*config);
        leo::decode(bytes, length, *config, *model);
    });
}

int32_t leo_checkpoint_save_atomic(const char* path, const LeoHostConfig* config, const LeoModelView* model,
                                   const char* config_toml, uint64_t config_length, uint32_t retain_previous) {
    return guarded([&] {
        if (!config || !model || (!config_toml && config_length))
            throw Error(LEO_ERR_INVALID_ARGUMENT, "null argument");
        if (config_length > leo::kMaxConfigBytes) throw Error(LEO_ERR_INVALID_ARGUMENT, "CONFIG section exceeds 1 MiB");
        leo::save_atomic(leo::need_path(path), *config, *model, config_toml, config_length, retain_previous != 0);
    });
}

int32_t leo_checkpoint_read_generation(const char* path, uint64_t* generation) {
    return guarded([&] {
        if (!generation) throw Error(LEO_ERR_INVALID_ARGUMENT, "null argument");
        *generation = leo::read_generation(leo::need_path(path));
    });
}

int32_t leo_checkpoint_prune_generations(const char* path, uint64_t keep_previous) {
    return guarded([&] { leo::prune(leo::need_path(path), keep_previous); });
}

int32_t leo_dataset_compute_id(uint32_t schema_version, uint64_t record_count, uint64_t bytes_length,
                               const LeoDigest* bytes_digest, const LeoDigest* records_digest,
                               const LeoDigest* provenance_digest, LeoDigest* out) {
    return guarded([&] {
        if (!bytes_digest || !records_digest || !provenance_digest || !out)
            throw Error(LEO_ERR_INVALID_ARGUMENT, "null argument");
        *out = leo::dataset_id(schema_version, record_count, bytes_length, *bytes_digest, *records_digest,
                               *provenance_digest);
    });
}

int32_t leo_dataset_write_index(const char* index_path, const char* bytes_path, const LeoStoryIndex* entries,
                                uint64_t count, const LeoDigest* provenance, LeoDatasetIdentity* identity) {
    return guarded([&] {
        if ((!entries && count) || !provenance) throw Error(LEO_ERR_INVALID_ARGUMENT, "null argument");
        const LeoDatasetIdentity id =
            leo::write_index(leo::need_path(index_path), leo::need_path(bytes_path), entries, count, *provenance);
        if (identity) *identity = id;
    });
}

int32_t leo_dataset_open(const char* bytes_path, const char* index_path, LeoDataset** out) {
    return guarded([&] {
        if (!out) throw Error(LEO_ERR_INVALID_ARGUMENT, "null argument");
        *out = nullptr;
        *out = leo::open_dataset(leo::need_path(bytes_path), leo::need_path(index_path));
    });
}

void leo_dataset_close(LeoDataset* dataset) { delete dataset; }

int32_t leo_dataset_identity(const LeoDataset* dataset, LeoDatasetIdentity* out) {
    return guarded([&] {
        if (!dataset || !out) throw Error(LEO_ERR_INVALID_ARGUMENT, "null argument");
        *out = dataset->identity;
    });
}

uint64_t leo_dataset_len(const LeoDataset* dataset) { return dataset ? dataset->entries.size() : 0; }

int32_t leo_dataset_entry(const LeoDataset* dataset, uint64_t index, LeoStoryIndex* out) {
    return guarded([&] {
        if (!dataset || !out) throw Error(LEO_ERR_INVALID_ARGUMENT, "null argument");
        if (index >= dataset->entries.size()) throw Error(LEO_ERR_INVALID_ARGUMENT, "story index out of range");
        *out = dataset->entries[index];
    });
}

int32_t leo_dataset_story(LeoDataset* dataset, uint64_t index, uint8_t* out, uint64_t capacity, uint64_t* length) {
    return guarded([&] {
        if (!dataset || !length) throw Error(LEO_ERR_INVALID_ARGUMENT, "null argument");
        if (index >= dataset->entries.size()) throw Error(LEO_ERR_INVALID_ARGUMENT, "story index out of range");
        const uint64_t n = dataset->entries[index].length;
        *length = n;
        if (!out || capacity < n) throw Error(LEO_ERR_INVALID_ARGUMENT, "story buffer is too small");
        leo::read_story(dataset, index, out);
    });
}

int32_t leo_dataset_pack(LeoDataset* dataset, uint64_t first, uint64_t count, uint8_t* bytes, uint64_t capacity,
                         uint64_t* offsets) {
    return guarded([&] {
        if (!dataset || !offsets) throw Error(LEO_ERR_INVALID_ARGUMENT, "null argument");
        if (first > dataset->entries.size() || count > dataset->entries.size() - first)
            throw Error(LEO_ERR_INVALID_ARGUMENT, "story range out of range");
        offsets[0] = 0;
        for (uint64_t i = 0; i < count; ++i) offsets[i + 1] = offsets[i] + dataset->entries[first + i].length;
        if (!bytes) return;
        if (capacity < offsets[count]) throw Error(LEO_ERR_INVALID_ARGUMENT, "story buffer is too small");
        for (uint64_t i = 0; i < count; ++i) leo::read_story(dataset, first + i, bytes + offsets[i]);
    });
}

}  // extern "C"
