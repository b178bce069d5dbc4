// One-pod segment executor: the MI355X counterpart of phobos-pod's Engine
// restricted to ALLOC / LOAD / COMPUTE / STORE / FREE on one GPU
// (phobos-pod/src/engine.rs:121-232 run loop, 355-398 issue, 424-509
// LOAD/STORE, 542-653 COMPUTE, 655-687 event polling, 752-793 alloc/complete).
//
// Semantics kept from the reference:
//   * an instruction is issued once all its deps have completed (host-observed
//     completion, so no cross-stream device hazards);
//   * ALLOC takes an exact size-class slab from the device arena and parks
//     while the arena is full; a segment that can never fit fails with
//     "arena exhausted" (engine.rs:752-775);
//   * COMPUTE marshals the exploded-memref argument list, scalars interleaved
//     by position (engine.rs:582-630), round-robin over the pod's streams,
//     and completes when its event has fired;
//   * LOAD / STORE move f32 regions of file:// tensors (storage.rs:22-79).
//
// MI355X design: the reference does a blocking file read then a synchronous
// cuMemcpy on the engine thread (tile_store.rs:153-181).  Here a LOAD or
// STORE moves in chunks through a bounded pool of pinned (hipHostMalloc)
// staging buffers: file reads and writes run on a worker pool, the copies
// are hipMemcpyAsync on two copy streams (one per direction), so reading
// chunk c+1 overlaps copying chunk c, and LOADs of later supertiles, STOREs
// of finished ones and COMPUTEs overlap.  The pool is allocated on first use
// and kept for the pod's lifetime, so the pinned host memory is bounded
// however large the segment.  Built-in leaf kernels get their grid from phx_grid_for (the reference's leaf grid would also be
// correct: every kernel strides over its work).
#include <fcntl.h>
#include <unistd.h>

#include <algorithm>
#include <chrono>
#include <condition_variable>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <functional>
#include <map>
#include <mutex>
#include <set>
#include <sstream>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "phx_internal.h"

using namespace phx;

namespace {

enum class OpKind { Alloc, Load, Compute, Store, Free };
enum class Mode { Read, Write, RMW };

struct Region {
    std::vector<uint64_t> offset, shape;
};

struct Instr {
    uint64_t iid = 0;
    std::vector<uint64_t> deps;
    OpKind kind = OpKind::Alloc;
    uint64_t tile = 0;
    std::vector<uint64_t> shape;  // ALLOC
    uint32_t tensor = 0;          // LOAD / STORE
    Region region;                // LOAD / STORE
    uint32_t kernel = 0;          // COMPUTE
    uint32_t serves = 0;          // FREE: expected_serves (no peer pods here)
    std::vector<std::pair<uint64_t, Mode>> args;
    std::vector<phx_scalar_arg> scalars;
    uint32_t grid[3] = {1, 1, 1}, cta[3] = {1, 1, 1};
};

struct TileBuf {
    uint64_t addr = 0;
    size_t cls = 0;
    std::vector<uint64_t> shape;
    size_t elems = 0;
};

struct TensorInfo {
    std::string path;
    std::vector<uint64_t> shape;
};

// file:// URI -> path, dropping the leading '/' of "/C:..." (storage.rs:9-20).
bool file_path(const std::string &uri, std::string *out) {
    const std::string pre = "file://";
    if (uri.compare(0, pre.size(), pre) != 0) return false;
    std::string rest = uri.substr(pre.size());
    if (rest.size() > 2 && rest[0] == '/' && rest[2] == ':') rest = rest.substr(1);
    *out = rest;
    return true;
}

// (byte offset, elements) runs of a rank<=2 region (storage.rs:22-46).
bool byte_spans(const std::vector<uint64_t> &tshape, const Region &r,
                std::vector<std::pair<uint64_t, size_t>> *out) {
    out->clear();
    if (r.shape.size() == 1) {
        out->push_back({r.offset[0] * 4, (size_t)r.shape[0]});
        return true;
    }
    if (r.shape.size() == 2 && tshape.size() == 2) {
        const uint64_t pitch = tshape[1];
        for (uint64_t row = 0; row < r.shape[0]; ++row)
            out->push_back({((r.offset[0] + row) * pitch + r.offset[1]) * 4, (size_t)r.shape[1]});
        return true;
    }
    return false;
}

// Staging chunk size and the most chunks a pod pins: 8 MiB x 32 by default;
// PHX_POD_STAGE_MIB (1..1024) and PHX_POD_STAGE_CHUNKS (2..256) override.
static size_t env_clamped(const char *name, size_t dflt, size_t lo, size_t hi) {
    const char *e = getenv(name);
    const long v = e ? atol(e) : (long)dflt;
    return v < (long)lo ? lo : v > (long)hi ? hi : (size_t)v;
}

// Fixed worker pool for file I/O.
// File reads and writes of LOAD/STORE run on a pool of host threads (the
// reference runs each on tokio's blocking pool, engine.rs:437-440, 489-492).
// Eight by default; PHX_POD_IO_THREADS (1..64) overrides.
static int io_threads() {
    const char *e = getenv("PHX_POD_IO_THREADS");
    const int n = e ? atoi(e) : 8;
    return n < 1 ? 1 : n > 64 ? 64 : n;
}

class IoPool {
   public:
    explicit IoPool(int n) {
        for (int i = 0; i < n; ++i) th_.emplace_back([this] { loop(); });
    }
    ~IoPool() {
        {
            std::lock_guard<std::mutex> l(mu_);
            stop_ = true;
        }
        cv_.notify_all();
        for (auto &t : th_) t.join();
    }
    void submit(std::function<void()> f) {
        {
            std::lock_guard<std::mutex> l(mu_);
            q_.push_back(std::move(f));
        }
        cv_.notify_one();
    }

   private:
    void loop() {
        for (;;) {
            std::function<void()> f;
            {
                std::unique_lock<std::mutex> l(mu_);
                cv_.wait(l, [this] { return stop_ || !q_.empty(); });
                if (stop_ && q_.empty()) return;
                f = std::move(q_.front());
                q_.pop_front();
            }
            f();
        }
    }
    std::mutex mu_;
    std::condition_variable cv_;
    std::deque<std::function<void()>> q_;
    std::vector<std::thread> th_;
    bool stop_ = false;
};

uint64_t now_ns() {
    return (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(
               std::chrono::steady_clock::now().time_since_epoch())
        .count();
}

}  // namespace

struct phx_pod_s {
    phx_arena arena = nullptr;
    std::vector<hipStream_t> streams;
    hipStream_t copy_stream = nullptr;   // LOAD: host -> device
    hipStream_t store_stream = nullptr;  // STORE: device -> host
    size_t next_stream = 0;
    std::unordered_map<uint32_t, TensorInfo> tensors;
    std::unordered_map<uint32_t, phx_kernel> kernels;
    // kernels loaded from code objects the caller supplies (SetKernels with a
    // gfx950 code object in place of PTX): function and index width
    std::unordered_map<uint32_t, std::pair<hipFunction_t, int>> functions;
    std::unordered_map<uint64_t, TileBuf> tiles;
    // pinned staging chunks of stage_bytes, at most stage_chunks of them
    size_t stage_bytes = 0, stage_chunks = 0;
    std::vector<void *> stage_free;
    std::vector<void *> stage_all;
    IoPool *io = nullptr;
};

namespace {

struct Inflight {
    enum Stage { H2D, D2H, Kernel } stage;
    size_t idx;         // instruction index
    size_t chunk = 0;   // H2D / D2H: chunk of the tile
    hipEvent_t start = nullptr, done = nullptr;
    void *staging = nullptr;
    // Kernel: the arena slab a split launch keeps its partial results in
    // (0: none), released when the launch completes
    uint64_t ws_addr = 0;
    size_t ws_cls = 0;
};

// A file read (LOAD) or write (STORE) of one chunk that a worker finished.
struct IoDone {
    size_t idx, chunk;
    bool ok;
    std::string err;
    uint64_t ns;
    void *staging;
};

// A LOAD or STORE in progress: the tile's bytes in chunks of
// the pod's staging size, each staged, copied and read or written on its own.
struct Xfer {
    bool load;
    uint64_t dev;  // tile address
    size_t bytes;  // tile bytes
    size_t nchunks, next = 0, landed = 0;
    std::string path;
    std::vector<std::pair<uint64_t, size_t>> spans;  // (file byte offset, bytes), tile order
};

// Reads (or writes) tile bytes [a, a + len) from (to) their file spans.
bool chunk_io(const Xfer &x, bool write, char *buf, size_t a, size_t len, std::string *err) {
    int fd = write ? open(x.path.c_str(), O_RDWR | O_CREAT, 0644) : open(x.path.c_str(), O_RDONLY);
    if (fd < 0) {
        *err = (write ? "cannot open/write " : "cannot open/read ") + x.path;
        return false;
    }
    size_t pos = 0;  // tile byte where the current span starts
    bool ok = true;
    for (auto &sp : x.spans) {
        const size_t s0 = pos;
        pos += sp.second;
        const size_t lo = std::max(s0, a), hi = std::min(pos, a + len);
        if (lo >= hi) {
            if (s0 >= a + len) break;
            continue;
        }
        const off_t fo = (off_t)(sp.first + (lo - s0));
        char *b = buf + (lo - a);
        const size_t want = hi - lo;
        size_t done = 0;
        while (done < want) {
            ssize_t r = write ? pwrite(fd, b + done, want - done, fo + (off_t)done)
                              : pread(fd, b + done, want - done, fo + (off_t)done);
            if (r <= 0) break;
            done += (size_t)r;
        }
        if (done != want) {
            *err = (write ? "short write to " : "short read from ") + x.path;
            ok = false;
            break;
        }
    }
    close(fd);
    return ok;
}

bool parse_u64_list(const std::string &s, char sep, std::vector<uint64_t> *out) {
    out->clear();
    if (s == "-") return true;
    std::stringstream ss(s);
    std::string tok;
    while (std::getline(ss, tok, sep)) {
        if (tok.empty()) return false;
        char *end = nullptr;
        uint64_t v = strtoull(tok.c_str(), &end, 0);
        if (*end) return false;
        out->push_back(v);
    }
    return true;
}

int parse_segment(const char *text, std::vector<Instr> *out) {
    std::stringstream in(text ? text : "");
    std::string line;
    int lineno = 0;
    while (std::getline(in, line)) {
        ++lineno;
        size_t hash = line.find('#');
        if (hash != std::string::npos) line = line.substr(0, hash);
        std::stringstream ls(line);
        std::vector<std::string> t;
        std::string w;
        while (ls >> w) t.push_back(w);
        if (t.empty()) continue;
        auto bad = [&](const char *why) {
            return set_error(PHX_E_SEGMENT, "segment line %d: %s", lineno, why);
        };
        if (t.size() < 4) return bad("expected '<iid> <deps> <OP> ...'");
        Instr I;
        I.iid = strtoull(t[0].c_str(), nullptr, 0);
        if (!parse_u64_list(t[1], ',', &I.deps)) return bad("bad deps");
        const std::string &op = t[2];
        I.tile = strtoull(t[3].c_str(), nullptr, 0);
        if (op == "ALLOC") {
            I.kind = OpKind::Alloc;
            if (t.size() < 5 || !parse_u64_list(t[4], 'x', &I.shape) || I.shape.empty())
                return bad("ALLOC <tile> <d0xd1..> [f32]");
            if (t.size() > 5 && t[5] != "f32") return bad("only f32 tiles (tile_store.rs:111)");
        } else if (op == "LOAD" || op == "STORE") {
            I.kind = op == "LOAD" ? OpKind::Load : OpKind::Store;
            if (t.size() < 7) return bad("LOAD/STORE <tile> <tensor> <offsets> <shape>");
            I.tensor = (uint32_t)strtoul(t[4].c_str(), nullptr, 0);
            if (!parse_u64_list(t[5], ',', &I.region.offset) ||
                !parse_u64_list(t[6], ',', &I.region.shape) ||
                I.region.offset.size() != I.region.shape.size())
                return bad("bad region");
        } else if (op == "COMPUTE") {
            I.kind = OpKind::Compute;
            // COMPUTE <kernel> <tile:mode,...> <pos:type:value,...|-> <gx,gy,gz> <cx,cy,cz>
            if (t.size() < 8) return bad("COMPUTE <kernel> <args> <scalars> <grid> <cta>");
            I.kernel = (uint32_t)strtoul(t[3].c_str(), nullptr, 0);
            std::stringstream as(t[4]);
            std::string a;
            while (std::getline(as, a, ',')) {
                size_t c = a.find(':');
                if (c == std::string::npos) return bad("arg is tile:mode");
                uint64_t tile = strtoull(a.substr(0, c).c_str(), nullptr, 0);
                std::string m = a.substr(c + 1);
                Mode mode = m == "r" ? Mode::Read : m == "w" ? Mode::Write : Mode::RMW;
                if (m != "r" && m != "w" && m != "rmw") return bad("mode is r|w|rmw");
                I.args.push_back({tile, mode});
            }
            if (t[5] != "-") {
                std::stringstream ss(t[5]);
                std::string s;
                while (std::getline(ss, s, ',')) {
                    size_t c1 = s.find(':'), c2 = s.find(':', c1 + 1);
                    if (c1 == std::string::npos || c2 == std::string::npos)
                        return bad("scalar is pos:type:value");
                    phx_scalar_arg sa;
                    sa.pos = (uint32_t)strtoul(s.substr(0, c1).c_str(), nullptr, 0);
                    std::string ty = s.substr(c1 + 1, c2 - c1 - 1), val = s.substr(c2 + 1);
                    if (ty == "f32") {
                        sa.bytes = 4;
                        if (val.rfind("0x", 0) == 0) {
                            sa.bits = strtoull(val.c_str(), nullptr, 16) & 0xffffffffu;
                        } else {
                            float f = strtof(val.c_str(), nullptr);
                            uint32_t u;
                            memcpy(&u, &f, 4);
                            sa.bits = u;
                        }
                    } else if (ty == "i32") {
                        sa.bytes = 4;
                        sa.bits = (uint32_t)strtol(val.c_str(), nullptr, 0);
                    } else if (ty == "i64" || ty == "f64") {
                        sa.bytes = 8;
                        if (ty == "i64") {
                            sa.bits = (uint64_t)strtoll(val.c_str(), nullptr, 0);
                        } else {
                            double d = strtod(val.c_str(), nullptr);
                            memcpy(&sa.bits, &d, 8);
                        }
                    } else if (ty == "bool") {
                        sa.bytes = 1;
                        sa.bits = strtoul(val.c_str(), nullptr, 0) ? 1 : 0;
                    } else {
                        return bad("scalar type is f32|i32|i64|f64|bool");
                    }
                    I.scalars.push_back(sa);
                }
            }
            std::vector<uint64_t> g, c;
            if (!parse_u64_list(t[6], ',', &g) || g.size() != 3 || !parse_u64_list(t[7], ',', &c) ||
                c.size() != 3)
                return bad("grid/cta are x,y,z");
            for (int i = 0; i < 3; ++i) {
                I.grid[i] = (uint32_t)g[i];
                I.cta[i] = (uint32_t)c[i];
            }
        } else if (op == "FREE") {
            I.kind = OpKind::Free;
            if (t.size() > 4) I.serves = (uint32_t)strtoul(t[4].c_str(), nullptr, 0);
        } else {
            return bad("unknown op");
        }
        out->push_back(std::move(I));
    }
    return PHX_OK;
}

// ------------------------------------------------------ protobuf decoding
// Hand decoder of the proto3 wire format for the scheduler's messages
// (phobos-cluster/proto/v1/phobos_v1_isa.proto, phobos_v1_scheduler.proto),
// with the same checks as the reference's converters (proto.rs:193-275):
// missing sub-messages and unknown enum values are errors.  Unknown fields
// are skipped; repeated scalars are accepted packed or unpacked.
class Pb {
   public:
    Pb(const void *b, size_t n) : p_((const uint8_t *)b), end_(p_ + n) {}
    bool done() const { return p_ >= end_; }
    bool varint(uint64_t *v) {
        uint64_t r = 0;
        for (int s = 0; s < 64 && p_ < end_; s += 7) {
            const uint8_t b = *p_++;
            r |= (uint64_t)(b & 0x7f) << s;
            if (!(b & 0x80)) {
                *v = r;
                return true;
            }
        }
        return false;
    }
    bool tag(uint32_t *field, uint32_t *wt) {
        uint64_t t;
        if (!varint(&t) || (t >> 3) == 0 || (t >> 3) > 0x1fffffff) return false;
        *field = (uint32_t)(t >> 3);
        *wt = (uint32_t)(t & 7);
        return true;
    }
    bool len(Pb *sub) {
        uint64_t l;
        if (!varint(&l) || l > (uint64_t)(end_ - p_)) return false;
        *sub = Pb(p_, (size_t)l);
        p_ += l;
        return true;
    }
    bool str(std::string *out) {
        Pb s(nullptr, 0);
        if (!len(&s)) return false;
        out->assign((const char *)s.p_, (size_t)(s.end_ - s.p_));
        return true;
    }
    bool fixed(void *out, size_t n) {
        if ((size_t)(end_ - p_) < n) return false;
        memcpy(out, p_, n);
        p_ += n;
        return true;
    }
    bool skip(uint32_t wt) {
        uint64_t v;
        Pb s(nullptr, 0);
        switch (wt) {
        case 0: return varint(&v);
        case 1: return fixed(&v, 8);
        case 2: return len(&s);
        case 5: return fixed(&v, 4);
        default: return false;
        }
    }
    // repeated uint64, packed (wire type 2) or one element (wire type 0)
    bool rep_u64(uint32_t wt, std::vector<uint64_t> *out) {
        uint64_t v;
        if (wt == 0) {
            if (!varint(&v)) return false;
            out->push_back(v);
            return true;
        }
        Pb s(nullptr, 0);
        if (wt != 2 || !len(&s)) return false;
        while (!s.done()) {
            if (!s.varint(&v)) return false;
            out->push_back(v);
        }
        return true;
    }

   private:
    const uint8_t *p_, *end_;
};

int pb_bad(const char *what) { return set_error(PHX_E_SEGMENT, "protobuf: %s", what); }

// Reads a varint field of the expected wire type.
#define PB_VARINT(var)                                       \
    do {                                                     \
        uint64_t v_;                                         \
        if (wt != 0 || !m.varint(&v_)) return pb_bad(#var); \
        var = v_;                                            \
    } while (0)

int pb_region(Pb m, Region *r) {
    uint32_t f, wt;
    while (!m.done()) {
        if (!m.tag(&f, &wt)) return pb_bad("Region tag");
        if (f == 1) {
            if (!m.rep_u64(wt, &r->offset)) return pb_bad("Region.offset");
        } else if (f == 2) {
            if (!m.rep_u64(wt, &r->shape)) return pb_bad("Region.shape");
        } else if (!m.skip(wt)) {
            return pb_bad("Region field");
        }
    }
    if (r->offset.size() != r->shape.size() || r->shape.empty()) return pb_bad("Region rank");
    return PHX_OK;
}

int pb_storage_ref(Pb m, Instr *I, const char *who) {
    uint32_t f, wt;
    bool have_region = false;
    while (!m.done()) {
        if (!m.tag(&f, &wt)) return pb_bad("StorageReference tag");
        if (f == 1) {
            uint64_t t = 0;
            PB_VARINT(t);
            I->tensor = (uint32_t)t;
        } else if (f == 2) {
            Pb s(nullptr, 0);
            if (wt != 2 || !m.len(&s)) return pb_bad("StorageReference.region");
            if (int rc = pb_region(s, &I->region)) return rc;
            have_region = true;
        } else if (!m.skip(wt)) {
            return pb_bad("StorageReference field");
        }
    }
    if (!have_region) return set_error(PHX_E_SEGMENT, "%s: StorageReference.region missing", who);
    return PHX_OK;
}

int pb_dim3(Pb m, uint32_t out[3]) {
    uint32_t f, wt;
    out[0] = out[1] = out[2] = 0;  // proto3 default
    while (!m.done()) {
        if (!m.tag(&f, &wt)) return pb_bad("Dim3 tag");
        if (f >= 1 && f <= 3) {
            uint64_t v = 0;
            PB_VARINT(v);
            out[f - 1] = (uint32_t)v;
        } else if (!m.skip(wt)) {
            return pb_bad("Dim3 field");
        }
    }
    return PHX_OK;
}

// ScalarValue oneof -> little-endian bits and byte width (tile.rs:74-84).
int pb_scalar_value(Pb m, phx_scalar_arg *sa) {
    uint32_t f, wt;
    bool have = false;
    while (!m.done()) {
        if (!m.tag(&f, &wt)) return pb_bad("ScalarValue tag");
        if (f == 1 && wt == 5) {  // f32
            uint32_t u;
            if (!m.fixed(&u, 4)) return pb_bad("ScalarValue.f32");
            sa->bits = u;
            sa->bytes = 4;
        } else if (f == 2 && wt == 1) {  // f64
            uint64_t u;
            if (!m.fixed(&u, 8)) return pb_bad("ScalarValue.f64");
            sa->bits = u;
            sa->bytes = 8;
        } else if (f == 3 && wt == 0) {  // i32 (negative values are 10-byte varints)
            uint64_t u;
            if (!m.varint(&u)) return pb_bad("ScalarValue.i32");
            sa->bits = (uint32_t)u;
            sa->bytes = 4;
        } else if (f == 4 && wt == 0) {  // i64
            uint64_t u;
            if (!m.varint(&u)) return pb_bad("ScalarValue.i64");
            sa->bits = u;
            sa->bytes = 8;
        } else if (f == 5 && wt == 0) {  // bool
            uint64_t u;
            if (!m.varint(&u)) return pb_bad("ScalarValue.boolean");
            sa->bits = u ? 1 : 0;
            sa->bytes = 1;
        } else {
            if (!m.skip(wt)) return pb_bad("ScalarValue field");
            continue;
        }
        have = true;  // a oneof: the last value on the wire wins
    }
    if (!have) return set_error(PHX_E_SEGMENT, "ScalarValue.value missing");
    return PHX_OK;
}

int pb_compute(Pb m, Instr *I) {
    uint32_t f, wt;
    bool have_grid = false, have_cta = false;
    while (!m.done()) {
        if (!m.tag(&f, &wt)) return pb_bad("Compute tag");
        Pb s(nullptr, 0);
        if (f == 1) {
            uint64_t k = 0;
            PB_VARINT(k);
            I->kernel = (uint32_t)k;
        } else if (f == 2) {  // ComputeArgument {tile, mode}
            if (wt != 2 || !m.len(&s)) return pb_bad("Compute.arguments");
            uint64_t tile = 0, mode = 0;
            uint32_t g, gwt;
            while (!s.done()) {
                if (!s.tag(&g, &gwt)) return pb_bad("ComputeArgument tag");
                uint64_t v;
                if ((g == 1 || g == 2) && gwt == 0) {
                    if (!s.varint(&v)) return pb_bad("ComputeArgument");
                    (g == 1 ? tile : mode) = v;
                } else if (!s.skip(gwt)) {
                    return pb_bad("ComputeArgument field");
                }
            }
            if (mode < 1 || mode > 3)
                return set_error(PHX_E_SEGMENT, "unknown AccessMode %llu", (unsigned long long)mode);
            I->args.push_back({tile, mode == 1 ? Mode::Read : mode == 2 ? Mode::Write : Mode::RMW});
        } else if (f == 3 || f == 4) {
            if (wt != 2 || !m.len(&s)) return pb_bad("Compute.grid/cta");
            if (int rc = pb_dim3(s, f == 3 ? I->grid : I->cta)) return rc;
            (f == 3 ? have_grid : have_cta) = true;
        } else if (f == 5) {  // ScalarArgument {position, value}
            if (wt != 2 || !m.len(&s)) return pb_bad("Compute.scalars");
            phx_scalar_arg sa{0, 0, 0};
            bool have_value = false;
            uint32_t g, gwt;
            while (!s.done()) {
                if (!s.tag(&g, &gwt)) return pb_bad("ScalarArgument tag");
                Pb v(nullptr, 0);
                if (g == 1 && gwt == 0) {
                    uint64_t pos;
                    if (!s.varint(&pos)) return pb_bad("ScalarArgument.position");
                    sa.pos = (uint32_t)pos;
                } else if (g == 2 && gwt == 2) {
                    if (!s.len(&v)) return pb_bad("ScalarArgument.value");
                    if (int rc = pb_scalar_value(v, &sa)) return rc;
                    have_value = true;
                } else if (!s.skip(gwt)) {
                    return pb_bad("ScalarArgument field");
                }
            }
            if (!have_value) return set_error(PHX_E_SEGMENT, "ScalarArgument.value missing");
            I->scalars.push_back(sa);
        } else if (!m.skip(wt)) {
            return pb_bad("Compute field");
        }
    }
    if (!have_grid) return set_error(PHX_E_SEGMENT, "Compute.grid missing");
    if (!have_cta) return set_error(PHX_E_SEGMENT, "Compute.cta missing");
    return PHX_OK;
}

// Operation oneof -> Instr fields.
int pb_operation(Pb m, Instr *I) {
    uint32_t f, wt;
    bool have = false;
    while (!m.done()) {
        if (!m.tag(&f, &wt)) return pb_bad("Operation tag");
        if (f < 1 || f > 6) {
            if (!m.skip(wt)) return pb_bad("Operation field");
            continue;
        }
        Pb s(nullptr, 0);
        if (wt != 2 || !m.len(&s)) return pb_bad("Operation kind");
        *I = Instr{I->iid, I->deps};  // a later kind on the wire replaces an earlier one
        uint32_t g, gwt;
        if (f == 3)
            return set_error(PHX_E_SEGMENT,
                             "FETCH (a tile from another pod) needs a peer; this executor runs "
                             "one pod");
        if (f == 4) {
            I->kind = OpKind::Compute;
            if (int rc = pb_compute(s, I)) return rc;
            have = true;
            continue;
        }
        I->kind = f == 1 ? OpKind::Alloc : f == 2 ? OpKind::Load : f == 5 ? OpKind::Store : OpKind::Free;
        bool have_ref = false;
        uint64_t dtype = 0;
        while (!s.done()) {
            if (!s.tag(&g, &gwt)) return pb_bad("op tag");
            if (g == 1 && gwt == 0) {
                if (!s.varint(&I->tile)) return pb_bad("op.tile");
            } else if (f == 6 && g == 2 && gwt == 0) {
                uint64_t v;
                if (!s.varint(&v)) return pb_bad("Free.expected_serves");
                I->serves = (uint32_t)v;
            } else if (f == 1 && g == 2) {
                if (!s.rep_u64(gwt, &I->shape)) return pb_bad("Allocate.shape");
            } else if (f == 1 && g == 3 && gwt == 0) {
                if (!s.varint(&dtype)) return pb_bad("Allocate.data_type");
            } else if ((f == 2 || f == 5) && g == 2 && gwt == 2) {
                Pb r(nullptr, 0);
                if (!s.len(&r)) return pb_bad("StorageReference");
                if (int rc = pb_storage_ref(r, I, f == 2 ? "Load" : "Store")) return rc;
                have_ref = true;
            } else if (!s.skip(gwt)) {
                return pb_bad("op field");
            }
        }
        if (f == 1) {
            if (dtype < 1 || dtype > 7)
                return set_error(PHX_E_SEGMENT, "unknown DataType %llu", (unsigned long long)dtype);
            if (dtype != 2) return set_error(PHX_E_SEGMENT, "only f32 tiles (tile_store.rs:111-131)");
            if (I->shape.empty()) return set_error(PHX_E_SEGMENT, "Allocate.shape empty");
        }
        if ((f == 2 || f == 5) && !have_ref)
            return set_error(PHX_E_SEGMENT, f == 2 ? "Load.source missing" : "Store.destination missing");
        have = true;
    }
    if (!have) return set_error(PHX_E_SEGMENT, "Operation.kind missing");
    return PHX_OK;
}

int pb_segment(const void *bytes, size_t n, std::vector<Instr> *out) {
    if (!bytes && n) return set_error(PHX_E_INVALID, "null segment bytes");
    Pb m(bytes, n);
    uint32_t f, wt;
    while (!m.done()) {
        if (!m.tag(&f, &wt)) return pb_bad("Segment tag");
        if (f != 2) {
            if (!m.skip(wt)) return pb_bad("Segment field");
            continue;
        }
        Pb ins(nullptr, 0);
        if (wt != 2 || !m.len(&ins)) return pb_bad("Segment.instructions");
        Instr I;
        bool have_op = false;
        uint32_t g, gwt;
        while (!ins.done()) {
            if (!ins.tag(&g, &gwt)) return pb_bad("Instruction tag");
            if (g == 1 && gwt == 0) {
                if (!ins.varint(&I.iid)) return pb_bad("Instruction.iid");
            } else if (g == 2) {
                if (!ins.rep_u64(gwt, &I.deps)) return pb_bad("Instruction.dependencies");
            } else if (g == 3 && gwt == 2) {
                Pb op(nullptr, 0);
                if (!ins.len(&op)) return pb_bad("Instruction.operation");
                Instr J{I.iid, I.deps};
                if (int rc = pb_operation(op, &J)) return rc;
                const uint64_t iid = I.iid;
                const std::vector<uint64_t> deps = I.deps;
                I = std::move(J);
                I.iid = iid;
                I.deps = deps;
                have_op = true;
            } else if (!ins.skip(gwt)) {
                return pb_bad("Instruction field");
            }
        }
        if (!have_op)
            return set_error(PHX_E_SEGMENT, "iid %llu: Instruction.operation missing",
                             (unsigned long long)I.iid);
        out->push_back(std::move(I));
    }
    return PHX_OK;
}

// The text form of an instruction list (the inverse of parse_segment).
std::string render_text(const std::vector<Instr> &ins) {
    std::string out;
    char buf[128];
    auto list = [](const std::vector<uint64_t> &v, char sep) {
        std::string r;
        for (size_t i = 0; i < v.size(); ++i) {
            if (i) r += sep;
            r += std::to_string((unsigned long long)v[i]);
        }
        return r.empty() ? std::string("-") : r;
    };
    for (const Instr &I : ins) {
        out += std::to_string((unsigned long long)I.iid) + " " + list(I.deps, ',') + " ";
        snprintf(buf, sizeof buf, "0x%llx", (unsigned long long)I.tile);
        switch (I.kind) {
        case OpKind::Alloc:
            out += std::string("ALLOC ") + buf + " " + list(I.shape, 'x') + " f32";
            break;
        case OpKind::Load:
        case OpKind::Store:
            out += std::string(I.kind == OpKind::Load ? "LOAD " : "STORE ") + buf + " " +
                   std::to_string(I.tensor) + " " + list(I.region.offset, ',') + " " +
                   list(I.region.shape, ',');
            break;
        case OpKind::Compute: {
            out += "COMPUTE " + std::to_string(I.kernel) + " ";
            for (size_t a = 0; a < I.args.size(); ++a) {
                snprintf(buf, sizeof buf, "%s0x%llx:%s", a ? "," : "",
                         (unsigned long long)I.args[a].first,
                         I.args[a].second == Mode::Read ? "r"
                         : I.args[a].second == Mode::Write ? "w" : "rmw");
                out += buf;
            }
            out += " ";
            if (I.scalars.empty()) out += "-";
            for (size_t k = 0; k < I.scalars.size(); ++k) {
                const phx_scalar_arg &sa = I.scalars[k];
                // only the width and bit pattern reach the kernel, so 4-byte
                // values print as f32 bits and 8-byte ones as i64: both exact
                if (sa.bytes == 1)
                    snprintf(buf, sizeof buf, "%u:bool:%u", sa.pos, (unsigned)sa.bits);
                else if (sa.bytes == 4)
                    snprintf(buf, sizeof buf, "%u:f32:0x%llx", sa.pos, (unsigned long long)sa.bits);
                else
                    snprintf(buf, sizeof buf, "%u:i64:%lld", sa.pos, (long long)sa.bits);
                out += (k ? "," : "") + std::string(buf);
            }
            snprintf(buf, sizeof buf, " %u,%u,%u %u,%u,%u", I.grid[0], I.grid[1], I.grid[2],
                     I.cta[0], I.cta[1], I.cta[2]);
            out += buf;
            break;
        }
        case OpKind::Free:
            out += std::string("FREE ") + buf + " " + std::to_string(I.serves);
            break;
        }
        out += "\n";
    }
    return out;
}

// Built-in kernels a JobManifest may name (KernelEntry.name, the entry
// point): the one-pod job's leaves (clustergen.rs:1285, 1353) and saxpy.
// The GEMM and flash entry names are shared by several .ph kernels, so those
// are bound by id with phx_pod_set_kernel instead.
bool builtin_by_name(const std::string &name, phx_kernel *k) {
    if (name == "matmul") *k = PHX_MATMUL;
    else if (name == "matmul_init") *k = PHX_MATMUL_INIT;
    else if (name == "saxpy") *k = PHX_SAXPY_FP32;
    else return false;
    return true;
}

}  // namespace

extern "C" {

int phx_pod_create(phx_pod *out, size_t arena_bytes, int nstreams) {
    if (nstreams < 1 || nstreams > 16) return set_error(PHX_E_INVALID, "nstreams must be 1..16");
    phx_pod p = new phx_pod_s;
    if (int rc = phx_arena_create(&p->arena, arena_bytes)) {
        delete p;
        return rc;
    }
    for (int i = 0; i < nstreams + 2; ++i) {
        hipStream_t s;
        hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
        if (e != hipSuccess) {
            phx_pod_destroy(p);
            return hip_error(e, "pod stream");
        }
        if (i == nstreams)
            p->copy_stream = s;
        else if (i == nstreams + 1)
            p->store_stream = s;
        else
            p->streams.push_back(s);
    }
    p->io = new IoPool(io_threads());
    p->stage_bytes = env_clamped("PHX_POD_STAGE_MIB", 8, 1, 1024) << 20;
    p->stage_chunks = env_clamped("PHX_POD_STAGE_CHUNKS", 32, 2, 256);
    *out = p;
    return PHX_OK;
}

int phx_pod_get_arena(phx_pod p, phx_arena *a) {
    if (!p || !a) return set_error(PHX_E_INVALID, "null pod or arena");
    *a = p->arena;
    return PHX_OK;
}

int phx_pod_destroy(phx_pod p) {
    if (!p) return PHX_OK;
    delete p->io;
    for (auto s : p->streams) (void)hipStreamDestroy(s);
    if (p->copy_stream) (void)hipStreamDestroy(p->copy_stream);
    if (p->store_stream) (void)hipStreamDestroy(p->store_stream);
    for (void *h : p->stage_all) (void)hipHostFree(h);
    phx_arena_destroy(p->arena);
    delete p;
    return PHX_OK;
}

int phx_pod_set_tensor(phx_pod p, uint32_t tensor, const char *uri, const uint64_t *shape,
                       uint32_t rank) {
    if (!p || !uri || rank < 1 || rank > 2)
        return set_error(PHX_E_INVALID, "set_tensor: bad argument (rank 1..2)");
    TensorInfo ti;
    if (!file_path(uri, &ti.path))
        return set_error(PHX_E_IO, "unsupported storage URI '%s' (expected file://)", uri);
    ti.shape.assign(shape, shape + rank);
    p->tensors[tensor] = ti;
    return PHX_OK;
}

int phx_pod_set_kernel(phx_pod p, uint32_t kernel_id, phx_kernel k) {
    if (!p || (int)k < 0 || k >= PHX_NUM_KERNELS) return set_error(PHX_E_INVALID, "set_kernel");
    hipFunction_t f;
    if (int rc = builtin(k, &f)) return rc;
    p->functions.erase(kernel_id);
    p->kernels[kernel_id] = k;
    return PHX_OK;
}

int phx_pod_set_kernel_function(phx_pod p, uint32_t kernel_id, phx_function f,
                                int index_bits) {
    if (!p || !f) return set_error(PHX_E_INVALID, "set_kernel_function: null pod or function");
    if (index_bits != 32 && index_bits != 64)
        return set_error(PHX_E_INVALID, "index_bits must be 32 or 64");
    p->kernels.erase(kernel_id);
    p->functions[kernel_id] = {(hipFunction_t)f, index_bits};
    return PHX_OK;
}

static int run_instrs(phx_pod p, std::vector<Instr> &ins, uint64_t stats[8]);

int phx_pod_run_segment(phx_pod p, const char *text, uint64_t stats[8]) {
    if (!p) return set_error(PHX_E_INVALID, "null pod");
    std::vector<Instr> ins;
    if (int rc = parse_segment(text, &ins)) return rc;
    return run_instrs(p, ins, stats);
}

int phx_pod_run_segment_pb(phx_pod p, const void *segment, size_t bytes, uint64_t stats[8]) {
    if (!p) return set_error(PHX_E_INVALID, "null pod");
    std::vector<Instr> ins;
    if (int rc = pb_segment(segment, bytes, &ins)) return rc;
    return run_instrs(p, ins, stats);
}

int phx_pod_set_manifest_pb(phx_pod p, const void *manifest, size_t bytes) {
    if (!p || (!manifest && bytes)) return set_error(PHX_E_INVALID, "set_manifest: bad argument");
    Pb m(manifest, bytes);
    uint32_t f, wt;
    while (!m.done()) {
        if (!m.tag(&f, &wt)) return pb_bad("JobManifest tag");
        Pb e(nullptr, 0);
        if ((f != 1 && f != 2) || wt != 2) {
            if (!m.skip(wt)) return pb_bad("JobManifest field");
            continue;  // kernel_holders and unknown fields: not used by one pod
        }
        if (!m.len(&e)) return pb_bad("JobManifest entry");
        uint64_t index = 0, dtype = 2;
        std::string uri, hash, name;
        std::vector<uint64_t> shape;
        uint32_t g, gwt;
        while (!e.done()) {
            if (!e.tag(&g, &gwt)) return pb_bad("entry tag");
            bool ok = true;
            if (g == 1 && gwt == 0) ok = e.varint(&index);
            else if (f == 1 && g == 2 && gwt == 2) ok = e.str(&uri);
            else if (f == 1 && g == 3 && gwt == 0) ok = e.varint(&dtype);
            else if (f == 1 && g == 4) ok = e.rep_u64(gwt, &shape);
            else if (f == 2 && g == 2 && gwt == 2) ok = e.str(&hash);
            else if (f == 2 && g == 3 && gwt == 2) ok = e.str(&name);
            else ok = e.skip(gwt);
            if (!ok) return pb_bad(f == 1 ? "TensorEntry field" : "KernelEntry field");
        }
        if (f == 1) {
            if (dtype != 2 && dtype != 0)
                return set_error(PHX_E_SEGMENT, "tensor %llu: only f32 tensors (storage.rs:48-79)",
                                 (unsigned long long)index);
            if (int rc = phx_pod_set_tensor(p, (uint32_t)index, uri.c_str(), shape.data(),
                                            (uint32_t)shape.size()))
                return rc;
        } else {
            phx_kernel k;
            if (!builtin_by_name(name, &k))
                return set_error(PHX_E_NOT_FOUND,
                                 "kernel %llu '%s' is not a built-in pod leaf; bind it with "
                                 "phx_pod_set_kernel",
                                 (unsigned long long)index, name.c_str());
            if (int rc = phx_pod_set_kernel(p, (uint32_t)index, k)) return rc;
        }
    }
    return PHX_OK;
}

int phx_segment_pb_to_text(const void *segment, size_t bytes, char *text, size_t cap,
                           size_t *needed) {
    std::vector<Instr> ins;
    if (int rc = pb_segment(segment, bytes, &ins)) return rc;
    const std::string t = render_text(ins);
    if (needed) *needed = t.size() + 1;
    if (!text || cap < t.size() + 1)
        return text ? set_error(PHX_E_INVALID, "text buffer of %zu bytes, %zu needed", cap,
                                t.size() + 1)
                    : PHX_OK;
    memcpy(text, t.c_str(), t.size() + 1);
    return PHX_OK;
}

static int run_instrs(phx_pod p, std::vector<Instr> &ins, uint64_t stats[8]) {
    const size_t n = ins.size();
    std::unordered_map<uint64_t, size_t> by_iid;
    for (size_t i = 0; i < n; ++i) {
        if (by_iid.count(ins[i].iid)) return set_error(PHX_E_SEGMENT, "duplicate iid %llu", (unsigned long long)ins[i].iid);
        by_iid[ins[i].iid] = i;
    }
    std::vector<size_t> pending(n, 0);
    std::vector<std::vector<size_t>> dependents(n);
    for (size_t i = 0; i < n; ++i)
        for (uint64_t d : ins[i].deps) {
            auto it = by_iid.find(d);
            if (it == by_iid.end())
                return set_error(PHX_E_SEGMENT, "iid %llu depends on unknown iid %llu",
                                 (unsigned long long)ins[i].iid, (unsigned long long)d);
            dependents[it->second].push_back(i);
            pending[i]++;
        }
    uint64_t st[8] = {0};
    const uint64_t t0 = now_ns();
    // compute_ns is the time at least one COMPUTE was running: leaves on the
    // pod's streams may overlap each other, so their intervals, timed from an
    // origin event recorded before any of them, are merged at the end rather
    // than their durations summed.
    struct Origin {
        hipEvent_t ev = nullptr;
        ~Origin() {
            if (ev) (void)hipEventDestroy(ev);
        }
    } origin;
    if (hipEventCreate(&origin.ev) != hipSuccess ||
        hipEventRecord(origin.ev, p->streams[0]) != hipSuccess) {
        if (origin.ev) (void)hipEventDestroy(origin.ev);
        origin.ev = nullptr;
    }
    std::vector<std::pair<float, float>> busy;  // kernel [start, end) in ms after origin

    std::set<size_t> ready;  // ordered by segment position
    for (size_t i = 0; i < n; ++i)
        if (pending[i] == 0) ready.insert(i);
    std::vector<size_t> parked_alloc;
    std::vector<Inflight> inflight;
    std::mutex io_mu;
    std::vector<IoDone> io_done;
    size_t io_pending = 0, completed = 0;
    int err = PHX_OK;

    auto complete = [&](size_t i) {
        ++completed;
        for (size_t d : dependents[i])
            if (--pending[d] == 0) ready.insert(d);
    };
    // LOADs and STOREs in progress, and those with chunks not yet staged
    // (first issued, first served, so the earliest transfer finishes first)
    std::map<size_t, Xfer> xfers;
    std::deque<size_t> xq;
    auto take_stage = [&](void **h) -> int {
        *h = nullptr;
        if (!p->stage_free.empty()) {
            *h = p->stage_free.back();
            p->stage_free.pop_back();
        } else if (p->stage_all.size() < p->stage_chunks) {
            if (hipHostMalloc(h, p->stage_bytes, hipHostMallocDefault) != hipSuccess) {
                *h = nullptr;
                if (p->stage_all.empty())  // none will ever come back
                    return set_error(PHX_E_IO, "pinned staging of %zu bytes failed",
                                     p->stage_bytes);
            } else {
                p->stage_all.push_back(*h);
            }
        }
        return PHX_OK;
    };
    auto chunk_range = [&](const Xfer &x, size_t c, size_t *a, size_t *len) {
        *a = c * p->stage_bytes;
        *len = std::min(p->stage_bytes, x.bytes - *a);
    };
    // stages every chunk that a free staging buffer allows: a LOAD chunk goes
    // to a worker for its file read, a STORE chunk to the D2H copy stream
    auto pump = [&]() -> int {
        while (!xq.empty()) {
            const size_t idx = xq.front();
            Xfer &x = xfers.at(idx);
            if (x.next == x.nchunks) {
                xq.pop_front();
                continue;
            }
            void *h;
            if (int rc = take_stage(&h)) return rc;
            if (!h) return PHX_OK;  // all chunks busy: wait for one to come back
            const size_t c = x.next++;
            size_t a, len;
            chunk_range(x, c, &a, &len);
            if (x.load) {
                const Xfer *xp = &x;  // map nodes stay put until the transfer ends
                io_pending++;
                p->io->submit([&, idx, c, h, a, len, xp]() {
                    const uint64_t s0 = now_ns();
                    IoDone d{idx, c, true, "", 0, h};
                    d.ok = chunk_io(*xp, false, (char *)h, a, len, &d.err);
                    d.ns = now_ns() - s0;
                    std::lock_guard<std::mutex> l(io_mu);
                    io_done.push_back(d);
                });
            } else {
                Inflight f{Inflight::D2H, idx};
                f.chunk = c;
                f.staging = h;
                inflight.push_back(f);  // the drain accounts for the chunk from here on
                Inflight &g = inflight.back();
                hipError_t e = hipMemcpyAsync(h, (void *)(uintptr_t)(x.dev + a), len,
                                              hipMemcpyDeviceToHost, p->store_stream);
                if (e == hipSuccess) e = hipEventCreateWithFlags(&g.done, hipEventDisableTiming);
                if (e == hipSuccess) e = hipEventRecord(g.done, p->store_stream);
                if (e != hipSuccess) return hip_error(e, "STORE hipMemcpyAsync");
            }
        }
        return PHX_OK;
    };
    // a transfer's chunk arrived (LOAD: on the device; STORE: in the file)
    auto chunk_landed = [&](size_t idx, void *h) {
        p->stage_free.push_back(h);
        Xfer &x = xfers.at(idx);
        if (++x.landed < x.nchunks) return;
        st[x.load ? 1 : 3]++;
        xfers.erase(idx);
        complete(idx);
    };
    auto tile_of = [&](uint64_t id, TileBuf **out) -> int {
        auto it = p->tiles.find(id);
        if (it == p->tiles.end())
            return set_error(PHX_E_SEGMENT, "unknown tile 0x%llx", (unsigned long long)id);
        *out = &it->second;
        return PHX_OK;
    };
    std::vector<uint64_t> allocated_here;  // released again if the segment fails
    auto region_ok = [&](const Instr &I, const TileBuf &tb, const TensorInfo &ti) -> int {
        uint64_t elems = 1;
        for (auto s : I.region.shape) elems *= s;
        if (elems != tb.elems)
            return set_error(PHX_E_SEGMENT, "region of %llu elements for a tile of %zu",
                             (unsigned long long)elems, tb.elems);
        if (I.region.shape.size() != ti.shape.size() && !(I.region.shape.size() == 1))
            return set_error(PHX_E_SEGMENT, "region rank != tensor rank");
        if (I.region.shape.size() == 1 && ti.shape.size() > 1) {
            // a rank-1 region over a higher-rank tensor is a flat element
            // range, as byte_spans reads it (storage.rs:22-79)
            uint64_t total = 1;
            for (auto s : ti.shape) total *= s;
            if (I.region.offset[0] + I.region.shape[0] > total)
                return set_error(PHX_E_SEGMENT, "region exceeds tensor bounds");
            return PHX_OK;
        }
        for (size_t d = 0; d < I.region.shape.size(); ++d)
            if (I.region.offset[d] + I.region.shape[d] > ti.shape[d])
                return set_error(PHX_E_SEGMENT, "region exceeds tensor bounds");
        return PHX_OK;
    };

    auto issue = [&](size_t i) -> int {
        Instr &I = ins[i];
        switch (I.kind) {
        case OpKind::Alloc: {
            size_t elems = 1;
            for (auto s : I.shape) elems *= (size_t)s;
            if (p->tiles.count(I.tile))
                return set_error(PHX_E_SEGMENT, "tile 0x%llx allocated twice", (unsigned long long)I.tile);
            if (!phx_arena_can_alloc(p->arena, elems * 4)) {
                parked_alloc.push_back(i);
                return PHX_OK;
            }
            TileBuf tb;
            if (int rc = phx_arena_alloc(p->arena, elems * 4, &tb.addr, &tb.cls)) return rc;
            tb.shape = I.shape;
            tb.elems = elems;
            p->tiles[I.tile] = tb;
            allocated_here.push_back(I.tile);
            st[0]++;
            complete(i);
            return PHX_OK;
        }
        case OpKind::Free: {
            auto it = p->tiles.find(I.tile);
            if (it == p->tiles.end())
                return set_error(PHX_E_SEGMENT, "free of unknown tile 0x%llx", (unsigned long long)I.tile);
            phx_arena_free(p->arena, it->second.addr, it->second.cls);
            p->tiles.erase(it);
            st[4]++;
            complete(i);
            // a release may unpark allocations
            for (size_t a : parked_alloc) ready.insert(a);
            parked_alloc.clear();
            return PHX_OK;
        }
        case OpKind::Load:
        case OpKind::Store: {
            const bool load = I.kind == OpKind::Load;
            TileBuf *tb;
            if (int rc = tile_of(I.tile, &tb)) return rc;
            auto tit = p->tensors.find(I.tensor);
            if (tit == p->tensors.end())
                return set_error(PHX_E_SEGMENT, load ? "LOAD of unregistered tensor %u"
                                                     : "STORE to unregistered tensor %u",
                                 I.tensor);
            if (int rc = region_ok(I, *tb, tit->second)) return rc;
            Xfer x;
            x.load = load;
            x.dev = tb->addr;
            x.bytes = tb->elems * 4;
            x.nchunks = (x.bytes + p->stage_bytes - 1) / p->stage_bytes;
            x.path = tit->second.path;
            if (!byte_spans(tit->second.shape, I.region, &x.spans))
                return set_error(PHX_E_IO, "cannot %s %s", load ? "open/read" : "open/write",
                                 x.path.c_str());
            for (auto &sp : x.spans) sp.second *= 4;
            if (x.nchunks == 0) {
                st[load ? 1 : 3]++;
                complete(i);
                return PHX_OK;
            }
            xfers.emplace(i, std::move(x));
            xq.push_back(i);
            return pump();
        }
        case OpKind::Compute: {
            auto kit = p->kernels.find(I.kernel);
            auto fit = p->functions.find(I.kernel);
            if (kit == p->kernels.end() && fit == p->functions.end())
                return set_error(PHX_E_SEGMENT, "kernel id %u not bound", I.kernel);
            std::vector<phx_tile_arg> targs;
            for (auto &a : I.args) {
                TileBuf *tb;
                if (int rc = tile_of(a.first, &tb)) return rc;
                phx_tile_arg ta;
                memset(&ta, 0, sizeof ta);
                ta.addr = tb->addr;
                ta.rank = (uint32_t)tb->shape.size();
                if (ta.rank < 1 || ta.rank > 3) return set_error(PHX_E_SEGMENT, "tile rank");
                for (uint32_t d = 0; d < ta.rank; ++d) ta.shape[d] = tb->shape[d];
                targs.push_back(ta);
            }
            // A caller-supplied kernel runs with the instruction's grid and
            // cta, as the reference launches every COMPUTE (engine.rs:632-647);
            // the built-in leaves take theirs from phx_grid_for.
            uint32_t grid[3] = {I.grid[0], I.grid[1], I.grid[2]};
            uint32_t block[3] = {I.cta[0], I.cta[1], I.cta[2]};
            int bits;
            hipFunction_t f;
            if (kit == p->kernels.end()) {
                f = fit->second.first;
                bits = fit->second.second;
            } else {
                const phx_kernel k = kit->second;
                kernel_abi(k, &bits, block);
                int64_t dims[4];
                int nd = 0;
                if ((k == PHX_MATMUL || k == PHX_GEMM_FP32) && targs.size() == 3) {
                    dims[0] = (int64_t)targs[0].shape[0];
                    dims[1] = (int64_t)targs[1].shape[1];
                    dims[2] = (int64_t)targs[0].shape[1];
                    nd = 3;
                } else if (k == PHX_MATMUL_INIT && targs.size() == 1 && targs[0].rank == 2) {
                    dims[0] = (int64_t)targs[0].shape[0];
                    dims[1] = (int64_t)targs[0].shape[1];
                    nd = 2;
                } else if (k == PHX_SAXPY_FP32 && targs.size() == 3) {
                    dims[0] = (int64_t)targs[0].shape[0];
                    nd = 1;
                }
                if (nd) {
                    if (int rc = grid_for(k, dims, nd, grid, block)) return rc;
                }
                if (int rc = builtin(k, &f)) return rc;
            }
            hipStream_t s = p->streams[p->next_stream];
            p->next_stream = (p->next_stream + 1) % p->streams.size();
            Inflight fl{Inflight::Kernel, i};
            // A built-in GEMM or flash leaf too small to fill the GPU runs
            // split; its partial results take an arena slab, as any tile
            // does (tile_store.rs:14-83), bound to the launch stream for this
            // one launch.  When the arena cannot hold it the leaf runs unsplit.
            size_t ws_bytes = 0;
            if (kit != p->kernels.end()) {
                const phx_kernel k = kit->second;
                int64_t dims[4];
                int nd = 0;
                const bool gemm = k == PHX_GEMM_FP32 || k == PHX_GEMM_FP16TC_FP32ACC ||
                                  k == PHX_GEMM_FP16;
                const bool flash = k == PHX_FLASH_FP32 || k == PHX_FLASH_FP16 ||
                                   k == PHX_FLASH_FP32_BH || k == PHX_FLASH_FP16_BH;
                if (gemm && targs.size() == 3 && targs[0].rank == 2 && targs[1].rank == 2) {
                    dims[0] = (int64_t)targs[0].shape[0];
                    dims[1] = (int64_t)targs[1].shape[1];
                    dims[2] = (int64_t)targs[0].shape[1];
                    nd = 3;
                } else if (flash && targs.size() == 4 && targs[0].rank == targs[1].rank &&
                           (targs[0].rank == 2 || targs[0].rank == 3)) {
                    const uint32_t r = targs[0].rank;
                    if (r == 3) dims[nd++] = (int64_t)targs[0].shape[0];
                    dims[nd++] = (int64_t)targs[0].shape[r - 2];
                    dims[nd++] = (int64_t)targs[1].shape[r - 2];
                    dims[nd++] = (int64_t)targs[0].shape[r - 1];
                }
                int sp = 1;
                // a shape the kernel does not take leaves ws_bytes 0, and the
                // launch below reports it
                if (nd && phx_split_plan(k, dims, nd, &sp, &ws_bytes) != PHX_OK) ws_bytes = 0;
                if (ws_bytes && phx_arena_can_alloc(p->arena, ws_bytes)) {
                    if (int rc = phx_arena_alloc(p->arena, ws_bytes, &fl.ws_addr, &fl.ws_cls))
                        return rc;
                    if (int rc = phx_stream_set_workspace((phx_stream)s, fl.ws_addr, ws_bytes)) {
                        phx_arena_free(p->arena, fl.ws_addr, fl.ws_cls);
                        return rc;
                    }
                }
            }
            // the slab goes back to the arena on any failure before the
            // launch is in flight
            auto drop_ws = [&]() {
                if (!fl.ws_addr) return;
                (void)phx_stream_set_workspace((phx_stream)s, 0, 0);
                phx_arena_free(p->arena, fl.ws_addr, fl.ws_cls);
                fl.ws_addr = 0;
            };
            hipError_t e;
            if ((e = hipEventCreate(&fl.start)) != hipSuccess) {
                drop_ws();
                return hip_error(e, "hipEventCreate");
            }
            if ((e = hipEventCreate(&fl.done)) != hipSuccess) {
                (void)hipEventDestroy(fl.start);
                drop_ws();
                return hip_error(e, "hipEventCreate");
            }
            if ((e = hipEventRecord(fl.start, s)) != hipSuccess) {
                (void)hipEventDestroy(fl.start);
                (void)hipEventDestroy(fl.done);
                drop_ws();
                return hip_error(e, "hipEventRecord");
            }
            const int crc = phx_compute((phx_function)f, bits, targs.data(),
                                        (uint32_t)targs.size(), I.scalars.data(),
                                        (uint32_t)I.scalars.size(), grid, block, (phx_stream)s);
            if (fl.ws_addr) (void)phx_stream_set_workspace((phx_stream)s, 0, 0);
            if (crc) {
                // a launch that failed to enqueue may still have enqueued its
                // first kernel (split launches are two), so the slab is only
                // released once the stream has drained
                (void)hipStreamSynchronize(s);
                (void)hipEventDestroy(fl.start);
                (void)hipEventDestroy(fl.done);
                if (fl.ws_addr) phx_arena_free(p->arena, fl.ws_addr, fl.ws_cls);
                return crc;
            }
            inflight.push_back(fl);  // the error drain destroys its events and slab from here on
            if ((e = hipEventRecord(fl.done, s)) != hipSuccess) return hip_error(e, "hipEventRecord");
            return PHX_OK;
        }
        }
        return PHX_OK;
    };

    while (completed < n && err == PHX_OK) {
        bool progress = false;
        // issue everything ready, in segment order
        while (!ready.empty() && err == PHX_OK) {
            size_t i = *ready.begin();
            ready.erase(ready.begin());
            err = issue(i);
            progress = true;
        }
        if (err) break;
        // chunks of queued transfers that staging buffers freed since
        if ((err = pump())) break;
        // file reads/writes that finished
        std::vector<IoDone> done;
        {
            std::lock_guard<std::mutex> l(io_mu);
            done.swap(io_done);
        }
        // every entry taken is accounted for before any is acted on, so an
        // error part-way through the batch still lets io_pending reach 0
        io_pending -= done.size();
        for (auto &d : done) {
            st[7] += d.ns;
            progress = true;
            if (err || !d.ok) {
                p->stage_free.push_back(d.staging);
                if (!err) err = set_error(PHX_E_IO, "%s", d.err.c_str());
                continue;
            }
            Xfer &x = xfers.at(d.idx);
            if (x.load) {  // chunk read from the file: copy it to the tile
                size_t a, len;
                chunk_range(x, d.chunk, &a, &len);
                Inflight f{Inflight::H2D, d.idx};
                f.chunk = d.chunk;
                f.staging = d.staging;
                inflight.push_back(f);
                Inflight &g = inflight.back();
                hipError_t e = hipMemcpyAsync((void *)(uintptr_t)(x.dev + a), d.staging, len,
                                              hipMemcpyHostToDevice, p->copy_stream);
                if (e == hipSuccess) e = hipEventCreateWithFlags(&g.done, hipEventDisableTiming);
                if (e == hipSuccess) e = hipEventRecord(g.done, p->copy_stream);
                if (e != hipSuccess) err = hip_error(e, "LOAD hipMemcpyAsync");
            } else {  // chunk written to the file
                chunk_landed(d.idx, d.staging);
            }
        }
        if (err) break;
        // device work that finished
        for (size_t j = 0; j < inflight.size();) {
            Inflight &f = inflight[j];
            if (!f.done) {
                ++j;
                continue;
            }
            hipError_t q = hipEventQuery(f.done);
            if (q == hipErrorNotReady) {
                ++j;
                continue;
            }
            if (q != hipSuccess) {
                err = hip_error(q, "event query");
                break;
            }
            progress = true;
            if (f.stage == Inflight::Kernel) {
                float a = 0, b = 0;
                if (origin.ev && hipEventElapsedTime(&a, origin.ev, f.start) == hipSuccess &&
                    hipEventElapsedTime(&b, origin.ev, f.done) == hipSuccess)
                    busy.push_back({a, b});
                else if (hipEventElapsedTime(&b, f.start, f.done) == hipSuccess)
                    st[5] += (uint64_t)(b * 1e6);  // no origin: the plain duration
                (void)hipEventDestroy(f.start);
                if (f.ws_addr) {  // the split's slab; a release may unpark allocations
                    phx_arena_free(p->arena, f.ws_addr, f.ws_cls);
                    for (size_t a : parked_alloc) ready.insert(a);
                    parked_alloc.clear();
                }
                st[2]++;
                complete(f.idx);
            } else if (f.stage == Inflight::H2D) {
                chunk_landed(f.idx, f.staging);
            } else {  // D2H landed: write the chunk to the file on the pool
                const Xfer *xp = &xfers.at(f.idx);
                const size_t idx = f.idx, c = f.chunk;
                void *h = f.staging;
                size_t a, len;
                chunk_range(*xp, c, &a, &len);
                io_pending++;
                p->io->submit([&, idx, c, h, a, len, xp]() {
                    const uint64_t s0 = now_ns();
                    IoDone d{idx, c, true, "", 0, h};
                    d.ok = chunk_io(*xp, true, (char *)h, a, len, &d.err);
                    d.ns = now_ns() - s0;
                    std::lock_guard<std::mutex> l(io_mu);
                    io_done.push_back(d);
                });
            }
            (void)hipEventDestroy(f.done);
            inflight.erase(inflight.begin() + (long)j);
        }
        if (err) break;
        if (!progress) {
            if (inflight.empty() && io_pending == 0 && ready.empty()) {
                if (!parked_alloc.empty()) {
                    err = set_error(PHX_E_EXHAUSTED,
                                    "device arena exhausted: %zu ALLOCs can never fit",
                                    parked_alloc.size());
                } else {
                    err = set_error(PHX_E_SEGMENT, "segment deadlocked (dependency cycle?)");
                }
                break;
            }
            std::this_thread::sleep_for(std::chrono::microseconds(20));
        }
    }
    // drain: never leave work in flight that references this call's state,
    // then hand back what the call took, so the pod can run a segment again
    if (err) {
        for (auto s : p->streams) (void)hipStreamSynchronize(s);
        (void)hipStreamSynchronize(p->copy_stream);
        (void)hipStreamSynchronize(p->store_stream);
        for (;;) {
            {
                std::lock_guard<std::mutex> l(io_mu);
                io_pending -= io_done.size();
                io_done.clear();
            }
            if (io_pending == 0) break;
            std::this_thread::sleep_for(std::chrono::microseconds(100));
        }
        for (auto &f : inflight) {
            if (f.start) (void)hipEventDestroy(f.start);
            if (f.done) (void)hipEventDestroy(f.done);
            if (f.ws_addr) phx_arena_free(p->arena, f.ws_addr, f.ws_cls);
        }
        p->stage_free = p->stage_all;  // nothing is in flight any more
        for (uint64_t id : allocated_here) {
            auto it = p->tiles.find(id);
            if (it == p->tiles.end()) continue;
            phx_arena_free(p->arena, it->second.addr, it->second.cls);
            p->tiles.erase(it);
        }
        return err;
    }
    std::sort(busy.begin(), busy.end());
    for (size_t a = 0; a < busy.size();) {  // union of the kernel intervals
        float lo = busy[a].first, hi = busy[a].second;
        size_t b = a + 1;
        for (; b < busy.size() && busy[b].first <= hi; ++b) hi = std::max(hi, busy[b].second);
        st[5] += (uint64_t)((double)(hi - lo) * 1e6);
        a = b;
    }
    st[6] = now_ns() - t0;
    if (stats) memcpy(stats, st, sizeof st);
    return PHX_OK;
}

}  // extern "C"
