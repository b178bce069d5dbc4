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
// cuMemcpy on the engine thread (tile_store.rs:153-181).  Here file I/O runs
// on a worker pool into pinned (hipHostMalloc) staging slabs, and the copy is
// a hipMemcpyAsync on a dedicated copy stream, so LOADs of later supertiles,
// STOREs of finished ones and COMPUTEs overlap.  Built-in leaf kernels get
// their grid from phx_grid_for (the reference's leaf grid would also be
// correct: every kernel strides over its work).
#include <fcntl.h>
#include <unistd.h>

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

// Fixed worker pool for file I/O.
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
    hipStream_t copy_stream = nullptr;
    size_t next_stream = 0;
    std::unordered_map<uint32_t, TensorInfo> tensors;
    std::unordered_map<uint32_t, phx_kernel> kernels;
    std::unordered_map<uint64_t, TileBuf> tiles;
    // pinned staging slabs, keyed by byte size
    std::multimap<size_t, void *> pinned_free;
    std::vector<void *> pinned_all;
    IoPool *io = nullptr;
};

namespace {

struct Inflight {
    enum Stage { H2D, D2H, Kernel } stage;
    size_t idx;  // instruction index
    hipEvent_t start = nullptr, done = nullptr;
    void *staging = nullptr;
    size_t staging_bytes = 0;
};

struct IoDone {
    size_t idx;
    bool ok;
    std::string err;
    uint64_t ns;
    void *staging;  // STORE: pinned slab to return once the file write is done
    size_t bytes;
};

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
                    } else {
                        return bad("scalar type is f32|i32|i64|f64");
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
        } else {
            return bad("unknown op");
        }
        out->push_back(std::move(I));
    }
    return PHX_OK;
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
    for (int i = 0; i <= nstreams; ++i) {
        hipStream_t s;
        hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
        if (e != hipSuccess) {
            phx_pod_destroy(p);
            return hip_error(e, "pod stream");
        }
        if (i == nstreams)
            p->copy_stream = s;
        else
            p->streams.push_back(s);
    }
    p->io = new IoPool(4);
    *out = p;
    return PHX_OK;
}

int phx_pod_destroy(phx_pod p) {
    if (!p) return PHX_OK;
    delete p->io;
    for (auto s : p->streams) (void)hipStreamDestroy(s);
    if (p->copy_stream) (void)hipStreamDestroy(p->copy_stream);
    for (void *h : p->pinned_all) (void)hipHostFree(h);
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
    p->kernels[kernel_id] = k;
    return PHX_OK;
}

int phx_pod_run_segment(phx_pod p, const char *text, uint64_t stats[8]) {
    if (!p) return set_error(PHX_E_INVALID, "null pod");
    std::vector<Instr> ins;
    if (int rc = parse_segment(text, &ins)) return rc;
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
    auto get_pinned = [&](size_t bytes) -> void * {
        auto it = p->pinned_free.find(bytes);
        if (it != p->pinned_free.end()) {
            void *h = it->second;
            p->pinned_free.erase(it);
            return h;
        }
        void *h = nullptr;
        if (hipHostMalloc(&h, bytes, hipHostMallocDefault) != hipSuccess) return nullptr;
        p->pinned_all.push_back(h);
        return h;
    };
    auto put_pinned = [&](void *h, size_t bytes) { p->pinned_free.insert({bytes, h}); };
    auto tile_of = [&](uint64_t id, TileBuf **out) -> int {
        auto it = p->tiles.find(id);
        if (it == p->tiles.end())
            return set_error(PHX_E_SEGMENT, "unknown tile 0x%llx", (unsigned long long)id);
        *out = &it->second;
        return PHX_OK;
    };
    auto region_ok = [&](const Instr &I, const TileBuf &tb, const TensorInfo &ti) -> int {
        uint64_t elems = 1;
        for (auto s : I.region.shape) elems *= s;
        if (elems != tb.elems)
            return set_error(PHX_E_SEGMENT, "region of %llu elements for a tile of %zu",
                             (unsigned long long)elems, tb.elems);
        if (I.region.shape.size() != ti.shape.size() && !(I.region.shape.size() == 1))
            return set_error(PHX_E_SEGMENT, "region rank != tensor rank");
        for (size_t d = 0; d < I.region.shape.size() && d < ti.shape.size(); ++d)
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
        case OpKind::Load: {
            TileBuf *tb;
            if (int rc = tile_of(I.tile, &tb)) return rc;
            auto tit = p->tensors.find(I.tensor);
            if (tit == p->tensors.end())
                return set_error(PHX_E_SEGMENT, "LOAD of unregistered tensor %u", I.tensor);
            if (int rc = region_ok(I, *tb, tit->second)) return rc;
            const size_t bytes = tb->elems * 4;
            void *h = get_pinned(bytes);
            if (!h) return set_error(PHX_E_IO, "pinned staging of %zu bytes failed", bytes);
            const TensorInfo ti = tit->second;
            const Region rg = I.region;
            io_pending++;
            p->io->submit([&, i, h, ti, rg]() {
                uint64_t s0 = now_ns();
                IoDone d{i, true, "", 0, nullptr, 0};
                std::vector<std::pair<uint64_t, size_t>> spans;
                int fd = open(ti.path.c_str(), O_RDONLY);
                if (fd < 0 || !byte_spans(ti.shape, rg, &spans)) {
                    d.ok = false;
                    d.err = "cannot open/read " + ti.path;
                } else {
                    char *dst = (char *)h;
                    for (auto &sp : spans) {
                        size_t want = sp.second * 4, got = 0;
                        while (got < want) {
                            ssize_t r = pread(fd, dst + got, want - got, (off_t)(sp.first + got));
                            if (r <= 0) break;
                            got += (size_t)r;
                        }
                        if (got != want) {
                            d.ok = false;
                            d.err = "short read from " + ti.path;
                            break;
                        }
                        dst += want;
                    }
                }
                if (fd >= 0) close(fd);
                d.ns = now_ns() - s0;
                std::lock_guard<std::mutex> l(io_mu);
                io_done.push_back(d);
            });
            Inflight f{Inflight::H2D, i};
            f.staging = h;
            f.staging_bytes = bytes;
            inflight.push_back(f);  // copy is enqueued once the read lands
            inflight.back().done = nullptr;
            return PHX_OK;
        }
        case OpKind::Store: {
            TileBuf *tb;
            if (int rc = tile_of(I.tile, &tb)) return rc;
            auto tit = p->tensors.find(I.tensor);
            if (tit == p->tensors.end())
                return set_error(PHX_E_SEGMENT, "STORE to unregistered tensor %u", I.tensor);
            if (int rc = region_ok(I, *tb, tit->second)) return rc;
            const size_t bytes = tb->elems * 4;
            void *h = get_pinned(bytes);
            if (!h) return set_error(PHX_E_IO, "pinned staging of %zu bytes failed", bytes);
            Inflight f{Inflight::D2H, i};
            f.staging = h;
            f.staging_bytes = bytes;
            hipError_t e = hipMemcpyAsync(h, (void *)(uintptr_t)tb->addr, bytes,
                                          hipMemcpyDeviceToHost, p->copy_stream);
            if (e != hipSuccess) return hip_error(e, "STORE hipMemcpyAsync");
            if ((e = hipEventCreateWithFlags(&f.done, hipEventDisableTiming)) != hipSuccess)
                return hip_error(e, "hipEventCreate");
            if ((e = hipEventRecord(f.done, p->copy_stream)) != hipSuccess)
                return hip_error(e, "hipEventRecord");
            inflight.push_back(f);
            return PHX_OK;
        }
        case OpKind::Compute: {
            auto kit = p->kernels.find(I.kernel);
            if (kit == p->kernels.end())
                return set_error(PHX_E_SEGMENT, "kernel id %u not bound", I.kernel);
            const phx_kernel k = kit->second;
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
            // grid from phx_grid_for for the built-in leaves
            uint32_t grid[3] = {I.grid[0], I.grid[1], I.grid[2]};
            uint32_t block[3];
            int bits;
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
            hipFunction_t f;
            if (int rc = builtin(k, &f)) return rc;
            hipStream_t s = p->streams[p->next_stream];
            p->next_stream = (p->next_stream + 1) % p->streams.size();
            Inflight fl{Inflight::Kernel, i};
            hipError_t e;
            if ((e = hipEventCreate(&fl.start)) != hipSuccess) return hip_error(e, "hipEventCreate");
            if ((e = hipEventCreate(&fl.done)) != hipSuccess) return hip_error(e, "hipEventCreate");
            if ((e = hipEventRecord(fl.start, s)) != hipSuccess) return hip_error(e, "hipEventRecord");
            if (int rc = phx_compute((phx_function)f, bits, targs.data(), (uint32_t)targs.size(),
                                     I.scalars.data(), (uint32_t)I.scalars.size(), grid, block,
                                     (phx_stream)s))
                return rc;
            if ((e = hipEventRecord(fl.done, s)) != hipSuccess) return hip_error(e, "hipEventRecord");
            inflight.push_back(fl);
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
        // file reads/writes that finished
        std::vector<IoDone> done;
        {
            std::lock_guard<std::mutex> l(io_mu);
            done.swap(io_done);
        }
        for (auto &d : done) {
            io_pending--;
            st[7] += d.ns;
            progress = true;
            if (!d.ok) {
                err = set_error(PHX_E_IO, "%s", d.err.c_str());
                break;
            }
            Instr &I = ins[d.idx];
            if (I.kind == OpKind::Load) {
                for (auto &f : inflight)
                    if (f.idx == d.idx && f.stage == Inflight::H2D && !f.done) {
                        TileBuf *tb;
                        if ((err = tile_of(I.tile, &tb))) break;
                        hipError_t e = hipMemcpyAsync((void *)(uintptr_t)tb->addr, f.staging,
                                                      f.staging_bytes, hipMemcpyHostToDevice,
                                                      p->copy_stream);
                        if (e == hipSuccess) e = hipEventCreateWithFlags(&f.done, hipEventDisableTiming);
                        if (e == hipSuccess) e = hipEventRecord(f.done, p->copy_stream);
                        if (e != hipSuccess) err = hip_error(e, "LOAD hipMemcpyAsync");
                        break;
                    }
            } else {  // STORE finished writing the file
                put_pinned(d.staging, d.bytes);
                st[3]++;
                complete(d.idx);
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
            Instr &I = ins[f.idx];
            if (f.stage == Inflight::Kernel) {
                float ms = 0;
                if (hipEventElapsedTime(&ms, f.start, f.done) == hipSuccess)
                    st[5] += (uint64_t)(ms * 1e6);
                (void)hipEventDestroy(f.start);
                st[2]++;
                complete(f.idx);
            } else if (f.stage == Inflight::H2D) {
                put_pinned(f.staging, f.staging_bytes);
                st[1]++;
                complete(f.idx);
            } else {  // D2H landed: write the file on the pool
                auto tit = p->tensors.find(I.tensor);
                const TensorInfo ti = tit->second;
                const Region rg = I.region;
                void *h = f.staging;
                size_t bytes = f.staging_bytes;
                size_t idx = f.idx;
                io_pending++;
                p->io->submit([&, idx, h, bytes, ti, rg]() {
                    uint64_t s0 = now_ns();
                    IoDone d{idx, true, "", 0, h, bytes};
                    std::vector<std::pair<uint64_t, size_t>> spans;
                    int fd = open(ti.path.c_str(), O_RDWR | O_CREAT, 0644);
                    if (fd < 0 || !byte_spans(ti.shape, rg, &spans)) {
                        d.ok = false;
                        d.err = "cannot open/write " + ti.path;
                    } else {
                        const char *src = (const char *)h;
                        for (auto &sp : spans) {
                            size_t want = sp.second * 4, put = 0;
                            while (put < want) {
                                ssize_t w = pwrite(fd, src + put, want - put, (off_t)(sp.first + put));
                                if (w <= 0) break;
                                put += (size_t)w;
                            }
                            if (put != want) {
                                d.ok = false;
                                d.err = "short write to " + ti.path;
                                break;
                            }
                            src += want;
                        }
                    }
                    if (fd >= 0) close(fd);
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
    // drain: never leave work in flight that references this call's state
    if (err) {
        for (auto s : p->streams) (void)hipStreamSynchronize(s);
        (void)hipStreamSynchronize(p->copy_stream);
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
        }
        return err;
    }
    st[6] = now_ns() - t0;
    if (stats) memcpy(stats, st, sizeof st);
    return PHX_OK;
}

}  // extern "C"
