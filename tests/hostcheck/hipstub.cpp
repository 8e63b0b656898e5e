// A recording stand-in for the HIP runtime, for checking the library's host
// bookkeeping on the CPU (no GPU, no kernels run).  Built with AddressSanitizer
// and linked, in place of libamdhip64, against host-only objects of the
// library (tests/hostcheck/Makefile); driven by tests/hostcheck/drive.py.
//
// "Device" memory is host memory from aligned_alloc that is never handed back
// while the process runs, so a freed buffer's address is never reused and any
// later use of it is seen.  Every kernel launch, eager or captured into a
// graph, is recorded with its pointer arguments (which arguments are pointers,
// and the sizes of by-value arguments, come from the kernel metadata of the
// real gfx950 build: kernel_args.tsv, made by kernel_args.py).  Streams carry a
// sequence number per operation and a "completed" mark that only host
// synchronisation (stream, event, device) advances, so work that may still be
// running is known.
//
// Violations (each printed to stderr when it happens and counted):
//   * launch of a destroyed graph exec; destroy of a destroyed exec/graph;
//   * a graph exec destroyed while its last launch may still be running;
//   * hipFree of a buffer that a live (not destroyed) graph exec references
//     (hipFree itself waits for the device, so eager work still running is
//     no hazard; a graph exec that is kept would use the freed buffer later);
//   * a kernel or graph launch whose pointer arguments lie in freed memory or
//     in no allocation, or an 8-byte aligned word of whose by-value
//     arguments lies in freed memory;
//   * memcpy/memset ranges outside their allocations;
//   * allocation, free, synchronisation or a second capture while a stream
//     is capturing; an event re-recorded while a host wait may still be
//     pending on it is counted (legal in HIP, reported as a statistic);
//   * unknown kernels, unknown streams, events or pointers.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <map>
#include <set>
#include <sstream>
#include <string>
#include <vector>

namespace {

struct Alloc {
    size_t size;
    bool alive;
    int kind;      // 0 device, 1 pinned host, 2 device symbol
    long id;
};

struct Arg {
    char kind;     // 'g' pointer, 'v' by value
    int size;
};

struct Node {
    std::string name;                 // kernel (mangled) or "memcpy"/"memset"
    std::vector<uintptr_t> ptrs;      // pointer arguments
    std::vector<uintptr_t> words;     // 8-byte words of by-value arguments
};

struct Graph {
    bool alive = true;
    std::vector<Node> nodes;
    long id = 0;
};

}  // namespace

struct ihipStream_t {
    bool alive = true;
    uint64_t seq = 0;     // operations enqueued
    uint64_t done = 0;    // operations known complete (host synchronised)
    Graph *cap = nullptr; // graph being captured
    long id = 0;
};
struct ihipEvent_t {
    bool alive = true;
    ihipStream_t *s = nullptr;
    uint64_t seq = 0;
    bool recorded = false;
};
struct ihipGraph {
    Graph g;
};
struct hipGraphExec {
    bool alive = true;
    std::vector<Node> nodes;
    ihipStream_t *last_s = nullptr;
    uint64_t last_seq = 0;
    long id = 0;
};

namespace {

std::map<uintptr_t, Alloc> g_allocs;            // base -> allocation
std::map<const void *, std::string> g_funcs;    // host stub -> device name
std::map<std::string, std::vector<Arg>> g_args; // device name -> explicit arguments
std::map<const void *, uintptr_t> g_vars;       // host shadow -> fake device memory
std::vector<hipGraphExec *> g_execs;
std::vector<ihipGraph *> g_graphs;
std::vector<ihipStream_t *> g_streams;
struct Pending {
    ihipStream_t *s;
    uint64_t seq;
    std::vector<uintptr_t> ptrs;
    std::string name;
};
std::vector<Pending> g_pending;                  // eager launches not known complete
long g_violations = 0, g_launches = 0, g_graph_launches = 0, g_captured = 0, g_allocs_n = 0,
     g_frees = 0, g_event_rerecord = 0, g_execs_made = 0, g_execs_destroyed = 0, g_suspect_words = 0;
long g_next_id = 1;
ihipStream_t g_null_stream;
bool g_table_loaded = false;
struct Config {
    dim3 grid, block;
    size_t shmem;
    hipStream_t stream;
};
std::vector<Config> g_cfg;

void violation(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    fprintf(stderr, "hipstub VIOLATION: ");
    vfprintf(stderr, fmt, ap);
    fprintf(stderr, "\n");
    fflush(stderr);
    va_end(ap);
    g_violations++;
}

ihipStream_t *S(hipStream_t s) { return s ? s : &g_null_stream; }

bool any_capturing() {
    for (auto *s : g_streams)
        if (s->alive && s->cap) return true;
    return false;
}

const Alloc *find(uintptr_t p, uintptr_t *base = nullptr) {
    auto it = g_allocs.upper_bound(p);
    if (it == g_allocs.begin()) return nullptr;
    --it;
    if (p >= it->first && p < it->first + std::max<size_t>(it->second.size, 1)) {
        if (base) *base = it->first;
        return &it->second;
    }
    return nullptr;
}

bool range_ok(const void *p, size_t n, const char *what) {
    if (n == 0) return true;
    uintptr_t base = 0;
    const Alloc *a = find((uintptr_t)p, &base);
    if (!a) { violation("%s: %p is in no allocation", what, p); return false; }
    if (!a->alive) { violation("%s: %p is in freed allocation #%ld", what, p, a->id); return false; }
    if ((uintptr_t)p + n > base + a->size) {
        violation("%s: %zu bytes at %p run past allocation #%ld (%zu bytes at %p)", what, n, p, a->id, a->size,
                  (void *)base);
        return false;
    }
    return true;
}

void load_table() {
    if (g_table_loaded) return;
    g_table_loaded = true;
    const char *path = getenv("HIPSTUB_KERNEL_ARGS");
    if (!path) { violation("HIPSTUB_KERNEL_ARGS is not set"); return; }
    std::ifstream f(path);
    if (!f) { violation("cannot read %s", path); return; }
    std::string line;
    while (std::getline(f, line)) {
        const size_t tab = line.find('\t');
        if (tab == std::string::npos) continue;
        std::vector<Arg> args;
        std::stringstream ss(line.substr(tab + 1));
        std::string tok;
        while (std::getline(ss, tok, ','))
            if (!tok.empty()) args.push_back(Arg{tok[0], atoi(tok.c_str() + 1)});
        g_args[line.substr(0, tab)] = args;
    }
}

// a recorded node's pointers must lie in live allocations (null is allowed);
// pointer-sized words of by-value arguments must not point into freed memory
void check_node(const Node &n, const char *where) {
    for (uintptr_t p : n.ptrs) {
        if (!p) continue;
        const Alloc *a = find(p);
        if (!a) violation("%s: %s: pointer %p is in no allocation", where, n.name.c_str(), (void *)p);
        else if (!a->alive)
            violation("%s: %s: pointer %p is in freed allocation #%ld", where, n.name.c_str(), (void *)p, a->id);
    }
    // By-value arguments are structs whose layout is not known here: a word
    // may be a pointer field, or a 4-byte field beside padding (stack bytes).
    // An 8-byte aligned word in freed memory is taken as a pointer field;
    // any other word that lands there is only counted and printed.
    for (uintptr_t w : n.words) {
        const Alloc *a = find(w);
        if (!a || a->alive) continue;
        if ((w & 7) == 0)
            violation("%s: %s: by-value word %p is in freed allocation #%ld", where, n.name.c_str(), (void *)w,
                      a->id);
        else if (g_suspect_words++ < 4)
            fprintf(stderr, "hipstub: %s: %s: unaligned by-value word %p in freed allocation #%ld "
                    "(a 4-byte field beside padding, most likely)\n", where, n.name.c_str(), (void *)w, a->id);
    }
}

// the node's pointer argument, or 8-byte aligned by-value word (taken as a
// pointer field, as in check_node), that lies in [base, base + size); 0 if none
uintptr_t node_uses(const Node &n, uintptr_t base, size_t size) {
    for (uintptr_t p : n.ptrs)
        if (p >= base && p < base + std::max<size_t>(size, 1)) return p;
    for (uintptr_t w : n.words)
        if ((w & 7) == 0 && w >= base && w < base + std::max<size_t>(size, 1)) return w;
    return 0;
}

void complete(ihipStream_t *s, uint64_t upto) {
    if (upto > s->done) s->done = upto;
    g_pending.erase(std::remove_if(g_pending.begin(), g_pending.end(),
                                   [&](const Pending &p) { return p.s == s && p.seq <= s->done; }),
                    g_pending.end());
}

void enqueue(ihipStream_t *s, const Node &n) {
    if (s->cap) {
        s->cap->nodes.push_back(n);
        g_captured++;
        return;
    }
    check_node(n, "eager launch");
    s->seq++;
    g_pending.push_back(Pending{s, s->seq, n.ptrs, n.name});
}

void *fake_alloc(size_t n, int kind) {
    const size_t sz = (std::max<size_t>(n, 1) + 255) & ~(size_t)255;
    void *p = aligned_alloc(256, sz);
    if (!p) return nullptr;
    memset(p, 0, sz);
    g_allocs[(uintptr_t)p] = Alloc{n, true, kind, g_next_id++};
    g_allocs_n++;
    return p;
}

hipError_t fake_free(void *p, int kind, const char *what) {
    if (!p) return hipSuccess;
    if (any_capturing()) violation("%s(%p) while a stream is capturing", what, p);
    auto it = g_allocs.find((uintptr_t)p);
    if (it == g_allocs.end() || it->second.kind != kind) {
        violation("%s(%p): not an allocation of this kind", what, p);
        return hipErrorInvalidValue;
    }
    if (!it->second.alive) {
        violation("%s(%p): allocation #%ld freed twice", what, p, it->second.id);
        return hipErrorInvalidValue;
    }
    for (auto *e : g_execs) {
        if (!e->alive) continue;
        for (const Node &n : e->nodes)
            if (const uintptr_t u = node_uses(n, it->first, it->second.size)) {
                violation("%s(%p): allocation #%ld (%zu bytes) is used by live graph exec #%ld (kernel %s, "
                          "argument %p)", what, p, it->second.id, it->second.size, e->id, n.name.c_str(), (void *)u);
                break;
            }
    }
    // hipFree waits for the device, so eager work in flight is not a hazard;
    // but a free inside a region the library believes unsynchronised is
    // worth knowing: count it as such only for exec launches in flight
    for (auto *e : g_execs) {
        if (!e->last_s || e->last_seq <= e->last_s->done) continue;
        for (const Node &n : e->nodes)
            if (node_uses(n, it->first, it->second.size)) {
                violation("%s(%p): allocation #%ld is used by graph exec #%ld whose last launch is not "
                          "synchronised", what, p, it->second.id, e->id);
                break;
            }
    }
    it->second.alive = false;   // the memory itself stays reserved: the address is never reused
    g_frees++;
    return hipSuccess;
}

}  // namespace

extern "C" {

// ---- registration (emitted by the compiler for every .hip translation unit)
void **__hipRegisterFatBinary(const void *data) {
    (void)data;
    static void *modules[4];
    return modules;
}
void __hipUnregisterFatBinary(void **modules) { (void)modules; }
void __hipRegisterFunction(void **modules, const void *hostFunction, char *deviceFunction, const char *deviceName,
                           unsigned int threadLimit, void *tid, void *bid, dim3 *blockDim, dim3 *gridDim,
                           int *wSize) {
    (void)modules; (void)deviceName; (void)threadLimit; (void)tid; (void)bid; (void)blockDim; (void)gridDim;
    (void)wSize;
    g_funcs[hostFunction] = deviceFunction;
}
void __hipRegisterVar(void **modules, void *var, char *hostVar, char *deviceVar, int ext, size_t size, int constant,
                      int global) {
    (void)modules; (void)hostVar; (void)deviceVar; (void)ext; (void)constant; (void)global;
    g_vars[var] = (uintptr_t)fake_alloc(size, 2);
}
hipError_t __hipPushCallConfiguration(dim3 gridDim, dim3 blockDim, size_t sharedMem, hipStream_t stream) {
    g_cfg.push_back(Config{gridDim, blockDim, sharedMem, stream});
    return hipSuccess;
}
hipError_t __hipPopCallConfiguration(dim3 *gridDim, dim3 *blockDim, size_t *sharedMem, hipStream_t *stream) {
    if (g_cfg.empty()) { violation("__hipPopCallConfiguration with nothing pushed"); return hipErrorInvalidValue; }
    const Config c = g_cfg.back();
    g_cfg.pop_back();
    *gridDim = c.grid;
    *blockDim = c.block;
    *sharedMem = c.shmem;
    *stream = c.stream;
    return hipSuccess;
}

hipError_t hipLaunchKernel(const void *function_address, dim3 numBlocks, dim3 dimBlocks, void **args,
                           size_t sharedMemBytes, hipStream_t stream) {
    (void)sharedMemBytes;
    load_table();
    ihipStream_t *s = S(stream);
    if (!s->alive) violation("launch on a destroyed stream");
    if ((size_t)numBlocks.x * numBlocks.y * numBlocks.z == 0 || (size_t)dimBlocks.x * dimBlocks.y * dimBlocks.z == 0)
        violation("launch with an empty grid or block");
    auto f = g_funcs.find(function_address);
    if (f == g_funcs.end()) {
        violation("launch of an unregistered function %p", function_address);
        return hipErrorInvalidDeviceFunction;
    }
    auto t = g_args.find(f->second);
    if (t == g_args.end()) {
        violation("kernel %s is not in the argument table", f->second.c_str());
        return hipErrorInvalidDeviceFunction;
    }
    Node n;
    n.name = f->second;
    for (size_t i = 0; i < t->second.size(); i++) {
        const Arg &a = t->second[i];
        if (a.kind == 'g') {
            n.ptrs.push_back(*(const uintptr_t *)args[i]);
        } else {
            for (int off = 0; off + 8 <= a.size; off += 8) {
                uintptr_t w;
                memcpy(&w, (const char *)args[i] + off, 8);
                n.words.push_back(w);
            }
        }
    }
    g_launches++;
    enqueue(s, n);
    return hipSuccess;
}

// ---- memory
hipError_t hipMalloc(void **p, size_t n) {
    if (any_capturing()) violation("hipMalloc(%zu) while a stream is capturing", n);
    *p = fake_alloc(n, 0);
    return *p ? hipSuccess : hipErrorOutOfMemory;
}
hipError_t hipFree(void *p) { return fake_free(p, 0, "hipFree"); }
hipError_t hipHostMalloc(void **p, size_t n, unsigned int flags) {
    (void)flags;
    if (any_capturing()) violation("hipHostMalloc(%zu) while a stream is capturing", n);
    *p = fake_alloc(n, 1);
    return *p ? hipSuccess : hipErrorOutOfMemory;
}
hipError_t hipHostFree(void *p) { return fake_free(p, 1, "hipHostFree"); }

static bool copy_ok(void *dst, const void *src, size_t n, hipMemcpyKind k, const char *what) {
    bool ok = true;
    if (k == hipMemcpyHostToDevice || k == hipMemcpyDeviceToDevice) ok &= range_ok(dst, n, what);
    if (k == hipMemcpyDeviceToHost || k == hipMemcpyDeviceToDevice) ok &= range_ok(src, n, what);
    return ok;
}
hipError_t hipMemcpy(void *dst, const void *src, size_t n, hipMemcpyKind k) {
    if (any_capturing()) violation("hipMemcpy while a stream is capturing");
    if (copy_ok(dst, src, n, k, "hipMemcpy")) memmove(dst, src, n);
    for (auto *s : g_streams) complete(s, s->seq);   // synchronous with the device
    complete(&g_null_stream, g_null_stream.seq);
    return hipSuccess;
}
hipError_t hipMemcpyAsync(void *dst, const void *src, size_t n, hipMemcpyKind k, hipStream_t stream) {
    ihipStream_t *s = S(stream);
    if (!copy_ok(dst, src, n, k, "hipMemcpyAsync")) return hipErrorInvalidValue;
    Node nd;
    nd.name = "memcpy";
    if (k != hipMemcpyHostToDevice) nd.ptrs.push_back((uintptr_t)src);
    if (k != hipMemcpyDeviceToHost) nd.ptrs.push_back((uintptr_t)dst);
    if (!s->cap) memmove(dst, src, n);
    enqueue(s, nd);
    return hipSuccess;
}
hipError_t hipMemset(void *p, int v, size_t n) {
    if (any_capturing()) violation("hipMemset while a stream is capturing");
    if (range_ok(p, n, "hipMemset")) memset(p, v, n);
    return hipSuccess;
}

// ---- device
hipError_t hipGetDeviceCount(int *n) { *n = 1; return hipSuccess; }
hipError_t hipSetDevice(int d) { return d == 0 ? hipSuccess : hipErrorInvalidDevice; }
hipError_t hipGetDevice(int *d) { *d = 0; return hipSuccess; }
hipError_t hipGetDevicePropertiesR0600(hipDeviceProp_t *p, int d) {
    if (d != 0) return hipErrorInvalidDevice;
    memset(p, 0, sizeof *p);
    strcpy(p->name, "hipstub");
    strcpy(p->gcnArchName, "gfx950:sramecc+:xnack-");
    p->multiProcessorCount = 256;
    p->totalGlobalMem = (size_t)288 << 30;
    p->sharedMemPerBlock = 65536;
    p->maxSharedMemoryPerMultiProcessor = 160 * 1024;
    p->warpSize = 64;
    p->maxThreadsPerBlock = 1024;
    p->l2CacheSize = 4 << 20;
    return hipSuccess;
}
hipError_t hipDeviceGetAttribute(int *v, hipDeviceAttribute_t attr, int d) {
    (void)d;
    *v = attr == hipDeviceAttributeMultiprocessorCount ? 256 : 0;
    return hipSuccess;
}
hipError_t hipFuncSetAttribute(const void *f, hipFuncAttribute attr, int value) {
    (void)attr; (void)value;
    if (!g_funcs.count(f)) violation("hipFuncSetAttribute on an unregistered function");
    return hipSuccess;
}
hipError_t hipOccupancyMaxActiveBlocksPerMultiprocessor(int *n, const void *f, int blockSize, size_t dyn) {
    (void)blockSize; (void)dyn;
    if (!g_funcs.count(f)) violation("occupancy query on an unregistered function");
    *n = 1;
    return hipSuccess;
}
hipError_t hipGetLastError(void) { return hipSuccess; }
const char *hipGetErrorString(hipError_t e) { return e == hipSuccess ? "no error" : "hipstub error"; }
hipError_t hipGetSymbolAddress(void **p, const void *sym) {
    auto it = g_vars.find(sym);
    if (it == g_vars.end()) { violation("hipGetSymbolAddress of an unregistered symbol"); return hipErrorInvalidSymbol; }
    *p = (void *)it->second;
    return hipSuccess;
}
hipError_t hipDeviceSynchronize(void) {
    if (any_capturing()) violation("hipDeviceSynchronize while a stream is capturing");
    for (auto *s : g_streams) complete(s, s->seq);
    complete(&g_null_stream, g_null_stream.seq);
    return hipSuccess;
}

// ---- streams and events
hipError_t hipStreamCreateWithFlags(hipStream_t *s, unsigned int flags) {
    (void)flags;
    auto *st = new ihipStream_t;
    st->id = g_next_id++;
    g_streams.push_back(st);
    *s = st;
    return hipSuccess;
}
hipError_t hipStreamDestroy(hipStream_t stream) {
    ihipStream_t *s = S(stream);
    if (!s->alive) { violation("stream destroyed twice"); return hipErrorInvalidHandle; }
    if (s->cap) violation("stream destroyed while capturing");
    s->alive = false;
    return hipSuccess;
}
hipError_t hipStreamSynchronize(hipStream_t stream) {
    ihipStream_t *s = S(stream);
    if (!s->alive) violation("synchronise of a destroyed stream");
    if (s->cap) { violation("hipStreamSynchronize while the stream is capturing"); return hipErrorStreamCaptureUnsupported; }
    complete(s, s->seq);
    return hipSuccess;
}
hipError_t hipEventCreate(hipEvent_t *e) {
    *e = new ihipEvent_t;
    return hipSuccess;
}
hipError_t hipEventDestroy(hipEvent_t e) {
    if (!e->alive) { violation("event destroyed twice"); return hipErrorInvalidHandle; }
    e->alive = false;
    return hipSuccess;
}
hipError_t hipEventRecord(hipEvent_t e, hipStream_t stream) {
    ihipStream_t *s = S(stream);
    if (!e->alive) { violation("record of a destroyed event"); return hipErrorInvalidHandle; }
    if (s->cap) violation("event recorded into a capturing stream");
    if (e->recorded && e->s && e->seq > e->s->done) g_event_rerecord++;
    s->seq++;
    e->s = s;
    e->seq = s->seq;
    e->recorded = true;
    return hipSuccess;
}
hipError_t hipEventSynchronize(hipEvent_t e) {
    if (!e->alive || !e->recorded) { violation("synchronise of a destroyed or unrecorded event"); return hipErrorInvalidHandle; }
    complete(e->s, e->seq);
    return hipSuccess;
}
hipError_t hipEventElapsedTime(float *ms, hipEvent_t a, hipEvent_t b) {
    if (!a->alive || !b->alive || !a->recorded || !b->recorded) {
        violation("elapsed time of a destroyed or unrecorded event");
        return hipErrorInvalidHandle;
    }
    if (b->seq > b->s->done || a->seq > a->s->done) violation("elapsed time of an event not yet waited for");
    const uint64_t d = b->seq > a->seq ? b->seq - a->seq : 1;
    *ms = 0.001f * (float)d;   // any positive figure: nothing runs
    return hipSuccess;
}

// ---- capture and graphs
hipError_t hipStreamBeginCapture(hipStream_t stream, hipStreamCaptureMode mode) {
    (void)mode;
    ihipStream_t *s = S(stream);
    if (s->cap) { violation("capture begun twice on one stream"); return hipErrorIllegalState; }
    auto *g = new ihipGraph;
    g->g.id = g_next_id++;
    s->cap = &g->g;
    g_graphs.push_back(g);
    return hipSuccess;
}
hipError_t hipStreamEndCapture(hipStream_t stream, hipGraph_t *graph) {
    ihipStream_t *s = S(stream);
    if (!s->cap) { violation("end of a capture that was not begun"); return hipErrorIllegalState; }
    for (auto *g : g_graphs)
        if (&g->g == s->cap) *graph = g;
    s->cap = nullptr;
    return hipSuccess;
}
hipError_t hipGraphInstantiate(hipGraphExec_t *exec, hipGraph_t graph, hipGraphNode_t *err, char *log, size_t n) {
    (void)err; (void)log; (void)n;
    if (!graph->g.alive) { violation("instantiate of a destroyed graph"); return hipErrorInvalidValue; }
    auto *e = new hipGraphExec;
    e->nodes = graph->g.nodes;
    e->id = g_next_id++;
    for (const Node &nd : e->nodes) check_node(nd, "instantiate");
    g_execs.push_back(e);
    g_execs_made++;
    *exec = e;
    return hipSuccess;
}
hipError_t hipGraphDestroy(hipGraph_t graph) {
    if (!graph->g.alive) { violation("graph destroyed twice"); return hipErrorInvalidValue; }
    graph->g.alive = false;
    return hipSuccess;
}
hipError_t hipGraphExecDestroy(hipGraphExec_t e) {
    if (!e->alive) { violation("graph exec #%ld destroyed twice", e->id); return hipErrorInvalidValue; }
    if (e->last_s && e->last_seq > e->last_s->done)
        violation("graph exec #%ld destroyed while its last launch may still run (stream not synchronised)", e->id);
    e->alive = false;
    g_execs_destroyed++;
    return hipSuccess;
}
hipError_t hipGraphLaunch(hipGraphExec_t e, hipStream_t stream) {
    ihipStream_t *s = S(stream);
    if (!e->alive) { violation("launch of destroyed graph exec #%ld", e->id); return hipErrorInvalidValue; }
    if (!s->alive) violation("graph launch on a destroyed stream");
    if (s->cap) violation("graph launched into a capturing stream");
    for (const Node &n : e->nodes) check_node(n, "graph launch");
    s->seq++;
    e->last_s = s;
    e->last_seq = s->seq;
    g_graph_launches++;
    return hipSuccess;
}

// ---- report
int hipstub_violations(void) { return (int)g_violations; }
void hipstub_report(void) {
    long live_execs = 0, live_dev = 0;
    size_t live_bytes = 0;
    for (auto *e : g_execs) live_execs += e->alive;
    for (auto &kv : g_allocs)
        if (kv.second.alive && kv.second.kind == 0) { live_dev++; live_bytes += kv.second.size; }
    fprintf(stderr,
            "hipstub: %ld kernel launches (%ld recorded into graphs), %ld graph launches, %ld execs made, "
            "%ld destroyed, %ld live; %ld allocations, %ld frees, %ld live device buffers (%.1f MB); "
            "%ld events re-recorded before a wait; %ld unaligned by-value words in freed memory; %ld violations\n",
            g_launches, g_captured, g_graph_launches, g_execs_made, g_execs_destroyed, live_execs, g_allocs_n, g_frees,
            live_dev, live_bytes / 1e6, g_event_rerecord, g_suspect_words, g_violations);
    fflush(stderr);
}

}  // extern "C"
