// Schedule executor behind kr_plan_run: the MI355X counterpart of the
// reference's nhp_exec (exec/exec_main.cpp:1325-1494).
//
// A schedule.json lists nodes (op, rows/cols/k/n, tiles) and, per engine
// stream, the ordered (node, tile) tasks with their cross-stream waits and
// publish marks plus explicit row geometry (in_row_off, in_rows,
// out_row_off). Engines map onto two HIP streams: "aic" (matrix work) on the
// producer stream, "aiv" (vector work) on the consumer stream; a schedule
// that also holds MIX ("aicore") tasks is merged into one stream in global
// topological order, as the reference does (NormalizeTopology,
// exec_main.cpp:243-341).
//
// Cross-stream dependencies are device flags by default (KR_SYNC=flag):
// a publishing task releases its tile from its own epilogue, and a waiting
// task either spins in its own prologue (row/elementwise consumers, one
// producer node, contiguous tiles) or behind a one-workgroup wait kernel.
// KR_SYNC=event uses hipEvents instead (the reference's default,
// exec_main.cpp:700-723).
//
// Inputs follow the reference convention (DetValue/NodeSeed, seeds +1 input,
// +2 weight, +3 second operand: exec_main.cpp:498-540) unless a node names
// input files ("inputs": {"in","b","x1","gamma"}). The checksum is the
// reference's: sum over ranks and nodes of the first 8192 16-bit outputs
// (exec_main.cpp:1292-1311).
#include <algorithm>
#include <cstdio>
#include <deque>
#include <fstream>
#include <map>
#include <memory>
#include <numeric>
#include <set>
#include <tuple>
#include <sstream>

#include "kr_gemm.h"
#include "kr_json.h"
#include "kr_misc.h"
#include "kr_rowops.h"
#include "kr_runtime.h"

namespace kr {
namespace plan {

using json::Value;

enum class Op { MatMul, Gelu, Softmax, Cast, Add, Silu, Mul, Swiglu, RmsNorm, AddRmsNorm, LayerNorm };

Op ParseOp(const std::string &s)
{
    if (s == "matmul") return Op::MatMul;
    if (s == "gelu") return Op::Gelu;
    if (s == "softmax") return Op::Softmax;
    if (s == "cast") return Op::Cast;
    if (s == "add") return Op::Add;
    if (s == "silu") return Op::Silu;
    if (s == "mul") return Op::Mul;
    if (s == "swiglu") return Op::Swiglu;
    if (s == "rmsnorm") return Op::RmsNorm;
    if (s == "add_rmsnorm") return Op::AddRmsNorm;
    if (s == "layernorm") return Op::LayerNorm;
    throw std::runtime_error("op '" + s + "' is not built on this target "
                             "(supported: matmul gelu softmax cast add silu mul swiglu rmsnorm add_rmsnorm layernorm)");
}

int ParseDType(const std::string &s)
{
    if (s.empty() || s == "fp16" || s == "float16" || s == "f16") return kF16;
    if (s == "bf16" || s == "bfloat16") return kBF16;
    if (s == "fp32" || s == "float32" || s == "f32") return kF32;
    throw std::runtime_error("unknown dtype '" + s + "'");
}

bool IsBinary(Op op) { return op == Op::Add || op == Op::Mul || op == Op::Swiglu || op == Op::AddRmsNorm; }

struct NodeSpec {
    std::string id;
    Op op = Op::Add;
    std::string opname;
    std::string engine;
    int dtype = kF16;
    int out_dtype = kF16;
    int64_t rows = 0, cols = 0, k = 0, n = 0;
    int tiles = 1;
    bool split = false;
    float eps = 1e-6f;
    std::vector<std::string> preds;
    std::map<std::string, std::string> inputs;
};

struct TaskSpec {
    std::string node;
    int tile = 0;
    std::vector<std::pair<std::string, int>> waits;
    bool publish = false;
    bool has_geom = false;
    int64_t in_row_off = 0, in_rows = 0, out_row_off = 0;
    int64_t n_off = 0, n_tile = 0;
};

struct Lane {
    std::string engine;
    std::vector<TaskSpec> tasks;
};

struct SchedDoc {
    std::string dag, group;
    int nranks = 1;
    std::vector<NodeSpec> nodes;
    std::map<std::string, size_t> index;
    std::vector<Lane> lanes;  // in engine order

    const NodeSpec &Node(const std::string &id) const
    {
        auto it = index.find(id);
        if (it == index.end()) throw std::runtime_error("missing plan for task: unknown node " + id);
        return nodes[it->second];
    }
};

int EngineRank(const std::string &e)
{
    if (e == "aicore" || e == "compute") return 0;
    if (e == "aic") return 1;
    if (e == "aiv") return 2;
    if (e == "aicpu") return 3;
    if (e == "hccl") return 4;
    throw std::runtime_error("unknown engine " + e);
}

SchedDoc ParseSchedule(const Value &root)
{
    SchedDoc doc;
    doc.dag = root.Str("dag");
    doc.group = root.Str("group");
    doc.nranks = std::max(1, int(root.Num("nranks", 1)));
    for (const auto &n : root.At("nodes").Items()) {
        NodeSpec s;
        s.id = n.Str("id");
        s.opname = n.Str("op");
        s.op = ParseOp(s.opname);
        s.engine = n.Str("engine", "aiv");
        s.dtype = ParseDType(n.Str("dtype", "fp16"));
        if (s.dtype == kF32) throw std::runtime_error("node " + s.id + ": fp32 inputs are not supported");
        s.rows = int64_t(n.Num("rows"));
        s.cols = int64_t(n.Num("cols"));
        s.k = int64_t(n.Num("k"));
        s.n = int64_t(n.Num("n"));
        s.tiles = std::max(1, int(n.Num("tiles", 1)));
        s.split = n.Flag("split", false);
        // aclnnLayerNorm runs with eps 1e-5 in the reference (op_impl.cpp:248)
        s.eps = float(n.Num("eps", s.op == Op::LayerNorm ? 1e-5 : 1e-6));
        if (n.Has("preds"))
            for (const auto &p : n.At("preds").Items()) s.preds.push_back(p.AsString());
        if (n.Has("inputs"))
            for (const auto &kv : n.At("inputs").Members()) s.inputs[kv.first] = kv.second.AsString();
        if (s.op == Op::Cast) {
            const std::string to = n.Str("to", "");
            s.out_dtype = !to.empty() ? ParseDType(to) : (s.dtype == kF16 ? kF32 : kF16);
        } else {
            s.out_dtype = s.dtype;
        }
        if (s.rows <= 0 || s.cols <= 0) throw std::runtime_error("node " + s.id + ": rows/cols must be > 0");
        if (s.op == Op::MatMul && (s.k <= 0 || s.n <= 0 || s.n != s.cols))
            throw std::runtime_error("node " + s.id + ": matmul needs k > 0 and n == cols");
        if (doc.index.count(s.id)) throw std::runtime_error("duplicate node id " + s.id);
        doc.index[s.id] = doc.nodes.size();
        doc.nodes.push_back(s);
    }
    std::map<std::string, Lane> by_engine;
    for (const auto &kv : root.At("streams").Members()) {
        const std::string name = kv.first == "compute" ? "aicore" : kv.first;
        (void)EngineRank(name);
        if (by_engine.count(name)) throw std::runtime_error("duplicate engine stream " + name);
        Lane lane;
        lane.engine = name;
        for (const auto &t : kv.second.Items()) {
            TaskSpec task;
            task.node = t.Str("node");
            task.tile = int(t.Num("tile", 0));
            task.publish = t.Flag("publish", false);
            if (t.Has("wait"))
                for (const auto &w : t.At("wait").Items())
                    task.waits.emplace_back(w.At(size_t(0)).AsString(), int(w.At(size_t(1)).AsNumber()));
            if (t.Has("in_row_off") && t.Has("in_rows")) {
                task.has_geom = true;
                task.in_row_off = int64_t(t.Num("in_row_off"));
                task.in_rows = int64_t(t.Num("in_rows"));
                task.out_row_off = t.Has("out_row_off") ? int64_t(t.Num("out_row_off")) : task.in_row_off;
                task.n_off = int64_t(t.Num("n_off", 0));
                task.n_tile = int64_t(t.Num("n_tiles", 0));
            }
            lane.tasks.push_back(task);
        }
        by_engine[name] = std::move(lane);
    }
    for (auto &kv : by_engine) doc.lanes.push_back(std::move(kv.second));
    std::sort(doc.lanes.begin(), doc.lanes.end(),
              [](const Lane &a, const Lane &b) { return EngineRank(a.engine) < EngineRank(b.engine); });
    return doc;
}

using Key = std::pair<std::string, int>;

// Global topological order over all tasks (hard edges: same-lane FIFO and
// every wait); ties broken by (engine rank, lane position).
std::vector<std::pair<size_t, size_t>> TopoOrder(const SchedDoc &doc)
{
    std::map<Key, std::pair<size_t, size_t>> pos;
    std::vector<std::pair<size_t, size_t>> keys;
    for (size_t l = 0; l < doc.lanes.size(); ++l)
        for (size_t i = 0; i < doc.lanes[l].tasks.size(); ++i) {
            const auto &t = doc.lanes[l].tasks[i];
            const Key k{t.node, t.tile};
            if (pos.count(k)) throw std::runtime_error("duplicate task for node " + t.node + " tile " + std::to_string(t.tile));
            pos[k] = {l, i};
            keys.emplace_back(l, i);
        }
    std::map<std::pair<size_t, size_t>, std::set<std::pair<size_t, size_t>>> deps;
    for (const auto &key : keys) {
        std::set<std::pair<size_t, size_t>> d;
        if (key.second > 0) d.insert({key.first, key.second - 1});
        for (const auto &w : doc.lanes[key.first].tasks[key.second].waits) {
            auto it = pos.find(w);
            if (it == pos.end()) throw std::runtime_error("wait on unpublished flag " + w.first + "#" + std::to_string(w.second));
            if (it->second != key) d.insert(it->second);
        }
        deps[key] = std::move(d);
    }
    auto rank = [&](const std::pair<size_t, size_t> &k) {
        return std::make_pair(EngineRank(doc.lanes[k.first].engine), k.second);
    };
    std::vector<std::pair<size_t, size_t>> order, ready;
    for (const auto &k : keys)
        if (deps[k].empty()) ready.push_back(k);
    std::set<std::pair<size_t, size_t>> done;
    while (!ready.empty()) {
        auto it = std::min_element(ready.begin(), ready.end(), [&](const auto &a, const auto &b) { return rank(a) < rank(b); });
        const auto cur = *it;
        ready.erase(it);
        order.push_back(cur);
        done.insert(cur);
        for (auto &kv : deps) {
            if (done.count(kv.first) || !kv.second.count(cur)) continue;
            kv.second.erase(cur);
            if (kv.second.empty()) ready.push_back(kv.first);
        }
    }
    if (order.size() != keys.size()) throw std::runtime_error("schedule contains wait cycle");
    return order;
}

// MIX (aicore) tasks may not overlap pure aic/aiv work: merge those lanes into
// one in global topological order (exec_main.cpp:243-341).
void NormalizeTopology(SchedDoc &doc)
{
    auto order = TopoOrder(doc);
    bool has_mix = false, has_pure = false;
    for (const auto &l : doc.lanes) {
        if (l.tasks.empty()) continue;
        if (l.engine == "aicore") has_mix = true;
        if (l.engine == "aic" || l.engine == "aiv") has_pure = true;
    }
    for (const auto &l : doc.lanes)
        if (!l.tasks.empty() && (l.engine == "aicpu" || l.engine == "hccl"))
            throw std::runtime_error("engine " + l.engine + " has no executor on this target");
    if (!(has_mix && has_pure)) {
        std::vector<Lane> keep;
        for (auto &l : doc.lanes)
            if (!l.tasks.empty()) keep.push_back(std::move(l));
        doc.lanes = std::move(keep);
        return;
    }
    Lane merged;
    merged.engine = "aicore";
    for (const auto &k : order) merged.tasks.push_back(doc.lanes[k.first].tasks[k.second]);
    doc.lanes.clear();
    doc.lanes.push_back(std::move(merged));
}

// ------------------------------------------------------------------ runtime
struct NodeBuf {
    DevBuf out, bt, own_in, aux, gamma, sum, beta;
    size_t out_bytes = 0;
};

struct Launch {
    int lane = 0;
    const TaskSpec *task = nullptr;
    const NodeSpec *node = nullptr;
    // relay wiring
    bool fused_wait = false;
    RelayWait wait{};
    int tile_rows = 0;
    std::vector<RelayWait> extra_waits;  // standalone one-workgroup waits
    bool publish = false;
    int flag = -1;
    hipEvent_t pub_event = nullptr;
    std::vector<hipEvent_t> wait_events;
    // coalescing: rows per released tile, tasks merged, fused consumer nodes
    // (fan[0] == node) and each one's state base
    int64_t pub_rows = 0;
    int merged = 1;
    bool coresident = false;
    std::vector<const NodeSpec *> fan;
    std::vector<int32_t> fan_states;
    // persistent-consumer tiles (those released before the producer GEMM's
    // last round of workgroups); -1 = every tile waits in-kernel
    int early_tiles = -1;
    // in-register relay (KR_PLAN_EPILOGUE=1): this consumer launch runs in
    // its producer GEMM's epilogue (skip), or this GEMM launch writes that
    // consumer's output beside C (epi)
    bool skip = false;
    const NodeSpec *epi = nullptr;
};

struct RankCtx {
    int rank = 0;
    std::map<std::string, NodeBuf> bufs;
};

class Executor {
public:
    Executor(SchedDoc doc, int device, std::string mode)
        : doc_(std::move(doc)), device_(device), mode_(std::move(mode))
    {
        sync_ = EnvStr("KR_SYNC", "flag");
        if (sync_ != "flag" && sync_ != "event") throw std::runtime_error("KR_SYNC must be flag or event");
        wait_kind_ = EnvStr("KR_RELAY_WAIT", "fused");
        relay_grid_ = EnvInt("KR_RELAY_GRID", 256);
        partition_ = std::max(0, EnvInt("KR_PLAN_PARTITION", 0));
        fan_max_ = EnvInt("KR_PLAN_FAN", kMaxFanOut);
        max_spins_ = uint32_t(EnvInt("KR_MAX_SPINS", int(kDefaultMaxSpins)));
        if (mode_ != "direct" && mode_ != "graph" && mode_ != "graph_per_stream" && mode_ != "graph_segment")
            throw std::runtime_error("mode '" + mode_ +
                                     "' is not built (direct, graph, graph_per_stream, graph_segment)");
        // graph_segment joins its graphs with events (the segments' waits and
        // publishes), whatever KR_SYNC says
        if (mode_ == "graph_segment") sync_ = "event";
        // a CU partition needs the two lanes on their own queues at launch
        // time; one multi-stream graph may run every node on one queue
        if (mode_ == "graph" || sync_ != "flag") partition_ = 0;
    }

    ~Executor()
    {
        for (auto &g : graphs_) {
            if (g.exec) (void)hipGraphExecDestroy(g.exec);
            if (g.graph) (void)hipGraphDestroy(g.graph);
        }
        for (auto &g : segments_) {
            if (g.exec) (void)hipGraphExecDestroy(g.exec);
            if (g.graph) (void)hipGraphDestroy(g.graph);
        }
        for (auto &L : launches_) {
            if (L.pub_event) (void)hipEventDestroy(L.pub_event);
        }
        if (ev0_) (void)hipEventDestroy(ev0_);
        if (ev1_) (void)hipEventDestroy(ev1_);
        if (ev2_) (void)hipEventDestroy(ev2_);
        if (ev3_) (void)hipEventDestroy(ev3_);
        streams_.Destroy();
    }

    // Host-only checks: every rejection happens before the device is touched.
    void Validate() { ValidateGeometry(); }

    void Prepare()
    {
        ValidateGeometry();
        Check(hipSetDevice(device_), "hipSetDevice");
        Check(hipDeviceGetAttribute(&ncu_, hipDeviceAttributeMultiprocessorCount, device_), "CU count");
        // a persistent consumer beside a GEMM: at most one workgroup per CU
        relay_grid_ = std::max(1, std::min(relay_grid_, ncu_));
        // KR_PLAN_PARTITION = n: lane 1 (the vector engine's lane) owns n CUs
        // of every XCD and lane 0 the rest, as the reference's vector and
        // cube cores are separate; the consumer grid is one workgroup per
        // lane-1 CU
        partition_ = std::min(partition_, ncu_ / 16);
        streams_.Create(device_, partition_);
        // there the lane-1 CUs are the consumer's alone: eight workgroups per
        // CU keep enough loads in flight for a memory-bound pass on a few CUs
        if (partition_ > 0) relay_grid_ = std::max(1, EnvInt("KR_RELAY_GRID", streams_.cons_cus * 8));
        Check(hipEventCreate(&ev0_), "event");
        Check(hipEventCreate(&ev1_), "event");
        Check(hipEventCreate(&ev2_), "event");
        Check(hipEventCreate(&ev3_), "event");
        ranks_.resize(doc_.nranks);
        for (int r = 0; r < doc_.nranks; ++r) {
            ranks_[r].rank = r;
            for (const auto &n : doc_.nodes) Allocate(ranks_[r], n);
            Upload(ranks_[r]);
        }
        Wire();
        Check(hipDeviceSynchronize(), "prepare sync");
        if (mode_ != "direct") Capture();
    }

    // One execution of every rank's program; returns the makespan (max over
    // ranks, ranks run back to back on the one device) in microseconds.
    double RunOnce(double *dev_us)
    {
        double makespan = 0.0, dev = 0.0;
        for (int r = 0; r < doc_.nranks; ++r) {
            Check(hipDeviceSynchronize(), "pre-run sync");
            const auto t0 = Clock::now();
            // each stream that runs work records its own start: the device
            // makespan runs from the earlier start to the later end, with no
            // cross-stream event wait of its own in the timed region
            const bool one_graph = sync_ == "event" && (mode_ == "graph" || mode_ == "graph_per_stream");
            const bool two = lanes_used_[1] && !one_graph;
            Check(hipEventRecord(ev0_, streams_.prod), "record start");
            if (two) Check(hipEventRecord(ev3_, streams_.cons), "record start cons");
            if (mode_ == "direct") {
                EnqueueRank(r);
            } else if (mode_ == "graph_segment") {
                RunSegments(r);
            } else {
                for (auto &g : graphs_)
                    if (g.rank == r) Check(hipGraphLaunch(g.exec, g.lane == 0 ? streams_.prod : streams_.cons), "graph launch");
            }
            Check(hipEventRecord(ev1_, streams_.prod), "record end prod");
            if (two) Check(hipEventRecord(ev2_, streams_.cons), "record end cons");
            Check(hipStreamSynchronize(streams_.prod), "sync prod");
            Check(hipStreamSynchronize(streams_.cons), "sync cons");
            const auto t1 = Clock::now();
            float a = 0.f, b = 0.f, c = 0.f;
            Check(hipEventElapsedTime(&a, ev0_, ev1_), "elapsed");
            if (two) {
                Check(hipEventElapsedTime(&b, ev0_, ev2_), "elapsed");
                Check(hipEventElapsedTime(&c, ev0_, ev3_), "elapsed");
            }
            makespan = std::max(makespan, Us(t0, t1));
            dev = std::max(dev, 1000.0 * (std::max(a, b) - std::min(0.f, c)));
        }
        if (dev_us) *dev_us = dev;
        return makespan;
    }

    int FlagTimeouts()
    {
        if (ctrl_words_ == 0) return 0;
        std::vector<int32_t> host(ctrl_words_);
        Check(hipMemcpy(host.data(), ctrl_.get(), ctrl_words_ * 4, hipMemcpyDeviceToHost), "ctrl d2h");
        int bad = 0;
        for (int s : consumed_states_)
            if (host[size_t(s) * kWords + kOffStatus] != 1) ++bad;
        return bad;
    }

    double Checksum()
    {
        double sum = 0.0;
        for (auto &rc : ranks_)
            for (const auto &n : doc_.nodes) {
                const NodeBuf &b = rc.bufs.at(n.id);
                const size_t elems = std::min<size_t>(b.out_bytes / 2, 8192);
                std::vector<uint16_t> host(elems);
                Check(hipMemcpy(host.data(), b.out.get(), elems * 2, hipMemcpyDeviceToHost), "checksum d2h");
                // 16-bit words are read in the output's 16-bit format; an fp32
                // output is read as fp16 halves, exactly as the reference does.
                const bool bf = n.out_dtype == kBF16;
                for (uint16_t h : host) sum += double(bf ? HostBF16ToF32(h) : HostF16ToF32(h));
            }
        return sum;
    }

    void Dump(const std::string &dir)
    {
        for (const auto &n : doc_.nodes) {
            const NodeBuf &b = ranks_[0].bufs.at(n.id);
            std::vector<char> host(b.out_bytes);
            Check(hipMemcpy(host.data(), b.out.get(), b.out_bytes, hipMemcpyDeviceToHost), "dump d2h");
            std::ofstream f(dir + "/" + n.id + ".bin", std::ios::binary);
            f.write(host.data(), std::streamsize(host.size()));
        }
    }

    const SchedDoc &doc() const { return doc_; }
    int edges() const { return int(consumed_states_.size()); }
    int epilogue_consumers() const
    {
        int n = 0;
        for (const auto &L : launches_) n += L.epi != nullptr;
        return n;
    }
    const std::string &sync() const { return sync_; }
    int consumer_cus() const { return streams_.cons_cus; }
    int partition() const { return partition_; }

private:
    int64_t OutRows(const NodeSpec &n) const { return n.rows; }
    int64_t InCols(const NodeSpec &n) const { return n.op == Op::MatMul ? n.k : n.cols; }

    void ValidateGeometry()
    {
        for (const auto &lane : doc_.lanes)
            for (const auto &t : lane.tasks) {
                const NodeSpec &n = doc_.Node(t.node);
                const int tiles = n.split ? n.tiles : 1;
                if (t.tile < 0 || t.tile >= tiles)
                    throw std::runtime_error("missing plan for task " + t.node + "#" + std::to_string(t.tile));
                const int64_t rt = n.rows / tiles;
                const int64_t in_off = t.has_geom ? t.in_row_off : t.tile * rt;
                const int64_t in_rows = t.has_geom ? t.in_rows : rt;
                const int64_t out_off = t.has_geom ? t.out_row_off : t.tile * rt;
                const int64_t limit = n.preds.empty() ? n.rows : OutRows(doc_.Node(n.preds[0]));
                if (in_off < 0 || in_rows <= 0 || in_off + in_rows > limit)
                    throw std::runtime_error("task " + t.node + "#" + std::to_string(t.tile) + " input rows [" +
                                             std::to_string(in_off) + "," + std::to_string(in_off + in_rows) +
                                             ") exceed " + std::to_string(limit));
                if (out_off < 0 || out_off + in_rows > OutRows(n))
                    throw std::runtime_error("task " + t.node + "#" + std::to_string(t.tile) + " output rows exceed " +
                                             std::to_string(OutRows(n)));
                if (t.n_tile > 0 && (t.n_off < 0 || t.n_off + t.n_tile > n.n))
                    throw std::runtime_error("task " + t.node + "#" + std::to_string(t.tile) + " N tile exceed " +
                                             std::to_string(n.n));
            }
        std::set<Key> publishing;
        for (const auto &lane : doc_.lanes)
            for (const auto &t : lane.tasks)
                if (t.publish) publishing.insert({t.node, t.tile});
        for (const auto &lane : doc_.lanes)
            for (const auto &t : lane.tasks)
                for (const auto &w : t.waits)
                    if (!publishing.count(w))
                        throw std::runtime_error("wait on unpublished flag " + w.first + "#" + std::to_string(w.second));
        (void)TopoOrder(doc_);
    }

    std::vector<uint16_t> HostInput(const NodeSpec &n, const std::string &role, size_t elems, uint32_t seed, int dtype)
    {
        std::vector<uint16_t> host(elems);
        auto it = n.inputs.find(role);
        if (it != n.inputs.end()) {
            std::ifstream f(it->second, std::ios::binary | std::ios::ate);
            if (!f) throw std::runtime_error("node " + n.id + ": cannot open input " + it->second);
            const size_t bytes = size_t(f.tellg());
            if (bytes != elems * 2)
                throw std::runtime_error("node " + n.id + ": input " + role + " has " + std::to_string(bytes) +
                                         " bytes, expected " + std::to_string(elems * 2));
            f.seekg(0);
            f.read(reinterpret_cast<char *>(host.data()), std::streamsize(bytes));
            return host;
        }
        for (size_t i = 0; i < elems; ++i) {
            const float v = DetValue(seed, i);
            host[i] = dtype == kBF16 ? HostF32ToBF16(v) : HostF32ToF16(v);
        }
        return host;
    }

    void Allocate(RankCtx &rc, const NodeSpec &n)
    {
        NodeBuf b;
        b.out_bytes = size_t(n.rows) * n.cols * DTypeBytes(n.out_dtype);
        b.out.Alloc(b.out_bytes);
        Check(hipMemset(b.out.get(), 0, b.out_bytes), "memset out");
        const size_t rows = size_t(n.rows), cols = size_t(n.cols);
        if (n.preds.empty()) b.own_in.Alloc(rows * InCols(n) * 2);
        if (n.op == Op::MatMul) b.bt.Alloc(size_t(n.k) * n.n * 2);
        if (IsBinary(n.op) && n.preds.size() < 2) b.aux.Alloc(rows * cols * 2);
        if (n.op == Op::RmsNorm || n.op == Op::AddRmsNorm || n.op == Op::LayerNorm) b.gamma.Alloc(cols * 2);
        if (n.op == Op::LayerNorm) b.beta.Alloc(cols * 2);
        if (n.op == Op::AddRmsNorm) b.sum.Alloc(rows * cols * 2);
        rc.bufs[n.id] = std::move(b);
    }

    void Upload(RankCtx &rc)
    {
        for (const auto &n : doc_.nodes) {
            NodeBuf &b = rc.bufs[n.id];
            const uint32_t seed = NodeSeed(n.id, uint32_t(rc.rank));
            const size_t rows = size_t(n.rows), cols = size_t(n.cols);
            if (b.own_in.get()) {
                auto h = HostInput(n, "in", rows * InCols(n), seed + 1, n.dtype);
                Check(hipMemcpy(b.own_in.get(), h.data(), h.size() * 2, hipMemcpyHostToDevice), "upload in");
            }
            if (n.op == Op::MatMul) {
                // weight generated / read as [K, N] (the reference's layout),
                // re-laid out once to [N, K] for the MFMA kernel.
                auto h = HostInput(n, "b", size_t(n.k) * n.n, seed + 2, n.dtype);
                DevBuf stage(h.size() * 2);
                Check(hipMemcpy(stage.get(), h.data(), h.size() * 2, hipMemcpyHostToDevice), "upload b");
                TransposeLaunch(stage.get(), b.bt.get(), int(n.k), int(n.n), nullptr);
                Check(hipDeviceSynchronize(), "transpose sync");
            }
            if (b.gamma.get()) {
                auto h = HostInput(n, "gamma", cols, seed + 2, n.dtype);
                Check(hipMemcpy(b.gamma.get(), h.data(), h.size() * 2, hipMemcpyHostToDevice), "upload gamma");
            }
            if (b.beta.get()) {
                // LayerNorm weight seed + 2, bias seed + 3 (exec_main.cpp:519-528)
                auto h = HostInput(n, "beta", cols, seed + 3, n.dtype);
                Check(hipMemcpy(b.beta.get(), h.data(), h.size() * 2, hipMemcpyHostToDevice), "upload beta");
            }
            if (b.aux.get()) {
                auto h = HostInput(n, "x1", rows * cols, seed + 3, n.dtype);
                Check(hipMemcpy(b.aux.get(), h.data(), h.size() * 2, hipMemcpyHostToDevice), "upload x1");
            }
        }
    }

    int LaneOf(const std::string &engine) const
    {
        // lane 0 = producer stream, lane 1 = consumer stream
        if (doc_.lanes.size() == 1) return 0;
        return engine == "aiv" ? 1 : 0;
    }

    int NodeTiles(const NodeSpec &n) const { return n.split ? n.tiles : 1; }

    int64_t TaskRows(const TaskSpec &t) const
    {
        const NodeSpec &n = doc_.Node(t.node);
        return t.has_geom ? t.in_rows : n.rows / NodeTiles(n);
    }
    int64_t TaskInOff(const TaskSpec &t) const
    {
        const NodeSpec &n = doc_.Node(t.node);
        return t.has_geom ? t.in_row_off : t.tile * (n.rows / NodeTiles(n));
    }
    int64_t TaskOutOff(const TaskSpec &t) const
    {
        const NodeSpec &n = doc_.Node(t.node);
        return t.has_geom ? t.out_row_off : t.tile * (n.rows / NodeTiles(n));
    }

    // A consumer task whose waits can be taken inside its own kernel: all on
    // one producer node, exactly the producer tiles its input rows intersect.
    bool InKernelWait(const TaskSpec &t, std::string *prod) const
    {
        if (t.waits.empty()) return false;
        const std::string &p = t.waits[0].first;
        std::vector<int> tiles;
        for (const auto &w : t.waits) {
            if (w.first != p) return false;
            tiles.push_back(w.second);
        }
        std::sort(tiles.begin(), tiles.end());
        const NodeSpec &P = doc_.Node(p);
        const int ptiles = NodeTiles(P);
        const int64_t prows = OutRows(P) / ptiles;
        const int64_t lo = TaskInOff(t), hi = lo + TaskRows(t);
        std::vector<int> hits;
        for (int k = 0; k < ptiles; ++k)
            if (k * prows < hi && (k + 1) * prows > lo) hits.push_back(k);
        if (hits != tiles) return false;
        if (prod) *prod = p;
        return true;
    }

    // Task t continues `run` (consecutive tasks of one lane) as one launch:
    // the next row tile of the same node, contiguous rows, and either a GEMM
    // with no waits (one launch releasing each tile in turn) or a consumer
    // waiting in-kernel on one producer (one persistent launch that waits for
    // each tile in turn).
    bool Extends(const std::vector<const TaskSpec *> &run, const TaskSpec &t) const
    {
        const TaskSpec &a = *run.back();
        if (t.node != a.node || t.tile != a.tile + 1 || t.publish != a.publish) return false;
        if (a.n_tile > 0 || t.n_tile > 0) return false;
        if (TaskRows(t) != TaskRows(a) || TaskInOff(t) != TaskInOff(a) + TaskRows(a) ||
            TaskOutOff(t) != TaskOutOff(a) + TaskRows(a))
            return false;
        const NodeSpec &n = doc_.Node(t.node);
        if (n.op == Op::MatMul) return a.waits.empty() && t.waits.empty();
        if (t.publish || wait_kind_ != "fused") return false;
        std::string pa, pt;
        return InKernelWait(a, &pa) && InKernelWait(t, &pt) && pa == pt;
    }

    static bool FanOp(Op op)
    {
        return op == Op::Gelu || op == Op::Silu || op == Op::Cast || op == Op::Softmax || op == Op::RmsNorm;
    }

    // Run r holds the same rows of another unary consumer of the producer
    // the runs of `group` consume: read the rows once for all of them.
    bool Sibling(const std::vector<std::vector<const TaskSpec *>> &group, const std::vector<const TaskSpec *> &r) const
    {
        if (int(group.size()) >= kMaxFanOut || fan_max_ < 2 || int(group.size()) >= fan_max_) return false;
        const auto &r0 = group[0];
        const NodeSpec &a = doc_.Node(r0[0]->node), &b = doc_.Node(r[0]->node);
        if (!FanOp(a.op) || !FanOp(b.op) || a.preds.size() != 1 || b.preds.size() != 1 || a.preds[0] != b.preds[0])
            return false;
        if (a.dtype != b.dtype || a.cols != b.cols || r.size() != r0.size()) return false;
        for (size_t i = 0; i < r.size(); ++i) {
            const TaskSpec &x = *r0[i], &y = *r[i];
            if (x.publish || y.publish || TaskInOff(x) != TaskInOff(y) || TaskRows(x) != TaskRows(y) ||
                TaskOutOff(x) != TaskOutOff(y))
                return false;
            std::string px, py;
            if (!InKernelWait(x, &px) || !InKernelWait(y, &py) || px != py || px != a.preds[0]) return false;
            auto wx = x.waits, wy = y.waits;
            std::sort(wx.begin(), wx.end());
            std::sort(wy.begin(), wy.end());
            if (wx != wy) return false;
        }
        return true;
    }

    // How many leading tiles of consumer launch L its producer launch PL
    // releases before its last round of workgroups starts: a persistent
    // consumer beside the GEMM can only overlap those; the rest are released
    // when the GEMM ends and run better at full width. -1 (every tile waits
    // in-kernel) when PL is not one GEMM launch releasing every tile of its
    // node, or when the tail is small enough for the persistent grid.
    // A GEMM released tile by tile runs co-resident tiles (room beside it
    // for a consumer's waves) only where that costs it nothing: where its
    // fastest tile is the 8-wave 256x256 kernel (every register of a CU) it
    // runs that, its consumers wait in a one-wave kernel (5 registers, which
    // fits beside it) and run at full width after it. Measured on the 4096^3
    // mm -> {softmax, gelu, cast} fan-out: co-resident 256x128 tiles made
    // the split 0.955x serial once the 256x256 kernel got faster.
    // KR_PLAN_CORESIDENT=1 keeps co-resident tiles throughout.
    bool CoresidentPays(const Launch &L) const
    {
        if (partition_ > 0) return false;  // its consumers run on CUs of their own
        if (EnvInt("KR_PLAN_CORESIDENT", 0) != 0) return true;
        const int64_t prows = L.pub_rows > 0 ? L.pub_rows : TaskRows(*L.task);
        const int N = int(L.task->n_tile > 0 ? L.task->n_tile : L.node->n);
        const GemmTile best = GemmPickTile(int(TaskRows(*L.task)), N, int(prows), false);
        return !(best.bm == 256 && best.bn == 256);
    }

    // In-register relay (KR_PLAN_EPILOGUE=1): a GELU / SiLU / cast consumer
    // that reads every row of one GEMM launch's output, and whose own output
    // no node reads, is computed in that GEMM's epilogue from each stored C
    // value with the elementwise kernel's arithmetic (the same bits); its
    // launch, waits and relay states go away. The tile reaches its consumer
    // in registers the moment it exists, instead of through HBM after a flag.
    template <class M>
    void FuseEpilogues(const M &launch_of)
    {
        for (Launch &L : launches_) {
            if (L.fan.size() != 1) continue;
            const NodeSpec &C = *L.node;
            if (C.op != Op::Gelu && C.op != Op::Silu && C.op != Op::Cast) continue;
            if (C.preds.size() != 1 || L.merged != NodeTiles(C)) continue;
            const NodeSpec &P = doc_.Node(C.preds[0]);
            if (P.op != Op::MatMul || C.rows != P.rows || C.cols != P.n) continue;
            if (TaskInOff(*L.task) != 0 || TaskOutOff(*L.task) != 0 || TaskRows(*L.task) != C.rows) continue;
            bool read = false;
            for (const auto &n : doc_.nodes)
                if (std::find(n.preds.begin(), n.preds.end(), C.id) != n.preds.end()) read = true;
            // a task that waits on C would wait on a release no launch makes
            for (const auto &lane : doc_.lanes)
                for (const auto &t : lane.tasks)
                    for (const auto &w : t.waits)
                        if (w.first == C.id) read = true;
            if (read) continue;
            // what GemmLaunch asks of the unary output: 16-byte rows (the
            // buffer itself is 256-byte aligned); otherwise the consumer
            // keeps its own launch
            if (C.out_dtype != kBF16 && C.out_dtype != kF16 && C.out_dtype != kF32) continue;
            if ((C.cols * int64_t(DTypeBytes(C.out_dtype))) % 16 != 0) continue;
            const auto it = launch_of.find({P.id, 0});
            if (it == launch_of.end()) continue;
            Launch &PL = launches_[it->second];
            if (PL.merged != NodeTiles(P) || PL.task->n_tile > 0 || PL.epi != nullptr) continue;
            if (TaskInOff(*PL.task) != 0 || TaskRows(*PL.task) != P.rows) continue;
            PL.epi = &C;
            L.skip = true;
        }
        // a producer whose every waiter now runs in its epilogue releases
        // nothing: it launches like an unreleased GEMM
        std::set<std::string> awaited;
        for (const Launch &L : launches_)
            if (!L.skip)
                for (const auto &w : L.task->waits) awaited.insert(w.first);
        for (Launch &L : launches_)
            if (L.epi != nullptr && !awaited.count(L.node->id)) L.publish = false;
    }

    int EarlyTiles(const Launch &PL, const Launch &L, int64_t in_off, int64_t in_rows) const
    {
        const NodeSpec &P = *PL.node;
        // with a CU partition the consumer's persistent grid has CUs of its
        // own: every tile waits in-kernel there
        if (partition_ > 0) return -1;
        // a GEMM that leaves no room beside it: a persistent consumer grid
        // would hold the CUs its own rows need, so its consumers take the
        // one-wave wait kernel and run at full width after it
        if (P.op == Op::MatMul && PL.publish && !PL.coresident) return 0;
        if (P.op != Op::MatMul || !PL.publish || PL.merged != NodeTiles(P) || PL.task->n_tile > 0) return -1;
        const int64_t prows = PL.pub_rows;
        if (prows <= 0 || L.tile_rows != prows || in_off % prows != 0) return -1;
        const int M = int(TaskRows(*PL.task)), N = int(P.n);
        const GemmTile gt = GemmPickTile(M, N, int(prows), PL.coresident);
        if (gt.bm <= 0) return -1;
        const int64_t tn = (N + gt.bn - 1) / gt.bn;
        const int64_t per = (prows / gt.bm) * tn;                 // workgroups per relay tile
        const int64_t total = ((M + gt.bm - 1) / gt.bm) * tn;
        const int64_t slots = int64_t(ncu_) * (gt.bm * gt.bn >= 256 * 128 ? 1 : 2);
        const int64_t last_round = ((total - 1) / slots) * slots;  // first workgroup of the last round
        const int k0 = int(in_off / prows);
        const int nt = int((in_rows + prows - 1) / prows);
        int early = 0;
        while (early < nt && (int64_t(k0 + early) + 1) * per <= last_round) ++early;
        // a tail the persistent grid clears in one pass (a wave per row,
        // four rows per workgroup) gains nothing from a second launch
        if (in_rows - int64_t(early) * prows <= int64_t(relay_grid_) * 4) return -1;
        return early;
    }

    void Wire()
    {
        // Launches. With device flags, consecutive row tiles of one node
        // become one launch (a GEMM that releases each tile as it completes,
        // or a persistent consumer that waits for each in turn), and sibling
        // unary consumers of the same producer rows share one pass over them
        // (KR_PLAN_COALESCE=0 keeps one launch per task, as the reference).
        const bool coalesce = sync_ == "flag" && EnvInt("KR_PLAN_COALESCE", 1) != 0;
        std::map<Key, size_t> launch_of;
        for (size_t l = 0; l < doc_.lanes.size(); ++l) {
            std::vector<std::vector<const TaskSpec *>> runs;
            for (const auto &t : doc_.lanes[l].tasks) {
                if (coalesce && !runs.empty() && Extends(runs.back(), t)) {
                    runs.back().push_back(&t);
                } else {
                    runs.push_back({&t});
                }
            }
            std::vector<std::vector<std::vector<const TaskSpec *>>> groups;
            for (auto &r : runs) {
                if (coalesce && !groups.empty() && Sibling(groups.back(), r)) {
                    groups.back().push_back(r);
                } else {
                    groups.push_back({r});
                }
            }
            for (const auto &g : groups) {
                Launch L;
                L.lane = LaneOf(doc_.lanes[l].engine);
                const auto &r0 = g[0];
                if (r0.size() == 1) {
                    L.task = r0[0];
                } else {
                    TaskSpec m = *r0[0];
                    m.has_geom = true;
                    m.in_row_off = TaskInOff(*r0[0]);
                    m.out_row_off = TaskOutOff(*r0[0]);
                    m.in_rows = 0;
                    m.waits.clear();
                    for (const TaskSpec *t : r0) {
                        m.in_rows += TaskRows(*t);
                        for (const auto &w : t->waits)
                            if (std::find(m.waits.begin(), m.waits.end(), w) == m.waits.end()) m.waits.push_back(w);
                    }
                    merged_.push_back(m);
                    L.task = &merged_.back();
                }
                L.node = &doc_.Node(r0[0]->node);
                L.publish = L.task->publish;
                L.pub_rows = TaskRows(*r0[0]);
                L.merged = int(r0.size());
                for (const auto &r : g) L.fan.push_back(&doc_.Node(r[0]->node));
                for (const auto &r : g)
                    for (const TaskSpec *t : r) launch_of[{t->node, t->tile}] = launches_.size();
                launches_.push_back(L);
            }
        }
        if (doc_.lanes.size() > 2) throw std::runtime_error("more than two engine lanes after normalization");
        if (coalesce && EnvInt("KR_PLAN_EPILOGUE", 0) != 0) FuseEpilogues(launch_of);
        // Which tasks are awaited: only cross-lane waits need a flag/event.
        std::map<std::string, int> flag_base;
        int next_block = 0;
        for (const auto &n : doc_.nodes) {
            flag_base[n.id] = next_block;
            next_block += NodeTiles(n);
        }
        // state blocks per (consumer node, producer node)
        std::map<std::pair<std::string, std::string>, int> state_base;
        // last waiter per (consumer node, producer node, producer tile)
        std::map<std::tuple<std::string, std::string, int>, size_t> last_waiter;
        for (size_t i = 0; i < launches_.size(); ++i) {
            Launch &L = launches_[i];
            if (L.skip) continue;
            for (const auto &w : L.task->waits) {
                auto it = launch_of.find(w);
                if (it == launch_of.end()) throw std::runtime_error("missing plan for task " + w.first);
                const Launch &P = launches_[it->second];
                if (!P.task->publish) throw std::runtime_error("wait on unpublished flag " + w.first + "#" + std::to_string(w.second));
                for (const NodeSpec *c : L.fan) {
                    const auto sk = std::make_pair(c->id, w.first);
                    if (!state_base.count(sk)) {
                        state_base[sk] = next_block;
                        next_block += NodeTiles(doc_.Node(w.first));
                    }
                    last_waiter[std::make_tuple(c->id, w.first, w.second)] = i;
                }
            }
        }
        ctrl_words_ = size_t(std::max(next_block, 1)) * kWords;
        ctrl_.Alloc(ctrl_words_ * 4);
        Check(hipMemset(ctrl_.get(), 0, ctrl_words_ * 4), "zero ctrl");
        int32_t *ctrl = ctrl_.as<int32_t>();

        // every producer's tile policy first: a consumer's early tiles follow it
        for (Launch &L : launches_)
            if (L.publish) L.coresident = L.node->op == Op::MatMul && CoresidentPays(L);
        for (size_t i = 0; i < launches_.size(); ++i) {
            Launch &L = launches_[i];
            const NodeSpec &n = *L.node;
            const TaskSpec &t = *L.task;
            const int64_t in_off = TaskInOff(t);
            const int64_t in_rows = TaskRows(t);
            if (L.publish) L.flag = flag_base.at(n.id) + t.tile;
            if (L.skip) continue;  // computed in its producer's epilogue
            if (sync_ == "event") {
                if (L.publish) Check(hipEventCreateWithFlags(&L.pub_event, hipEventDisableTiming), "event");
                continue;
            }
            // group waits by producer node
            std::map<std::string, std::vector<int>> by_prod;
            for (const auto &w : t.waits) by_prod[w.first].push_back(w.second);
            for (auto &kv : by_prod) {
                const NodeSpec &P = doc_.Node(kv.first);
                std::sort(kv.second.begin(), kv.second.end());
                const int ptiles = NodeTiles(P);
                const int64_t prows = OutRows(P) / ptiles;
                // per fused consumer: its state base and the tiles it consumes here
                std::vector<int> sbases;
                std::vector<int> adv;
                for (size_t c = 0; c < L.fan.size(); ++c) {
                    const int sb = state_base.at({L.fan[c]->id, P.id});
                    sbases.push_back(sb);
                    for (int k : kv.second)
                        if (last_waiter.at(std::make_tuple(L.fan[c]->id, P.id, k)) == i) {
                            if (c == 0) adv.push_back(k);
                            consumed_states_.push_back(sb + k);
                        }
                }
                // tiles intersecting this task's input rows in P's output row space
                std::vector<int> hits;
                for (int k = 0; k < ptiles; ++k)
                    if (k * prows < in_off + in_rows && (k + 1) * prows > in_off) hits.push_back(k);
                const bool contiguous_adv =
                    adv.empty() || (adv.back() - adv.front() + 1 == int(adv.size()));
                // a GEMM consumer waits in its own workgroups only when they
                // cannot hold CUs its producer needs (a CU partition between
                // the lanes); otherwise behind one-workgroup wait kernels
                const bool gemm_ok =
                    n.op != Op::MatMul ||
                    (partition_ > 0 && L.fan.size() == 1 && launches_[launch_of.at({P.id, kv.second.front()})].lane != L.lane);
                const bool fusable = wait_kind_ == "fused" && by_prod.size() == 1 && gemm_ok &&
                                     hits == kv.second && contiguous_adv;
                if (fusable) {
                    L.fused_wait = true;
                    L.wait.ctrl = ctrl;
                    L.wait.flag0 = flag_base.at(P.id);
                    L.wait.state0 = sbases[0];
                    L.wait.prod_rows = int(prows);
                    L.wait.row_off = int(in_off);
                    L.wait.adv_lo = adv.empty() ? 0 : adv.front();
                    L.wait.adv_hi = adv.empty() ? 0 : adv.back() + 1;
                    L.wait.max_spins = max_spins_;
                    L.tile_rows = int(std::min<int64_t>(in_rows, prows));
                    L.fan_states = sbases;
                    L.early_tiles = EarlyTiles(launches_[launch_of.at({P.id, kv.second.front()})], L, in_off, in_rows);
                } else {
                    // one-workgroup wait kernels before the launch, one per
                    // (consumer, producer tile)
                    for (size_t c = 0; c < L.fan.size(); ++c)
                        for (int k : kv.second) {
                            RelayWait w{};
                            w.ctrl = ctrl;
                            w.flag0 = flag_base.at(P.id) + k;
                            w.state0 = sbases[c] + k;
                            w.prod_rows = 1;
                            w.row_off = 0;
                            const bool advance = last_waiter.at(std::make_tuple(L.fan[c]->id, P.id, k)) == i;
                            w.adv_lo = 0;
                            w.adv_hi = advance ? 1 : 0;
                            w.max_spins = max_spins_;
                            L.extra_waits.push_back(w);
                        }
                }
            }
        }
        if (sync_ == "event") {
            for (auto &L : launches_)
                for (const auto &w : L.task->waits) L.wait_events.push_back(launches_[launch_of.at(w)].pub_event);
        }
        // enqueue order: global topological order (records before waits); a
        // merged launch goes where its first task would
        auto order = TopoOrder(doc_);
        std::set<size_t> queued;
        for (const auto &o : order) {
            const auto &t = doc_.lanes[o.first].tasks[o.second];
            const size_t li = launch_of.at({t.node, t.tile});
            if (queued.insert(li).second) enqueue_order_.push_back(li);
        }
        for (const Launch &L : launches_)
            if (!L.skip) lanes_used_[L.lane] = true;
    }

    hipStream_t StreamOf(int lane) const { return lane == 0 ? streams_.prod : streams_.cons; }

    // One consumer kernel over rows [r0, r0 + nrows) of launch L (local
    // numbering), waiting in-kernel through `wait` (ctrl == nullptr: none).
    void LaunchConsumer(RankCtx &rc, Launch &L, hipStream_t s, int64_t r0, int64_t nrows, const RelayWait &wait,
                        int grid, const RelayPub &pub)
    {
        const NodeSpec &n = *L.node;
        const TaskSpec &t = *L.task;
        NodeBuf &b = rc.bufs.at(n.id);
        const int64_t in_off = TaskInOff(t) + r0;
        const int64_t out_off = TaskOutOff(t) + r0;
        const void *in_base = n.preds.empty() ? b.own_in.get() : rc.bufs.at(n.preds[0]).out.get();
        const auto *in_tile = static_cast<const char *>(in_base) + size_t(in_off) * InCols(n) * 2;
        const void *x1 = nullptr;
        if (IsBinary(n.op)) {
            const void *x1base = n.preds.size() > 1 ? rc.bufs.at(n.preds[1]).out.get() : b.aux.get();
            x1 = static_cast<const char *>(x1base) + size_t(in_off) * n.cols * 2;
        }
        char *out_tile = static_cast<char *>(b.out.get()) + size_t(out_off) * n.cols * DTypeBytes(n.out_dtype);
        const int tile_rows = wait.ctrl != nullptr ? L.tile_rows : 0;

        if (L.fan.size() > 1) {
            // sibling unary consumers of the same rows: one pass, every output
            FanDesc d;
            d.dtype_in = n.dtype;
            d.x = in_tile;
            d.rows = int(nrows);
            d.cols = int(n.cols);
            d.eps = n.eps;
            d.n_out = int(L.fan.size());
            for (size_t i = 0; i < L.fan.size(); ++i) {
                const NodeSpec &c = *L.fan[i];
                NodeBuf &cb = rc.bufs.at(c.id);
                FanOutDesc &o = d.out[i];
                o.op = c.op == Op::Gelu ? kEwGelu
                     : c.op == Op::Silu ? kEwSilu
                     : c.op == Op::Cast ? kEwCast
                     : c.op == Op::Softmax ? kFanSoftmax
                                           : kFanRmsNorm;
                o.dtype = c.out_dtype;
                o.y = static_cast<char *>(cb.out.get()) + size_t(out_off) * c.cols * DTypeBytes(c.out_dtype);
                o.gamma = cb.gamma.get();
                d.states[i] = L.fan_states.empty() ? 0 : L.fan_states[i];
            }
            d.tile_rows = tile_rows;
            d.grid = grid;
            d.wait = wait;
            FanLaunch(d, s);
            return;
        }
        switch (n.op) {
            case Op::Gelu:
            case Op::Silu:
            case Op::Cast:
            case Op::Add:
            case Op::Mul:
            case Op::Swiglu: {
                EwDesc d;
                d.op = n.op == Op::Gelu ? kEwGelu
                     : n.op == Op::Silu ? kEwSilu
                     : n.op == Op::Cast ? kEwCast
                     : n.op == Op::Add  ? kEwAdd
                     : n.op == Op::Mul  ? kEwMul
                                        : kEwSwiglu;
                d.dtype_in = n.dtype;
                d.dtype_out = n.out_dtype;
                d.x0 = in_tile;
                d.x1 = x1;
                d.y = out_tile;
                d.rows = int(nrows);
                d.cols = int(n.cols);
                d.tile_rows = tile_rows;
                d.grid = grid;
                d.wait = wait;
                d.pub = pub;
                if (pub.ctrl && d.tile_rows > 0 && d.tile_rows != d.rows) {
                    // publish once for the whole task: release after the kernel
                    d.pub = RelayPub{};
                    EwLaunch(d, s);
                    PublishLaunch(pub, 0, s);
                } else {
                    EwLaunch(d, s);
                }
                break;
            }
            case Op::Softmax:
            case Op::RmsNorm:
            case Op::AddRmsNorm:
            case Op::LayerNorm: {
                RowDesc d;
                d.op = n.op == Op::Softmax     ? kRowSoftmax
                       : n.op == Op::RmsNorm   ? kRowRmsNorm
                       : n.op == Op::LayerNorm ? kRowLayerNorm
                                               : kRowAddRmsNorm;
                d.dtype = n.dtype;
                d.x0 = in_tile;
                d.x1 = n.op == Op::LayerNorm ? b.beta.get() : x1;
                d.gamma = b.gamma.get();
                d.y = out_tile;
                d.sum_out = b.sum.get() ? static_cast<char *>(b.sum.get()) + size_t(out_off) * n.cols * 2 : nullptr;
                d.rows = int(nrows);
                d.cols = int(n.cols);
                d.eps = n.eps;
                d.tile_rows = tile_rows;
                d.grid = grid;
                d.wait = wait;
                d.pub = pub;
                if (pub.ctrl && d.tile_rows > 0 && d.tile_rows != d.rows) {
                    d.pub = RelayPub{};
                    RowLaunch(d, s);
                    PublishLaunch(pub, 0, s);
                } else {
                    RowLaunch(d, s);
                }
                break;
            }
            case Op::MatMul:
                throw std::logic_error("LaunchConsumer: matmul");
        }
    }

    // events = false: leave the launch's event waits and records to the
    // caller (graph_segment puts them between its graphs)
    void EnqueueTask(RankCtx &rc, Launch &L, hipStream_t s, bool events = true)
    {
        if (L.skip) return;  // computed in its producer GEMM's epilogue
        const NodeSpec &n = *L.node;
        const TaskSpec &t = *L.task;
        NodeBuf &b = rc.bufs.at(n.id);
        const int64_t in_off = TaskInOff(t);
        const int64_t in_rows = TaskRows(t);
        const int64_t out_off = TaskOutOff(t);

        if (sync_ == "event" && events) {
            for (hipEvent_t e : L.wait_events) Check(hipStreamWaitEvent(s, e, 0), "stream wait event");
        }
        for (const auto &w : L.extra_waits) WaitLaunch(w, 0, 1, s);

        RelayPub pub{};
        if (L.publish && sync_ == "flag") {
            pub.ctrl = ctrl_.as<int32_t>();
            pub.flag0 = L.flag;
            pub.rows_per_tile = int(L.pub_rows > 0 ? L.pub_rows : in_rows);
        }

        if (n.op == Op::MatMul) {
            const void *in_base = n.preds.empty() ? b.own_in.get() : rc.bufs.at(n.preds[0]).out.get();
            GemmDesc d;
            d.dtype = n.dtype;
            d.A = static_cast<const char *>(in_base) + size_t(in_off) * n.k * 2;
            d.lda = n.k;
            const int64_t ncols = t.n_tile > 0 ? t.n_tile : n.n;
            d.Bt = b.bt.as<uint16_t>() + size_t(t.n_off) * n.k;
            d.ldb = n.k;
            d.C = reinterpret_cast<uint16_t *>(static_cast<char *>(b.out.get()) + size_t(out_off) * n.cols * 2) +
                  (t.n_tile > 0 ? t.n_off : 0);
            d.ldc = n.n;
            d.M = int(in_rows);
            d.N = int(ncols);
            d.K = int(n.k);
            d.coresident = L.coresident;
            // each workgroup waits for the producer tiles of the A rows it
            // reads (a CU partition keeps it off the producer's CUs)
            if (L.fused_wait) d.wait = L.wait;
            if (L.epi != nullptr) {
                // the in-register relay: the consumer's rows leave with C's
                const NodeSpec &c = *L.epi;
                d.y = static_cast<char *>(rc.bufs.at(c.id).out.get()) + size_t(out_off) * c.cols * DTypeBytes(c.out_dtype);
                d.y_op = c.op == Op::Gelu ? kEwGelu : (c.op == Op::Silu ? kEwSilu : kEwCast);
                d.y_dtype = c.out_dtype;
                d.ld_y = c.cols;
            }
            if (pub.ctrl && GemmPickTile(d.M, d.N, pub.rows_per_tile, d.coresident).bm < 0) {
                // the tile cannot be one GEMM relay tile: release after the GEMM
                GemmLaunch(d, s);
                for (int k = 0; k < L.merged; ++k) PublishLaunch(pub, k, s);
            } else {
                d.pub = pub;
                GemmLaunch(d, s);
            }
        } else if (!L.fused_wait) {
            LaunchConsumer(rc, L, s, 0, in_rows, RelayWait{}, 0, pub);
        } else if (L.early_tiles < 0) {
            // persistent consumer: waits for each producer tile in turn
            LaunchConsumer(rc, L, s, 0, in_rows, L.wait, relay_grid_, pub);
        } else {
            // tiles released before the producer's last round: a persistent
            // consumer beside the GEMM; tiles released at its end: a wait
            // kernel, then the consumer at full width
            const int64_t rows_a = std::min<int64_t>(in_rows, int64_t(L.early_tiles) * L.tile_rows);
            const int split_tile = int((in_off + rows_a) / L.wait.prod_rows);
            RelayWait wa = L.wait, wb = L.wait;
            wa.adv_hi = std::min(wa.adv_hi, split_tile);
            wb.adv_lo = std::max(wb.adv_lo, split_tile);
            if (wa.adv_hi < wa.adv_lo) wa.adv_hi = wa.adv_lo;
            if (wb.adv_hi < wb.adv_lo) wb.adv_hi = wb.adv_lo;
            if (rows_a > 0) LaunchConsumer(rc, L, s, 0, rows_a, wa, relay_grid_, RelayPub{});
            if (rows_a < in_rows) {
                const std::vector<int32_t> st = L.fan_states.empty() ? std::vector<int32_t>{wb.state0} : L.fan_states;
                wb.state0 = st[0];
                WaitLaunchMulti(wb, int(rows_a), int(in_rows), st.data(), int(st.size()), s);
                LaunchConsumer(rc, L, s, rows_a, in_rows - rows_a, RelayWait{}, 0, RelayPub{});
            }
            // a consumer that is itself a producer (mm -> GELU -> mm): its
            // rows may span both launches, so it releases its tiles behind
            // the last one (nothing when it publishes nothing)
            for (int k = 0; k < L.merged; ++k) PublishLaunch(pub, k, s);
        }
        Check(hipGetLastError(), "task launch");
        if (L.publish && sync_ == "event" && events) Check(hipEventRecord(L.pub_event, s), "record event");
    }

    void EnqueueRank(int r)
    {
        for (size_t idx : enqueue_order_) {
            Launch &L = launches_[idx];
            EnqueueTask(ranks_[r], L, StreamOf(L.lane));
        }
    }

    // graph_segment (the reference's NHP_GRAPH_SEGMENT, exec_main.cpp:
    // 1150-1273): each stream's launches are cut into runs, a run ending
    // after a launch that publishes and a new one starting at a launch that
    // waits on an event; each run is captured as one graph. A run's waits
    // are its first launch's, its publishes its last launch's.
    void CaptureSegments()
    {
        for (int r = 0; r < doc_.nranks; ++r)
            for (int lane = 0; lane < 2; ++lane) {
                std::vector<size_t> run;
                auto close = [&]() {
                    if (run.empty()) return;
                    Segment g{};
                    g.rank = r;
                    g.lane = lane;
                    g.waits = launches_[run.front()].wait_events;
                    for (size_t i : run)
                        if (launches_[i].publish) g.pubs.push_back(launches_[i].pub_event);
                    hipStream_t s = StreamOf(lane);
                    Check(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), "begin capture");
                    for (size_t i : run) EnqueueTask(ranks_[r], launches_[i], s, false);
                    Check(hipStreamEndCapture(s, &g.graph), "end capture");
                    Check(hipGraphInstantiate(&g.exec, g.graph, nullptr, nullptr, 0), "instantiate");
                    segments_.push_back(g);
                    run.clear();
                };
                for (size_t idx : enqueue_order_) {
                    const Launch &L = launches_[idx];
                    if (L.lane != lane) continue;
                    if (!run.empty() && !L.wait_events.empty()) close();
                    run.push_back(idx);
                    if (L.publish) close();
                }
                close();
            }
    }

    // Launch rank r's segments in dependency order: a segment goes out once
    // every event it waits on has been recorded in this run, behind
    // hipStreamWaitEvent on them; its publishes are recorded right after it.
    void RunSegments(int r)
    {
        std::set<hipEvent_t> recorded;
        std::vector<char> done(segments_.size(), 0);
        size_t remaining = 0;
        for (const auto &g : segments_) remaining += g.rank == r;
        while (remaining > 0) {
            bool progress = false;
            for (size_t i = 0; i < segments_.size(); ++i) {
                Segment &g = segments_[i];
                if (g.rank != r || done[i]) continue;
                bool ready = true;
                for (hipEvent_t e : g.waits)
                    if (recorded.count(e) == 0) {
                        ready = false;
                        break;
                    }
                if (!ready) continue;
                hipStream_t s = StreamOf(g.lane);
                for (hipEvent_t e : g.waits) Check(hipStreamWaitEvent(s, e, 0), "segment wait");
                Check(hipGraphLaunch(g.exec, s), "segment launch");
                for (hipEvent_t e : g.pubs) {
                    Check(hipEventRecord(e, s), "segment record");
                    recorded.insert(e);
                }
                done[i] = 1;
                --remaining;
                progress = true;
            }
            if (!progress) throw std::runtime_error("segment wait cycle");
        }
    }

    void Capture()
    {
        if (mode_ == "graph_segment") {
            CaptureSegments();
            return;
        }
        for (int r = 0; r < doc_.nranks; ++r) {
            if (sync_ == "event") {
                // one multi-stream graph: fork the consumer stream off the producer
                hipGraph_t g = nullptr;
                Check(hipStreamBeginCapture(streams_.prod, hipStreamCaptureModeThreadLocal), "begin capture");
                hipEvent_t fork = nullptr, join = nullptr;
                Check(hipEventCreateWithFlags(&fork, hipEventDisableTiming), "fork event");
                Check(hipEventCreateWithFlags(&join, hipEventDisableTiming), "join event");
                Check(hipEventRecord(fork, streams_.prod), "fork");
                Check(hipStreamWaitEvent(streams_.cons, fork, 0), "fork wait");
                EnqueueRank(r);
                Check(hipEventRecord(join, streams_.cons), "join");
                Check(hipStreamWaitEvent(streams_.prod, join, 0), "join wait");
                Check(hipStreamEndCapture(streams_.prod, &g), "end capture");
                hipGraphExec_t ex = nullptr;
                Check(hipGraphInstantiate(&ex, g, nullptr, nullptr, 0), "instantiate");
                graphs_.push_back({g, ex, 0, r});
                (void)hipEventDestroy(fork);
                (void)hipEventDestroy(join);
                continue;
            }
            // flags: one graph per stream, replayed on that stream. A lane
            // whose first launch waits on the other lane is launched second,
            // so that the host's launch of its graph does not delay the lane
            // that can start at once.
            int first_waits[2] = {-1, -1};
            for (size_t idx : enqueue_order_) {
                const Launch &L = launches_[idx];
                if (L.skip || first_waits[L.lane] >= 0) continue;
                first_waits[L.lane] = (L.fused_wait || !L.extra_waits.empty()) ? 1 : 0;
            }
            const int order[2] = {first_waits[0] == 1 && first_waits[1] == 0 ? 1 : 0,
                                  first_waits[0] == 1 && first_waits[1] == 0 ? 0 : 1};
            for (int lane : order) {
                bool any = false;
                for (size_t idx : enqueue_order_)
                    if (launches_[idx].lane == lane && !launches_[idx].skip) any = true;
                if (!any) continue;
                hipStream_t s = StreamOf(lane);
                hipGraph_t g = nullptr;
                Check(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), "begin capture");
                for (size_t idx : enqueue_order_) {
                    Launch &L = launches_[idx];
                    if (L.lane == lane) EnqueueTask(ranks_[r], L, s);
                }
                Check(hipStreamEndCapture(s, &g), "end capture");
                hipGraphExec_t ex = nullptr;
                Check(hipGraphInstantiate(&ex, g, nullptr, nullptr, 0), "instantiate");
                graphs_.push_back({g, ex, lane, r});
            }
        }
    }

    struct Graph {
        hipGraph_t graph;
        hipGraphExec_t exec;
        int lane;
        int rank;
    };
    struct Segment {
        hipGraph_t graph;
        hipGraphExec_t exec;
        int lane;
        int rank;
        std::vector<hipEvent_t> waits;
        std::vector<hipEvent_t> pubs;
    };
    std::vector<Segment> segments_;

    SchedDoc doc_;
    int device_;
    std::string mode_;
    std::string sync_;
    std::string wait_kind_;
    int relay_grid_ = 256;
    int ncu_ = 256;
    int partition_ = 0;  // CUs per XCD owned by lane 1 (0: both lanes share every CU)
    int fan_max_ = kMaxFanOut;
    std::deque<TaskSpec> merged_;
    uint32_t max_spins_ = kDefaultMaxSpins;
    StreamPair streams_;
    hipEvent_t ev0_ = nullptr, ev1_ = nullptr, ev2_ = nullptr, ev3_ = nullptr;
    bool lanes_used_[2] = {false, false};  // a lane with at least one launch
    std::vector<RankCtx> ranks_;
    std::vector<Launch> launches_;
    std::vector<size_t> enqueue_order_;
    std::vector<int> consumed_states_;
    DevBuf ctrl_;
    size_t ctrl_words_ = 0;
    std::vector<Graph> graphs_;
};

int ParseDevice(const char *devices)
{
    if (devices == nullptr || *devices == '\0') return 0;
    std::string s(devices);
    int dev = -1;
    std::stringstream ss(s);
    std::string tok;
    while (std::getline(ss, tok, ',')) {
        if (tok.empty()) throw std::runtime_error("devices has an empty entry");
        const int d = std::stoi(tok);
        if (dev >= 0 && d != dev) throw std::runtime_error("all ranks must run on the one device of this target");
        dev = d;
    }
    return dev < 0 ? 0 : dev;
}

// Cross-stream sync micro-benchmark (the reference's NHP_SYNC_BENCH,
// exec/exec_main.cpp:751-833): n producer/consumer kernel pairs on two
// streams with hardware queues of their own. Every mode launches the same two
// one-workgroup kernels per pair (a publish on the producer stream, a wait on
// the consumer stream) and changes only the synchronisation: "nosync" (the
// wait targets a block published beforehand, so it returns at once),
// "event" (a hipEvent record / stream wait between them as well) and "flag"
// (the wait spins on the block this pair's publish releases). Wall time per
// pair, median over rounds; event/flag minus nosync is the cost of the sync.
double SyncBenchMode(const std::string &mode, int n, int rounds, int warmup, const StreamPair &sp, DevBuf &ctrl,
                     std::vector<hipEvent_t> &events, int *timeouts)
{
    std::vector<double> samples;
    int32_t *blocks = ctrl.as<int32_t>();
    std::vector<int32_t> ready(size_t(n) * kWords, 0);
    for (int i = 0; i < n; ++i) ready[size_t(i) * kWords + kOffPublished] = 1 << 30;
    for (int r = 0; r < warmup + rounds; ++r) {
        // blocks [0, n): released by this round's publishes; [n, 2n): already released
        Check(hipMemset(blocks, 0, size_t(n) * kWords * 4), "sync clear flags");
        Check(hipMemcpy(blocks + size_t(n) * kWords, ready.data(), ready.size() * 4, hipMemcpyHostToDevice),
              "sync preset flags");
        Check(hipDeviceSynchronize(), "sync reset");
        const auto t0 = Clock::now();
        for (int i = 0; i < n; ++i) {
            RelayPub pub{};
            pub.ctrl = blocks;
            pub.flag0 = i;
            pub.rows_per_tile = 1;
            PublishLaunch(pub, 0, sp.prod);
            if (mode == "event") {
                Check(hipEventRecord(events[i], sp.prod), "sync record");
                Check(hipStreamWaitEvent(sp.cons, events[i], 0), "sync wait event");
            }
            RelayWait w{};
            w.ctrl = blocks;
            w.flag0 = mode == "flag" ? i : n + i;
            w.state0 = i;
            w.prod_rows = 1;
            w.adv_lo = 0;
            w.adv_hi = 1;
            w.max_spins = kDefaultMaxSpins;
            WaitLaunch(w, 0, 1, sp.cons);
        }
        Check(hipStreamSynchronize(sp.prod), "sync prod");
        Check(hipStreamSynchronize(sp.cons), "sync cons");
        const auto t1 = Clock::now();
        if (r >= warmup) samples.push_back(Us(t0, t1) / n);
    }
    std::vector<int32_t> host(size_t(n) * kWords);
    Check(hipMemcpy(host.data(), blocks, host.size() * 4, hipMemcpyDeviceToHost), "sync status copy");
    *timeouts = 0;
    for (int i = 0; i < n; ++i)
        if (host[size_t(i) * kWords + kOffStatus] != 1) ++*timeouts;
    return Median(samples);
}

int RunSyncBench(const std::string &out_path, int device)
{
    const int n = 256, rounds = 10;
    Check(hipSetDevice(device), "hipSetDevice");
    StreamPair sp;
    sp.Create(device);
    DevBuf ctrl(size_t(2 * n) * kWords * 4);
    std::vector<hipEvent_t> events(n, nullptr);
    for (auto &e : events) Check(hipEventCreateWithFlags(&e, hipEventDisableTiming), "sync event");
    int to_none = 0, to_event = 0, to_flag = 0;
    const double none = SyncBenchMode("nosync", n, rounds, 2, sp, ctrl, events, &to_none);
    const double event = SyncBenchMode("event", n, rounds, 2, sp, ctrl, events, &to_event);
    const double flag = SyncBenchMode("flag", n, rounds, 2, sp, ctrl, events, &to_flag);
    for (auto e : events) (void)hipEventDestroy(e);
    sp.Destroy();
    Value r = Value::MakeObject();
    r.Set("n", Value::MakeNumber(n));
    r.Set("rounds", Value::MakeNumber(rounds));
    r.Set("us_per_pair_nosync", Value::MakeNumber(none));
    r.Set("us_per_pair_event", Value::MakeNumber(event));
    r.Set("us_per_pair_flag", Value::MakeNumber(flag));
    r.Set("event_minus_nosync_us", Value::MakeNumber(event - none));
    r.Set("flag_minus_nosync_us", Value::MakeNumber(flag - none));
    r.Set("timeouts_nosync", Value::MakeNumber(to_none));
    r.Set("timeouts_event", Value::MakeNumber(to_event));
    r.Set("timeouts_flag", Value::MakeNumber(to_flag));
    std::ofstream f(out_path);
    f << r.Dump() << "\n";
    std::printf("sync bench: nosync %.3f us/pair (to %d), event %.3f (to %d), flag %.3f (to %d), "
                "event-base %.3f, flag-base %.3f\n",
                none, to_none, event, to_event, flag, to_flag, event - none, flag - none);
    return 0;
}

int RunPlan(const char *schedule_json, int iters, int warmup, const char *devices, const char *mode,
            const char *out_json)
{
    try {
        if (const char *sync_out = std::getenv("NHP_SYNC_BENCH")) return RunSyncBench(sync_out, ParseDevice(devices));
        if (iters < 1 || warmup < 0) {
            std::fprintf(stderr, "kr_plan_run: iters must be >= 1 and warmup >= 0\n");
            return 2;
        }
        const Value root = json::ParseFile(schedule_json);
        SchedDoc doc = ParseSchedule(root);
        NormalizeTopology(doc);
        const int device = ParseDevice(devices);
        Executor ex(std::move(doc), device, mode ? mode : "direct");
        ex.Prepare();
        for (int i = 0; i < warmup; ++i) (void)ex.RunOnce(nullptr);
        std::vector<double> times, dev;
        for (int i = 0; i < iters; ++i) {
            double d = 0.0;
            times.push_back(ex.RunOnce(&d));
            dev.push_back(d);
        }
        const int timeouts = ex.FlagTimeouts();
        const double checksum = ex.Checksum();
        const std::string dump = EnvStr("KR_DUMP_DIR", "");
        if (!dump.empty()) ex.Dump(dump);

        Value result = Value::MakeObject();
        result.Set("dag", Value::MakeString(ex.doc().dag));
        result.Set("group", Value::MakeString(ex.doc().group));
        result.Set("nranks", Value::MakeNumber(ex.doc().nranks));
        result.Set("iters", Value::MakeNumber(iters));
        result.Set("warmup", Value::MakeNumber(warmup));
        result.Set("p50_us", Value::MakeNumber(Median(times)));
        result.Set("gate_timeouts", Value::MakeNumber(timeouts));
        result.Set("checksum", Value::MakeNumber(checksum));
        result.Set("ok", Value::MakeBool(timeouts == 0));
        Value arr = Value::MakeArray();
        for (double t : times) arr.Push(Value::MakeNumber(t));
        result.Set("times_us", arr);
        result.Set("best_us", Value::MakeNumber(Min(times)));
        Value darr = Value::MakeArray();
        for (double t : dev) darr.Push(Value::MakeNumber(t));
        result.Set("device_us", darr);
        result.Set("device_best_us", Value::MakeNumber(Min(dev)));
        result.Set("device_p50_us", Value::MakeNumber(Median(dev)));
        result.Set("sync", Value::MakeString(ex.sync()));
        result.Set("mode", Value::MakeString(mode ? mode : "direct"));
        result.Set("flag_edges", Value::MakeNumber(ex.edges()));
        result.Set("epilogue_consumers", Value::MakeNumber(ex.epilogue_consumers()));
        result.Set("consumer_cus", Value::MakeNumber(ex.consumer_cus()));
        result.Set("cu_partition_per_xcd", Value::MakeNumber(ex.partition()));
        json::WriteFile(out_json, result);
        std::printf("%s\n", result.Dump().c_str());
        std::fflush(stdout);
        return 0;
    } catch (const std::exception &e) {
        std::fprintf(stderr, "kr_plan_run error: %s\n", e.what());
        std::fflush(stderr);
        return 1;
    }
}

}  // namespace plan
}  // namespace kr

extern "C" int kr_plan_run(const char *schedule_json, int iters, int warmup, const char *devices, const char *mode,
                           const char *out_json)
{
    if (schedule_json == nullptr || out_json == nullptr) return 2;
    return kr::plan::RunPlan(schedule_json, iters, warmup, devices, mode, out_json);
}
