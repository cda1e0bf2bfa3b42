// The recognition head inside a model file's graph (host code): the segment the
// engine-level fused hook replaces, MatMul(x, W) -> Add(bias) (optional) -> Softmax(axis
// -1) -> graph output.  The rules follow the reference's load-time passes: Identity nodes
// are aliases (src/engine/model.rs:67-95); a MatMul whose output is used once folds the
// bias of the Add that uses it when the Add's other input is a weight
// (src/engine/model.rs:96-166); Softmax takes attribute "axis", default -1, normalised
// against the input's rank at run time (src/engine/model.rs:1286-1302,
// src/ops/softmax.rs:199-212).  The hook needs the softmax over the classes, the last axis:
// axis -1, or a non-negative axis equal to the rank minus one, where the rank is traced
// back from the MatMul's activation through MatMul with a weight, Add with a weight and
// Identity (each keeps the rank) to a Transpose (its perm's length).  The PP-OCRv6 graphs
// carry Transpose.8 perm [0,2,1] -> MatMul.12 -> Add -> Identity -> Softmax.2 axis 2 (the
// small model) and Transpose -> MatMul.0 -> Add -> MatMul.1 -> Add -> Softmax.0 axis 2 (the
// tiny one).  Graph validity checks are those of Model::load (src/engine/model.rs:40-66).
#include "model_graph.hpp"

#include <map>

#include "../../include/ppocr_rechead.h"
#include "json.hpp"

namespace ppocr {

int fail(int code, const std::string& msg);  // api.hip: sets the thread's last error

namespace {

int model_fail(const std::string& msg) { return fail(PPOCR_ERR_MODEL, "Model: " + msg); }

struct GNode {
    std::string name, op;
    std::vector<std::string> in, out;
    const JVal* attrs = nullptr;
};

bool str_array(const JVal* v, std::vector<std::string>* out) {
    if (!v || v->kind != JVal::kArr) return false;
    for (const JVal& e : v->arr) {
        if (e.kind != JVal::kStr) return false;
        out->push_back(e.s);
    }
    return true;
}

}  // namespace

int find_rec_head(const StFile& f, RecHeadNames* out) {
    const std::string* g = f.metadata("graph");
    if (!g) return model_fail("model metadata missing 'graph' definition");
    Json js{g->data(), g->data() + g->size(), {}};
    JVal root;
    if (!js.value(&root)) return model_fail("failed to parse graph JSON: " + js.err);
    js.ws();
    if (js.p != js.end || root.kind != JVal::kObj) return model_fail("failed to parse graph JSON: not one object");
    std::vector<std::string> g_in, g_out;
    if (!str_array(root.get("inputs"), &g_in) || !str_array(root.get("outputs"), &g_out))
        return model_fail("graph inputs and outputs must be lists of names");
    if (g_in.empty()) return model_fail("graph declares no inputs");
    if (g_out.empty()) return model_fail("graph declares no outputs");
    const JVal* jn = root.get("nodes");
    if (!jn || jn->kind != JVal::kArr) return model_fail("graph has no node list");

    std::vector<GNode> nodes;
    for (const JVal& v : jn->arr) {
        GNode n;
        const JVal* name = v.get("name");
        const JVal* op = v.get("op");
        if (!name || name->kind != JVal::kStr || !op || op->kind != JVal::kStr || !str_array(v.get("inputs"), &n.in) ||
            !str_array(v.get("outputs"), &n.out))
            return model_fail("a node lacks name, op, inputs or outputs");
        n.name = name->s;
        n.op = op->s;
        if (n.in.empty() || n.out.empty())
            return model_fail("node '" + n.name + "' (" + n.op + ") has " + std::to_string(n.in.size()) + " inputs and " +
                              std::to_string(n.out.size()) + " outputs; both must be non-empty");
        n.attrs = v.get("attrs");
        nodes.push_back(std::move(n));
    }

    // Identity nodes are aliases of their input
    std::map<std::string, std::string> alias;
    for (const GNode& n : nodes)
        if (n.op == "Identity") alias[n.out[0]] = n.in[0];
    auto resolve = [&](std::string s) {
        for (int hops = 0; hops < 1000; ++hops) {
            auto it = alias.find(s);
            if (it == alias.end()) break;
            s = it->second;
        }
        return s;
    };
    std::map<std::string, int> usage;
    std::map<std::string, size_t> producer;
    for (size_t i = 0; i < nodes.size(); ++i) {
        const GNode& n = nodes[i];
        if (n.op == "Identity") continue;
        for (const std::string& x : n.in) ++usage[resolve(x)];
        producer[n.out[0]] = i;
    }
    for (const std::string& o : g_out) ++usage[resolve(o)];
    auto is_output = [&](const std::string& s) {
        for (const std::string& o : g_out)
            if (resolve(o) == s) return true;
        return false;
    };
    auto made_by = [&](const std::string& s, const char* op) -> const GNode* {
        auto it = producer.find(s);
        return (it != producer.end() && nodes[it->second].op == op) ? &nodes[it->second] : nullptr;
    };
    auto is_weight = [&](const std::string& s) { return f.find(s.c_str()) != nullptr; };

    // rank of an activation, traced back to a Transpose through rank-keeping nodes (0: unknown)
    auto rank_of = [&](std::string x) -> int64_t {
        for (int hops = 0; hops < 64; ++hops) {
            x = resolve(x);
            auto it = producer.find(x);
            if (it == producer.end()) return 0;
            const GNode& p = nodes[it->second];
            if (p.op == "Transpose") {
                const JVal* perm = p.attrs ? p.attrs->get("perm") : nullptr;
                return (perm && perm->kind == JVal::kArr) ? (int64_t)perm->arr.size() : 0;
            }
            if (p.op == "MatMul" && p.in.size() == 2 && is_weight(resolve(p.in[1]))) {
                x = p.in[0];
            } else if (p.op == "Add" && p.in.size() == 2 && is_weight(resolve(p.in[1]))) {
                x = p.in[0];
            } else if (p.op == "Add" && p.in.size() == 2 && is_weight(resolve(p.in[0]))) {
                x = p.in[1];
            } else {
                return 0;
            }
        }
        return 0;
    };
    auto known_rank = [&](const GNode* mm) -> int64_t { return rank_of(mm->in[0]); };
    for (const GNode& sm : nodes) {
        if (sm.op != "Softmax") continue;
        const JVal* axis = sm.attrs ? sm.attrs->get("axis") : nullptr;
        if (axis && !(axis->kind == JVal::kNum && axis->is_int)) continue;
        const int64_t ax = axis ? axis->i : -1;
        if (ax != -1 && ax < 0) continue;
        if (!is_output(sm.out[0])) continue;
        const std::string x = resolve(sm.in[0]);
        const GNode* mm = nullptr;
        std::string bias;
        if (const GNode* add = made_by(x, "Add")) {
            if (add->in.size() != 2 || usage[x] != 1) continue;
            const std::string a0 = resolve(add->in[0]), a1 = resolve(add->in[1]);
            if (made_by(a0, "MatMul") && is_weight(a1) && usage[a0] == 1) {
                mm = made_by(a0, "MatMul");
                bias = a1;
            } else if (made_by(a1, "MatMul") && is_weight(a0) && usage[a1] == 1) {
                mm = made_by(a1, "MatMul");
                bias = a0;
            }
        } else {
            mm = made_by(x, "MatMul");
            if (mm && usage[x] != 1) mm = nullptr;
        }
        if (!mm || mm->in.size() != 2) continue;
        if (ax != -1 && known_rank(mm) != ax + 1) continue;  // softmax over the classes only
        const StTensor* w = f.find(resolve(mm->in[1]).c_str());
        if (!w || w->dtype != "F32" || w->shape.size() != 2) continue;
        const int64_t k = w->shape[0], n = w->shape[1];
        if (!bias.empty()) {
            const StTensor* b = f.find(bias.c_str());
            if (!b || b->dtype != "F32" || (int64_t)(b->bytes / 4) != n) continue;
        }
        out->weight = w->name;
        out->bias = bias;
        out->softmax = sm.name;
        out->n = n;
        out->k = k;
        return PPOCR_OK;
    }
    return model_fail("no MatMul -> [Add] -> Softmax(last axis) segment ending at a graph output");
}

}  // namespace ppocr
