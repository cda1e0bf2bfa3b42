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

#include <cmath>
#include <cstring>
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

namespace {

// The graph of a model file: its nodes in order, Identity aliases resolved, the producer
// and the number of uses of every value (Identity nodes excluded, graph outputs counted).
struct Graph {
    std::vector<std::string> in, out;
    std::vector<GNode> nodes;
    std::map<std::string, std::string> alias;
    std::map<std::string, int> usage;
    std::map<std::string, size_t> producer;
    JVal root;
    std::string resolve(std::string s) const {
        for (int hops = 0; hops < 1000; ++hops) {
            auto it = alias.find(s);
            if (it == alias.end()) break;
            s = it->second;
        }
        return s;
    }
};

int load_graph(const StFile& f, Graph* gr) {
    const std::string* g = f.metadata("graph");
    if (!g) return model_fail("model metadata missing 'graph' definition");
    Json js{g->data(), g->data() + g->size(), {}};
    JVal& root = gr->root;
    if (!js.value(&root)) return model_fail("failed to parse graph JSON: " + js.err);
    js.ws();
    if (js.p != js.end || root.kind != JVal::kObj) return model_fail("failed to parse graph JSON: not one object");
    std::vector<std::string>& g_in = gr->in;
    std::vector<std::string>& g_out = gr->out;
    if (!str_array(root.get("inputs"), &g_in) || !str_array(root.get("outputs"), &g_out))
        return model_fail("graph inputs and outputs must be lists of names");
    if (g_in.empty()) return model_fail("graph declares no inputs");
    if (g_out.empty()) return model_fail("graph declares no outputs");
    const JVal* jn = root.get("nodes");
    if (!jn || jn->kind != JVal::kArr) return model_fail("graph has no node list");

    std::vector<GNode>& nodes = gr->nodes;
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
    for (const GNode& n : nodes)
        if (n.op == "Identity") gr->alias[n.out[0]] = n.in[0];
    for (size_t i = 0; i < nodes.size(); ++i) {
        const GNode& n = nodes[i];
        if (n.op == "Identity") continue;
        for (const std::string& x : n.in) ++gr->usage[gr->resolve(x)];
        gr->producer[n.out[0]] = i;
    }
    for (const std::string& o : g_out) ++gr->usage[gr->resolve(o)];
    return PPOCR_OK;
}

}  // namespace

int find_rec_head(const StFile& f, RecHeadNames* out) {
    Graph gr;
    if (int e = load_graph(f, &gr)) return e;
    const std::vector<GNode>& nodes = gr.nodes;
    const std::vector<std::string>& g_out = gr.out;
    auto resolve = [&](const std::string& s) { return gr.resolve(s); };
    std::map<std::string, int>& usage = gr.usage;
    const std::map<std::string, size_t>& producer = gr.producer;
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

// The neck is read in graph order, node by node (Identity nodes are aliases and skipped),
// with each step's activation input checked against the previous step's output:
//   LayerNorm (the nine-node sub-graph the reference fuses, src/engine/model.rs:2143-2245:
//   ReduceMean, Sub, Pow(2), ReduceMean, Add(eps), Sqrt, Div, Mul(w), Add(b)),
//   MatMul [D][3D] + Add, Reshape [0, -1, 3, H, D/H], the attention (up to the next MatMul
//   with a weight: one Mul by a scalar constant, two MatMuls of activations, one Softmax),
//   MatMul [D][D] + Add, Add(residual), LayerNorm, MatMul [D][F] + Add, Sigmoid, Mul,
//   MatMul [F][D] + Add, Add(residual); blocks repeat while a LayerNorm is followed by a
//   MatMul [D][3D]; then the final LayerNorm, Reshape (after the nodes computing its shape),
//   Transpose [0,3,1,2], Add(shortcut), Squeeze and the Transpose [0,2,1] that feeds the
//   head's MatMul.
int find_rec_neck(const StFile& f, RecNeckNames* out) {
    RecHeadNames head;
    if (int e = find_rec_head(f, &head)) return e;
    Graph gr;
    if (int e = load_graph(f, &gr)) return e;
    auto bad = [](const std::string& why) { return model_fail("no SVTR neck tail before the head: " + why); };
    std::vector<const GNode*> ord;
    for (const GNode& n : gr.nodes)
        if (n.op != "Identity") ord.push_back(&n);
    auto R = [&](const std::string& s) { return gr.resolve(s); };
    auto weight = [&](const std::string& s) { return f.find(R(s).c_str()); };
    auto f32_vec = [&](const std::string& s, int64_t n) {
        const StTensor* t = weight(s);
        return t && t->dtype == "F32" && (int64_t)(t->bytes / 4) == n && t->shape.size() >= 1;
    };
    auto f32_mat = [&](const std::string& s, int64_t k, int64_t n) {
        const StTensor* t = weight(s);
        return t && t->dtype == "F32" && t->shape.size() == 2 && t->shape[0] == k && (n < 0 || t->shape[1] == n);
    };
    auto scalar = [&](const std::string& s, float* v) {
        const StTensor* t = weight(s);
        if (!t || t->dtype != "F32" || t->bytes != 4) return false;
        std::memcpy(v, t->data, 4);
        return true;
    };
    auto perm_is = [&](const GNode* n, std::initializer_list<int64_t> want) {
        const JVal* perm = n->attrs ? n->attrs->get("perm") : nullptr;
        if (!perm || perm->kind != JVal::kArr || perm->arr.size() != want.size()) return false;
        size_t i = 0;
        for (int64_t v : want)
            if (!perm->arr[i].is_int || perm->arr[i++].i != v) return false;
        return true;
    };
    auto other = [&](const GNode* n, const std::string& x, std::string* o) {
        if (n->in.size() != 2) return false;
        if (R(n->in[0]) == x) *o = R(n->in[1]);
        else if (R(n->in[1]) == x) *o = R(n->in[0]);
        else return false;
        return true;
    };
    size_t p = 0;
    auto at = [&](const char* op) { return p < ord.size() && ord[p]->op == op; };

    // LayerNorm sub-graph at p over activation x (empty: any); advances p past it
    struct Ln {
        std::string x, out, w, b;
        float eps = 0.0f;
    };
    auto layer_norm = [&](size_t q, Ln* ln) {
        static const char* kOps[9] = {"ReduceMean", "Sub", "Pow", "ReduceMean", "Add", "Sqrt", "Div", "Mul", "Add"};
        if (q + 9 > ord.size()) return false;
        for (int i = 0; i < 9; ++i)
            if (ord[q + i]->op != kOps[i]) return false;
        const GNode *rm = ord[q], *sub = ord[q + 1], *pw = ord[q + 2], *rm2 = ord[q + 3], *ae = ord[q + 4],
                    *sq = ord[q + 5], *dv = ord[q + 6], *mu = ord[q + 7], *ad = ord[q + 8];
        const std::string x = R(rm->in[0]), mean = rm->out[0], diff = sub->out[0];
        std::string two, eps, w, b;
        float v2 = 0.0f;
        if (sub->in.size() != 2 || R(sub->in[0]) != x || R(sub->in[1]) != mean) return false;
        if (pw->in.size() != 2 || R(pw->in[0]) != diff || !scalar(pw->in[1], &v2) || v2 != 2.0f) return false;
        if (R(rm2->in[0]) != pw->out[0] || !other(ae, rm2->out[0], &eps) || !scalar(eps, &ln->eps)) return false;
        if (R(sq->in[0]) != ae->out[0] || dv->in.size() != 2 || R(dv->in[0]) != diff || R(dv->in[1]) != sq->out[0])
            return false;
        if (!other(mu, dv->out[0], &w) || !other(ad, mu->out[0], &b)) return false;
        ln->x = x;
        ln->out = ad->out[0];
        ln->w = w;
        ln->b = b;
        return true;
    };
    // MatMul(x, W [k][n]) + Add(bias [n]) at p; advances p; n < 0: any, returned in *n
    auto linear = [&](const std::string& x, int64_t k, int64_t* n, std::string* w, std::string* b,
                      std::string* y) {
        if (!at("MatMul") || ord[p]->in.size() != 2 || R(ord[p]->in[0]) != x || !f32_mat(ord[p]->in[1], k, *n))
            return false;
        *w = R(ord[p]->in[1]);
        *n = weight(*w)->shape[1];
        const std::string mm = ord[p]->out[0];
        ++p;
        if (!at("Add") || !other(ord[p], mm, b) || !f32_vec(*b, *n)) return false;
        *y = ord[p]->out[0];
        ++p;
        return true;
    };

    // The attention at p, from the qkv Reshape's output r up to the next MatMul with a weight,
    // node by node, each input checked against what the steps before it produced:
    //   Transpose(r) perm [2,0,3,1,4]; q, k and v as parts 0, 1 and 2 of its first axis
    //   (Slice [i, i+1) on axis 0 then Squeeze axis 0, or Gather index i on axis 0);
    //   Mul(q, scalar) (optionally Reshape'd to Shape(q)); Transpose(k) perm [0,1,3,2];
    //   MatMul(q * scale, k^T); Softmax over the last axis; MatMul(p, v);
    //   Transpose perm [0,2,1,3]; Reshape [0,-1,D].
    // Any other node in the span (a mask or bias Add, another scaling, another Softmax
    // axis, operands wired otherwise) refuses the graph: the kernels compute exactly
    // softmax(q * scale * k^T) v per head.  Advances p to the projection MatMul.
    std::string att_why;
    auto i64s = [&](const std::string& s, std::vector<int64_t>* v) {
        const StTensor* t = weight(s);
        if (!t || t->dtype != "I64" || t->bytes % 8 != 0) return false;
        v->resize(t->bytes / 8);
        std::memcpy(v->data(), t->data, t->bytes);
        return true;
    };
    auto int_attr = [&](const GNode* n, const char* key, int64_t dflt, int64_t* v) {
        const JVal* a = n->attrs ? n->attrs->get(key) : nullptr;
        if (!a) {
            *v = dflt;
            return true;
        }
        if (!a->is_int) return false;
        *v = a->i;
        return true;
    };
    auto axes_attr_is0 = [&](const GNode* n) {
        const JVal* a = n->attrs ? n->attrs->get("axes") : nullptr;
        if (a) return a->kind == JVal::kArr && a->arr.size() == 1 && a->arr[0].is_int && a->arr[0].i == 0;
        std::vector<int64_t> v;  // opset 13: axes as a second input
        return n->in.size() == 2 && i64s(n->in[1], &v) && v.size() == 1 && v[0] == 0;
    };
    auto attention = [&](const std::string& r, int64_t D, float* scale, std::string* att) {
        enum Role { kR, kT, kSlice0, kSlice1, kSlice2, kQ, kK, kV, kQs, kShapeQ, kKt, kS, kP, kO, kOt, kAtt };
        std::map<std::string, int> role;
        role[R(r)] = kR;
        bool have[kAtt + 1] = {};
        auto role_of = [&](const std::string& x) {
            auto it = role.find(R(x));
            return it == role.end() ? -1 : it->second;
        };
        auto give = [&](const GNode* n, int rl) {
            if (have[rl]) return false;  // each value of the pattern is made once
            have[rl] = true;
            role[n->out[0]] = rl;
            return true;
        };
        auto fail_at = [&](const GNode* n, const char* why) {
            att_why = std::string(why) + " at node '" + n->name + "' (" + n->op + ")";
            return false;
        };
        for (; p < ord.size(); ++p) {
            const GNode* n = ord[p];
            if (n->op == "MatMul" && n->in.size() == 2 && weight(n->in[1])) break;
            const int r0 = role_of(n->in[0]);
            if (n->op == "Transpose") {
                if (n->in.size() != 1) return fail_at(n, "Transpose inputs");
                if (r0 == kR && perm_is(n, {2, 0, 3, 1, 4})) {
                    if (!give(n, kT)) return fail_at(n, "second q/k/v Transpose");
                } else if (r0 == kK && perm_is(n, {0, 1, 3, 2})) {
                    if (!give(n, kKt)) return fail_at(n, "second k Transpose");
                } else if (r0 == kO && perm_is(n, {0, 2, 1, 3})) {
                    if (!give(n, kOt)) return fail_at(n, "second output Transpose");
                } else {
                    return fail_at(n, "unexpected Transpose");
                }
            } else if (n->op == "Slice") {
                // Slice(data, starts, ends[, axes[, steps]]): [i, i+1) on axis 0
                std::vector<int64_t> st, en, ax{0}, sp{1};
                if (r0 != kT || n->in.size() < 3 || n->in.size() > 5 || !i64s(n->in[1], &st) || !i64s(n->in[2], &en) ||
                    (n->in.size() > 3 && !i64s(n->in[3], &ax)) || (n->in.size() > 4 && !i64s(n->in[4], &sp)))
                    return fail_at(n, "Slice of q, k, v");
                if (st.size() != 1 || en.size() != 1 || ax.size() != 1 || sp.size() != 1 || ax[0] != 0 ||
                    sp[0] != 1 || st[0] < 0 || st[0] > 2 || en[0] != st[0] + 1)
                    return fail_at(n, "Slice other than one part of axis 0");
                if (!give(n, kSlice0 + (int)st[0])) return fail_at(n, "part sliced twice");
            } else if (n->op == "Squeeze") {
                if (r0 < kSlice0 || r0 > kSlice2 || !axes_attr_is0(n)) return fail_at(n, "Squeeze of a q, k, v part");
                if (!give(n, kQ + (r0 - kSlice0))) return fail_at(n, "part squeezed twice");
            } else if (n->op == "Gather") {
                std::vector<int64_t> ix;
                int64_t axis = 0;
                if (r0 != kT || n->in.size() != 2 || !i64s(n->in[1], &ix) || ix.size() != 1 || ix[0] < 0 ||
                    ix[0] > 2 || !int_attr(n, "axis", 0, &axis) || axis != 0)
                    return fail_at(n, "Gather other than one part of axis 0");
                if (!give(n, kQ + (int)ix[0])) return fail_at(n, "part gathered twice");
            } else if (n->op == "Mul") {
                float v = 0.0f;
                if (n->in.size() != 2) return fail_at(n, "Mul inputs");
                const int r1 = role_of(n->in[1]);
                const bool ok = (r0 == kQ && r1 < 0 && scalar(n->in[1], &v)) || (r1 == kQ && r0 < 0 && scalar(n->in[0], &v));
                if (!ok) return fail_at(n, "Mul other than q by a scalar constant");
                if (!std::isfinite(v)) return fail_at(n, "non-finite attention scale");
                if (!give(n, kQs)) return fail_at(n, "second scaling of q");
                *scale = v;
            } else if (n->op == "Shape") {
                if (r0 != kQ || n->in.size() != 1) return fail_at(n, "Shape other than q's");
                if (!give(n, kShapeQ)) return fail_at(n, "second Shape");
            } else if (n->op == "Reshape") {
                if (n->in.size() != 2) return fail_at(n, "Reshape inputs");
                std::vector<int64_t> shape;
                if (r0 == kQs && role_of(n->in[1]) == kShapeQ) {
                    role[n->out[0]] = kQs;  // q * scale back to q's own shape
                } else if (r0 == kOt && i64s(n->in[1], &shape) && shape.size() == 3 && shape[0] == 0 &&
                           shape[1] == -1 && shape[2] == D) {
                    if (!give(n, kAtt)) return fail_at(n, "second output Reshape");
                } else {
                    return fail_at(n, "unexpected Reshape");
                }
            } else if (n->op == "MatMul") {
                if (n->in.size() != 2) return fail_at(n, "MatMul inputs");
                const int r1 = role_of(n->in[1]);
                if (r0 == kQs && r1 == kKt) {
                    if (!give(n, kS)) return fail_at(n, "second score MatMul");
                } else if (r0 == kP && r1 == kV) {
                    if (!give(n, kO)) return fail_at(n, "second value MatMul");
                } else {
                    return fail_at(n, "MatMul other than (q * scale) k^T or p v");
                }
            } else if (n->op == "Softmax") {
                int64_t axis = -1;
                if (r0 != kS || n->in.size() != 1 || !int_attr(n, "axis", -1, &axis) || (axis != -1 && axis != 3))
                    return fail_at(n, "Softmax other than over the keys of the scores");
                if (!give(n, kP)) return fail_at(n, "second Softmax");
            } else {
                return fail_at(n, "node outside the attention pattern");
            }
        }
        if (p >= ord.size()) {
            att_why = "no projection MatMul after it";
            return false;
        }
        if (!have[kAtt]) {
            att_why = "the pattern is incomplete";
            return false;
        }
        for (const auto& kv : role)
            if (kv.second == kAtt) *att = kv.first;
        return true;
    };

    Ln ln;
    while (p < ord.size() && !layer_norm(p, &ln)) ++p;
    if (p >= ord.size()) return bad("no LayerNorm sub-graph");
    {
        auto it = gr.producer.find(ln.x);
        if (it == gr.producer.end() || gr.nodes[it->second].op != "Transpose" ||
            !perm_is(&gr.nodes[it->second], {0, 2, 1}))
            return bad("the first LayerNorm does not read a Transpose [0,2,1]");
        out->input = R(gr.nodes[it->second].in[0]);
    }
    const StTensor* lw = weight(ln.w);
    if (!lw || lw->dtype != "F32" || lw->shape.empty()) return bad("LayerNorm weight");
    const int64_t D = (int64_t)(lw->bytes / 4);
    out->dim = D;
    std::string x = ln.x;
    for (;;) {
        RecNeckBlockNames bk;
        if (!layer_norm(p, &ln) || ln.x != x || !f32_vec(ln.w, D) || !f32_vec(ln.b, D)) break;
        // a block starts with LayerNorm -> MatMul [D][3D]; otherwise this is the final LayerNorm
        const size_t save = p;
        p += 9;
        int64_t n3 = 3 * D;
        std::string qkv;
        if (!linear(ln.out, D, &n3, &bk.qkv_w, &bk.qkv_b, &qkv)) {
            p = save;
            break;
        }
        bk.ln1_w = R(ln.w);
        bk.ln1_b = R(ln.b);
        bk.ln1_eps = ln.eps;
        if (!at("Reshape") || ord[p]->in.size() != 2 || R(ord[p]->in[0]) != qkv) return bad("qkv Reshape");
        const StTensor* shp = weight(ord[p]->in[1]);
        if (!shp || shp->dtype != "I64" || shp->bytes != 40) return bad("qkv Reshape shape");
        int64_t sv[5];
        std::memcpy(sv, shp->data, 40);
        if (sv[0] != 0 || sv[1] != -1 || sv[2] != 3 || sv[3] <= 0 || sv[4] <= 0 || sv[3] * sv[4] != D)
            return bad("qkv Reshape [0,-1,3,H,D/H]");
        if (out->heads && out->heads != sv[3]) return bad("blocks with different head counts");
        out->heads = sv[3];
        const std::string rsh = ord[p]->out[0];
        ++p;
        float scale = 0.0f;
        std::string att;
        if (!attention(rsh, D, &scale, &att)) return bad("attention: " + att_why);
        if (out->scale != 0.0f && out->scale != scale) return bad("blocks with different attention scales");
        out->scale = scale;
        if (!at("MatMul") || ord[p]->in.size() != 2 || !weight(ord[p]->in[1]) || R(ord[p]->in[0]) != att)
            return bad("attention output is not the projection MatMul's input");
        int64_t nd = D;
        std::string proj;
        if (!linear(att, D, &nd, &bk.proj_w, &bk.proj_b, &proj)) return bad("attention projection MatMul [D][D] + Add");
        std::string res;
        if (!at("Add") || !other(ord[p], R(proj), &res) || res != x) return bad("attention residual Add");
        x = ord[p]->out[0];
        ++p;
        if (!layer_norm(p, &ln) || ln.x != R(x) || !f32_vec(ln.w, D) || !f32_vec(ln.b, D)) return bad("second LayerNorm");
        bk.ln2_w = R(ln.w);
        bk.ln2_b = R(ln.b);
        bk.ln2_eps = ln.eps;
        p += 9;
        int64_t hdim = -1;
        std::string h;
        if (!linear(ln.out, D, &hdim, &bk.fc1_w, &bk.fc1_b, &h)) return bad("MLP MatMul [D][F] + Add");
        if (out->hidden && out->hidden != hdim) return bad("blocks with different MLP widths");
        out->hidden = hdim;
        if (!at("Sigmoid") || R(ord[p]->in[0]) != R(h)) return bad("MLP Sigmoid");
        const std::string sg = ord[p]->out[0];
        ++p;
        std::string o2;
        if (!at("Mul") || !other(ord[p], R(h), &o2) || o2 != R(sg)) return bad("MLP swish Mul");
        const std::string hs = ord[p]->out[0];
        ++p;
        nd = D;
        std::string f2;
        if (!linear(R(hs), hdim, &nd, &bk.fc2_w, &bk.fc2_b, &f2)) return bad("MLP MatMul [F][D] + Add");
        if (!at("Add") || !other(ord[p], R(f2), &res) || res != R(x)) return bad("MLP residual Add");
        x = ord[p]->out[0];
        ++p;
        x = R(x);
        out->blocks.push_back(bk);
    }
    if (out->blocks.empty()) return bad("no transformer block");
    if (!layer_norm(p, &ln) || ln.x != x || !f32_vec(ln.w, D) || !f32_vec(ln.b, D)) return bad("final LayerNorm");
    out->lnf_w = R(ln.w);
    out->lnf_b = R(ln.b);
    out->lnf_eps = ln.eps;
    p += 9;
    // shape arithmetic of the Reshape (Unsqueeze, Concat, ...) may come first
    for (int skip = 0; skip < 16 && p < ord.size() && !(ord[p]->op == "Reshape" && R(ord[p]->in[0]) == R(ln.out));
         ++skip) {
        for (const std::string& i : ord[p]->in)
            if (R(i) == R(ln.out)) return bad("the final LayerNorm is read before its Reshape");
        ++p;
    }
    if (!at("Reshape") || R(ord[p]->in[0]) != R(ln.out)) return bad("Reshape after the final LayerNorm");
    const std::string rs = ord[p]->out[0];
    ++p;
    if (!at("Transpose") || R(ord[p]->in[0]) != R(rs) || !perm_is(ord[p], {0, 3, 1, 2}))
        return bad("Transpose [0,3,1,2] after the final LayerNorm");
    const std::string tr = ord[p]->out[0];
    ++p;
    if (!at("Add") || !other(ord[p], R(tr), &out->shortcut)) return bad("shortcut Add");
    const std::string sum = ord[p]->out[0];
    ++p;
    if (!at("Squeeze") || R(ord[p]->in[0]) != R(sum)) return bad("Squeeze before the head");
    const std::string sq = ord[p]->out[0];
    ++p;
    if (!at("Transpose") || R(ord[p]->in[0]) != R(sq) || !perm_is(ord[p], {0, 2, 1})) return bad("Transpose [0,2,1] before the head");
    const std::string t8 = ord[p]->out[0];
    ++p;
    if (!at("MatMul") || ord[p]->in.size() != 2 || R(ord[p]->in[0]) != R(t8) || R(ord[p]->in[1]) != head.weight)
        return bad("the tail does not feed the head's MatMul");
    return PPOCR_OK;
}

}  // namespace ppocr
