// Binning, prediction and the model file format (host side).
#include "mb_host.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <exception>
#include <fstream>
#include <mutex>
#include <sstream>
#include <stdexcept>
#include <thread>

#include "mb_math.h"

namespace mb {

namespace {

// Runs fn(0 .. n_tasks - 1) on up to 16 threads. An exception thrown by a
// task stops that thread's remaining tasks and the first one is rethrown on
// the calling thread after every thread has joined.
template <class Fn>
void parallel_for(int64_t n_tasks, Fn fn) {
    int hw = (int)std::max(1u, std::thread::hardware_concurrency());
    int nt = (int)std::min<int64_t>(n_tasks, std::min(hw, 16));
    if (nt <= 1) {
        for (int64_t i = 0; i < n_tasks; ++i) fn(i);
        return;
    }
    std::mutex mu;
    std::exception_ptr first;
    std::vector<std::thread> th;
    for (int t = 0; t < nt; ++t)
        th.emplace_back([&, t] {
            try {
                for (int64_t i = t; i < n_tasks; i += nt) fn(i);
            } catch (...) {
                std::lock_guard<std::mutex> lock(mu);
                if (!first) first = std::current_exception();
            }
        });
    for (auto &x : th) x.join();
    if (first) std::rethrow_exception(first);
}

std::string bits(double x) {
    uint64_t u;
    std::memcpy(&u, &x, 8);
    return std::to_string(u);
}

double from_bits(const std::string &tok) {
    uint64_t u = std::stoull(tok);
    double d;
    std::memcpy(&d, &u, 8);
    return d;
}

// A feature name as one whitespace-free token of the model file
// (serialize._escape_name, src/mojotrees/serialize.mojo:276-319): space, tab,
// newline, carriage return and the backslash become two-character escapes,
// other control bytes are refused, every other byte (UTF-8 included) is
// copied; an empty name travels as the token "\e".
std::string escape_name(const std::string &name) {
    if (name.empty()) return "\\e";
    std::string out;
    for (unsigned char b : name) {
        switch (b) {
            case ' ': out += "\\s"; break;
            case '\t': out += "\\t"; break;
            case '\n': out += "\\n"; break;
            case '\r': out += "\\r"; break;
            case '\\': out += "\\\\"; break;
            default:
                if (b < 32 || b == 127)
                    throw std::runtime_error("feature name contains control byte " + std::to_string((int)b) +
                                             ", which the model file format cannot carry");
                out += (char)b;
        }
    }
    return out;
}

// The exact inverse (serialize._unescape_name, serialize.mojo:321-355).
std::string unescape_name(const std::string &tok) {
    if (tok == "\\e") return "";
    std::string out;
    for (size_t i = 0; i < tok.size(); ++i) {
        if (tok[i] != '\\') {
            out += tok[i];
            continue;
        }
        if (i + 1 >= tok.size()) throw std::runtime_error("corrupt feature name: token ends in an escape");
        const char c = tok[++i];
        if (c == 's') out += ' ';
        else if (c == 't') out += '\t';
        else if (c == 'n') out += '\n';
        else if (c == 'r') out += '\r';
        else if (c == '\\') out += '\\';
        else throw std::runtime_error("corrupt feature name: unknown escape");
    }
    return out;
}

// Whitespace tokens of a model file.
std::vector<std::string> file_tokens(const std::string &path) {
    std::ifstream f(path);
    if (!f) throw std::runtime_error("cannot open '" + path + "'");
    std::vector<std::string> tok;
    for (std::string s; f >> s;) tok.push_back(s);
    return tok;
}

// serialize._read_version (serialize.mojo:1372-1398): the magic, then v1..v4.
// v5 (linear leaves, CTR tables) is outside this library's models.
int read_version(const std::vector<std::string> &tok, size_t &i) {
    if (i >= tok.size() || tok[i] != "mojotrees") throw std::runtime_error("not a mojotrees model file");
    ++i;
    if (i >= tok.size()) throw std::runtime_error("truncated model file");
    const std::string &v = tok[i++];
    if (v == "v1") return 1;
    if (v == "v2") return 2;
    if (v == "v3") return 3;
    if (v == "v4") return 4;
    if (v == "v5")
        throw std::runtime_error("model file version 'v5' (linear leaves or CTR tables) is not served by this library");
    throw std::runtime_error("unsupported model file version '" + v + "'");
}

// serialize._read_feature_names (serialize.mojo:401-415): the optional
// section right after the version.
std::vector<std::string> read_feature_names(const std::vector<std::string> &tok, size_t &i) {
    std::vector<std::string> names;
    if (i >= tok.size() || tok[i] != "feature_names") return names;
    ++i;
    if (i >= tok.size()) throw std::runtime_error("truncated model file");
    const long long n = std::stoll(tok[i++]);
    if (n < 1) throw std::runtime_error("corrupt feature_names section: nonpositive count");
    if ((size_t)n > tok.size() - i) throw std::runtime_error("truncated model file");
    for (long long k = 0; k < n; ++k) names.push_back(unescape_name(tok[i++]));
    return names;
}

}  // namespace

bool BinMapper::any_cat() const {
    for (uint8_t c : is_cat)
        if (c) return true;
    return false;
}

int BinMapper::n_categories(int f) const {
    return cat_offsets.empty() ? 0 : (int)(cat_offsets[f + 1] - cat_offsets[f]);
}

int BinMapper::bin_of(int f, double v) const {
    if (!is_cat.empty() && is_cat[f]) {
        // CategoricalSpec.bin_of (categorical.mojo:296-322): missing, codes
        // out of range and unseen codes take bin 0; a fraction truncates
        if (!(v >= 0.0) || v >= 2147483648.0) return 0;
        const int64_t code = (int64_t)v;
        const int64_t *a = cat_codes.data() + cat_offsets[f], *b = cat_codes.data() + cat_offsets[f + 1];
        const int64_t *it = std::lower_bound(a, b, code);
        return (it != b && *it == code) ? (int)(it - a) + 1 : 0;
    }
    if (v != v) {
        if (missing_bin[f] >= 0) return missing_bin[f];
        v = 0.0;
    }
    const double *e = edges.data() + edge_offsets[f];
    int64_t lo = 0, hi = edge_offsets[f + 1] - edge_offsets[f];
    while (lo < hi) {
        int64_t mid = (lo + hi) / 2;
        if (v <= e[mid]) hi = mid;
        else lo = mid + 1;
    }
    return (int)lo;
}

void BinMapper::transform(const double *x, int64_t n, uint8_t *out) const {
    const int64_t blocks_per_col = (n + 262143) / 262144;
    parallel_for((int64_t)n_features * blocks_per_col, [&](int64_t task) {
        const int f = (int)(task / blocks_per_col);
        const int64_t b = task % blocks_per_col;
        const int64_t lo = b * 262144, hi = std::min(n, lo + 262144);
        for (int64_t r = lo; r < hi; ++r)
            out[(size_t)f * n + r] = (uint8_t)bin_of(f, x[(size_t)f * n + r]);
    });
}

// fit_categorical_spec's per-column table (categorical.mojo:325-464): the
// distinct non-negative codes, the keep most frequent (ties toward the smaller
// code), returned ascending.
static std::vector<int64_t> fit_category_codes(const double *col, int64_t n, int keep) {
    std::vector<int64_t> present;
    present.reserve(n);
    for (int64_t r = 0; r < n; ++r) {
        const double v = col[r];
        if (!(v >= 0.0)) continue;
        if (v >= 2147483648.0)
            throw std::invalid_argument("categorical feature values must be below 2^31; use smaller integer codes");
        present.push_back((int64_t)v);
    }
    std::sort(present.begin(), present.end());
    std::vector<int64_t> codes, counts;
    for (size_t i = 0; i < present.size();) {
        size_t j = i;
        while (j < present.size() && present[j] == present[i]) ++j;
        codes.push_back(present[i]);
        counts.push_back((int64_t)(j - i));
        i = j;
    }
    if ((int)codes.size() <= keep) return codes;
    std::vector<int> order(codes.size());
    for (size_t i = 0; i < order.size(); ++i) order[i] = (int)i;
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return counts[a] > counts[b]; });
    std::vector<int64_t> kept;
    for (int i = 0; i < keep; ++i) kept.push_back(codes[order[i]]);
    std::sort(kept.begin(), kept.end());
    return kept;
}

BinMapper fit_bins(const double *x, int64_t n, int nf, int max_bins, int min_data_in_bin,
                   bool use_missing, int64_t sample_cnt, int64_t seed, const std::vector<int> &categorical) {
    if (max_bins < 2 || max_bins > 256) throw std::invalid_argument("max_bin must be in [2, 256]");
    if (min_data_in_bin < 1) throw std::invalid_argument("min_data_in_bin must be positive");
    std::vector<uint8_t> is_cat(nf, 0);
    for (int f : categorical) {
        if (f < 0 || f >= nf) throw std::invalid_argument("categorical feature index out of range");
        if (is_cat[f]) throw std::invalid_argument("duplicate categorical feature index");
        is_cat[f] = 1;
    }
    // bin_construct_sample_rows (binning.mojo:1745): sequential selection
    // sampling keyed by the data seed.
    std::vector<int64_t> sample;
    if (!(sample_cnt <= 0 || sample_cnt >= n)) {
        uint64_t base = (uint64_t)seed * kGolden;
        int64_t need = sample_cnt;
        for (int64_t r = 0; r < n && need > 0; ++r) {
            int64_t left = n - r;
            if (need >= left || uniform53(base + (uint64_t)r) * (double)left < (double)need) {
                sample.push_back(r);
                --need;
            }
        }
    }
    const bool sampled = !sample.empty();
    const int64_t n_sample = sampled ? (int64_t)sample.size() : n;
    std::vector<std::vector<double>> per(nf);
    std::vector<int32_t> missing(nf, -1);
    std::vector<std::vector<int64_t>> codes(nf);
    parallel_for(nf, [&](int64_t fi) {
        const int f = (int)fi;
        const double *colp = x + (size_t)f * n;
        if (is_cat[f]) {  // categorical columns never enter quantile binning
            codes[f] = fit_category_codes(colp, n, max_bins - 1);
            return;
        }
        std::vector<double> col;
        col.reserve(n_sample);
        for (int64_t i = 0; i < n_sample; ++i) {
            double v = colp[sampled ? sample[i] : i];
            if (v == v) col.push_back(v);
        }
        const int64_t n_valid = (int64_t)col.size();
        const bool reserve = use_missing && n_valid < n_sample;
        const int n_ordinary = reserve ? max_bins - 1 : max_bins;
        std::sort(col.begin(), col.end());
        std::vector<double> below, above;
        // few distinct levels: edges between levels, merging levels until a
        // bin holds min_data_in_bin rows (collect_distinct, binning.mojo:1531)
        std::vector<double> lv;
        std::vector<int64_t> lc;
        bool few = true;
        for (int64_t i = 0; i < n_valid;) {
            int64_t j = i;
            while (j < n_valid && col[j] == col[i]) ++j;
            lv.push_back(col[i]);
            lc.push_back(j - i);
            if ((int64_t)lv.size() > n_ordinary) {
                few = false;
                break;
            }
            i = j;
        }
        if (few) {
            int64_t acc = 0;
            for (size_t j = 0; j + 1 < lv.size(); ++j) {
                acc += lc[j];
                if (min_data_in_bin <= 1 || acc >= min_data_in_bin) {
                    below.push_back(lv[j]);
                    above.push_back(lv[j + 1]);
                    acc = 0;
                }
            }
        } else {
            // quantile boundaries (quantile_boundary_indices, :558)
            int64_t n_ord = n_ordinary;
            if (min_data_in_bin > 1) n_ord = std::min<int64_t>(n_ord, std::max<int64_t>(1, n_valid / min_data_in_bin));
            for (int64_t b = 1; b < n_ord; ++b) {
                const int64_t idx = b * n_valid / n_ord;
                if (idx <= 0 || idx >= n_valid) continue;
                const double w = col[idx - 1];
                const int64_t e = std::upper_bound(col.begin() + idx, col.end(), w) - col.begin();
                below.push_back(w);
                above.push_back(e < n_valid ? col[e] : w);
            }
        }
        // emit_quantile_edges (:583): midpoints, strictly increasing, clamped
        std::vector<double> &out = per[f];
        for (size_t j = 0; j < below.size(); ++j) {
            const double lo = below[j], hi = above[j];
            if (hi <= lo) continue;
            double edge = (lo + hi) / 2.0;
            if (edge != edge) edge = 0.0;
            else if (edge >= 1e300) edge = 1e300;
            else if (edge <= -1e300) edge = -1e300;
            if (!out.empty() && edge <= out.back()) continue;
            out.push_back(edge);
        }
        missing[f] = reserve ? (int32_t)out.size() + 1 : -1;
    });
    BinMapper m;
    m.n_features = nf;
    m.n_bins = max_bins;
    m.missing_bin = missing;
    m.edge_offsets.assign(1, 0);
    for (int f = 0; f < nf; ++f) {
        m.edges.insert(m.edges.end(), per[f].begin(), per[f].end());
        m.edge_offsets.push_back((int64_t)m.edges.size());
    }
    if (!categorical.empty()) {
        m.is_cat = is_cat;
        m.cat_offsets.assign(1, 0);
        for (int f = 0; f < nf; ++f) {
            m.cat_codes.insert(m.cat_codes.end(), codes[f].begin(), codes[f].end());
            m.cat_offsets.push_back((int64_t)m.cat_codes.size());
        }
    }
    return m;
}

void Model::predict_raw(const double *x, int64_t n, int64_t it0, int64_t it1, double *out) const {
    const int K = num_class;
    const int64_t t0 = it0 * K, t1 = std::min<int64_t>(it1 * K, num_trees());
    const int64_t blocks = (n + 4095) / 4096;
    parallel_for(blocks, [&](int64_t b) {
        const int64_t lo = b * 4096, hi = std::min(n, lo + 4096);
        for (int64_t r = lo; r < hi; ++r) {
            for (int k = 0; k < K; ++k) out[r * K + k] = it0 == 0 ? base[k] : 0.0;
            for (int64_t t = t0; t < t1; ++t) {
                const int64_t o = offsets[t];
                int node = 0;
                while (feature[o + node] >= 0) {
                    const int f = feature[o + node];
                    const int bn = mapper.bin_of(f, x[(size_t)f * n + r]);
                    node = goes_left(o + node, bn) ? left[o + node] : right[o + node];
                }
                double &s = out[r * K + (int)(t % K)];
                s = fma(learning_rate, value[o + node], s);  // predict_raw_row, fused
            }
        }
    });
}

void Model::response(double *raw, int64_t n) const {
    if (num_class == 1) {
        if (objective == 1)
            for (int64_t r = 0; r < n; ++r) raw[r] = sigmoid(raw[r]);
        return;
    }
    const int K = num_class;
    for (int64_t r = 0; r < n; ++r) {
        double *p = raw + r * K;
        double m = p[0];
        for (int k = 1; k < K; ++k) m = std::max(m, p[k]);
        double tot = 0.0;
        for (int k = 0; k < K; ++k) {
            p[k] = ref_exp(p[k] - m);
            tot += p[k];
        }
        for (int k = 0; k < K; ++k) p[k] = p[k] / tot;
    }
}

// The reference's v4 text model format (src/mojotrees/serialize.mojo:184-545,
// :999-1121): whitespace-separated tokens, floats as the decimal of their
// IEEE-754 bits, numerical features only.
void Model::save(const std::string &path) const {
    std::ostringstream o;
    o << "mojotrees v4\n";
    if (!feature_names.empty()) {  // _write_feature_names (serialize.mojo:389-398)
        if ((int)feature_names.size() != mapper.n_features)
            throw std::runtime_error("feature_names has " + std::to_string(feature_names.size()) + " entries for " +
                                     std::to_string(mapper.n_features) + " features");
        o << "feature_names " << feature_names.size() << "\n";
        for (const std::string &nm : feature_names) o << escape_name(nm) << " ";
        o << "\n";
    }
    if (num_class == 1) {
        o << "objective " << objective << "\n";
        o << "learning_rate " << bits(learning_rate) << "\n";
        o << "base_score " << bits(base[0]) << "\n";
    } else {
        o << "multiclass " << num_class << "\n";
        o << "learning_rate " << bits(learning_rate) << "\n";
        o << "base_scores";
        for (int k = 0; k < num_class; ++k) o << " " << bits(base[k]);
        o << "\n";
    }
    o << "mapper " << mapper.n_features << " " << mapper.n_bins << " " << mapper.edges.size() << "\n";
    for (double e : mapper.edges) o << bits(e) << " ";
    o << "\n";
    for (int64_t v : mapper.edge_offsets) o << v << " ";
    o << "\n";
    for (int32_t v : mapper.missing_bin) o << v << " ";
    o << "\n";
    if (mapper.any_cat()) {  // _write_categorical (serialize.mojo:545-566)
        o << "categorical " << mapper.n_features << " " << mapper.cat_codes.size() << "\n";
        for (int f = 0; f < mapper.n_features; ++f) o << (mapper.is_cat[f] ? 1 : 0) << " ";
        o << "\n";
        for (int64_t c : mapper.cat_codes) o << c << " ";
        o << "\n";
        for (int64_t c : mapper.cat_offsets) o << c << " ";
        o << "\n";
    }
    if (!monotone.empty()) {  // _write_monotone (serialize.mojo:964-973)
        o << "monotone " << monotone.size();
        for (int32_t v : monotone) o << " " << v;
        o << "\n";
    }
    o << "trees " << num_trees() << "\n";
    for (int64_t t = 0; t < num_trees(); ++t) {
        const int64_t a = offsets[t], b = offsets[t + 1];
        o << "tree " << (b - a) << " " << n_leaves[t] << "\n";
        auto ints = [&](const std::vector<int32_t> &v) {
            for (int64_t i = a; i < b; ++i) o << v[i] << " ";
            o << "\n";
        };
        auto dbls = [&](const std::vector<double> &v) {
            for (int64_t i = a; i < b; ++i) o << bits(v[i]) << " ";
            o << "\n";
        };
        ints(feature);
        ints(threshold);
        ints(left);
        ints(right);
        dbls(value);
        ints(default_left);
        ints(missing_bin);
        bool covers = true, gains = false;
        for (int64_t i = a; i < b; ++i) {
            covers = covers && count[i] > 0.0;
            gains = gains || gain[i] > 0.0;
        }
        o << "counts " << (covers ? 1 : 0) << "\n";
        if (covers) dbls(count);
        o << "gains " << (gains ? 1 : 0) << "\n";
        if (gains) dbls(gain);
        // category sets, only for a tree with a categorical node
        // (serialize.mojo:533-543): offsets into the tree's pool, -1 numerical
        int64_t n_cat = 0;
        for (int64_t i = a; i < b; ++i) n_cat += is_cat_node[i] ? 1 : 0;
        if (n_cat > 0) {
            o << "cat " << 4 * n_cat << "\n";
            int64_t off = 0;
            for (int64_t i = a; i < b; ++i) {
                o << (is_cat_node[i] ? off : -1) << " ";
                if (is_cat_node[i]) off += 4;
            }
            o << "\n";
            for (int64_t i = a; i < b; ++i)
                if (is_cat_node[i])
                    for (int w = 0; w < 4; ++w) o << cat_bits[4 * (size_t)i + w] << " ";
            o << "\n";
        }
    }
    std::ofstream f(path);
    if (!f) throw std::runtime_error("cannot open '" + path + "' for writing");
    f << o.str();
    if (!f) throw std::runtime_error("cannot write '" + path + "'");
}

// serialize.load_model / load_multiclass_model (serialize.mojo:1463-1560)
// over the reader functions of that file: _read_version, _read_feature_names,
// _read_kind, _read_mapper (:1121-1165; v1 reserves no missing bins),
// _read_categorical (:1168-1232), _read_monotone (:976-995) and _read_trees
// (:1235-1369: v1 nodes carry no missing routing, v3 covers have no presence
// flag, v4 flags covers and gains, category sets from v2 on).
Model Model::load(const std::string &path) {
    const std::vector<std::string> tok = file_tokens(path);
    size_t i = 0;
    auto next = [&]() -> const std::string & {
        if (i >= tok.size()) throw std::runtime_error("truncated model file");
        return tok[i++];
    };
    auto peek_is = [&](const char *w) { return i < tok.size() && tok[i] == w; };
    auto expect = [&](const char *w) {
        if (next() != w) throw std::runtime_error(std::string("malformed model file: expected '") + w + "'");
    };
    auto geti = [&]() { return std::stoll(next()); };
    Model m;
    const int version = read_version(tok, i);
    m.feature_names = read_feature_names(tok, i);
    const std::string kind = next();
    if (kind == "objective") {
        m.objective = (int)geti();
        if (m.objective != 0 && m.objective != 1 && m.objective != 7)
            throw std::runtime_error("objective " + std::to_string(m.objective) + " is not served by this library");
        expect("learning_rate");
        m.learning_rate = from_bits(next());
        expect("base_score");
        m.base.push_back(from_bits(next()));
    } else if (kind == "multiclass") {
        m.objective = -1;
        m.num_class = (int)geti();
        if (m.num_class < 2) throw std::runtime_error("multiclass needs at least 2 classes");
        expect("learning_rate");
        m.learning_rate = from_bits(next());
        expect("base_scores");
        for (int k = 0; k < m.num_class; ++k) m.base.push_back(from_bits(next()));
    } else {
        throw std::runtime_error("corrupt model file: unknown model kind '" + kind + "'");
    }
    expect("mapper");
    m.mapper.n_features = (int)geti();
    m.mapper.n_bins = (int)geti();
    const int64_t ne = geti();
    if (m.mapper.n_features < 1 || ne < 0) throw std::runtime_error("corrupt mapper header");
    if (m.mapper.n_bins < 1 || m.mapper.n_bins > 256)
        throw std::runtime_error("corrupt mapper: n_bins must be in [1, 256]");
    if ((size_t)ne > tok.size() - i) throw std::runtime_error("truncated model file");
    for (int64_t k = 0; k < ne; ++k) m.mapper.edges.push_back(from_bits(next()));
    m.mapper.edge_offsets.clear();
    for (int k = 0; k <= m.mapper.n_features; ++k) m.mapper.edge_offsets.push_back(geti());
    if (m.mapper.edge_offsets[0] != 0 || m.mapper.edge_offsets.back() != ne)
        throw std::runtime_error("corrupt mapper offsets");
    for (int f = 0; f < m.mapper.n_features; ++f) {
        const int64_t w = m.mapper.edge_offsets[f + 1] - m.mapper.edge_offsets[f];
        if (w < 0) throw std::runtime_error("corrupt mapper offsets");
        if (w > m.mapper.n_bins - 1) throw std::runtime_error("corrupt mapper: more edges than bins allow");
    }
    for (int f = 0; f < m.mapper.n_features; ++f) {
        int32_t mb = -1;
        if (version >= 2) {
            mb = (int32_t)geti();
            if (mb < -1 || mb >= m.mapper.n_bins) throw std::runtime_error("corrupt mapper: missing bin out of range");
        }
        m.mapper.missing_bin.push_back(mb);
    }
    if (peek_is("categorical")) {
        next();
        const int64_t nfl = geti(), ncodes = geti();
        if (nfl != m.mapper.n_features || ncodes < 0) throw std::runtime_error("corrupt categorical header");
        for (int f = 0; f < m.mapper.n_features; ++f) m.mapper.is_cat.push_back(geti() != 0 ? 1 : 0);
        for (int64_t k = 0; k < ncodes; ++k) m.mapper.cat_codes.push_back(geti());
        for (int f = 0; f <= m.mapper.n_features; ++f) m.mapper.cat_offsets.push_back(geti());
        if (m.mapper.cat_offsets[0] != 0 || m.mapper.cat_offsets.back() != ncodes)
            throw std::runtime_error("corrupt categorical offsets");
        for (int f = 0; f < m.mapper.n_features; ++f) {
            const int64_t c0 = m.mapper.cat_offsets[f], c1 = m.mapper.cat_offsets[f + 1];
            if (c1 < c0 || c1 - c0 >= m.mapper.n_bins) throw std::runtime_error("corrupt categorical offsets");
            if (c1 > c0 && !m.mapper.is_cat[f]) throw std::runtime_error("corrupt categorical: table on a numerical feature");
            for (int64_t k = c0 + 1; k < c1; ++k)
                if (m.mapper.cat_codes[k] <= m.mapper.cat_codes[k - 1])
                    throw std::runtime_error("corrupt categorical: codes are not ascending");
        }
    }
    // _check_feature_names (serialize.mojo:417-430)
    if (!m.feature_names.empty() && (int)m.feature_names.size() != m.mapper.n_features)
        throw std::runtime_error("corrupt model file: feature_names has " + std::to_string(m.feature_names.size()) +
                                 " entries for " + std::to_string(m.mapper.n_features) + " features");
    if (peek_is("monotone")) {
        next();
        const int64_t n = geti();
        if (n != m.mapper.n_features)
            throw std::runtime_error("corrupt model file: monotone section has " + std::to_string(n) + " entries for " +
                                     std::to_string(m.mapper.n_features) + " features");
        for (int64_t k = 0; k < n; ++k) {
            const int64_t v = geti();
            if (v < -1 || v > 1) throw std::runtime_error("corrupt model file: monotone sign out of range");
            m.monotone.push_back((int32_t)v);
        }
    }
    const std::string tr = next();
    if (tr != "trees") throw std::runtime_error("section '" + tr + "' is not served by this library");
    const int64_t nt = geti();
    if (nt < 0) throw std::runtime_error("corrupt model file: negative tree count");
    for (int64_t t = 0; t < nt; ++t) {
        expect("tree");
        const int64_t nn = geti();
        const int64_t nl = geti();
        // validation.check_tree_header (src/mojotrees/validation.mojo:1253-1290)
        if (nn < 1 || nl < 1 || nl > nn || nn > 2 * nl - 1 || (size_t)nn > tok.size() - i)
            throw std::runtime_error("corrupt tree header");
        m.n_leaves.push_back((int32_t)nl);
        auto ints = [&](std::vector<int32_t> &v) {
            for (int64_t k = 0; k < nn; ++k) v.push_back((int32_t)geti());
        };
        auto dbls = [&](std::vector<double> &v) {
            for (int64_t k = 0; k < nn; ++k) v.push_back(from_bits(next()));
        };
        ints(m.feature);
        ints(m.threshold);
        ints(m.left);
        ints(m.right);
        dbls(m.value);
        if (version >= 2) {
            ints(m.default_left);
            const size_t mb0 = m.missing_bin.size();
            ints(m.missing_bin);
            for (size_t k = mb0; k < m.missing_bin.size(); ++k)
                if (m.missing_bin[k] < -1 || m.missing_bin[k] >= m.mapper.n_bins)
                    throw std::runtime_error("corrupt tree: missing bin out of range");
        } else {
            m.default_left.insert(m.default_left.end(), (size_t)nn, 0);
            m.missing_bin.insert(m.missing_bin.end(), (size_t)nn, -1);
        }
        bool has_counts = version == 3;
        if (version >= 4) {
            expect("counts");
            has_counts = geti() != 0;
        }
        if (has_counts) {
            const size_t c0 = m.count.size();
            dbls(m.count);
            int64_t zeros = 0;
            for (size_t k = c0; k < m.count.size(); ++k) {
                if (m.count[k] == 0.0) ++zeros;
                else if (!(m.count[k] > 0.0)) throw std::runtime_error("corrupt tree: node cover must be positive");
            }
            if (zeros > 0 && zeros != nn) throw std::runtime_error("corrupt tree: node cover must be positive");
        } else {
            m.count.insert(m.count.end(), (size_t)nn, 0.0);
        }
        bool has_gains = false;
        if (version >= 4) {
            expect("gains");
            has_gains = geti() != 0;
        }
        if (has_gains) {
            const size_t g0 = m.gain.size();
            dbls(m.gain);
            for (size_t k = g0; k < m.gain.size(); ++k)
                if (m.gain[k] != m.gain[k]) throw std::runtime_error("corrupt tree: split gain is NaN");
        } else {
            m.gain.insert(m.gain.end(), (size_t)nn, 0.0);
        }
        const size_t base_node = m.is_cat_node.size();
        m.is_cat_node.insert(m.is_cat_node.end(), (size_t)nn, 0);
        m.cat_bits.insert(m.cat_bits.end(), 4 * (size_t)nn, 0ULL);
        if (version >= 2 && peek_is("cat")) {
            next();
            const int64_t pool = geti();
            if (pool < 0 || pool % 4) throw std::runtime_error("corrupt cat section");
            std::vector<int64_t> off(nn);
            for (int64_t k = 0; k < nn; ++k) off[k] = geti();
            std::vector<uint64_t> words(pool);
            for (int64_t k = 0; k < pool; ++k) words[k] = std::stoull(next());
            for (int64_t k = 0; k < nn; ++k) {
                if (off[k] < 0) continue;
                if (off[k] % 4 || off[k] + 4 > pool) throw std::runtime_error("corrupt cat section: offset out of range");
                m.is_cat_node[base_node + k] = 1;
                for (int w = 0; w < 4; ++w) m.cat_bits[4 * (base_node + k) + w] = words[off[k] + w];
            }
        }
        m.offsets.push_back((int64_t)m.feature.size());
        for (int64_t k = m.offsets[t]; k < m.offsets[t + 1]; ++k) {
            const int fe = m.feature[k];
            if (fe >= m.mapper.n_features) throw std::runtime_error("node feature out of range");
            if (fe >= 0 && (m.left[k] < 0 || m.left[k] >= nn || m.right[k] < 0 || m.right[k] >= nn))
                throw std::runtime_error("node child out of range");
        }
    }
    if (i != tok.size()) throw std::runtime_error("unexpected trailing section in model file");
    if (m.num_trees() % m.num_class != 0) throw std::runtime_error("tree count is not a multiple of the class count");
    return m;
}

std::vector<std::string> Model::load_feature_names(const std::string &path) {
    const std::vector<std::string> tok = file_tokens(path);
    size_t i = 0;
    read_version(tok, i);
    return read_feature_names(tok, i);
}

std::string Model::dump_json() const {
    std::ostringstream o;
    o.precision(17);
    o << "{\"format\":\"mojotrees-inspection\",\"num_class\":" << num_class
      << ",\"objective\":" << objective << ",\"learning_rate\":" << learning_rate
      << ",\"num_features\":" << mapper.n_features << ",\"num_trees\":" << num_trees()
      << ",\"num_iterations\":" << num_iterations() << ",\"base_score\":[";
    for (int k = 0; k < num_class; ++k) o << (k ? "," : "") << base[k];
    o << "],\"feature_names\":[";
    for (int f = 0; f < mapper.n_features; ++f) o << (f ? "," : "") << "\"Column_" << f << "\"";
    bool any_gain = false;
    for (double g : gain) any_gain = any_gain || g > 0.0;
    o << "],\"has_split_gain\":" << (any_gain ? "true" : "false") << ",\"bin_mapper\":[";
    for (int f = 0; f < mapper.n_features; ++f) {
        o << (f ? "," : "") << "{\"feature\":" << f << ",\"missing_bin\":" << mapper.missing_bin[f]
          << ",\"upper_edges\":[";
        for (int64_t e = mapper.edge_offsets[f]; e < mapper.edge_offsets[f + 1]; ++e)
            o << (e > mapper.edge_offsets[f] ? "," : "") << mapper.edges[e];
        o << "]}";
    }
    o << "],\"trees\":[";
    for (int64_t t = 0; t < num_trees(); ++t) {
        const int64_t a = offsets[t], b = offsets[t + 1];
        o << (t ? "," : "") << "{\"tree_index\":" << t << ",\"class\":" << (t % num_class)
          << ",\"num_leaves\":" << n_leaves[t] << ",\"nodes\":[";
        for (int64_t k = a; k < b; ++k) {
            o << (k > a ? "," : "") << "{\"id\":" << (k - a);
            if (feature[k] >= 0) {
                const int f = feature[k];
                const int bn = threshold[k];
                const int64_t eo = mapper.edge_offsets[f];
                const int64_t ne = mapper.edge_offsets[f + 1] - eo;
                o << ",\"split_feature\":" << f << ",\"threshold_bin\":" << bn;
                if (is_cat_node[k]) {
                    // the raw category codes routed left
                    o << ",\"categories_left\":[";
                    bool first = true;
                    for (int b = 1; b < 256; ++b)
                        if ((cat_bits[4 * (size_t)k + (b >> 6)] >> (b & 63)) & 1ULL) {
                            const int64_t c = mapper.cat_offsets.empty() || b > mapper.n_categories(f)
                                                  ? -1 : mapper.cat_codes[mapper.cat_offsets[f] + b - 1];
                            o << (first ? "" : ",") << c;
                            first = false;
                        }
                    o << "]";
                } else if (bn < ne) o << ",\"threshold\":" << mapper.edges[eo + bn];
                else o << ",\"threshold\":1e300";
                o << ",\"default_left\":" << (default_left[k] ? "true" : "false")
                  << ",\"left\":" << left[k] << ",\"right\":" << right[k] << ",\"split_gain\":" << gain[k];
            } else {
                o << ",\"leaf_value\":" << value[k];
            }
            o << ",\"count\":" << count[k] << "}";
        }
        o << "]}";
    }
    o << "]}";
    return o.str();
}

}  // namespace mb
