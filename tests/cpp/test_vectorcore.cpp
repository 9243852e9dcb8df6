// C++ suite of the VectorCore runtime, linked against libvectorcore.so (or
// compiled with its sources under ASan+UBSan or TSan).
//
// It restates the known-answer cases of the reference's C++ suite
// (tests/cpp/test_vectorcore.cpp) and runs each on every device named in
// VECTORCORE_TEST_DEVICES ("cpu", "hip"; default "cpu,hip", hip skipped when
// no GPU is present), plus cases the reference does not have: cpu kernels
// driven from several threads at once, a small MLP train step on hip against
// the cpu device, and the oracle's C kernels against the cpu device. Exit
// status 0 when every case passes.
#include "vectorcore/vectorcore.hpp"

extern "C" {
#include "vc_oracle.h"
}

#include <cmath>
#include <cstdlib>
#include <functional>
#include <iostream>
#include <random>
#include <sstream>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

using namespace vectorcore;

namespace {

struct Failure : std::runtime_error {
    using std::runtime_error::runtime_error;
};

void expect(bool ok, const std::string& what) {
    if (!ok) throw Failure(what);
}

void expect_values(const Tensor& t, const std::vector<float>& want, float tol = 1e-5F) {
    const std::vector<float> got = t.to(Device::cpu()).to_vector();
    expect(got.size() == want.size(), "size " + std::to_string(got.size()) + " != " + std::to_string(want.size()));
    for (std::size_t i = 0; i < got.size(); ++i) {
        if (!(std::fabs(got[i] - want[i]) <= tol)) {
            std::ostringstream s;
            s << "element " << i << ": " << got[i] << " != " << want[i];
            throw Failure(s.str());
        }
    }
}

template <class F>
void expect_throw(F&& f, const std::string& what) {
    try {
        f();
    } catch (const Failure&) {
        throw;
    } catch (const std::exception&) {
        return;
    }
    throw Failure("no exception: " + what);
}

std::vector<float> random_values(std::size_t n, unsigned seed) {
    std::mt19937 gen(seed);
    std::uniform_real_distribution<float> dist(-1.0F, 1.0F);
    std::vector<float> v(n);
    for (auto& x : v) x = dist(gen);
    return v;
}

struct Case {
    std::string name;
    std::function<void(Device)> run;
    bool cpu_only = false;
};

std::vector<Case> cases() {
    std::vector<Case> c;
    c.push_back({"shape, strides, scalar and indexing", [](Device d) {
        Tensor t({1, 2, 3, 4, 5, 6}, {2, 3}, false, d);
        expect(t.shape() == Shape({2, 3}) && t.strides() == Strides({3, 1}), "shape/strides");
        expect(t.at({1, 2}) == 6.0F, "at");
        expect(Tensor::scalar(4.0F, false, d).shape().empty(), "scalar rank");
        expect_throw([&] { (void)t.at({3, 0}); }, "index out of range");
        expect_throw([&] { Tensor({1, 2}, {3}, false, d); }, "values do not fill the shape");
    }});
    c.push_back({"reshape shares storage", [](Device d) {
        Tensor t({1, 2, 3, 4}, {2, 2});
        Tensor flat = t.flatten();
        flat.set_at({2}, 8.0F);
        expect(t.at({1, 0}) == 8.0F, "view write not visible");
        expect(flat.shape() == Shape({4}), "flatten shape");
        expect_throw([&] { (void)Tensor({1, 2, 3, 4}, {2, 2}, false, d).reshape({3, 2}); }, "bad reshape");
    }, true});
    c.push_back({"elementwise ops and scalars", [](Device d) {
        Tensor a({1, 2, 3, 4}, {2, 2}, false, d), b({4, 3, 2, 1}, {2, 2}, false, d);
        expect_values(a + b, {5, 5, 5, 5});
        expect_values(a - b, {-3, -1, 1, 3});
        expect_values(a * b, {4, 6, 6, 4});
        expect_values(a / b, {0.25F, 2.0F / 3.0F, 1.5F, 4});
        expect_values(-a, {-1, -2, -3, -4});
        expect_values(2.0F + a * 2.0F, {4, 6, 8, 10});
    }});
    c.push_back({"broadcasting", [](Device d) {
        Tensor m({1, 2, 3, 4, 5, 6}, {2, 3}, false, d);
        expect_values(m + Tensor({10, 20, 30}, {3}, false, d), {11, 22, 33, 14, 25, 36});
        expect_values(m + Tensor({10, 20, 30}, {1, 3}, false, d), {11, 22, 33, 14, 25, 36});
        expect_values(m + Tensor::scalar(2.0F, false, d), {3, 4, 5, 6, 7, 8});
        std::vector<float> pattern;
        for (int r = 0; r < 6; ++r) pattern.insert(pattern.end(), {1, 2, 3, 4});
        expect_values(Tensor::ones({2, 3, 4}, false, d) * Tensor({1, 2, 3, 4}, {1, 4}, false, d), pattern);
        expect_throw([&] { (void)(m + Tensor::ones({2, 2}, false, d)); }, "incompatible broadcast");
    }});
    c.push_back({"matmul and transpose", [](Device d) {
        Tensor a({1, 2, 3, 4, 5, 6}, {2, 3}, false, d), b({7, 8, 9, 10, 11, 12}, {3, 2}, false, d);
        expect_values(a.matmul(b), {58, 64, 139, 154});
        expect_values(a.transpose(), {1, 4, 2, 5, 3, 6});
        expect_throw([&] { (void)a.matmul(Tensor::ones({4, 2}, false, d)); }, "inner mismatch");
    }});
    c.push_back({"reductions and activations", [](Device d) {
        Tensor v({-2, -1, 0, 1, 2}, {5}, false, d);
        expect(v.sum().item() == 0.0F && v.mean().item() == 0.0F, "sum/mean");
        expect_values(v.relu(), {0, 0, 0, 1, 2});
        expect(std::fabs(v.sigmoid().to_vector()[2] - 0.5F) < 1e-6F, "sigmoid(0)");
        expect(Tensor::zeros({0}, false, d).sum().item() == 0.0F, "empty sum");
        expect_throw([&] { (void)Tensor::zeros({0}, false, d).mean(); }, "mean of nothing");
    }});
    c.push_back({"gradient of a repeated use", [](Device d) {
        Tensor x({1, 2, 3}, {3}, true, d);
        ((x * x) + x).sum().backward();
        expect_values(x.grad(), {3, 5, 7});
        x.zero_grad();
        expect(!x.has_grad(), "zero_grad");
    }});
    c.push_back({"broadcast gradient is summed", [](Device d) {
        Tensor x({1, 2, 3, 4, 5, 6}, {2, 3}, true, d), bias({0.1F, 0.2F, 0.3F}, {3}, true, d);
        (x + bias).sum().backward();
        expect_values(x.grad(), {1, 1, 1, 1, 1, 1});
        expect_values(bias.grad(), {2, 2, 2});
    }});
    c.push_back({"matmul gradients", [](Device d) {
        Tensor a({1, 2, 3, 4, 5, 6}, {2, 3}, true, d), b({1, 2, 3, 4, 5, 6}, {3, 2}, true, d);
        a.matmul(b).sum().backward();
        expect_values(a.grad(), {3, 7, 11, 3, 7, 11});
        expect_values(b.grad(), {5, 5, 7, 7, 9, 9});
    }});
    c.push_back({"sigmoid through a reshape", [](Device d) {
        Tensor x({-1, 0, 1, 2}, {2, 2}, true, d);
        x.reshape({4}).sigmoid().sum().backward();
        std::vector<float> want;
        for (float y : x.detach().sigmoid().to_vector()) want.push_back(y * (1.0F - y));
        expect_values(x.grad(), want);
    }});
    c.push_back({"finite differences", [](Device d) {
        const std::vector<float> base{0.3F, -0.7F, 1.2F};
        Tensor x(base, {3}, true, d);
        (x * x).sigmoid().sum().backward();
        const std::vector<float> analytic = x.grad().to_vector();
        const float h = 1e-3F;
        for (std::size_t i = 0; i < base.size(); ++i) {
            std::vector<float> up = base, down = base;
            up[i] += h;
            down[i] -= h;
            const auto f = [&](const std::vector<float>& v) {
                Tensor t(v, {3}, false, d);
                return (t * t).sigmoid().sum().item();
            };
            expect(std::fabs(analytic[i] - (f(up) - f(down)) / (2 * h)) < 3e-3F, "finite difference");
        }
    }});
    c.push_back({"gradients accumulate across backward calls", [](Device d) {
        Tensor x({1, 2}, {2}, true, d);
        (x * 3.0F).sum().backward();
        (x * 4.0F).sum().backward();
        expect_values(x.grad(), {7, 7});
    }});
    c.push_back({"linear regression converges", [](Device d) {
        Tensor input({-2, -1, 0, 1, 2}, {5, 1}, false, d), target({-3, -1, 1, 3, 5}, {5, 1}, false, d);
        nn::Linear model(1, 1, 7);
        model.weight = model.weight.to(d).detach();
        model.weight.set_requires_grad(true);
        model.bias = model.bias.to(d).detach();
        model.bias.set_requires_grad(true);
        const float first = nn::mse_loss(model(input), target).item();
        for (int epoch = 0; epoch < 150; ++epoch) {
            nn::mse_loss(model(input), target).backward();
            nn::sgd_step(model.parameters(), 0.08F);
            nn::zero_grad(model.parameters());
        }
        const float last = nn::mse_loss(model(input), target).item();
        expect(last < first * 1e-3F && last < 1e-4F, "did not converge");
    }});
    c.push_back({"metal is reported unavailable", [](Device) {
        expect(!metal_available(), "no Metal device in this build");
        expect_throw([] { (void)Tensor::ones({2}).to(Device::metal()); }, "to(metal)");
    }, true});
    c.push_back({"version counter shared by views", [](Device d) {
        // set_at writes cpu tensors only (as in the reference); sgd_step is
        // the in-place write every device has.
        Tensor v({1, 2, 3, 4}, {2, 2}, true, d);
        Tensor view = v.reshape({4});
        const auto start = v.version();
        (void)(v + v);
        expect(v.version() == start, "out-of-place op bumped the version");
        (v * 1.0F).sum().backward();
        nn::sgd_step({&v}, 0.5F);
        expect(v.version() == start + 1 && view.version() == v.version(), "update not counted on both views");
        if (d == Device::cpu()) {
            view.set_at({0}, 5.0F);
            expect(v.version() == start + 2 && v.at({0, 0}) == 5.0F, "set_at");
        } else {
            expect_throw([&] { view.set_at({0}, 5.0F); }, "set_at on a device tensor");
        }
    }});
    c.push_back({"in-place writes between forward and backward are rejected", [](Device d) {
        Tensor w({2.0F}, {1}, true, d), x({3.0F}, {1}, true, d);
        Tensor loss = (w * x).sum();
        (w * 1.0F).sum().backward();
        nn::sgd_step({&w}, 1.0F);
        expect_throw([&] { loss.backward(); }, "stale saved operand");
        Tensor a({1, 2, 3, 4}, {2, 2}, true, d), b({1, 0, 0, 1}, {2, 2}, true, d);
        Tensor product = a.matmul(b).sum();
        (b * 1.0F).sum().backward();
        nn::sgd_step({&b}, 0.0F);
        expect_throw([&] { product.backward(); }, "update after forward");
        if (d == Device::cpu()) {
            Tensor s({0.5F, -0.5F}, {2}, true, d);
            Tensor y = s.sigmoid();
            Tensor sig_loss = y.sum();
            Tensor alias = y.detach();
            alias.set_at({0}, 0.0F);
            expect_throw([&] { sig_loss.backward(); }, "saved output modified");
        }
    }});
    c.push_back({"only leaves keep gradients unless retained", [](Device d) {
        Tensor a({1, 2}, {2}, true, d);
        Tensor hidden = a * 2.0F, kept = a * 3.0F;
        kept.retain_grad();
        ((hidden * hidden).sum() + kept.sum()).backward();
        expect(a.is_leaf() && !hidden.is_leaf() && !hidden.has_grad(), "leaf flags");
        expect_values(kept.grad(), {1, 1});
        expect_values(a.grad(), {11, 19});
        expect_throw([&] { Tensor({1.0F}, {1}, false, d).retain_grad(); }, "retain_grad without grad");
    }});
    c.push_back({"axis reductions, exp, log, softmax", [](Device d) {
        Tensor x({1, 5, 3, 4, 2, 6}, {2, 3}, false, d);
        expect_values(x.sum(0), {5, 7, 9});
        expect_values(x.sum(-1, true), {9, 12});
        expect(x.sum(1, true).shape() == Shape({2, 1}), "keepdim");
        expect_values(x.mean(1), {3, 4});
        expect_values(x.max(1), {5, 6});
        expect_values(x.argmax(1), {1, 2});
        expect_values(x.max(), {6});
        expect_values(Tensor({0.0F, 1.0F}, {2}, false, d).exp(), {1.0F, std::exp(1.0F)});
        expect_values(Tensor({1.0F, std::exp(2.0F)}, {2}, false, d).log(), {0.0F, 2.0F});
        expect_values(x.softmax(1).sum(1), {1, 1}, 1e-6F);
        expect_throw([&] { (void)x.sum(2); }, "axis 2");
        expect_throw([&] { (void)x.max(-3); }, "axis -3");
        expect_throw([&] { (void)Tensor::scalar(1.0F, false, d).sum(0); }, "axis of a scalar");
    }});
    c.push_back({"cross-entropy value and gradient", [](Device d) {
        Tensor logits({0, 0, 0, 0}, {2, 2}, true, d);
        Tensor loss = nn::cross_entropy(logits, {0, 1});
        expect(std::fabs(loss.item() - std::log(2.0F)) < 1e-6F, "uniform logits give log 2");
        loss.backward();
        expect_values(logits.grad(), {-0.25F, 0.25F, 0.25F, -0.25F});
        expect_throw([&] { (void)nn::cross_entropy(logits, {0}); }, "target count");
        expect_throw([&] { (void)nn::cross_entropy(logits, {0, 2}); }, "target out of range");
    }});
    c.push_back({"batched and broadcast matmul", [](Device d) {
        Tensor a({1, 2, 3, 4}, {2, 1, 2}, true, d), w({1, 0, 0, 2}, {2, 2}, true, d);
        Tensor y = a.matmul(w);
        expect(y.shape() == Shape({2, 1, 2}), "batched shape");
        expect_values(y, {1, 4, 3, 8});
        y.sum().backward();
        expect_values(w.grad(), {4, 4, 6, 6});
        expect_values(a.grad(), {1, 2, 1, 2});
        expect_values(Tensor({1, 2, 3, 4, 5, 6, 7, 8}, {2, 2, 2}, false, d).transpose(), {1, 3, 2, 4, 5, 7, 6, 8});
        expect_throw([&] { (void)Tensor::ones({2, 2, 3}, false, d).matmul(Tensor::ones({3, 3, 1}, false, d)); },
                     "batch mismatch");
    }});
    c.push_back({"relu and bias gradients, and an SGD step", [](Device d) {
        Tensor gx({-1, 2, 3, -4, 5, 6}, {2, 3}, true, d), gb({0.5F, 1.0F, -2.0F}, {3}, true, d);
        (gx + gb).relu().sum().backward();
        expect_values(gx.grad(), {0, 1, 1, 0, 1, 1});
        expect_values(gb.grad(), {0, 2, 2});
        Tensor p({1, 2}, {2}, true, d);
        (p * p).sum().backward();
        nn::sgd_step({&p}, 0.5F);
        expect_values(p, {0, 0});
    }});
    c.push_back({"threaded cpu kernels against double sums", [](Device d) {
        const std::size_t m = 150, k = 300, n = 130;
        const auto av = random_values(m * k, 3), bv = random_values(k * n, 4);
        Tensor a(av, {m, k}, false, d), b(bv, {k, n}, false, d);
        const std::vector<float> c = a.matmul(b).to_vector();
        for (std::size_t i = 0; i < m; i += 7)
            for (std::size_t j = 0; j < n; j += 5) {
                double want = 0.0;
                for (std::size_t p = 0; p < k; ++p) want += double(av[i * k + p]) * bv[p * n + j];
                expect(std::fabs(c[i * n + j] - want) < 1e-3, "product element");
            }
        Tensor x(av, {m, k}, true, d), w(bv, {k, n}, true, d);
        x.matmul(w).sum().backward();
        const std::vector<float> gx = x.grad().to_vector();
        for (std::size_t p = 0; p < k; p += 11) {
            double row = 0.0;
            for (std::size_t j = 0; j < n; ++j) row += bv[p * n + j];
            expect(std::fabs(gx[p] - row) < 1e-3, "gradient through the transposed operand");
        }
        const auto big = random_values(1000 * 300, 7), row = random_values(300, 8);
        Tensor tb(big, {1000, 300}, false, d), tr(row, {300}, false, d);
        const float s1 = (tb + tr).sum().item(), s2 = (tb + tr).sum().item();
        expect(s1 == s2, "sum is not deterministic");
        double want = 0.0;
        for (std::size_t i = 0; i < big.size(); ++i) want += double(big[i] + row[i % 300]);
        expect(std::fabs(s1 - want) < 1e-2, "broadcast sum");
    }});
    c.push_back({"cpu kernels from several threads at once", [](Device) {
        // Each thread runs parallel reductions and products on the shared
        // pool; results must equal the single-threaded ones bit for bit.
        const auto data = random_values(700 * 513, 11), w = random_values(513 * 70, 12);
        Tensor x(data, {700, 513}), tw(w, {513, 70});
        const std::vector<float> col = x.sum(0).to_vector(), prod = x.matmul(tw).to_vector();
        const float total = x.sum().item();
        std::vector<std::thread> threads;
        std::vector<int> ok(6, 0);
        for (int t = 0; t < 6; ++t) {
            threads.emplace_back([&, t] {
                bool same = true;
                for (int rep = 0; rep < 4; ++rep) {
                    same = same && x.sum(0).to_vector() == col;
                    same = same && x.matmul(tw).to_vector() == prod;
                    same = same && x.sum().item() == total;
                }
                ok[t] = same ? 1 : 0;
            });
        }
        for (auto& th : threads) th.join();
        for (int t = 0; t < 6; ++t) expect(ok[t] == 1, "thread " + std::to_string(t) + " saw different bits");
    }, true});
    c.push_back({"an exception inside a parallel region reaches the caller", [](Device) {
        // Mismatched shapes are caught before the kernels; a NaN-free sum
        // after a failed call shows the pool is still usable.
        for (int i = 0; i < 3; ++i)
            expect_throw([] { (void)Tensor::ones({300, 200}).matmul(Tensor::ones({100, 3})); }, "shape error");
        expect(Tensor::ones({1000, 1000}).sum().item() == 1e6F, "pool unusable after an error");
    }, true});
    c.push_back({"cpu device equals the oracle's C kernels", [](Device) {
        const std::size_t m = 37, k = 300, n = 45;
        const auto av = random_values(m * k, 21), bv = random_values(k * n, 22);
        std::vector<float> want(m * n);
        vco_matmul(av.data(), bv.data(), want.data(), m, k, n, 0, 0);
        expect(Tensor(av, {m, k}).matmul(Tensor(bv, {k, n})).to_vector() == want, "GEMM bits");
        const auto big = random_values(3 * 65536 + 7, 23);
        expect(Tensor(big, {big.size()}).sum().item() == vco_sum(big.data(), big.size()), "sum bits");
        std::vector<float> colsum(45);
        const auto grid = random_values(900 * 45, 24);
        vco_reduce_axis(grid.data(), colsum.data(), 1, 900, 45, 0);
        expect(Tensor(grid, {900, 45}).sum(0).to_vector() == colsum, "axis sum bits");
    }, true});
    c.push_back({"MLP train step on hip against the cpu device", [](Device d) {
        if (d != Device::hip()) return;
        const std::size_t rows = 96, in = 40, hidden = 72, classes = 10;
        const auto xv = random_values(rows * in, 31), w1 = random_values(in * hidden, 32),
                   w2 = random_values(hidden * classes, 33);
        std::vector<std::size_t> targets(rows);
        for (std::size_t r = 0; r < rows; ++r) targets[r] = (r * 7) % classes;
        std::vector<std::vector<float>> results;
        for (Device dev : {Device::cpu(), Device::hip()}) {
            Tensor x(xv, {rows, in}, false, dev);
            Tensor a(w1, {in, hidden}, true, dev), b(std::vector<float>(hidden, 0.01F), {hidden}, true, dev);
            Tensor c2(w2, {hidden, classes}, true, dev);
            std::vector<Tensor*> params{&a, &b, &c2};
            std::vector<float> out;
            for (int step = 0; step < 3; ++step) {
                Tensor loss = nn::cross_entropy((x.matmul(a) + b).relu().matmul(c2), targets);
                loss.backward();
                nn::sgd_step(params, 0.1F);
                nn::zero_grad(params);
                out.push_back(loss.item());
            }
            for (Tensor* p : params)
                for (float v : p->to(Device::cpu()).to_vector()) out.push_back(v);
            results.push_back(out);
        }
        expect(results[0].size() == results[1].size(), "result sizes");
        for (std::size_t i = 0; i < results[0].size(); ++i)
            expect(std::fabs(results[0][i] - results[1][i]) <= 1e-4F * (1.0F + std::fabs(results[0][i])),
                   "hip and cpu differ at value " + std::to_string(i));
    }});
    return c;
}

std::vector<Device> devices() {
    const char* env = std::getenv("VECTORCORE_TEST_DEVICES");
    const std::string spec = env ? env : "cpu,hip";
    std::vector<Device> out;
    std::stringstream s(spec);
    std::string item;
    while (std::getline(s, item, ',')) {
        if (item == "cpu") out.push_back(Device::cpu());
        else if (item == "hip") {
            if (hip_available()) out.push_back(Device::hip());
            else std::cout << "hip unavailable: " << HipBackend::instance().last_error() << "\n";
        } else if (!item.empty()) {
            std::cerr << "unknown device " << item << "\n";
            std::exit(2);
        }
    }
    return out;
}

}  // namespace

int main() {
    int run = 0, failed = 0;
    const auto devs = devices();
    for (const Case& c : cases()) {
        for (Device d : devs) {
            if (c.cpu_only && d != Device::cpu()) continue;
            ++run;
            try {
                c.run(d);
                std::cout << "[PASS] " << c.name << " (" << d.str() << ")\n";
            } catch (const std::exception& e) {
                ++failed;
                std::cout << "[FAIL] " << c.name << " (" << d.str() << "): " << e.what() << "\n";
            }
        }
    }
    synchronize();
    std::cout << run - failed << "/" << run << " cases passed\n";
    return failed == 0 ? 0 : 1;
}
