"""Weight-initialisation functions (ref: src/CppNet/utils/init.cpp:21-130) on
the host, no GPU: a C++ program linked against libcppnet.so draws each
method's matrix after Utils::set_seed and prints it; the test checks each
draw against the distribution the reference fixes for that method:

  xavier / glorot              U(+-sqrt(6/(rows+cols)))   (init.cpp:21-33)
  xavier_normal                N(0, sqrt(2/(rows+cols)))  (init.cpp:35-47)
  he / kaiming                 U(+-sqrt(6/rows))          (init.cpp:49-61)
  he_normal                    N(0, sqrt(2/rows))         (init.cpp:63-75)
  uniform (defaults)           U(-1, 1)                   (init.hpp default args)
  normal (defaults)            N(0, 0.01)
  zeros / ones                 constants                  (init.cpp:101-106)

A uniform draw is pinned by its support (every |w| <= L and the largest
within 25/n of L, which fails with probability e^-25 for a correct draw)
and its first two moments (6-sigma bounds); a normal draw by mean and
variance (6 sigma).  A wrong fan (rows instead of rows + cols), a sqrt(2)
for a sqrt(6), or a swapped uniform/normal each miss these bounds by a
wide margin.  Seeding: equal seeds give equal draws, different seeds differ.
The reference's generator is seeded from std::random_device (init.cpp:17),
so draws themselves are not comparable with it; the distributions are.
"""
import json
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

from init_stats import check_normal, check_uniform

ROOT = Path(__file__).resolve().parents[1]
LIB = ROOT / "cppnet_amd" / "_lib"

PROGRAM = r'''
#include <CppNet/utils/init.hpp>
#include <cstdio>
#include <stdexcept>
#include <string>
using namespace CppNet;

static void dump(const char* name, const Tensor<float, 2>& w) {
    std::printf("\"%s\": [%lld, %lld, [", name, (long long)w.dimension(0), (long long)w.dimension(1));
    for (long long i = 0; i < w.size(); ++i) std::printf(i ? ",%.9g" : "%.9g", w.data()[i]);
    std::printf("]],\n");
}

int main() {
    const int R = 150, C = 250;
    std::printf("{\n");
    const char* methods[] = {"xavier", "glorot", "xavier_normal", "glorot_normal", "he", "kaiming",
                             "he_normal", "kaiming_normal", "uniform", "normal", "zeros", "ones"};
    for (const char* m : methods) {
        Utils::set_seed(7);
        dump(m, Utils::init_weights(R, C, m));
    }
    Utils::set_seed(7);
    dump("xavier_direct", Utils::xavier_uniform(R, C));
    Utils::set_seed(8);
    dump("xavier_seed8", Utils::xavier_uniform(R, C));
    Utils::set_seed(7);
    dump("uniform_range", Utils::uniform_init(R, C, 2.0f, 3.0f));
    Utils::set_seed(7);
    dump("normal_args", Utils::normal_init(R, C, 5.0f, 0.5f));
    dump("constant", Utils::constant_init(3, 4, 2.5f));
    std::string msg;
    try { Utils::init_weights(2, 2, "bogus"); } catch (const std::invalid_argument& e) { msg = e.what(); }
    std::printf("\"unknown_msg\": \"%s\"\n}\n", msg.c_str());
    return 0;
}
'''


@pytest.fixture(scope="module")
def draws(tmp_path_factory):
    if shutil.which("g++") is None:
        pytest.skip("no host C++ compiler")
    if not (LIB / "libcppnet.so").exists():
        pytest.skip("libraries not built (python -m cppnet_amd.build)")
    d = tmp_path_factory.mktemp("init")
    (d / "init.cpp").write_text(PROGRAM)
    exe = d / "init"
    cmd = ["g++", "-std=c++17", "-O1", f"-I{ROOT / 'cppnet_amd' / 'include'}", f"-I{ROOT / 'include'}",
           str(d / "init.cpp"), f"-L{LIB}", "-lcppnet", "-lcnhip", f"-Wl,-rpath,{LIB}", "-o", str(exe)]
    res = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stderr[-4000:]
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, run.stderr[-4000:]
    raw = json.loads(run.stdout)
    out = {"unknown_msg": raw.pop("unknown_msg")}
    for k, (r, c, vals) in raw.items():
        # ColMajor [r, c] -> logical (r, c) array
        out[k] = np.asarray(vals, np.float64).reshape(c, r).T
    return out


R, C = 150, 250


@pytest.mark.parametrize("m", ["xavier", "glorot", "xavier_direct"])
def test_xavier_uniform(draws, m):
    L = np.sqrt(6.0 / (R + C))
    check_uniform(draws[m], -L, L)


@pytest.mark.parametrize("m", ["xavier_normal", "glorot_normal"])
def test_xavier_normal(draws, m):
    check_normal(draws[m], 0.0, np.sqrt(2.0 / (R + C)))


@pytest.mark.parametrize("m", ["he", "kaiming"])
def test_he_uniform(draws, m):
    L = np.sqrt(6.0 / R)
    check_uniform(draws[m], -L, L)


@pytest.mark.parametrize("m", ["he_normal", "kaiming_normal"])
def test_he_normal(draws, m):
    check_normal(draws[m], 0.0, np.sqrt(2.0 / R))


def test_default_ranges(draws):
    check_uniform(draws["uniform"], -1.0, 1.0)
    check_normal(draws["normal"], 0.0, 0.01)
    check_uniform(draws["uniform_range"], 2.0, 3.0)
    check_normal(draws["normal_args"], 5.0, 0.5)


def test_constants(draws):
    assert np.all(draws["zeros"] == 0.0) and draws["zeros"].shape == (R, C)
    assert np.all(draws["ones"] == 1.0)
    assert np.all(draws["constant"] == 2.5) and draws["constant"].shape == (3, 4)


def test_seeding(draws):
    # aliases draw the same matrix from the same seed; another seed differs
    assert np.array_equal(draws["xavier"], draws["glorot"])
    assert np.array_equal(draws["xavier"], draws["xavier_direct"])
    assert np.array_equal(draws["he_normal"], draws["kaiming_normal"])
    assert not np.array_equal(draws["xavier"], draws["xavier_seed8"])
    # he and xavier differ only by their limit: the same underlying uniforms
    # scaled, so the ratio is the ratio of limits
    ratio = np.sqrt(6.0 / R) / np.sqrt(6.0 / (R + C))
    np.testing.assert_allclose(draws["he"], draws["xavier"] * ratio, rtol=2e-6, atol=1e-7)


def test_unknown_method_message(draws):
    # init.cpp:127-128
    assert draws["unknown_msg"] == "Unknown weight initialization method: bogus"
