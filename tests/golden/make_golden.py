"""Writes tests/golden/known_answers.json.

The fixtures are the known-answer vectors that the reference's own test suite
(LoqmanSamani/CppNet, tests/) asserts for the ops on the hot path, transcribed
as data: inputs, expected outputs, the reference's tolerance and the test
file:line they come from.  Matrices are given logically, row by row
(``[[row0...], [row1...]]``), exactly as the reference's ``setValues`` calls
write them; tests convert to Eigen ColMajor memory order.

Where the reference only asserts a sign or an inequality, the entry states
that predicate ("check") and, when the mathematics fixes the exact value, the
exact value as well ("exact", derived by hand in the "derivation" field).

Run:  python tests/golden/make_golden.py
"""
import json
import math
from pathlib import Path

HERE = Path(__file__).resolve().parent


def sig(x):
    return 1.0 / (1.0 + math.exp(-x))


def softmax(row):
    m = max(row)
    e = [math.exp(v - m) for v in row]
    s = sum(e)
    return [v / s for v in e]


CASES = [
    # ---- Linear ------------------------------------------------------------
    dict(op="linear_forward", source="tests/layers/test_linear.cpp:108-129",
         X=[[3.0, 4.0]], W=[[1.0, 0.0], [0.0, 1.0]], b=[0.5, -0.5],
         expected=[[3.5, 3.5]], tol=1e-4),
    dict(op="linear_forward", source="tests/kernels/test_matmul_gpu.cu:69-90",
         X=[[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]],
         W=[[1.0, 0.0, 0.0], [0.0, 1.0, 0.0], [0.0, 0.0, 1.0]], b=None,
         expected=[[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]], tol=1e-3),
    dict(op="linear_forward", source="tests/kernels/test_matmul_gpu.cu:92-109",
         X=[[3.0, 4.0]], W=[[1.0, 0.0], [0.0, 1.0]], b=[0.5, -0.5],
         expected=[[3.5, 3.5]], tol=1e-3),
    # ---- ReLU ----------------------------------------------------------------
    dict(op="relu_backward", source="tests/activations/test_relu.cpp:100-118",
         X=[[-1.0, 2.0, -3.0], [4.0, -5.0, 0.0]], dY=[[1.0, 1.0, 1.0], [1.0, 1.0, 1.0]],
         check="zero where input <= 0, positive where input > 0",
         exact=[[0.0, 1.0, 0.0], [1.0, 0.0, 0.0]],
         derivation="mask = (relu(x) > 0); dx = dy * mask; relu(0) = 0 so x = 0 is gated",
         tol=1e-6),
    # ---- Sigmoid -------------------------------------------------------------
    dict(op="sigmoid_forward", source="tests/activations/test_sigmoid.cpp:79-89",
         X=[[-2.0, -1.0, 1.0, 2.0]], expected=[[sig(-2.0), sig(-1.0), sig(1.0), sig(2.0)]],
         tol=1e-5),
    dict(op="sigmoid_forward", source="tests/activations/test_sigmoid.cpp:92-110",
         X=[[50.0, -50.0]], expected=[[1.0, 0.0]], tol=1e-5),
    dict(op="sigmoid_backward", source="tests/activations/test_sigmoid.cpp:131-148",
         X=[[-1.0, 0.0, 1.0]], dY=[[1.0, 1.0, 1.0]],
         expected=[[sig(-1.0) * (1 - sig(-1.0)), 0.25, sig(1.0) * (1 - sig(1.0))]], tol=1e-5),
    # ---- BinaryCrossEntropy --------------------------------------------------
    dict(op="bce_forward", source="tests/losses/test_binary_cross_entropy.cpp:97-109",
         P=[[0.5]], T=[[1.0]], expected=-math.log(0.5), tol=0.05),
    dict(op="bce_forward", source="tests/losses/test_binary_cross_entropy.cpp:47-58",
         P=[[0.999, 0.001, 0.999]], T=[[1.0, 0.0, 1.0]], check="loss < 0.01",
         exact=-math.log(0.999), derivation="each term is -log(0.999); mean of three equal terms",
         tol=1e-6),
    dict(op="bce_forward", source="tests/losses/test_binary_cross_entropy.cpp:61-72",
         P=[[0.01, 0.99]], T=[[1.0, 0.0]], check="loss > 1",
         exact=-math.log(0.01), derivation="each term is -log(0.01)", tol=1e-5),
    dict(op="bce_backward", source="tests/losses/test_binary_cross_entropy.cpp:144-157",
         P=[[0.5]], T=[[1.0]], check="grad < 0",
         exact=[[-2.0]], derivation="(0.5-1)/(0.5*0.5)/1 = -2", tol=1e-6),
    # ---- MSE -----------------------------------------------------------------
    dict(op="mse_forward", source="tests/losses/test_mse.cpp:74-86",
         P=[[0.0, 0.0, 0.0]], T=[[1.0, 2.0, 3.0]], expected=14.0 / 3.0, tol=0.1),
    dict(op="mse_forward", source="tests/losses/test_mse.cpp:47-57",
         P=[[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]], T=[[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]],
         expected=0.0, tol=1e-6),
    dict(op="mse_backward", source="tests/losses/test_mse.cpp:132-145",
         P=[[5.0, 10.0]], T=[[1.0, 1.0]], check="grad > 0",
         exact=[[2.0 * 4.0 / 2.0, 2.0 * 9.0 / 2.0]], derivation="2*(p-t)/n with n = 2",
         tol=1e-6),
    # ---- SoftmaxCrossEntropy -------------------------------------------------
    dict(op="softmax_ce_forward", source="tests/losses/test_softmax_cross_entropy.cpp:32-40",
         Z=[[10.0, -10.0, -10.0]], T=[[1.0, 0.0, 0.0]], check="loss < 0.1",
         exact=-math.log(softmax([10.0, -10.0, -10.0])[0]),
         derivation="-log softmax_0", tol=1e-6),
    dict(op="softmax_ce_forward", source="tests/losses/test_softmax_cross_entropy.cpp:42-50",
         Z=[[-10.0, 10.0, -10.0]], T=[[1.0, 0.0, 0.0]], check="loss > 10",
         exact=-math.log(softmax([-10.0, 10.0, -10.0])[0]),
         derivation="-log softmax_0 = 20 + log(1 + 2 e^-20)", tol=1e-4),
    dict(op="softmax_ce_backward", source="tests/losses/test_softmax_cross_entropy.cpp:77-90",
         Z=[[1.0, 2.0, 3.0]], T=[[0.0, 0.0, 1.0]], expected=[[0.0900, 0.2447, -0.3348]],
         exact=[[a - b for a, b in zip(softmax([1.0, 2.0, 3.0]), [0.0, 0.0, 1.0])]],
         derivation="softmax - target over a batch of 1", tol=0.02),
    # ---- MaxPool2D (4-D logical [n][c][h][w]) ------------------------------
    dict(op="maxpool2d_forward", source="tests/layers/test_max_pool2d.cpp:80-99",
         X=[[[[1.0, 2.0, 3.0, 4.0], [5.0, 6.0, 7.0, 8.0], [9.0, 10.0, 11.0, 12.0],
              [13.0, 14.0, 15.0, 16.0]]]], pool=2, stride=2,
         expected=[[[[6.0, 8.0], [14.0, 16.0]]]],
         exact_argmax=[[[[3, 3], [3, 3]]]],
         derivation="each window's max is its bottom-right element: ph=1, pw=1 -> 1*2+1 = 3",
         tol=1e-5),
    dict(op="maxpool2d_forward", source="tests/layers/test_max_pool2d.cpp:164-175",
         X=[[[[5.0] * 4] * 4]], pool=2, stride=2, expected=[[[[5.0, 5.0], [5.0, 5.0]]]],
         exact_argmax=[[[[0, 0], [0, 0]]]],
         derivation="all ties: strict > keeps the first element of each window (index 0)",
         tol=1e-5),
    dict(op="maxpool2d_shape", source="tests/layers/test_max_pool2d.cpp:147-160",
         shape=[1, 1, 5, 5], pool=3, stride=1, expected_shape=[1, 1, 3, 3]),
    # ---- Flatten ---------------------------------------------------------------
    dict(op="flatten_forward", source="tests/layers/test_flatten.cpp:60-79",
         X=[[[[1.0, 2.0], [3.0, 4.0]], [[5.0, 6.0], [7.0, 8.0]]]],
         expected_shape=[1, 8], check="sum preserved (36)",
         exact=[[1.0, 5.0, 3.0, 7.0, 2.0, 6.0, 4.0, 8.0]],
         derivation="ColMajor reshape [1,2,2,2] -> [1,8]: feature = c + 2*(h + 2*w)"),
    # ---- Adam ----------------------------------------------------------------
    dict(op="adam_first_step", source="src/CppNet/optimizers/adam.cpp:98-133",
         W=[1.0, -2.0, 0.5, 3.0], G=[0.1, -0.3, 2.0, -1e-3],
         lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8,
         exact=[w - 1e-3 * g / (abs(g) + 1e-8)
                for w, g in zip([1.0, -2.0, 0.5, 3.0], [0.1, -0.3, 2.0, -1e-3])],
         derivation="t=1: m/bc1 = g and v/bc2 = g^2, so W1 = W0 - lr*g/(|g|+eps)", tol=1e-6),
    # ---- LeakyReLU (leacky_relu.cpp) ------------------------------------------
    dict(op="leaky_relu_forward", source="tests/activations/test_leacky_relu.cpp:47-58",
         alpha=0.01, X=[[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]], expected=[[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]],
         tol=1e-6),
    dict(op="leaky_relu_forward", source="tests/activations/test_leacky_relu.cpp:61-72",
         alpha=0.01, X=[[-1.0, -2.0, -0.5, -100.0]], expected=[[-0.01, -0.02, -0.005, -1.0]], tol=1e-5),
    dict(op="leaky_relu_forward", source="tests/activations/test_leacky_relu.cpp:75-87",
         alpha=0.1, X=[[-2.0, 3.0, -0.5, 1.0]], expected=[[-0.2, 3.0, -0.05, 1.0]], tol=1e-5),
    dict(op="leaky_relu_forward", source="tests/activations/test_leacky_relu.cpp:91-102",
         alpha=0.2, X=[[-5.0, 5.0]], expected=[[-1.0, 5.0]], tol=1e-5),
    dict(op="leaky_relu_backward", source="tests/activations/test_leacky_relu.cpp:148-165",
         alpha=0.1, X=[[-2.0, 3.0, -0.5, 1.0]], dY=[[2.0, 3.0, 4.0, 5.0]],
         expected=[[0.2, 3.0, 0.4, 5.0]], tol=1e-5),
    # ---- Softmax (softmax.cpp) ---------------------------------------------------
    dict(op="softmax_forward", source="tests/activations/test_softmax.cpp:78-87",
         X=[[1.0, 1.0, 1.0, 1.0, 1.0]], expected=[[0.2, 0.2, 0.2, 0.2, 0.2]], tol=1e-5),
    dict(op="softmax_forward", source="tests/activations/test_softmax.cpp:106-114",
         X=[[42.0]], expected=[[1.0]], tol=1e-5),
    dict(op="softmax_forward", source="tests/activations/test_softmax.cpp:91-103",
         X=[[1.0, 2.0, 5.0, 0.5]], expected=[softmax([1.0, 2.0, 5.0, 0.5])], tol=1e-5,
         check="index 2 (value 5) is the largest"),
    dict(op="softmax_backward_constant", source="tests/activations/test_softmax.cpp:151-167",
         X=[[1.0, 2.0, 3.0, 4.0]], dY=[[1.0, 1.0, 1.0, 1.0]], expected=[[0.0, 0.0, 0.0, 0.0]], tol=1e-5,
         derivation="a constant upstream gradient c gives y*(c - c*sum(y)) = 0"),
    # ---- Losses -------------------------------------------------------------------
    dict(op="mae_forward", source="tests/losses/test_mae.cpp:60-72",
         P=[[0.0, 0.0, 0.0]], T=[[1.0, 2.0, 3.0]], expected=2.0, tol=1e-6,
         derivation="(1 + 2 + 3) / 3 (the reference test's own tolerance is 0.1)"),
    dict(op="huber_forward", source="tests/losses/test_huber.cpp:68-82",
         delta=10.0, P=[[0.5]], T=[[0.0]], expected=0.125, tol=1e-6),
    dict(op="huber_forward", source="tests/losses/test_huber.cpp:85-99",
         delta=1.0, P=[[5.0]], T=[[0.0]], expected=4.5, tol=1e-6,
         derivation="delta * (|5| - delta/2) (the reference test's own tolerance is 0.1)"),
    # ---- Global pools (global_pool.cpp) --------------------------------------------
    dict(op="global_avgpool_forward", source="tests/layers/test_global_pool.cpp:36-42",
         X=[[[[1.0, 3.0], [5.0, 7.0]]]], expected=[[4.0]], tol=1e-5),
    dict(op="global_avgpool_backward", source="tests/layers/test_global_pool.cpp:63-75",
         shape=[1, 1, 2, 3], dY=[[6.0]], expected_all=1.0, tol=1e-5),
    dict(op="global_maxpool_forward", source="tests/layers/test_global_pool.cpp:87-93",
         X=[[[[1.0, 3.0], [5.0, 7.0]]]], expected=[[7.0]], tol=1e-5),
    dict(op="global_maxpool_backward", source="tests/layers/test_global_pool.cpp:114-127",
         X=[[[[1.0, 3.0], [5.0, 7.0]]]], dY=[[1.0]], expected=[[[[0.0, 0.0], [0.0, 1.0]]]], tol=1e-6),
    # ---- Residual (residual.cpp) ----------------------------------------------
    dict(op="residual_forward", source="tests/layers/test_residual.cpp:68-84",
         block=[dict(W=[[0.0, 0.0], [0.0, 0.0]], b=None)], Wp=None,
         X=[[3.0, 7.0]], expected=[[3.0, 7.0]], tol=0.1,
         exact=[[3.0, 7.0]],
         derivation="bias-free Linear(2,2) with zero weights: block(x) = 0, identity shortcut, y = x"),
    dict(op="residual_forward", source="src/CppNet/layers/residual.cpp:31-36, 44-87",
         block=[dict(W=[[1.0, 0.0, 0.0], [0.0, 1.0, 0.0]], b=[0.0, 0.0, 1.0])],
         Wp=[[1.0, 1.0, 1.0], [0.0, 0.0, 0.0]],
         X=[[3.0, 7.0]],
         exact=[[6.0, 10.0, 4.0]],
         derivation="in 2 != out 3, so the shortcut is the bias-free projection x Wp = [3, 3, 3]; "
                    "block(x) = x W + b = [3, 7, 1]; y = [6, 10, 4]", tol=1e-6),
    dict(op="residual_backward", source="src/CppNet/layers/residual.cpp:89-131",
         block=[dict(W=[[2.0, 0.0], [0.0, 3.0]], b=[0.0, 0.0])], Wp=None,
         X=[[1.0, 1.0]], dY=[[1.0, 1.0]],
         exact=[[3.0, 4.0]], exact_gW=[[[1.0, 1.0], [1.0, 1.0]]], exact_gb=[[1.0, 1.0]],
         derivation="dX = dY W^T + dY = [2, 3] + [1, 1]; gW = x^T dY; gb = sum_batch dY", tol=1e-6),
    # ---- Dropout (dropout.cpp) ----------------------------------------------------
    dict(op="dropout_scale", source="tests/layers/test_dropout.cpp:51-62",
         p=0.5, x=1.0, expected_kept=2.0, tol=1e-5,
         derivation="kept entries are x * 1 * 1/(1-p)"),
]


def main():
    out = HERE / "known_answers.json"
    out.write_text(json.dumps({"convention": "matrices logical row-major, as setValues",
                               "cases": CASES}, indent=1) + "\n")
    print("wrote", out, len(CASES), "cases")


if __name__ == "__main__":
    main()
