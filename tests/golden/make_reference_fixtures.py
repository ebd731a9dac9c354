"""Writes reference_fixtures.json: the closed-form cases of Mantle's own tests for this path,
transcribed as data (inputs, attributes, expected outputs, tolerance class).

Nothing is imported or run from the reference: each case restates the constants of one test
function (file:line in "source"). Tensor specs:
  {"shape": [...], "fill": v}                 every element v
  {"shape": [...], "arange1": true}           element i = i + 1
  {"shape": [...], "data": [...]}             explicit values
  optional "set": {"i": v}                    element overrides
"tol": "exact" (assert_equal) or "almost" (rtol = atol = 1e-5, testing_utils.mojo:16-27).
"""
import json
import math
import os

import numpy as np

T = "tests/mojo/"


def fill(shape, v):
    return {"shape": shape, "fill": v}


def ar(shape, **kw):
    d = {"shape": shape, "arange1": True}
    d.update(kw)
    return d


def data(shape, vals):
    return {"shape": shape, "data": vals}


cases = []


def fwd(id_, src, op, t1, expected, t2=None, axis=None, tol="almost"):
    cases.append({"id": id_, "source": src, "kind": "forward", "op": op, "t1": t1, "t2": t2,
                  "axis": axis, "expected": expected, "tol": tol})


def bwd(id_, src, op, t1, ug, g1, t2=None, g2=None, axis=None, tol="almost"):
    cases.append({"id": id_, "source": src, "kind": "backward", "op": op, "t1": t1, "t2": t2, "ug": ug,
                  "axis": axis, "grad1": g1, "grad2": g2, "tol": tol})


S23 = [2, 3]
# ---- test_ops.mojo (forward through a one-node graph) ----
fwd("ops_add", T + "test_ops.mojo:13-24", "ADD", fill(S23, 1.0), fill(S23, 2.0), t2=fill(S23, 1.0))
fwd("ops_sub", T + "test_ops.mojo:27-38", "SUB", fill(S23, 2.0), fill(S23, 1.0), t2=fill(S23, 1.0))
fwd("ops_mul", T + "test_ops.mojo:41-52", "MUL", fill(S23, 2.0), fill(S23, 6.0), t2=fill(S23, 3.0))
fwd("ops_div", T + "test_ops.mojo:55-66", "DIV", fill(S23, 6.0), fill(S23, 3.0), t2=fill(S23, 2.0))
fwd("ops_exp", T + "test_ops.mojo:83-91", "EXP", fill(S23, 2.0), fill(S23, math.exp(2.0)))
fwd("ops_log", T + "test_ops.mojo:94-102", "LOG", fill(S23, 2.0), fill(S23, math.log(2.0)))
fwd("ops_pow", T + "test_ops.mojo:105-117", "POW", fill(S23, 2.0), fill(S23, 4.0), t2=fill([1], 2.0))
fwd("ops_sum_all", T + "test_ops.mojo:120-128", "SUM", fill([2, 3, 4], 1.0), fill([1], 24.0))
fwd("ops_sum_ax1", T + "test_ops.mojo:130-134", "SUM", fill([2, 3, 4], 1.0), fill([2, 1, 4], 3.0), axis=1)
fwd("ops_max_all", T + "test_ops.mojo:137-146", "MAX", ar([2, 3, 2]), fill([1], 12.0))
fwd("ops_max_ax0", T + "test_ops.mojo:154-159", "MAX", ar([2, 3, 2]), data([1, 3, 2], [7, 8, 9, 10, 11, 12]), axis=0)
fwd("ops_max_ax1", T + "test_ops.mojo:161-166", "MAX", ar([2, 3, 2]), data([2, 1, 2], [5, 6, 11, 12]), axis=1)
fwd("ops_max_ax2", T + "test_ops.mojo:168-173", "MAX", ar([2, 3, 2]), data([2, 3, 1], [2, 4, 6, 8, 10, 12]), axis=2)
fwd("ops_mean_all", T + "test_ops.mojo:177-186", "MEAN", fill(S23, 5.0), fill([1], 5.0))
fwd("ops_mean_ax0", T + "test_ops.mojo:188-191", "MEAN", fill(S23, 5.0), fill([1, 3], 5.0), axis=0)
fwd("ops_mean_ax1", T + "test_ops.mojo:193-196", "MEAN", fill(S23, 5.0), fill([2, 1], 5.0), axis=1)

# ---- test_backward.mojo (backward_op into a zeroed grad) ----
bwd("bw_add", T + "test_backward.mojo:18-33", "ADD", fill(S23, 1.0), fill(S23, 1.0), fill(S23, 1.0),
    t2=fill(S23, 2.0), g2=fill(S23, 1.0))
bwd("bw_sub", T + "test_backward.mojo:36-54", "SUB", fill(S23, 2.0), fill(S23, 1.0), fill(S23, 1.0),
    t2=fill(S23, 1.0), g2=fill(S23, -1.0))
bwd("bw_mul", T + "test_backward.mojo:57-75", "MUL", fill(S23, 1.0), fill(S23, 1.0), fill(S23, 2.0),
    t2=fill(S23, 2.0), g2=fill(S23, 1.0))
bwd("bw_div", T + "test_backward.mojo:78-96", "DIV", fill(S23, 1.0), fill(S23, 1.0), fill(S23, 0.5),
    t2=fill(S23, 2.0), g2=fill(S23, -0.25))
bwd("bw_exp", T + "test_backward.mojo:116-126", "EXP", fill(S23, 2.0), fill(S23, 5.0),
    fill(S23, 5.0 * math.exp(2.0)))
bwd("bw_log", T + "test_backward.mojo:129-139", "LOG", fill(S23, 2.0), fill(S23, 5.0), fill(S23, 2.5))
bwd("bw_pow", T + "test_backward.mojo:142-160", "POW", fill(S23, 2.0), fill(S23, 1.0), fill(S23, 4.0),
    t2=fill([1], 2.0), g2=fill([1], 6 * 4 * math.log(2.0)))
bwd("bw_pow_zero", T + "test_backward.mojo:162-168", "POW", fill(S23, 0.0), fill(S23, 1.0), fill(S23, 0.0),
    t2=fill([1], 0.0), g2=fill([1], 0.0))
bwd("bw_sum_all", T + "test_backward.mojo:170-181", "SUM", fill(S23, 1.0), fill([1], 9.0), fill(S23, 9.0))
bwd("bw_sum_ax0", T + "test_backward.mojo:184-201", "SUM", fill(S23, 1.0), data([1, 3], [0, 1, 2]),
    data(S23, [0, 1, 2, 0, 1, 2]), axis=0)
bwd("bw_sum_ax1", T + "test_backward.mojo:204-219", "SUM", fill(S23, 1.0), data([2, 1], [0, 1]),
    data(S23, [0, 0, 0, 1, 1, 1]), axis=1)
bwd("bw_max_all", T + "test_backward.mojo:222-236", "MAX", {"shape": S23, "fill": 1.0, "set": {"0": 2.0, "1": 2.0}},
    fill([1], 9.0), data(S23, [4.5, 4.5, 0, 0, 0, 0]))
bwd("bw_max_ax0", T + "test_backward.mojo:239-260", "MAX", ar([2, 3, 2], set={"0": 7.0}), fill([1, 3, 2], 2.0),
    data([2, 3, 2], [1, 0, 0, 0, 0, 0, 1, 2, 2, 2, 2, 2]), axis=0)
bwd("bw_max_ax1", T + "test_backward.mojo:263-283", "MAX", ar([2, 3, 2], set={"0": 5.0}), fill([2, 1, 2], 2.0),
    data([2, 3, 2], [1, 0, 0, 0, 1, 2, 0, 0, 0, 0, 2, 2]), axis=1)
bwd("bw_max_ax2", T + "test_backward.mojo:286-309", "MAX", ar([2, 3, 2], set={"0": 2.0}), fill([2, 3, 1], 2.0),
    data([2, 3, 2], [1, 1, 0, 2, 0, 2, 0, 2, 0, 2, 0, 2]), axis=2)
bwd("bw_mean_all", T + "test_backward.mojo:312-323", "MEAN", fill(S23, 1.0), fill([1], 9.0), fill(S23, 1.5))
bwd("bw_mean_ax0", T + "test_backward.mojo:326-340", "MEAN", fill(S23, 1.0), fill([1, 3], 3.0), fill(S23, 1.5), axis=0)
bwd("bw_mean_ax1", T + "test_backward.mojo:343-358", "MEAN", fill(S23, 1.0), fill([2, 1], 3.0), fill(S23, 1.0), axis=1)

# ---- test_mlops.mojo ----
fwd("ml_sigmoid", T + "test_mlops.mojo:26-34", "SIGMOID", fill(S23, 0.0), fill(S23, 0.5))
bwd("ml_sigmoid_bw", T + "test_mlops.mojo:37-52", "SIGMOID", fill(S23, 0.0), fill(S23, 5.0), fill(S23, 1.25))
fwd("ml_relu", T + "test_mlops.mojo:55-71", "RELU", data(S23, [3, 3, 3, -3, -3, -3]), data(S23, [3, 3, 3, 0, 0, 0]))
bwd("ml_relu_bw", T + "test_mlops.mojo:74-89", "RELU", data(S23, [3, 3, 3, -3, -3, -3]), fill(S23, 5.0),
    data(S23, [5, 5, 5, 0, 0, 0]))
fwd("ml_tanh", T + "test_mlops.mojo:138-146", "TANH", fill(S23, 0.0), fill(S23, 0.0))
bwd("ml_tanh_bw", T + "test_mlops.mojo:149-158", "TANH", fill(S23, 0.0), fill(S23, 5.0), fill(S23, 5.0))

# ---- test_tensorutils.mojo ----
fwd("tu_pow", T + "test_tensorutils.mojo:84-94", "POW", data([1, 10], list(range(10))),
    data([1, 10], [i * i for i in range(10)]), t2=fill([1], 2.0), tol="exact")
for op, v in (("ADD", 6.0), ("SUB", 0.0), ("MUL", 9.0), ("DIV", 1.0)):
    fwd("tu_tt_" + op.lower(), T + "test_tensorutils.mojo:97-128", op, fill([2, 10], 3.0), fill([2, 10], v),
        t2=fill([2, 10], 3.0), tol="exact")
fwd("tu_ts_add", T + "test_tensorutils.mojo:136-139", "ADD", fill([2, 10], 1.0), fill([2, 10], 3.0), t2=fill([1], 2.0), tol="exact")
fwd("tu_st_add", T + "test_tensorutils.mojo:141-142", "ADD", fill([1], 2.0), fill([2, 10], 3.0), t2=fill([2, 10], 1.0), tol="exact")
fwd("tu_ts_sub", T + "test_tensorutils.mojo:144-147", "SUB", fill([2, 10], 1.0), fill([2, 10], -1.0), t2=fill([1], 2.0), tol="exact")
fwd("tu_st_mul", T + "test_tensorutils.mojo:149-152", "MUL", fill([1], 2.0), fill([2, 10], 2.0), t2=fill([2, 10], 1.0), tol="exact")
fwd("tu_ts_div", T + "test_tensorutils.mojo:154-157", "DIV", fill([2, 10], 1.0), fill([2, 10], 0.5), t2=fill([1], 2.0), tol="exact")
exp_b = [0.0] * 120
for i in range(40):
    for j in range(3):
        exp_b[(i % 4) + (i // 4) * 12 + j * 4] = 3.0 + (i + 1)
fwd("tu_bcast", T + "test_tensorutils.mojo:161-181", "ADD", fill([2, 3, 4], 3.0), data([5, 2, 3, 4], exp_b),
    t2=ar([5, 2, 1, 4]), tol="exact")
fwd("tu_sum_all_2x10", T + "test_tensorutils.mojo:186-195", "SUM", ar([2, 10]), fill([1], 210.0), tol="exact")
fwd("tu_mean_all_2x10", T + "test_tensorutils.mojo:200-201", "MEAN", ar([2, 10]), fill([1], 10.5), tol="exact")
fwd("tu_sum_ax0_2x10", T + "test_tensorutils.mojo:213-219", "SUM", ar([2, 10]),
    data([1, 10], [(i + 1) + (i + 11) for i in range(10)]), axis=0, tol="exact")
fwd("tu_mean_ax0_2x10", T + "test_tensorutils.mojo:221-226", "MEAN", ar([2, 10]),
    data([1, 10], [((i + 1) + (i + 11)) / 2 for i in range(10)]), axis=0, tol="exact")
fwd("tu_sum_ax1_2x10", T + "test_tensorutils.mojo:235-241", "SUM", ar([2, 10]), data([2, 1], [55, 155]), axis=1, tol="exact")
fwd("tu_mean_ax1_2x10", T + "test_tensorutils.mojo:243-248", "MEAN", ar([2, 10]), data([2, 1], [5.5, 15.5]), axis=1, tol="exact")
fwd("tu_sum_all_3x4x5", T + "test_tensorutils.mojo:256-266", "SUM", ar([3, 4, 5]), fill([1], 1830.0), tol="exact")
fwd("tu_mean_all_3x4x5", T + "test_tensorutils.mojo:268-269", "MEAN", ar([3, 4, 5]), fill([1], 30.5), tol="exact")
D = T + "test_tensorutils_data.mojo"
fwd("tu_sum_ax0_3x4x5", D + ":667-688", "SUM", ar([3, 4, 5]), data([1, 4, 5], list(range(63, 121, 3))), axis=0)
fwd("tu_mean_ax0_3x4x5", D + ":690-711", "MEAN", ar([3, 4, 5]), data([1, 4, 5], list(range(21, 41))), axis=0)
fwd("tu_sum_ax1_3x4x5", D + ":722-738", "SUM", ar([3, 4, 5]),
    data([3, 1, 5], [34, 38, 42, 46, 50, 114, 118, 122, 126, 130, 194, 198, 202, 206, 210]), axis=1)
fwd("tu_mean_ax1_3x4x5", D + ":740-756,764", "MEAN", ar([3, 4, 5]),
    data([3, 1, 5], [v + 0.5 for v in [8, 9, 10, 11, 12, 28, 29, 30, 31, 32, 48, 49, 50, 51, 52]]), axis=1)
fwd("tu_sum_ax2_3x4x5", D + ":773-786", "SUM", ar([3, 4, 5]), data([3, 4, 1], list(range(15, 291, 25))), axis=2)
fwd("tu_mean_ax2_3x4x5", D + ":788-801", "MEAN", ar([3, 4, 5]), data([3, 4, 1], list(range(3, 59, 5))), axis=2)
# tstd (test_tensorutils.mojo:204-210, 228-232, 249-253, 269-275; SumMeanStdData expected_std,
# test_tensorutils_data.mojo:711, 760, 804). The all-element expectations are the test's own
# f32 loop: sqrt(sum((f32(i + 1) - mean)^2) / n).


def f32_std_loop(n):
    mean = np.float32(sum(range(1, n + 1))) / np.float32(n)
    acc = np.float32(0)
    for i in range(n):
        d = np.float32(i + 1) - mean
        acc = np.float32(acc + d * d)
    return float(np.sqrt(np.float32(acc / np.float32(n))))


def tstd_case(id_, src, t1, expected, axis=None, tol="almost"):
    cases.append({"id": id_, "source": src, "kind": "tstd", "t1": t1, "axis": axis, "expected": expected,
                  "tol": tol})


tstd_case("tu_std_all_2x10", T + "test_tensorutils.mojo:204-210", ar([2, 10]), fill([1], f32_std_loop(20)), tol="exact")
tstd_case("tu_std_ax0_2x10", T + "test_tensorutils.mojo:228-232", ar([2, 10]), fill([1, 10], 5.0), axis=0)
tstd_case("tu_std_ax1_2x10", T + "test_tensorutils.mojo:249-253", ar([2, 10]), fill([2, 1], 2.8722813129425049), axis=1)
tstd_case("tu_std_all_3x4x5", T + "test_tensorutils.mojo:269-275", ar([3, 4, 5]), fill([1], f32_std_loop(60)),
          tol="exact")
tstd_case("tu_std_ax0_3x4x5", D + ":711", ar([3, 4, 5]), fill([1, 4, 5], 16.32993162), axis=0)
tstd_case("tu_std_ax1_3x4x5", D + ":760", ar([3, 4, 5]), fill([3, 1, 5], 5.59016994), axis=1)
tstd_case("tu_std_ax2_3x4x5", D + ":804", ar([3, 4, 5]), fill([3, 4, 1], 1.41421356), axis=2)

cases.append({"id": "tu_accum_36", "source": T + "test_tensorutils.mojo:397-407", "kind": "accumulate",
              "grad_shape": [2, 1, 1], "rg": fill([2, 3, 4], 3.0), "expected": fill([2, 1, 1], 36.0), "tol": "exact"})
cases.append({"id": "tu_accum_24_noncompliant", "source": T + "test_tensorutils.mojo:409-414", "kind": "accumulate",
              "grad_shape": [2, 1], "rg": fill([2, 3, 4], 3.0), "expected": fill([2, 1], 24.0), "tol": "exact",
              "reject": "(2,1) does not broadcast to (2,3,4) under numpy rules; the reference indexes past "
                        "the 2-element grad (tensorutils.mojo:149-175, 482-484). Out of contract: rejected."})

# ---- composite graphs ----
for axis, v in ((0, 0.5), (1, 1.0 / 3.0), (2, 0.5)):
    cases.append({"id": f"act_softmax_ax{axis}", "source": T + "test_activations.mojo:105-121", "kind": "graph",
                  "graph": "softmax", "axis": axis, "t1": fill([2, 3, 2], 4.0), "expected": fill([2, 3, 2], v),
                  "tol": "almost"})
for axis, v in ((0, -0.69314718), (1, -1.09861231), (2, -0.69314718)):
    cases.append({"id": f"act_logsoftmax_ax{axis}", "source": T + "test_activations.mojo:124-140", "kind": "graph",
                  "graph": "logsoftmax", "axis": axis, "t1": fill([2, 3, 2], 4.0), "expected": fill([2, 3, 2], v),
                  "tol": "almost"})
cases.append({"id": "loss_mse_perfect", "source": T + "test_loss.mojo:9-38", "kind": "graph", "graph": "mse",
              "t1": fill([2, 10], 1.0), "t2": fill([2, 10], 1.0), "expected": fill([1], 0.0), "tol": "almost"})
cases.append({"id": "loss_mse_imperfect", "source": T + "test_loss.mojo:41-83", "kind": "graph", "graph": "mse",
              "t1": fill([1, 10], 1.0), "t2": data([1, 10], list(range(10))), "expected": fill([1], 20.5),
              "tol": "almost"})
cases.append({"id": "loss_ce_perfect", "source": T + "test_loss.mojo:86-127", "kind": "graph", "graph": "crossentropy",
              "t1": data([2, 3], [0.1, 0.2, 0.7, 0.7, 0.2, 0.1]), "t2": data([2, 3], [0, 0, 1, 1, 0, 0]),
              "expected": fill([1], 0.76794958), "tol": "almost6"})
cases.append({"id": "loss_ce_imperfect", "source": T + "test_loss.mojo:130-171", "kind": "graph",
              "graph": "crossentropy", "t1": data([2, 3], [0.1, 0.2, 0.7, 0.7, 0.2, 0.1]),
              "t2": data([2, 3], [0, 1, 0, 0, 0, 1]), "expected": fill([1], 1.31794953), "tol": "almost6"})

# ---- FMA (test_ops.mojo:256-271), LEAKYRELU and CLIP (test_mlops.mojo:91-135, 161-248) ----
cases.append({"id": "ops_fma", "source": T + "test_ops.mojo:256-271", "kind": "forward", "op": "FMA",
              "t1": fill(S23, 1.0), "t2": fill(S23, 2.0), "t3": fill(S23, 3.0), "axis": None,
              "expected": fill(S23, 5.0), "tol": "exact"})
LR_X = data(S23, [3, 3, 3, -3, -3, -3])
SLOPE = {"negative_slope": 0.1}
fwd("ml_leakyrelu", T + "test_mlops.mojo:91-110", "LEAKYRELU", LR_X, data(S23, [3, 3, 3, -0.3, -0.3, -0.3]))
cases[-1]["attrs"] = SLOPE
bwd("ml_leakyrelu_bw", T + "test_mlops.mojo:113-135", "LEAKYRELU", LR_X, fill(S23, 5.0),
    data(S23, [5, 5, 5, 0.5, 0.5, 0.5]))
cases[-1]["attrs"] = SLOPE
CL_X = data(S23, [i - 3 for i in range(6)])
for tag, attrs, fexp, bexp in [
        ("none", {}, [-3, -2, -1, 0, 1, 2], [5] * 6),
        ("min", {"min": -1.1}, [-1.1, -1.1, -1, 0, 1, 2], [0, 0, 5, 5, 5, 5]),
        ("max", {"max": 1.1}, [-3, -2, -1, 0, 1, 1.1], [5, 5, 5, 5, 5, 0]),
        ("minmax", {"min": -1.1, "max": 1.1}, [-1.1, -1.1, -1, 0, 1, 1.1], [0, 0, 5, 5, 5, 0])]:
    fwd(f"ml_clip_{tag}", T + "test_mlops.mojo:161-203", "CLIP", CL_X, data(S23, fexp))
    cases[-1]["attrs"] = attrs
    bwd(f"ml_clip_bw_{tag}", T + "test_mlops.mojo:206-248", "CLIP", CL_X, fill(S23, 5.0), data(S23, bexp))
    cases[-1]["attrs"] = attrs

here = os.path.dirname(os.path.abspath(__file__))
with open(os.path.join(here, "reference_fixtures.json"), "w") as f:
    json.dump({"note": "closed-form cases of Mantle's tests (see make_reference_fixtures.py)", "cases": cases}, f,
              indent=1)
print(len(cases), "cases")
