"""Weight initialisers and default init maps with NovaNN's behaviour.

The layers' default weights have to be the reference's own: a caller that
seeds numpy's global generator and builds a Linear or Conv2d gets the same
float32 weights from both frameworks.  So every function here draws from the
global legacy ``np.random`` stream, with the same call, shape and dtype
conversion as the reference (novann/core/init.py):

  - gain by nonlinearity (init.py:13-38): linear / sigmoid 1, tanh 5/3,
    relu sqrt(2), leakyrelu sqrt(2 / (1 + slope^2)) with slope 0.01 by default;
  - fans (init.py:55-90): a weight of shape (out, in, *kernel) has
    fan_in = in * prod(kernel), fan_out = out * prod(kernel); 2 to 5 dims;
  - kaiming_normal_ (init.py:155-179): normal(0, gain / sqrt(fan));
    kaiming_uniform_ (:182-207): uniform(-gain sqrt(3 / fan), +gain sqrt(3 / fan));
    xavier_normal_ (:93-111): normal(0, gain sqrt(2 / (fan_in + fan_out)));
    xavier_uniform_ (:114-132): uniform(+-gain sqrt(6 / (fan_in + fan_out)));
    each drawn in float64 and rounded to float32;
  - random_init_ (init.py:210-219): standard normals rounded to float32, then
    times ``gain`` (0.001) in float32 arithmetic;
  - the default maps of novann/core/config.py:24-40, which Linear
    (DEFAULT_NORMAL_INIT_MAP["default"], linear.py:55) and Conv2d
    (DEFAULT_UNIFORM_INIT_MAP["relu"], conv2d.py:62) fall back to.
"""
from __future__ import annotations

from typing import Callable, Dict, Optional, Tuple, Union

import numpy as np

Shape = Tuple[int, ...]
InitFn = Callable[[Shape], np.ndarray]


def calculate_gain(nonlinearity: str, param: Optional[float] = None) -> float:
    """Recommended gain for a nonlinearity; ValueError for an unknown name."""
    if nonlinearity in ("linear", "sigmoid"):
        return 1.0
    if nonlinearity == "tanh":
        return 5.0 / 3.0
    if nonlinearity == "relu":
        return float(np.sqrt(2.0))
    if nonlinearity == "leakyrelu":
        slope = 0.01 if param is None else float(param)
        return float(np.sqrt(2.0 / (1 + slope ** 2)))
    raise ValueError(f"Unsupported activation function: {nonlinearity}")


def fans(shape: Shape) -> Tuple[int, int]:
    """(fan_in, fan_out) of a weight (out, in, *kernel) of 2 to 5 dims."""
    if len(shape) < 2:
        raise ValueError(f"Shape must have at least 2 dimensions, got {len(shape)}")
    if len(shape) > 5:
        raise ValueError(f"Shape must have 2 to 5 dimensions, got {len(shape)}")
    receptive = 1
    for k in shape[2:]:
        receptive *= int(k)
    return int(shape[1]) * receptive, int(shape[0]) * receptive


def shape_validation(shape: Shape, mode: str = "fan_in") -> Union[int, Tuple[int, int]]:
    """fan_in, fan_out or both, as the reference's helper of that name."""
    if mode not in ("both", "fan_in", "fan_out"):
        raise ValueError(f"Mode must be ('both', 'fan_in', 'fan_out'), got '{mode}'")
    fan_in, fan_out = fans(shape)
    if mode == "both":
        return fan_in, fan_out
    return fan_in if mode == "fan_in" else fan_out


def kaiming_normal_(shape: Shape, a: Optional[float] = None, nonlinearity: str = "relu",
                    mode: str = "fan_in") -> np.ndarray:
    fan = shape_validation(shape, mode)
    std = calculate_gain(nonlinearity, a) / np.sqrt(fan)
    return np.random.normal(0.0, std, shape).astype(np.float32)


def kaiming_uniform_(shape: Shape, a: Optional[float] = None, nonlinearity: str = "relu",
                     mode: str = "fan_in") -> np.ndarray:
    fan = shape_validation(shape, mode)
    bound = calculate_gain(nonlinearity, a) * np.sqrt(3.0 / fan)
    return np.random.uniform(-bound, bound, shape).astype(np.float32)


def xavier_normal_(shape: Shape, gain: float = 1.0) -> np.ndarray:
    fan_in, fan_out = shape_validation(shape, "both")
    std = gain * np.sqrt(2.0 / (fan_in + fan_out))
    return np.random.normal(0.0, std, shape).astype(np.float32)


def xavier_uniform_(shape: Shape, gain: float = 1.0) -> np.ndarray:
    fan_in, fan_out = shape_validation(shape, "both")
    bound = gain * np.sqrt(6.0 / (fan_in + fan_out))
    return np.random.uniform(-bound, bound, shape).astype(np.float32)


def random_init_(shape: Shape, gain: float = 0.001) -> np.ndarray:
    return np.random.randn(*shape).astype(np.float32) * gain


DEFAULT_NORMAL_INIT_MAP: Dict[str, InitFn] = {
    "relu": lambda shape: kaiming_normal_(shape, a=0.0, nonlinearity="relu"),
    "leakyrelu": lambda shape: kaiming_normal_(shape, a=0.01, nonlinearity="leakyrelu"),
    "tanh": lambda shape: xavier_normal_(shape, gain=calculate_gain("tanh")),
    "sigmoid": lambda shape: xavier_normal_(shape, gain=calculate_gain("sigmoid")),
    "default": lambda shape: random_init_(shape),
}

DEFAULT_UNIFORM_INIT_MAP: Dict[str, InitFn] = {
    "relu": lambda shape: kaiming_uniform_(shape, a=0.0, nonlinearity="relu"),
    "leakyrelu": lambda shape: kaiming_uniform_(shape, a=0.01, nonlinearity="leakyrelu"),
    "tanh": lambda shape: xavier_uniform_(shape, gain=calculate_gain("tanh")),
    "sigmoid": lambda shape: xavier_uniform_(shape, gain=calculate_gain("sigmoid")),
    "default": lambda shape: random_init_(shape),
}
