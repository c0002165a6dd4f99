"""Enum types of the reference operator surface (nkilib ``common_types``).

Same member names as the reference uses at its call sites:
RouterActFnType (router_topk.py:78), ActFnType (moe_tkg.py:74),
ExpertAffinityScaleMode (moe_tkg.py:73), QuantizationType
(attention_block_tkg.py:94, moe_tkg.py:318-328).
"""
from enum import Enum


class RouterActFnType(Enum):
    SOFTMAX = 0
    SIGMOID = 1


class ActFnType(Enum):
    SiLU = 0
    Swish = 1      # GPT-OSS: g * sigmoid(1.702 g)
    GELU = 2
    GELU_Tanh_Approx = 3


class ExpertAffinityScaleMode(Enum):
    NO_SCALE = 0
    POST_SCALE = 1
    PRE_SCALE = 2
    PRE_SCALE_DELAYED = 3


class QuantizationType(Enum):
    NONE = 0
    STATIC = 1
    ROW = 2
    MX = 3


# x layouts of router_topk (router_topk.py:60-66)
XHBMLayout_H_T__0 = 0
XHBMLayout_T_H__1 = 1
XSBLayout_tp102__0 = 0
XSBLayout_tp2013__1 = 1
XSBLayout_tp201__2 = 2
XSBLayout__128_Hdiv128_T__3 = 3
