"""Seeded random-weight KataGo models and synthetic inputs.

There is no network access for real checkpoints, so every model this
repository measures or checks is written here, in KataGo's model-file format,
from a fixed seed. The writer follows the grammar that the parser reads
(/root/reference/cpp/neuralnet/desc.cpp:104-2445), which is also the grammar
of KataGo's exporter (/root/reference/python/export_model_pytorch.py:94-560):
whitespace-separated header tokens, and float arrays either as text or as
"@BIN@" followed by little-endian float32.

Architectures are those of BASELINE.json's configs (C0..C4), with the channel
layouts of /root/reference/python/katago/train/modelconfigs.py (b6c96 :142-166,
b10c128 :168-196, b18c384nbt :945-981; nested-bottleneck gpool blocks put the
gpool convolution in the first inner block, model_pytorch.py:910-916).

Random numbers: SplitMix64 with Box-Muller normals, so any implementation can
regenerate identical weights and inputs from the seed. Seeds are 1000+cfg for
weights and 2000+cfg for inputs.
"""
from __future__ import annotations

import gzip
import io
import math
import struct
from dataclasses import dataclass, field

import numpy as np

# ---------------------------------------------------------------------------
# Random numbers

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


class SplitMix64:
    """SplitMix64 (Steele, Lea, Flood 2014), vectorized over a block of draws."""

    def __init__(self, seed: int):
        self.state = np.uint64(seed & 0xFFFFFFFFFFFFFFFF)

    def next_u64(self, n: int) -> np.ndarray:
        with np.errstate(over="ignore"):
            idx = np.arange(1, n + 1, dtype=np.uint64)
            z = self.state + idx * _GAMMA
            self.state = self.state + np.uint64(n) * _GAMMA
            z = (z ^ (z >> np.uint64(30))) * _M1
            z = (z ^ (z >> np.uint64(27))) * _M2
            z = z ^ (z >> np.uint64(31))
        return z

    def uniform(self, n: int) -> np.ndarray:
        """U[0,1) with 53 random bits."""
        return (self.next_u64(n) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)

    def normal(self, n: int) -> np.ndarray:
        """Standard normals by Box-Muller on pairs of uniforms."""
        m = (n + 1) // 2
        u = self.uniform(2 * m)
        u1 = 1.0 - u[0::2]  # (0, 1]
        u2 = u[1::2]
        r = np.sqrt(-2.0 * np.log(u1))
        z = np.empty(2 * m)
        z[0::2] = r * np.cos(2.0 * math.pi * u2)
        z[1::2] = r * np.sin(2.0 * math.pi * u2)
        return z[:n]


# ---------------------------------------------------------------------------
# File writer


class ModelWriter:
    """Emits a model file token by token; binary=True writes the .bin form."""

    def __init__(self, binary: bool = True):
        self.binary = binary
        self.buf = io.BytesIO()

    def line(self, s) -> None:
        self.buf.write((str(s) + "\n").encode("ascii"))

    def floats(self, arr) -> None:
        a = np.ascontiguousarray(np.asarray(arr, dtype=np.float32).reshape(-1))
        if self.binary:
            self.buf.write(b"@BIN@")
            self.buf.write(a.astype("<f4").tobytes())
            self.buf.write(b"\n")
        else:
            self.buf.write((" ".join(repr(float(x)) for x in a) + "\n").encode("ascii"))

    def data(self) -> bytes:
        return self.buf.getvalue()


@dataclass
class Arch:
    """A KataGo network architecture (the subset this backend targets)."""
    name: str
    version: int
    trunk_c: int
    mid_c: int
    gpool_c: int
    blocks: list  # entries: "regular", "regulargpool", "bottlenest2", "bottlenest2gpool", "attention", "ffn"
    p1_c: int
    g1_c: int
    v1_c: int
    v2_c: int
    activation: str = "ACTIVATION_RELU"
    # transformer options
    heads: int = 0
    kv_heads: int = 0
    q_head_dim: int = 0
    v_head_dim: int = 0
    ffn_c: int = 0
    learnable_rope: bool = True
    rope_theta: float = 100.0
    trunk_rmsnorm: bool = False
    transformer_std: float = 0.02
    # Gain on the last convolution of each residual branch. KataGo's own init
    # zeroes those ("fixup", model_pytorch.py:722-725,930-935); a small
    # nonzero gain keeps every branch live while the residual stream stays in
    # fp16 range over deep stacks.
    residual_gain: float = 1.0
    num_input: int = 22
    num_global: int = 19
    # SGF metadata encoder (version >= 15; 1 = the 192 metadata channels of
    # sgfmetadata.cpp): written with random weights for the tests of its
    # rejection, not evaluated.
    meta_encoder_version: int = 0


def _he(rng: SplitMix64, shape, fan_in: int, gain: float = 1.0) -> np.ndarray:
    n = int(np.prod(shape))
    return (rng.normal(n) * (gain * math.sqrt(2.0 / fan_in))).reshape(shape)


class _Builder:
    def __init__(self, arch: Arch, seed: int, binary: bool):
        self.a = arch
        self.rng = SplitMix64(seed)
        self.w = ModelWriter(binary)

    # layers -----------------------------------------------------------------
    def conv(self, name, ky, kx, cin, cout, gain=1.0):
        w = self.w
        w.line(name)
        for v in (ky, kx, cin, cout, 1, 1):
            w.line(v)
        # file order (y, x, ic, oc)
        w.floats(_he(self.rng, (ky, kx, cin, cout), ky * kx * cin, gain))

    def bn(self, name, c):
        # Folded form as KataGo's exporter writes it: mean 0, variance 1-eps,
        # eps 1e-20, so mergedScale == scale exactly.
        w = self.w
        w.line(name)
        w.line(c)
        w.line(1e-20)
        w.line(1)
        w.line(1)
        w.floats(np.zeros(c))
        w.floats(np.full(c, 1.0 - 1e-20))
        w.floats(0.8 + 0.4 * self.rng.uniform(c))
        w.floats(0.1 * self.rng.normal(c))

    def act(self, name, kind=None):
        self.w.line(name)
        self.w.line(kind or self.a.activation)

    def matmul(self, name, cin, cout, std=None):
        w = self.w
        w.line(name)
        w.line(cin)
        w.line(cout)
        if std is None:
            w.floats(_he(self.rng, (cin, cout), cin))
        else:
            w.floats(self.rng.normal(cin * cout) * std)

    def matbias(self, name, c, std=0.1):
        self.w.line(name)
        self.w.line(c)
        self.w.floats(self.rng.normal(c) * std)

    def trmsnorm(self, name, c):
        self.w.line(name)
        self.w.line(c)
        self.w.line(1e-6)
        self.w.floats(1.0 + 0.1 * self.rng.normal(c))

    # blocks -----------------------------------------------------------------
    def ordinary(self, name, c, mid):
        self.w.line("ordinary_block")
        self.w.line(name)
        self.bn(name + ".norm1", c)
        self.act(name + ".act1")
        self.conv(name + ".conv1", 3, 3, c, mid)
        self.bn(name + ".norm2", mid)
        self.act(name + ".act2")
        self.conv(name + ".conv2", 3, 3, mid, c, self.a.residual_gain)

    def gpool(self, name, c, mid, gp):
        reg = mid - gp
        self.w.line("gpool_block")
        self.w.line(name)
        self.bn(name + ".norm1", c)
        self.act(name + ".act1")
        self.conv(name + ".conv1r", 3, 3, c, reg)
        self.conv(name + ".conv1g", 3, 3, c, gp)
        self.bn(name + ".normg", gp)
        self.act(name + ".actg")
        self.matmul(name + ".linear_g", 3 * gp, reg)
        self.bn(name + ".norm2", reg)
        self.act(name + ".act2")
        self.conv(name + ".conv2", 3, 3, reg, c, self.a.residual_gain)

    def nbt(self, name, c, mid, gp, use_gpool):
        self.w.line("nested_bottleneck_block")
        self.w.line(name)
        self.w.line(2)
        self.bn(name + ".normp", c)
        self.act(name + ".actp")
        self.conv(name + ".convp", 1, 1, c, mid)
        if use_gpool:
            self.gpool(name + ".blockstack.0", mid, mid, gp)
        else:
            self.ordinary(name + ".blockstack.0", mid, mid)
        self.ordinary(name + ".blockstack.1", mid, mid)
        self.bn(name + ".normq", mid)
        self.act(name + ".actq")
        self.conv(name + ".convq", 1, 1, mid, c, self.a.residual_gain)

    def attention(self, name, c):
        a = self.a
        w = self.w
        w.line("transformer_attention_block")
        w.line(name)
        for v in (a.heads, a.kv_heads, a.q_head_dim, a.v_head_dim, 1, 1 if a.learnable_rope else 0):
            w.line(v)
        self.trmsnorm(name + ".norm1", c)
        self.matmul(name + ".q_proj", c, a.heads * a.q_head_dim, a.transformer_std)
        self.matmul(name + ".k_proj", c, a.kv_heads * a.q_head_dim, a.transformer_std)
        self.matmul(name + ".v_proj", c, a.kv_heads * a.v_head_dim, a.transformer_std)
        self.matmul(name + ".out_proj", a.heads * a.v_head_dim, c, a.transformer_std)
        if a.learnable_rope:
            w.line(name + ".rope_freqs")
            w.line(a.kv_heads)
            w.line(a.q_head_dim // 2)
            w.line(2)
            pairs = a.q_head_dim // 2
            freqs = []
            for _h in range(a.kv_heads):
                for p in range(pairs):
                    base = a.rope_theta ** (-(2.0 * (p % max(1, pairs // 2))) / max(1, pairs))
                    ang = 2.0 * math.pi * self.rng.uniform(1)[0]
                    freqs += [base * math.cos(ang), base * math.sin(ang)]
            w.floats(freqs)
        else:
            w.line(name + ".rope_theta")
            w.line(a.rope_theta)

    def ffn(self, name, c):
        a = self.a
        self.w.line("transformer_ffn_block")
        self.w.line(name)
        self.w.line(c)
        self.w.line(a.ffn_c)
        self.w.line(1)
        self.trmsnorm(name + ".norm", c)
        self.matmul(name + ".ffn_linear1", c, a.ffn_c, a.transformer_std)
        self.matmul(name + ".ffn_linear_gate", c, a.ffn_c, a.transformer_std)
        self.matmul(name + ".ffn_linear2", a.ffn_c, c, a.transformer_std)

    # model ------------------------------------------------------------------
    def model(self) -> bytes:
        a = self.a
        w = self.w
        w.line(a.name)
        w.line(a.version)
        w.line(a.num_input)
        w.line(a.num_global)
        for v in (20.0, 20.0, 20.0, 20.0, 40.0, 0.25, 30.0):  # post-process multipliers (v >= 13)
            w.line(v)
        if a.version >= 15:
            w.line(a.meta_encoder_version)
            for _ in range(7):  # seven reserved zeros
                w.line(0)
        # trunk
        w.line("trunk")
        w.line(len(a.blocks))
        w.line(a.trunk_c)
        w.line(a.mid_c)
        w.line(a.mid_c - a.gpool_c)
        w.line(a.gpool_c)
        w.line(a.gpool_c)
        if a.version >= 15:
            w.line(1 if a.trunk_rmsnorm else 0)
            for _ in range(5):
                w.line(0)
        self.conv("model.conv_spatial", 3, 3, a.num_input, a.trunk_c)
        self.matmul("model.linear_global", a.num_global, a.trunk_c)
        if a.meta_encoder_version > 0:
            # SGFMetadataEncoderDesc (desc.cpp): name, input channels, then
            # mul, bias, act, mul, bias, act, mul to the trunk width.
            w.line("model.metadata_encoder")
            w.line(192)
            self.matmul("model.metadata_encoder.mul1", 192, 32)
            self.matbias("model.metadata_encoder.bias1", 32)
            self.act("model.metadata_encoder.act1")
            self.matmul("model.metadata_encoder.mul2", 32, 32)
            self.matbias("model.metadata_encoder.bias2", 32)
            self.act("model.metadata_encoder.act2")
            self.matmul("model.metadata_encoder.mul3", 32, a.trunk_c)
        for i, kind in enumerate(a.blocks):
            name = f"model.blocks.{i}"
            if kind == "regular":
                self.ordinary(name, a.trunk_c, a.mid_c)
            elif kind == "regulargpool":
                self.gpool(name, a.trunk_c, a.mid_c, a.gpool_c)
            elif kind in ("bottlenest2", "bottlenest2gpool"):
                self.nbt(name, a.trunk_c, a.mid_c, a.gpool_c, kind.endswith("gpool"))
            elif kind == "attention":
                self.attention(name, a.trunk_c)
            elif kind == "ffn":
                self.ffn(name, a.trunk_c)
            else:
                raise ValueError(kind)
        if a.trunk_rmsnorm:
            w.line("model.norm_trunkfinal")
            w.line(a.trunk_c)
            w.line(1e-6)
            w.line(0)
            w.line(0)
            w.floats(1.0 + 0.1 * self.rng.normal(a.trunk_c))
            w.floats(0.1 * self.rng.normal(a.trunk_c))
        else:
            self.bn("model.norm_trunkfinal", a.trunk_c)
        self.act("model.act_trunkfinal")
        # policy head (version >= 15 layout)
        w.line("model.policy_head")
        if a.version >= 17:
            w.line(2)
            for _ in range(3):
                w.line(0)
        self.conv("model.policy_head.conv1p", 1, 1, a.trunk_c, a.p1_c)
        self.conv("model.policy_head.conv1g", 1, 1, a.trunk_c, a.g1_c)
        self.bn("model.policy_head.biasg", a.g1_c)
        self.act("model.policy_head.actg")
        self.matmul("model.policy_head.linear_g", 3 * a.g1_c, a.p1_c)
        self.bn("model.policy_head.bias2", a.p1_c)
        self.act("model.policy_head.act2")
        self.conv("model.policy_head.conv2p", 1, 1, a.p1_c, 2)
        self.matmul("model.policy_head.linear_pass", 3 * a.g1_c, a.p1_c)
        self.matbias("model.policy_head.linear_pass_bias", a.p1_c)
        self.act("model.policy_head.act_pass")
        self.matmul("model.policy_head.linear_pass2", a.p1_c, 2)
        # value head
        w.line("model.value_head")
        if a.version >= 17:
            for _ in range(3):
                w.line(0)
        self.conv("model.value_head.conv1", 1, 1, a.trunk_c, a.v1_c)
        self.bn("model.value_head.bias1", a.v1_c)
        self.act("model.value_head.act1")
        self.matmul("model.value_head.linear2", 3 * a.v1_c, a.v2_c)
        self.matbias("model.value_head.bias2", a.v2_c)
        self.act("model.value_head.act2")
        self.matmul("model.value_head.linear_valuehead", a.v2_c, 3)
        self.matbias("model.value_head.bias_valuehead", 3)
        self.matmul("model.value_head.linear_miscvaluehead", a.v2_c, 6)
        self.matbias("model.value_head.bias_miscvaluehead", 6)
        self.conv("model.value_head.conv_ownership", 1, 1, a.v1_c, 1)
        return w.data()


def write_model(arch: Arch, seed: int, path: str, binary: bool = True, gz: bool | None = None) -> str:
    """Writes arch with weights from seed to path (.bin, .bin.gz, .txt or .txt.gz)."""
    data = _Builder(arch, seed, binary).model()
    if gz is None:
        gz = path.endswith(".gz")
    if gz:
        data = gzip.compress(data, compresslevel=1, mtime=0)
    with open(path, "wb") as f:
        f.write(data)
    return path


# ---------------------------------------------------------------------------
# Configurations (BASELINE.json "configs")

def b6c96() -> Arch:
    return Arch("b6c96-synthetic", 15, 96, 96, 32,
                ["regular", "regular", "regulargpool", "regular", "regulargpool", "regular"],
                32, 32, 32, 64, "ACTIVATION_RELU", residual_gain=0.5)


def b10c128() -> Arch:
    return Arch("b10c128-synthetic", 15, 128, 128, 32,
                ["regular", "regular", "regular", "regular", "regulargpool",
                 "regular", "regular", "regulargpool", "regular", "regular"],
                32, 32, 32, 80, "ACTIVATION_MISH", residual_gain=0.25)


def b18c384nbt() -> Arch:
    kinds = []
    for i in range(18):
        kinds.append("bottlenest2gpool" if i in (2, 5, 8, 11, 14) else "bottlenest2")
    return Arch("b18c384nbt-synthetic", 15, 384, 192, 64, kinds, 48, 48, 96, 128, "ACTIVATION_MISH",
                residual_gain=0.25)


def transformer_d384() -> Arch:
    kinds = []
    for _ in range(12):
        kinds += ["attention", "ffn"]
    return Arch("t12d384h6-synthetic", 17, 384, 384, 64, kinds, 48, 48, 96, 128, "ACTIVATION_SILU",
                heads=6, kv_heads=6, q_head_dim=64, v_head_dim=64, ffn_c=1024, learnable_rope=True,
                trunk_rmsnorm=True)


@dataclass
class Config:
    index: int
    arch: Arch
    batch: int
    fp16: bool
    board_sizes: list = field(default_factory=lambda: [19])

    @property
    def weight_seed(self) -> int:
        return 1000 + self.index

    @property
    def input_seed(self) -> int:
        return 2000 + self.index


def configs() -> list[Config]:
    return [
        Config(0, b6c96(), 8, False),
        Config(1, b10c128(), 64, True),
        Config(2, b18c384nbt(), 256, True),
        Config(3, b18c384nbt(), 256, True, [9, 13, 19]),
        Config(4, transformer_d384(), 128, True),
    ]


# ---------------------------------------------------------------------------
# Synthetic inputs


def board_xy(bs):
    """(x, y) size of a board given as a side length or an (x, y) pair."""
    return (bs, bs) if np.isscalar(bs) else (int(bs[0]), int(bs[1]))


def synthetic_inputs(seed: int, n: int, nn_x: int = 19, nn_y: int = 19, board_sizes=(19,), num_spatial: int = 22,
                     num_global: int = 19):
    """Rows of NHWC spatial features and global features.

    Plane 0 is the on-board mask (1 where x < bs and y < bs, board anchored
    top-left as in nninputs.h:23-38); plane 1 is Bernoulli(0.35) on-board;
    plane 2 is Bernoulli(0.35) on on-board points not in plane 1; planes 3..
    are Bernoulli(0.1) on-board. Globals are U(-1, 1). Board sizes cycle per
    row through board_sizes; an entry is a side length or an (x, y) pair for
    a rectangular board.
    """
    rng = SplitMix64(seed)
    hw = nn_x * nn_y
    spatial = np.zeros((n, nn_y, nn_x, num_spatial), dtype=np.float32)
    for i in range(n):
        bx, by = board_xy(board_sizes[i % len(board_sizes)])
        on = np.zeros((nn_y, nn_x), dtype=bool)
        on[:min(by, nn_y), :min(bx, nn_x)] = True
        u = rng.uniform(hw * num_spatial).reshape(nn_y, nn_x, num_spatial)
        spatial[i, :, :, 0] = on
        p1 = (u[:, :, 1] < 0.35) & on
        p2 = (u[:, :, 2] < 0.35) & on & ~p1
        spatial[i, :, :, 1] = p1
        spatial[i, :, :, 2] = p2
        spatial[i, :, :, 3:] = (u[:, :, 3:] < 0.1) & on[:, :, None]
    glob = (rng.uniform(n * num_global).reshape(n, num_global) * 2.0 - 1.0).astype(np.float32)
    return spatial.reshape(n, hw * num_spatial), glob


def model_path(cache_dir: str, cfg: Config) -> str:
    return f"{cache_dir}/{cfg.arch.name}-s{cfg.weight_seed}.bin.gz"


def ensure_model(cache_dir: str, cfg: Config) -> str:
    """Writes the config's model into cache_dir unless already there."""
    import os
    os.makedirs(cache_dir, exist_ok=True)
    path = model_path(cache_dir, cfg)
    if not os.path.exists(path):
        tmp = path + f".tmp{os.getpid()}"
        write_model(cfg.arch, cfg.weight_seed, tmp, binary=True, gz=True)
        os.replace(tmp, path)
    return path
