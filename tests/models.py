"""Small models used by the backend tests, with the shapes the reference's tests use on purpose
(tests/test_backend.py:19-31, :97-109, :203-217, :268-277 in the reference): K=200 and N=300 that are
not block multiples, q/k/v linears sharing an input, and 3x3 convs with and without bias, padding
"same", a stride-2 conv the pass must leave alone, and odd channel counts / image sizes."""
import torch
import torch.nn.functional as F


class Net(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.a = torch.nn.Linear(200, 300)
        self.b = torch.nn.Linear(300, 1024, bias=False)
        self.w = torch.nn.Parameter(torch.randn(1024, 520) * 0.03)

    def forward(self, x):
        h = F.gelu(self.a(x))
        h = F.silu(self.b(h))
        return h @ self.w


class Attn(torch.nn.Module):
    """q/k/v read the same input -> one fused GEMM; o reads another."""

    def __init__(self):
        super().__init__()
        self.q = torch.nn.Linear(256, 256)
        self.k = torch.nn.Linear(256, 128, bias=False)
        self.v = torch.nn.Linear(256, 128)
        self.o = torch.nn.Linear(256, 256)

    def forward(self, x):
        q, k, v = self.q(x), self.k(x), self.v(x)
        return self.o(q * torch.cat([k, v], -1).sigmoid())


class CNN(torch.nn.Module):
    """A conv with bias (its ReLU stays a graph op), one without (ReLU fused), padding "same", and a
    stride-2 conv the op does not take."""

    def __init__(self):
        super().__init__()
        self.c1 = torch.nn.Conv2d(64, 128, 3, padding=1)
        self.c2 = torch.nn.Conv2d(128, 128, 3, padding=1, bias=False)
        self.c3 = torch.nn.Conv2d(128, 32, 3, padding="same")
        self.down = torch.nn.Conv2d(32, 32, 3, stride=2, padding=1)

    def forward(self, x):
        h = torch.relu(self.c1(x))
        h = torch.relu(self.c2(h))
        return self.down(self.c3(h))


class OddCNN(torch.nn.Module):
    """Channel counts the kernel pads (Ci 3, Co 48) and an odd image size."""

    def __init__(self):
        super().__init__()
        self.c1 = torch.nn.Conv2d(3, 64, 3, padding=1)
        self.c2 = torch.nn.Conv2d(64, 48, 3, padding=1, bias=False)

    def forward(self, x):
        return torch.relu(self.c2(torch.relu(self.c1(x))))


class VGGBlock(torch.nn.Module):
    """Bias-free 3x3 convs, each followed by a ReLU (BASELINE config 3 shape at 256 channels)."""

    def __init__(self, c, layers):
        super().__init__()
        self.convs = torch.nn.ModuleList(torch.nn.Conv2d(c, c, 3, padding=1, bias=False) for _ in range(layers))

    def forward(self, x):
        for conv in self.convs:
            x = torch.relu(conv(x))
        return x


class VGGStack(torch.nn.Module):
    """A VGG-style stack: biased convs with in-place ReLUs and 2x2 max-pools (torchvision's layout),
    bias-free convs whose ReLU the rewrite fuses, channel counts that are and are not multiples of 64."""

    def __init__(self):
        super().__init__()
        self.features = torch.nn.Sequential(
            torch.nn.Conv2d(3, 32, 3, padding=1), torch.nn.ReLU(inplace=True),
            torch.nn.Conv2d(32, 64, 3, padding=1), torch.nn.ReLU(inplace=True), torch.nn.MaxPool2d(2, 2),
            torch.nn.Conv2d(64, 48, 3, padding=1, bias=False), torch.nn.ReLU(),
            torch.nn.MaxPool2d(2),
            torch.nn.Conv2d(48, 64, 3, padding=1), torch.nn.ReLU(inplace=True),
            torch.nn.Conv2d(64, 40, 3, padding=1))

    def forward(self, x):
        return torch.relu(self.features(x))


class Stack(torch.nn.Module):
    """A transformers Qwen3Model of Qwen3-0.6B's widths (random init) into a linear head, fed
    embeddings and a 4-D attention mask (the reference's stack test model, OmniVoice's backbone in
    miniature)."""

    def __init__(self, layers=2, out=1000, bias=False):
        super().__init__()
        from transformers import Qwen3Config, Qwen3Model

        cfg = Qwen3Config(hidden_size=1024, intermediate_size=3072, num_hidden_layers=layers, num_attention_heads=16,
                          num_key_value_heads=8, head_dim=128, vocab_size=16, rms_norm_eps=1e-6,
                          rope_parameters={"rope_type": "default", "rope_theta": 1e6}, attn_implementation="sdpa")
        self.llm = Qwen3Model(cfg)
        self.head = torch.nn.Linear(1024, out, bias=bias)

    def forward(self, x, mask):
        return self.head(self.llm(inputs_embeds=x, attention_mask=mask)[0])


def prefix_mask(lens, L, device="cpu"):
    """Sequence b's first n positions see those n; each padding position after them sees itself."""
    m = torch.zeros(len(lens), 1, L, L, dtype=torch.bool)
    for b, n in enumerate(lens):
        m[b, :, :n, :n] = True
        i = torch.arange(n, L)
        m[b, :, i, i] = True
    return m.to(device)


def run(net, x, **opts):
    """torch.compile with the xdna backend from a fresh Dynamo cache and fresh stats."""
    from torch_xdna import runtime

    torch._dynamo.reset()
    runtime.stats.reset()
    m = torch.compile(net, backend="xdna", options=opts)
    with torch.no_grad():
        return m(x)


def rel_err(y, ref):
    return ((y.float() - ref.float()).norm() / ref.float().norm()).item()
