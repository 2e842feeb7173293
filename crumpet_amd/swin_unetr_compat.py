"""A MONAI-compatible 3D Swin UNETR, for when MONAI is not installed.

crumpet's MONAI integration (torch-ext/crumpet/monai_patch.py) patches three
methods of ``monai.networks.nets.swin_unetr`` (MONAI 1.5.2):
``SwinTransformerBlock.forward_part1``, ``BasicLayer.forward`` and
``WindowAttention.forward``.  MONAI is not part of this build, so this
module restates the parts of that MONAI module the patch and the
end-to-end benchmark need, with the same class names, constructor
arguments, attribute names (``qkv``, ``proj``, ``relative_position_bias_table``,
``relative_position_index``, ``norm1``, ``attn``, ``blocks``, ``downsample``
...) and forward semantics, so that ``crumpet_amd.patch_monai_swin_unetr``
patches it exactly as it would patch MONAI.

The forwards here are MONAI's eager math (torch.roll + view/permute window
partition, q*scale @ k^T + bias + mask, softmax, @ v), i.e. the unpatched
baseline.  Compatibility with real MONAI's numerics is by construction from
MONAI's published architecture (Hatamizadeh et al., "Swin UNETR", 2022;
Liu et al., "Swin Transformer", 2021); it cannot be checked against MONAI
here (MONAI is absent).  Known MONAI details kept on purpose:

* ``get_window_size`` shrinks the window to the feature size and zeroes the
  shift on axes where the size does not exceed the window;
* the relative-position index is built for the configured window and
  sliced ``[:n, :n]`` when the effective window is smaller;
* ``PatchMerging`` (the ``"merging"`` default) concatenates the eight
  sub-grids in MONAI's v0.9 order, which repeats two of them;
* ``compute_mask`` labels the 27 slice regions and sets -100 where labels
  differ.
"""

from __future__ import annotations

import itertools
from typing import Sequence

import torch
import torch.nn as nn
import torch.nn.functional as F

__all__ = [
    "SwinUNETR",
    "SwinTransformer",
    "BasicLayer",
    "SwinTransformerBlock",
    "WindowAttention",
    "PatchMerging",
    "PatchMergingV2",
    "PatchEmbed",
    "MLPBlock",
    "UnetResBlock",
    "UnetrBasicBlock",
    "UnetrUpBlock",
    "UnetOutBlock",
    "get_window_size",
    "compute_mask",
    "window_partition",
    "window_reverse",
]


def get_window_size(x_size, window_size, shift_size=None):
    """Effective window (and shift): an axis no longer than the window uses
    its full size as the window and no shift."""
    win = list(window_size)
    sh = list(shift_size) if shift_size is not None else None
    for i, size in enumerate(x_size):
        if size <= window_size[i]:
            win[i] = size
            if sh is not None:
                sh[i] = 0
    if sh is None:
        return tuple(win)
    return tuple(win), tuple(sh)


def window_partition(x: torch.Tensor, window_size) -> torch.Tensor:
    """[b, d, h, w, c] -> [b * nW, wd * wh * ww, c], windows in (d, h, w) order."""
    b, d, h, w, c = x.shape
    wd, wh, ww = window_size
    x = x.view(b, d // wd, wd, h // wh, wh, w // ww, ww, c)
    return x.permute(0, 1, 3, 5, 2, 4, 6, 7).contiguous().view(-1, wd * wh * ww, c)


def window_reverse(windows: torch.Tensor, window_size, dims) -> torch.Tensor:
    """Inverse of ``window_partition``; dims = (b, d, h, w)."""
    b, d, h, w = dims
    wd, wh, ww = window_size
    x = windows.view(b, d // wd, h // wh, w // ww, wd, wh, ww, -1)
    return x.permute(0, 1, 4, 2, 5, 3, 6, 7).contiguous().view(b, d, h, w, -1)


def compute_mask(dims, window_size, shift_size, device) -> torch.Tensor:
    """Shifted-window mask [nW, n, n] (fp32): the padded volume is cut into
    three slices per axis ([:-ws], [-ws:-ss], [-ss:]); tokens of one window
    in different slice regions get -100."""
    d, h, w = dims
    img = torch.zeros((1, d, h, w, 1), device=device)
    label = 0
    cuts = [(slice(-ws), slice(-ws, -ss), slice(-ss, None)) for ws, ss in zip(window_size, shift_size)]
    for sd in cuts[0]:
        for sh in cuts[1]:
            for sw in cuts[2]:
                img[:, sd, sh, sw, :] = label
                label += 1
    win = window_partition(img, window_size).squeeze(-1)
    diff = win.unsqueeze(1) - win.unsqueeze(2)
    return diff.masked_fill(diff != 0, -100.0).masked_fill(diff == 0, 0.0)


class MLPBlock(nn.Module):
    """linear1 -> GELU -> dropout -> linear2 -> dropout (MONAI "swin" dropout mode)."""

    def __init__(self, hidden_size: int, mlp_dim: int, dropout_rate: float = 0.0):
        super().__init__()
        self.linear1 = nn.Linear(hidden_size, mlp_dim)
        self.linear2 = nn.Linear(mlp_dim, hidden_size)
        self.fn = nn.GELU()
        self.drop1 = nn.Dropout(dropout_rate)
        self.drop2 = self.drop1

    def forward(self, x):
        return self.drop2(self.linear2(self.drop1(self.fn(self.linear1(x)))))


def _relative_position_index(window_size) -> torch.Tensor:
    wd, wh, ww = window_size
    grid = torch.stack(torch.meshgrid(torch.arange(wd), torch.arange(wh), torch.arange(ww), indexing="ij"))
    flat = grid.flatten(1)
    rel = (flat[:, :, None] - flat[:, None, :]).permute(1, 2, 0).contiguous()
    rel[:, :, 0] += wd - 1
    rel[:, :, 1] += wh - 1
    rel[:, :, 2] += ww - 1
    rel[:, :, 0] *= (2 * wh - 1) * (2 * ww - 1)
    rel[:, :, 1] *= 2 * ww - 1
    return rel.sum(-1)


class WindowAttention(nn.Module):
    """Window multi-head self-attention with a learned 3D relative-position bias."""

    def __init__(self, dim: int, num_heads: int, window_size: Sequence[int], qkv_bias: bool = False,
                 attn_drop: float = 0.0, proj_drop: float = 0.0):
        super().__init__()
        self.dim = dim
        self.window_size = tuple(window_size)
        self.num_heads = num_heads
        head_dim = dim // num_heads
        self.scale = head_dim ** -0.5
        wd, wh, ww = self.window_size
        self.relative_position_bias_table = nn.Parameter(
            torch.zeros((2 * wd - 1) * (2 * wh - 1) * (2 * ww - 1), num_heads))
        self.register_buffer("relative_position_index", _relative_position_index(self.window_size))
        self.qkv = nn.Linear(dim, dim * 3, bias=qkv_bias)
        self.attn_drop = nn.Dropout(attn_drop)
        self.proj = nn.Linear(dim, dim)
        self.proj_drop = nn.Dropout(proj_drop)
        nn.init.trunc_normal_(self.relative_position_bias_table, std=0.02)
        self.softmax = nn.Softmax(dim=-1)

    def forward(self, x, mask):
        b, n, c = x.shape
        qkv = self.qkv(x).reshape(b, n, 3, self.num_heads, c // self.num_heads).permute(2, 0, 3, 1, 4)
        q, k, v = qkv[0], qkv[1], qkv[2]
        q = q * self.scale
        # the transposed operand is made contiguous before the batched product
        attn = q @ k.transpose(-2, -1).contiguous()
        idx = self.relative_position_index.clone()[:n, :n].reshape(-1)
        bias = self.relative_position_bias_table[idx].reshape(n, n, -1).permute(2, 0, 1).contiguous()
        attn = attn + bias.unsqueeze(0)
        if mask is not None:
            nw = mask.shape[0]
            attn = attn.view(b // nw, nw, self.num_heads, n, n) + mask.unsqueeze(1).unsqueeze(0)
            attn = attn.view(-1, self.num_heads, n, n)
        attn = self.softmax(attn)
        attn = self.attn_drop(attn).to(v.dtype)
        x = (attn @ v).transpose(1, 2).reshape(b, n, c)
        return self.proj_drop(self.proj(x))


class SwinTransformerBlock(nn.Module):
    """norm1 -> (shifted) window attention -> residual; norm2 -> MLP -> residual."""

    def __init__(self, dim: int, num_heads: int, window_size: Sequence[int], shift_size: Sequence[int],
                 mlp_ratio: float = 4.0, qkv_bias: bool = True, drop: float = 0.0,
                 attn_drop: float = 0.0, drop_path: float = 0.0, norm_layer=nn.LayerNorm,
                 use_checkpoint: bool = False):
        super().__init__()
        self.dim = dim
        self.num_heads = num_heads
        self.window_size = tuple(window_size)
        self.shift_size = tuple(shift_size)
        self.mlp_ratio = mlp_ratio
        self.use_checkpoint = use_checkpoint
        self.norm1 = norm_layer(dim)
        self.attn = WindowAttention(dim, num_heads=num_heads, window_size=self.window_size,
                                    qkv_bias=qkv_bias, attn_drop=attn_drop, proj_drop=drop)
        if drop_path > 0.0:
            raise ValueError("drop_path > 0 is not supported by this inference-only restatement")
        self.drop_path = nn.Identity()
        self.norm2 = norm_layer(dim)
        self.mlp = MLPBlock(hidden_size=dim, mlp_dim=int(dim * mlp_ratio), dropout_rate=drop)

    def forward_part1(self, x, mask_matrix):
        x = self.norm1(x)
        b, d, h, w, c = x.shape
        window_size, shift_size = get_window_size((d, h, w), self.window_size, self.shift_size)
        pad_d1 = (window_size[0] - d % window_size[0]) % window_size[0]
        pad_b = (window_size[1] - h % window_size[1]) % window_size[1]
        pad_r = (window_size[2] - w % window_size[2]) % window_size[2]
        x = F.pad(x, (0, 0, 0, pad_r, 0, pad_b, 0, pad_d1))
        _, dp, hp, wp, _ = x.shape
        if any(s > 0 for s in shift_size):
            shifted = torch.roll(x, shifts=tuple(-s for s in shift_size), dims=(1, 2, 3))
            attn_mask = mask_matrix
        else:
            shifted = x
            attn_mask = None
        windows = window_partition(shifted, window_size)
        attn_windows = self.attn(windows, mask=attn_mask)
        attn_windows = attn_windows.view(-1, *(tuple(window_size) + (c,)))
        shifted = window_reverse(attn_windows, window_size, (b, dp, hp, wp))
        if any(s > 0 for s in shift_size):
            x = torch.roll(shifted, shifts=tuple(shift_size), dims=(1, 2, 3))
        else:
            x = shifted
        if pad_d1 > 0 or pad_r > 0 or pad_b > 0:
            x = x[:, :d, :h, :w, :].contiguous()
        return x

    def forward_part2(self, x):
        return self.drop_path(self.mlp(self.norm2(x)))

    def forward(self, x, mask_matrix):
        x = x + self.drop_path(self.forward_part1(x, mask_matrix))
        return x + self.forward_part2(x)


class PatchMergingV2(nn.Module):
    """2x2x2 neighbourhood concat (itertools order) -> LayerNorm(8C) -> Linear(8C, 2C)."""

    def __init__(self, dim: int, norm_layer=nn.LayerNorm, spatial_dims: int = 3):
        super().__init__()
        if spatial_dims != 3:
            raise ValueError("only 3D patch merging is restated here")
        self.dim = dim
        self.reduction = nn.Linear(8 * dim, 2 * dim, bias=False)
        self.norm = norm_layer(8 * dim)

    @staticmethod
    def _pad(x):
        _, d, h, w, _ = x.shape
        if d % 2 or h % 2 or w % 2:
            x = F.pad(x, (0, 0, 0, w % 2, 0, h % 2, 0, d % 2))
        return x

    def forward(self, x):
        x = self._pad(x)
        x = torch.cat([x[:, i::2, j::2, k::2, :] for i, j, k in itertools.product(range(2), range(2), range(2))], -1)
        return self.reduction(self.norm(x))


class PatchMerging(PatchMergingV2):
    """MONAI's ``"merging"`` downsampling (the v0.9 sub-grid order, kept by MONAI
    for checkpoint compatibility: the 6th and 7th slices repeat the 3rd and 4th)."""

    def forward(self, x):
        x = self._pad(x)
        parts = [
            x[:, 0::2, 0::2, 0::2, :],
            x[:, 1::2, 0::2, 0::2, :],
            x[:, 0::2, 1::2, 0::2, :],
            x[:, 0::2, 0::2, 1::2, :],
            x[:, 1::2, 0::2, 1::2, :],
            x[:, 0::2, 1::2, 0::2, :],
            x[:, 0::2, 0::2, 1::2, :],
            x[:, 1::2, 1::2, 1::2, :],
        ]
        return self.reduction(self.norm(torch.cat(parts, -1)))


MERGING_MODE = {"merging": PatchMerging, "mergingv2": PatchMergingV2}


class BasicLayer(nn.Module):
    """One Swin stage: ``depth`` blocks alternating unshifted / shifted windows,
    then optional downsampling.  Input and output are channels-first."""

    def __init__(self, dim: int, depth: int, num_heads: int, window_size: Sequence[int], drop_path,
                 mlp_ratio: float = 4.0, qkv_bias: bool = False, drop: float = 0.0,
                 attn_drop: float = 0.0, norm_layer=nn.LayerNorm, downsample=None,
                 use_checkpoint: bool = False):
        super().__init__()
        self.window_size = tuple(window_size)
        self.shift_size = tuple(i // 2 for i in self.window_size)
        self.no_shift = tuple(0 for _ in self.window_size)
        self.depth = depth
        self.use_checkpoint = use_checkpoint
        self.blocks = nn.ModuleList([
            SwinTransformerBlock(dim=dim, num_heads=num_heads, window_size=self.window_size,
                                 shift_size=self.no_shift if i % 2 == 0 else self.shift_size,
                                 mlp_ratio=mlp_ratio, qkv_bias=qkv_bias, drop=drop, attn_drop=attn_drop,
                                 drop_path=drop_path[i] if isinstance(drop_path, list) else drop_path,
                                 norm_layer=norm_layer, use_checkpoint=use_checkpoint)
            for i in range(depth)
        ])
        self.downsample = downsample(dim=dim, norm_layer=norm_layer, spatial_dims=3) if callable(downsample) else downsample

    def forward(self, x):
        b, c, d, h, w = x.shape
        window_size, shift_size = get_window_size((d, h, w), self.window_size, self.shift_size)
        x = x.permute(0, 2, 3, 4, 1)
        dp = -(-d // window_size[0]) * window_size[0]
        hp = -(-h // window_size[1]) * window_size[1]
        wp = -(-w // window_size[2]) * window_size[2]
        attn_mask = compute_mask((dp, hp, wp), window_size, shift_size, x.device)
        for blk in self.blocks:
            x = blk(x, attn_mask)
        x = x.view(b, d, h, w, -1)
        if self.downsample is not None:
            x = self.downsample(x)
        return x.permute(0, 4, 1, 2, 3)


class PatchEmbed(nn.Module):
    """Non-overlapping patch embedding: a strided Conv3d (inputs padded up to a multiple of the patch)."""

    def __init__(self, patch_size=(2, 2, 2), in_chans: int = 1, embed_dim: int = 48, norm_layer=None,
                 spatial_dims: int = 3):
        super().__init__()
        self.patch_size = tuple(patch_size)
        self.embed_dim = embed_dim
        self.proj = nn.Conv3d(in_chans, embed_dim, kernel_size=self.patch_size, stride=self.patch_size)
        self.norm = norm_layer(embed_dim) if norm_layer is not None else None

    def forward(self, x):
        _, _, d, h, w = x.shape
        pd, ph, pw = self.patch_size
        if w % pw:
            x = F.pad(x, (0, pw - w % pw))
        if h % ph:
            x = F.pad(x, (0, 0, 0, ph - h % ph))
        if d % pd:
            x = F.pad(x, (0, 0, 0, 0, 0, pd - d % pd))
        x = self.proj(x)
        if self.norm is not None:
            b, c, d2, h2, w2 = x.shape
            x = self.norm(x.flatten(2).transpose(1, 2)).transpose(1, 2).view(b, c, d2, h2, w2)
        return x


class SwinTransformer(nn.Module):
    """Patch embedding plus four Swin stages; returns the five multi-scale features."""

    def __init__(self, in_chans: int, embed_dim: int, window_size, patch_size, depths, num_heads,
                 mlp_ratio: float = 4.0, qkv_bias: bool = True, drop_rate: float = 0.0,
                 attn_drop_rate: float = 0.0, drop_path_rate: float = 0.0, norm_layer=nn.LayerNorm,
                 patch_norm: bool = False, use_checkpoint: bool = False, spatial_dims: int = 3,
                 downsample="merging"):
        super().__init__()
        self.num_layers = len(depths)
        self.embed_dim = embed_dim
        self.patch_norm = patch_norm
        self.window_size = tuple(window_size)
        self.patch_size = tuple(patch_size)
        self.patch_embed = PatchEmbed(patch_size=self.patch_size, in_chans=in_chans, embed_dim=embed_dim,
                                      norm_layer=norm_layer if patch_norm else None, spatial_dims=spatial_dims)
        self.pos_drop = nn.Dropout(p=drop_rate)
        dpr = [float(v) for v in torch.linspace(0, drop_path_rate, sum(depths))]
        down = MERGING_MODE[downsample] if isinstance(downsample, str) else downsample
        for i in range(self.num_layers):
            layer = BasicLayer(dim=int(embed_dim * 2 ** i), depth=depths[i], num_heads=num_heads[i],
                               window_size=self.window_size,
                               drop_path=dpr[sum(depths[:i]):sum(depths[:i + 1])], mlp_ratio=mlp_ratio,
                               qkv_bias=qkv_bias, drop=drop_rate, attn_drop=attn_drop_rate,
                               norm_layer=norm_layer, downsample=down, use_checkpoint=use_checkpoint)
            setattr(self, f"layers{i + 1}", nn.ModuleList([layer]))
        self.num_features = int(embed_dim * 2 ** self.num_layers)

    @staticmethod
    def proj_out(x, normalize: bool = False):
        if normalize:
            c = x.shape[1]
            x = F.layer_norm(x.permute(0, 2, 3, 4, 1), [c]).permute(0, 4, 1, 2, 3)
        return x

    def forward(self, x, normalize: bool = True):
        x0 = self.pos_drop(self.patch_embed(x))
        outs = [self.proj_out(x0, normalize)]
        xi = x0
        for i in range(self.num_layers):
            xi = getattr(self, f"layers{i + 1}")[0](xi.contiguous())
            outs.append(self.proj_out(xi, normalize))
        return outs


class UnetResBlock(nn.Module):
    """conv-norm-lrelu-conv-norm (+ 1x1 conv-norm residual projection) -> add -> lrelu."""

    def __init__(self, spatial_dims: int, in_channels: int, out_channels: int, kernel_size: int = 3,
                 stride: int = 1, norm_name: str = "instance"):
        super().__init__()
        if norm_name != "instance" or spatial_dims != 3:
            raise ValueError("only 3D instance-norm residual blocks are restated here")
        pad = (kernel_size - stride + 1) // 2
        self.conv1 = nn.Conv3d(in_channels, out_channels, kernel_size, stride=stride, padding=pad, bias=False)
        self.conv2 = nn.Conv3d(out_channels, out_channels, kernel_size, stride=1,
                               padding=(kernel_size - 1 + 1) // 2, bias=False)
        self.lrelu = nn.LeakyReLU(negative_slope=0.01, inplace=True)
        self.norm1 = nn.InstanceNorm3d(out_channels)
        self.norm2 = nn.InstanceNorm3d(out_channels)
        self.downsample = in_channels != out_channels or stride != 1
        if self.downsample:
            self.conv3 = nn.Conv3d(in_channels, out_channels, 1, stride=stride, bias=False)
            self.norm3 = nn.InstanceNorm3d(out_channels)

    def forward(self, inp):
        out = self.lrelu(self.norm1(self.conv1(inp)))
        out = self.norm2(self.conv2(out))
        residual = self.norm3(self.conv3(inp)) if self.downsample else inp
        out += residual
        return self.lrelu(out)


class UnetrBasicBlock(nn.Module):
    def __init__(self, spatial_dims: int, in_channels: int, out_channels: int, kernel_size: int,
                 stride: int, norm_name: str = "instance", res_block: bool = True):
        super().__init__()
        if not res_block:
            raise ValueError("only the residual variant (res_block=True) is restated here")
        self.layer = UnetResBlock(spatial_dims, in_channels, out_channels, kernel_size, stride, norm_name)

    def forward(self, inp):
        return self.layer(inp)


class UnetrUpBlock(nn.Module):
    """Transposed-conv upsampling, concat with the skip, residual block."""

    def __init__(self, spatial_dims: int, in_channels: int, out_channels: int, kernel_size: int,
                 upsample_kernel_size: int, norm_name: str = "instance", res_block: bool = True):
        super().__init__()
        if not res_block:
            raise ValueError("only the residual variant (res_block=True) is restated here")
        self.transp_conv = nn.ConvTranspose3d(in_channels, out_channels, upsample_kernel_size,
                                              stride=upsample_kernel_size, bias=False)
        self.conv_block = UnetResBlock(spatial_dims, 2 * out_channels, out_channels, kernel_size, 1, norm_name)

    def forward(self, inp, skip):
        return self.conv_block(torch.cat((self.transp_conv(inp), skip), dim=1))


class UnetOutBlock(nn.Module):
    def __init__(self, spatial_dims: int, in_channels: int, out_channels: int):
        super().__init__()
        self.conv = nn.Conv3d(in_channels, out_channels, 1, bias=True)

    def forward(self, inp):
        return self.conv(inp)


class SwinUNETR(nn.Module):
    """Swin UNETR (patch 2, window 7): Swin encoder with a residual conv U-Net decoder."""

    def __init__(self, in_channels: int, out_channels: int, depths=(2, 2, 2, 2), num_heads=(3, 6, 12, 24),
                 feature_size: int = 24, norm_name: str = "instance", drop_rate: float = 0.0,
                 attn_drop_rate: float = 0.0, dropout_path_rate: float = 0.0, normalize: bool = True,
                 use_checkpoint: bool = False, spatial_dims: int = 3, downsample="merging",
                 use_v2: bool = False, img_size=None):
        super().__init__()
        if spatial_dims != 3:
            raise ValueError("only spatial_dims=3 is restated here")
        if use_v2:
            raise ValueError("use_v2=True is not restated here")
        if feature_size % 12 != 0:
            raise ValueError("feature_size should be divisible by 12")
        self.normalize = normalize
        fs = feature_size
        self.swinViT = SwinTransformer(in_chans=in_channels, embed_dim=fs, window_size=(7, 7, 7),
                                       patch_size=(2, 2, 2), depths=depths, num_heads=num_heads,
                                       mlp_ratio=4.0, qkv_bias=True, drop_rate=drop_rate,
                                       attn_drop_rate=attn_drop_rate, drop_path_rate=dropout_path_rate,
                                       norm_layer=nn.LayerNorm, use_checkpoint=use_checkpoint,
                                       spatial_dims=spatial_dims, downsample=downsample)
        self.encoder1 = UnetrBasicBlock(3, in_channels, fs, 3, 1, norm_name)
        self.encoder2 = UnetrBasicBlock(3, fs, fs, 3, 1, norm_name)
        self.encoder3 = UnetrBasicBlock(3, 2 * fs, 2 * fs, 3, 1, norm_name)
        self.encoder4 = UnetrBasicBlock(3, 4 * fs, 4 * fs, 3, 1, norm_name)
        self.encoder10 = UnetrBasicBlock(3, 16 * fs, 16 * fs, 3, 1, norm_name)
        self.decoder5 = UnetrUpBlock(3, 16 * fs, 8 * fs, 3, 2, norm_name)
        self.decoder4 = UnetrUpBlock(3, 8 * fs, 4 * fs, 3, 2, norm_name)
        self.decoder3 = UnetrUpBlock(3, 4 * fs, 2 * fs, 3, 2, norm_name)
        self.decoder2 = UnetrUpBlock(3, 2 * fs, fs, 3, 2, norm_name)
        self.decoder1 = UnetrUpBlock(3, fs, fs, 3, 2, norm_name)
        self.out = UnetOutBlock(3, fs, out_channels)

    def forward(self, x_in):
        hidden = self.swinViT(x_in, self.normalize)
        enc0 = self.encoder1(x_in)
        enc1 = self.encoder2(hidden[0])
        enc2 = self.encoder3(hidden[1])
        enc3 = self.encoder4(hidden[2])
        dec4 = self.encoder10(hidden[4])
        dec3 = self.decoder5(dec4, hidden[3])
        dec2 = self.decoder4(dec3, enc3)
        dec1 = self.decoder3(dec2, enc2)
        dec0 = self.decoder2(dec1, enc1)
        out = self.decoder1(dec0, enc0)
        return self.out(out)
