"""Pins of the oracle's model-level stream loop (oracle/runtime.py) on the CPU.

The loop's order is fixed by the reference:
  * per block: conditioning from the memory, denoise over the pre-block
    layers, renorm, colour correction, clean commit from the pre-block
    layers, set_reference (block 0) and update, then retention
    (taomate/inference/model.py:200-243; model_runtime.py:1160-1325);
  * inside the denoise: the prefix-only cache every step, x0 = x - v*sigma,
    re-noise with the NEXT sigma while it is above 0
    (model_runtime.py:847-962);
  * on a prompt change: the sink block plus the last warm prefix blocks,
    each re-run at its segment's global block position
    (taomate/inference/runtime.py:365-371, 400-414).

Each pin is a closed form, an invariant or a known answer worked out from
those lines, and each is also run on a mutant of the oracle carrying a
plausible slip, where it must fail.
"""
import pytest
import torch

from oracle import cache as OC
from oracle import memory as OM
from oracle import runtime as ORT
from taomate_amd import dit as D
from taomate_amd import runtime as RT

HW = (4, 8)
C = 8
B = 2


def _cfg():
    return D.AVConfig(num_layers=1, video_dim=32, audio_dim=16, video_heads=2, audio_heads=2, video_d_head=16,
                      audio_d_head=8, in_channels=C, out_channels=C)


def _params(cfg, seed=3):
    m = D.build_model(cfg, "cpu", seed=seed, dtype=torch.float32)
    return {n: p.detach().float().clone() for n, p in m.named_parameters()}


def _cond(cfg, seed=11):
    g = torch.Generator().manual_seed(seed)
    keep = torch.ones(B, 6, dtype=torch.int64)
    keep[:, -2:] = 0
    return dict(video_context=torch.randn(B, 6, cfg.video_dim, generator=g),
                audio_context=torch.randn(B, 6, cfg.audio_dim, generator=g),
                video_context_mask=keep, audio_context_mask=keep)


class Tape:
    """Seeded Gaussians, every draw kept in order for replay."""

    def __init__(self, seed):
        self.g = torch.Generator().manual_seed(seed)
        self.draws = []

    def __call__(self, shape):
        x = torch.randn(shape, generator=self.g)
        self.draws.append(x)
        return x


# ---------------------------------------------------------------------------
# (a) denoise: closed form with a constant velocity
# ---------------------------------------------------------------------------

def _closed_form_denoise(draws, bias, sig):
    """x = n0; x <- x - b*s0; x <- (1 - s1) x + s1 n1; x <- x - b*s1;
    x <- (1 - s2) x + s2 n2; x <- x - b*s2 (s3 = 0: no re-noise), with the
    tape's draws in the loop's order (video, audio initial; then per
    re-noise video, audio)."""
    s0, s1, s2, s3 = (float(v) for v in sig)
    assert s3 == 0.0
    v0, a0, v1, a1, v2, a2 = draws
    out = []
    for n0, n1, n2, b in ((v0, v1, v2, bias[0]), (a0, a1, a2, bias[1])):
        x = n0 - b * s0
        x = (1 - s1) * x + s1 * n1
        x = x - b * s1
        x = (1 - s2) * x + s2 * n2
        out.append(x - b * s2)
    return out


class RenoiseWithCurrentSigma(ORT.StreamOracle):
    """Planted slip: re-noise with sigma[si] instead of sigma[si + 1]."""

    def _denoise(self, blk, B_, C_, c, pre):
        _, vs, ve, as_, ae = blk
        H, W = self.hw
        video = self.noise((B_, ve - vs, C_, H, W))
        audio = self.noise((B_, ae - as_, C_))
        sig = self.sigmas
        for si in range(len(sig) - 1):
            s = sig[si].expand(B_)
            v_vel, a_vel, _ = self._forward(blk, video, audio, s, c, pre)
            video, audio = ORT.velocity_to_x0(video, v_vel, s), ORT.velocity_to_x0(audio, a_vel, s)
            if float(sig[si + 1]) > 0.0:
                video = ORT.add_noise(video, self.noise(tuple(video.shape)), s)
                audio = ORT.add_noise(audio, self.noise(tuple(audio.shape)), s)
        return video, audio


def _denoise_matches_closed_form(cls) -> bool:
    cfg = _cfg()
    p = _params(cfg)
    g = torch.Generator().manual_seed(5)
    bv, ba = torch.randn(C, generator=g), torch.randn(C, generator=g)
    p["proj_out.weight"].zero_()
    p["proj_out.bias"].copy_(bv)
    p["audio_proj_out.weight"].zero_()
    p["audio_proj_out.bias"].copy_(ba)
    tape = Tape(7)
    orc = cls(p, cfg, HW, noise=tape, renorm=False)
    out = orc.first_window(B, C, _cond(cfg), frames=7)          # blocks of 4 and 3 frames
    assert len(tape.draws) == 12
    sig = orc.sigmas
    ok = True
    for i, (blk, v, a) in enumerate(out):
        wv, wa = _closed_form_denoise(tape.draws[6 * i:6 * i + 6], (bv.view(1, 1, C, 1, 1), ba.view(1, 1, C)), sig)
        ok &= torch.allclose(v, wv, rtol=1e-5, atol=1e-5) and torch.allclose(a, wa, rtol=1e-5, atol=1e-5)
    return ok


def test_denoise_closed_form_with_constant_velocity():
    """With the output heads' weights zeroed the velocity is the heads'
    bias, whatever the blocks compute, so the 3-step denoise is a closed form
    in the noise tape and the four sigmas (1, ~0.757, ~0.522, 0)."""
    sig = ORT.denoising_sigmas()
    assert sig.numel() == 4 and sig[0].item() == 1.0 and sig[-1].item() == 0.0
    assert _denoise_matches_closed_form(ORT.StreamOracle)
    assert not _denoise_matches_closed_form(RenoiseWithCurrentSigma)


# ---------------------------------------------------------------------------
# (b) renorm: alpha 1 carries block 0's channel statistics
# ---------------------------------------------------------------------------

class AnchorEveryBlock(ORT.StreamOracle):
    """Planted slip: the renorm anchor captured again on every block."""

    def _stabilize(self, bi, video):
        self.anchor = ORT.channel_stats(video)
        return video


def _renorm_carries_block0(cls) -> bool:
    cfg = _cfg()
    orc = cls(_params(cfg), cfg, HW, noise=Tape(8), renorm=True, alpha=1.0)
    out = orc.first_window(B, C, _cond(cfg), frames=10)         # blocks of 4, 3, 3 frames
    m0, s0 = ORT.channel_stats(out[0][1])
    ok = True
    for _, v, _ in out[1:]:
        m, s = ORT.channel_stats(v)
        ok &= torch.allclose(m, m0, atol=1e-5) and torch.allclose(s, s0, atol=1e-5)
    return ok


def test_renorm_alpha_one_carries_block0_statistics():
    """_maybe_renorm_block with alpha 1 (model_runtime.py:24-46, 732-770):
    block 0 sets the anchor; every later block leaves with block 0's
    per-(batch, channel) mean and standard deviation over frames, rows and
    columns."""
    assert _renorm_carries_block0(ORT.StreamOracle)
    assert not _renorm_carries_block0(AnchorEveryBlock)


# ---------------------------------------------------------------------------
# (c) commit: from the renormed, colour-corrected latents
# ---------------------------------------------------------------------------

class Recorder(ORT.StreamOracle):
    """Keeps the conditioning and pre-block layers each commit received."""

    def __init__(self, *a, **kw):
        super().__init__(*a, **kw)
        self.commits = []

    def _commit(self, blk, video, audio, c, pre, first_of_stream):
        self.commits.append((blk, c, pre, first_of_stream))
        super()._commit(blk, video, audio, c, pre, first_of_stream)


class CommitBeforeColour(Recorder):
    """Planted slip: the clean commit runs on the latents before the colour
    correction."""

    def _block(self, blk, B_, C_, cond, first_of_stream):
        c = self._cond(cond)
        pre = self.layers
        video, audio = self._denoise(blk, B_, C_, c, pre)
        video = self._stabilize(blk[0], video)
        self._commit(blk, video, audio, c, pre, first_of_stream)
        video = torch.from_numpy(self.memory.apply_color(video.double().numpy())).float()
        if first_of_stream:
            self.memory.set_reference(video.double().numpy(), audio.double().numpy())
        self.memory.update(video.double().numpy(), audio.double().numpy())
        return video, audio


def _commit_is_of_final_latents(cls) -> bool:
    cfg = _cfg()
    mem = OM.MemoryOracle(color_alpha=0.5, color_proto_alpha=0.3)
    orc = cls(_params(cfg), cfg, HW, noise=Tape(9), memory=mem)
    out = orc.first_window(B, C, _cond(cfg), frames=7)
    blk, v, a = out[1]
    rec_blk, c, pre, first = orc.commits[1]
    assert rec_blk == blk and not first and pre is not None
    L = v.shape[1] * HW[0] * HW[1]
    _, _, direct = ORT.StreamOracle._forward(orc, blk, v, a, torch.zeros(B), c, pre)
    ok = True
    for key in ("video_self_k", "video_self_v", "v2a_k", "audio_self_k", "a2v_v"):
        n = L if key in ("video_self_k", "video_self_v", "v2a_k") else a.shape[1]
        ok &= torch.allclose(orc.layers[0][key][:, -n:], direct[0][key][:, -n:], rtol=1e-5, atol=1e-5)
        # the committed layers are the pre-block layers with this block appended
        ok &= torch.equal(orc.layers[0][key][:, :-n], pre[0][key])
    return ok


def test_commit_is_a_sigma0_pass_over_the_final_latents():
    """_commit_clean_block (model.py:88-129) after _stabilize_video and
    apply_color_memory (model.py:217-232): the committed K/V of a block are
    those of a sigma-0 pass over its renormed, colour-corrected latents,
    appended to the pre-block layers.  The colour correction is made strong
    here so that its order is visible."""
    assert _commit_is_of_final_latents(Recorder)
    assert not _commit_is_of_final_latents(CommitBeforeColour)


# ---------------------------------------------------------------------------
# (d) memory: set_reference on block 0 only, update after the commit
# ---------------------------------------------------------------------------

class SpyMemory:
    def __init__(self, log):
        self.m, self.log = OM.MemoryOracle(), log

    def conditioning(self):
        self.log.append("conditioning")
        return self.m.conditioning()

    def apply_color(self, video):
        self.log.append("colour")
        return self.m.apply_color(video)

    def set_reference(self, video, audio):
        self.log.append("set_reference")
        self.m.set_reference(video, audio)

    def update(self, video, audio):
        self.log.append("update")
        self.m.update(video, audio)


class Logged(ORT.StreamOracle):
    def __init__(self, *a, log=None, **kw):
        super().__init__(*a, **kw)
        self.log = log

    def _forward(self, blk, video, audio, sigma, cond, layers):
        self.log.append("denoise" if float(sigma.max()) > 0 else "forward0")
        return super()._forward(blk, video, audio, sigma, cond, layers)

    def _commit(self, *a):
        self.log.append("commit")
        super()._commit(*a)


class UpdateBeforeCommit(Logged):
    """Planted slip: the memory is fed the block before its clean commit."""

    def _block(self, blk, B_, C_, cond, first_of_stream):
        c = self._cond(cond)
        pre = self.layers
        video, audio = self._denoise(blk, B_, C_, c, pre)
        video = self._stabilize(blk[0], video)
        video = torch.from_numpy(self.memory.apply_color(video.double().numpy())).float()
        if first_of_stream:
            self.memory.set_reference(video.double().numpy(), audio.double().numpy())
        self.memory.update(video.double().numpy(), audio.double().numpy())
        self._commit(blk, video, audio, c, pre, first_of_stream)
        return video, audio


class ReferenceEveryBlock(Logged):
    """Planted slip: set_reference on every block."""

    def _block(self, blk, B_, C_, cond, first_of_stream):
        return super()._block(blk, B_, C_, cond, True if self.layers is not None else first_of_stream)


def _order(cls, monkeypatch):
    log = []
    real = OC.retain_streaming_context

    def retain(layers, segments, keep):
        log.append("retain")
        return real(layers, segments, keep)

    monkeypatch.setattr(OC, "retain_streaming_context", retain)
    cfg = _cfg()
    orc = cls(_params(cfg), cfg, HW, noise=Tape(10), memory=SpyMemory(log), log=log)
    orc.first_window(B, C, _cond(cfg), frames=7)
    first = list(log)
    log.clear()
    orc.next_window(B, C, _cond(cfg), first_block_index=2, n_blocks=2)
    return first, list(log)


def test_memory_and_commit_order(monkeypatch):
    """Per block (model_runtime.py:1160-1325 for the first window, model.py:
    200-243 for the next): conditioning, three denoise forwards, colour, the
    clean commit (a sigma-0 forward), set_reference on block 0 only, update;
    in the next window the retention after the update."""
    body = ["conditioning", "denoise", "denoise", "denoise", "colour", "commit", "forward0"]
    first, nxt = _order(Logged, monkeypatch)
    assert first == body + ["set_reference", "update"] + body + ["update"]
    assert nxt == (body + ["update", "retain"]) * 2
    bad_first, _ = _order(UpdateBeforeCommit, monkeypatch)
    assert bad_first != first
    bad_first, _ = _order(ReferenceEveryBlock, monkeypatch)
    assert bad_first != first


# ---------------------------------------------------------------------------
# (e) refresh: which prefix blocks re-run, at which global positions
# ---------------------------------------------------------------------------

# (block_idx, video_start, video_end, audio_start, audio_end): block 0 has 4
# video and 26 audio frames, block k >= 1 the video frames [4 + 3(k-1), 4 + 3k)
# and the audio frames [26 + 25(k-1), 26 + 25k) (mask_builder.py:125-134).
def _blk(k):
    return (0, 0, 4, 0, 26) if k == 0 else (k, 4 + 3 * (k - 1), 4 + 3 * k, 26 + 25 * (k - 1), 26 + 25 * k)


REFRESH_CASES = [
    # segments' block indices, prefix frames, next frames, (local, global) pairs
    ([0, 3, 4], 16, 15, [((0, 0, 4, 0, 26), _blk(0)), ((3, 10, 13, 76, 101), _blk(3)),
                         ((4, 13, 16, 101, 126), _blk(4))]),
    ([0, 8, 9], 10, 15, [((0, 0, 4, 0, 26), _blk(0)), ((1, 4, 7, 26, 51), (8, 25, 28, 201, 226)),
                         ((2, 7, 10, 51, 76), (9, 28, 31, 226, 251))]),
    ([3, 4], 7, 15, [((0, 0, 4, 0, 26), (3, 10, 13, 76, 101)), ((1, 4, 7, 26, 51), (4, 13, 16, 101, 126))]),
    ([0], 4, 15, [((0, 0, 4, 0, 26), (0, 0, 4, 0, 26))]),
    ([0, 7], 7, 15, [((0, 0, 4, 0, 26), _blk(0)), ((1, 4, 7, 26, 51), (7, 22, 25, 176, 201))]),
]


def _segs(ids):
    return [{"block_idx": k} for k in ids]


def _first_warm(segments, prefix_frames, next_frames):
    """Planted slip: the first warm prefix blocks instead of the last."""
    blocks = [b for b in ORT.compute_blocks(prefix_frames + next_frames) if b[2] <= prefix_frames]
    sink = segments[0]["block_idx"] == 0
    warm = len(segments) - int(sink)
    cands = blocks[1:] if sink else blocks
    sel = ([blocks[0]] if sink else []) + cands[:warm]
    return [(lb, ORT.global_block(s["block_idx"])) for lb, s in zip(sel, segments)]


def _local_positions(segments, prefix_frames, next_frames):
    """Planted slip: the segments re-run at their local prefix positions."""
    return [(lb, lb) for lb, _ in ORT.refresh_selection(segments, prefix_frames, next_frames)]


@pytest.mark.parametrize("ids,prefix,nxt,want", REFRESH_CASES)
def test_refresh_selection_known_answers(ids, prefix, nxt, want):
    assert tuple(ORT.global_block(ids[-1])) == want[-1][1]
    assert ORT.refresh_selection(_segs(ids), prefix, nxt) == want
    # the product picks the same blocks
    tup = lambda b: (b.block_idx, b.video_start, b.video_end, b.audio_start, b.audio_end)
    got = RT.refresh_selection(_segs(ids), prefix, nxt)
    assert [(tup(l), tup(g)) for l, g in got] == want


def test_refresh_selection_slips_are_caught():
    assert any(_first_warm(_segs(i), p, n) != w for i, p, n, w in REFRESH_CASES)
    assert any(_local_positions(_segs(i), p, n) != w for i, p, n, w in REFRESH_CASES)


def test_refresh_selection_rejects_a_short_prefix():
    """A prefix with fewer blocks than the cache's segments is the
    reference's layout error."""
    with pytest.raises(RuntimeError):
        ORT.refresh_selection(_segs([0, 3, 4]), 7, 15)
    with pytest.raises(RuntimeError):
        RT.refresh_selection(_segs([0, 3, 4]), 7, 15)
