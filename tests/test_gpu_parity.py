"""HIP step vs the CPU oracle, bit for bit, through the C ABI on the GPU.

Integer/index leaves (contact slots, candidate indices, keys, manifold point counts and feature ids, TOI counts and
flags) and float leaves (positions, angles, velocities, impulses, manifold geometry) must be identical at every step:
both sides perform the reference's float32 operations in the same order, so a float tolerance (1e-4 abs /
1e-3 rel per step would be allowed) is not needed; any difference is a bug. Island ids and solve order (not State leaves) are
compared through the debug outputs.
"""
import numpy as np
import pytest

from util import b2, leaf_mismatches, perturbed, wd

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _run(model, state, settings, dt, steps, oracle, actions=None):
    dev = b2.layout.to_device(state, "cuda")
    ref = oracle.copy(state)
    for k in range(steps):
        if actions is not None:
            a = actions[k]
            b2.scenes.apply_actions(ref.joints.motor_speed, ref.joints.max_motor, a)
            b2.scenes.apply_actions(dev.joints.motor_speed, dev.joints.max_motor, torch.from_numpy(a).cuda())
        b2.step_(model, dev, settings, dt)
        oracle.step_(model, ref, settings, dt)
        got = b2.layout.to_host(dev)
        bad = leaf_mismatches(ref, got)
        assert bad == [], f"step {k + 1}: {bad[:4]}"
    return ref


@pytest.mark.parametrize("name", list(b2.scenes.TEST_SCENES))
def test_scene_parity(name, oracle):
    """Every test scene, 64 perturbed copies, 90 steps, stock iteration counts."""
    s, m, st = b2.scenes.build_test_scene(name, iterations=(8, 3))
    _run(m, perturbed(st, 64), s, 1.0 / 60.0, 90, oracle)


@pytest.mark.parametrize("name", ["pile", "hammer_chain", "island_walk", "joints"])
def test_scene_parity_game_iterations(name, oracle):
    """The game's 300 / 30 iterations on the heavier scenes."""
    s, m, st = b2.scenes.build_test_scene(name)
    _run(m, perturbed(st, 16, seed=3), s, b2.GAME_DT, 60, oracle)


@pytest.mark.parametrize("k,n,steps,edges", [(1, 1, 200, "quad"), (3, 512, 30, "quad"), (4, 512, 30, "quad"),
                                              (5, 128, 20, "quad"), (4, 512, 30, "native"), (5, 128, 20, "native")])
def test_config_parity(k, n, steps, edges, oracle):
    """The benchmark configurations; "native" builds the terrain chain from b2EdgeShape children instead of thin
    quads (parity with the oracle only: the reference has no edge shape)."""
    s, m, st, cfg = b2.scenes.make_config(k, n, edges=edges)
    rng = np.random.default_rng(5)
    acts = [b2.scenes.actions(rng, n) for _ in range(steps)]
    ref = _run(m, st, s, cfg.dt, steps, oracle, acts)
    assert np.isfinite(np.asarray(ref.bodies.c)).all()


@pytest.mark.parametrize("oldest", [False, True])
@pytest.mark.parametrize("max_events", [1, None])
def test_toi_tie_parity(oracle, oldest, max_events):
    """scene_toi_tie over 64 worlds that keep its mirror symmetry (only the fall speed varies, 40 to 80 m/s), so
    every world's two TOIs tie to the bit and the device's pick must follow the tie rule as the oracle does
    (toi.py:552-556); max_events=1 leaves the rule's contact as the one with toi.count 1."""
    s = b2.Settings.stock(gravity=(0.0, 0.0), continuous_physics=True, toi_tie_oldest=oldest,
                          max_events=max_events)
    model, state = b2.scenes.scene_toi_tie(s).build(8)
    m = wd.compact_model(model, state)
    st = wd.batch(wd.compact_state(m, state), 64)
    st.bodies.v[:, 1, 1] = -np.random.default_rng(11).uniform(40.0, 80.0, 64).astype(np.float32)
    ref = _run(m, st, s, np.float32(1.0 / 60.0), 8, oracle)
    c = np.asarray(ref.bodies.c)[:, 1]
    assert (c[:, 1] > 0).all()  # every ball was stopped above the circles
    # the contact solved first pushes the ball away from its circle: fixture 1 (+x, newest) under the stock rule
    assert (np.sign(c[:, 0]) == (1 if oldest else -1)).all()


@pytest.mark.parametrize("xy_newer", [True, False])
def test_wake_cascade_parity(oracle, xy_newer):
    """scene_wake_cascade on the device and in the oracle in lockstep, bit for bit at every step, with the sleeping
    box moved by hand between steps as the oracle pin does (test_collide_wake_cascade_in_list_order): the device's
    Collide walk must wake Z in the step where X first touches Y only when the X-Y contact is the newer."""
    from test_oracle_pins import wake_cascade_run
    s = b2.Settings.stock(gravity=(0.0, 0.0))
    model, state = b2.scenes.scene_wake_cascade(s, xy_newer).build(8)
    m = wd.compact_model(model, state)
    dt = np.float32(1.0 / 60.0)

    def step(x):
        dev = b2.layout.to_device(x, "cuda")
        b2.step_(m, dev, s, dt)
        got = b2.layout.to_host(dev)
        ref = oracle.copy(x)
        oracle.step_(m, ref, s, dt)
        bad = leaf_mismatches(ref, got)
        assert bad == [], bad[:4]
        for dst, src in zip(wd.leaves(x), wd.leaves(got)):
            dst[...] = src

    got = wake_cascade_run(step, wd.batch(wd.compact_state(m, state), 1), xy_newer)
    assert got == ([(True, True), (True, True)] if xy_newer else [(False, False), (True, True)])


def test_model_without_body_types(oracle):
    """A compact Model as the reference's compact_model returns it (no body types: they stay in the State,
    world.py:437-472) steps the same; the body types come from the State."""
    s, m, st = b2.scenes.build_test_scene("pile", iterations=(8, 3))
    ref_style = m._replace(body_type=None, centroid=None, edge_flags=None)
    st = perturbed(st, 32, seed=4)
    dev = b2.layout.to_device(st, "cuda")
    ref = oracle.copy(st)
    for k in range(20):
        b2.step_(ref_style, dev, s, 1.0 / 60.0)
        oracle.step_(m, ref, s, 1.0 / 60.0)
    assert leaf_mismatches(ref, b2.layout.to_host(dev)) == []


def test_collide_config2(oracle):
    """Broadphase + narrowphase only over 4096 worlds (the collide-only workload, seed-1 terrain): candidate pairs, slots, keys, point
    counts and manifolds bit for bit."""
    s, m, st, cfg = b2.scenes.make_config(2)
    dev = b2.layout.to_device(st, "cuda")
    ref = oracle.copy(st)
    b2.collide_(m, dev, s)
    oracle.collide_(m, ref, s)
    got = b2.layout.to_host(dev)
    assert leaf_mismatches(ref, got) == []
    live = np.asarray(got.contacts.pair) >= 0
    assert live.sum() > 1000 and (np.asarray(got.contacts.count)[live] > 0).any()


def test_island_debug_outputs(oracle):
    """Island ids and solve order of the device Solve equal the oracle's."""
    s, m, st = b2.scenes.build_test_scene("pile", iterations=(8, 3))
    st = perturbed(st, 64, seed=9)
    dev = b2.layout.to_device(st, "cuda")
    ref = oracle.copy(st)
    B, R, J, C = wd.dims(st)
    for _ in range(40):
        dbg, t = b2.make_debug(64, (B, R, J, C))
        b2.step_(m, dev, s, 1.0 / 60.0, debug=dbg)
        d = {k: np.zeros(v.shape, np.int32) for k, v in t.items()}
        oracle.step_(m, ref, s, 1.0 / 60.0, debug=d)
        torch.cuda.synchronize()
        for k in d:
            assert np.array_equal(d[k], t[k].cpu().numpy()), k


def test_sincos_correctly_rounded(oracle):
    """The kernels' sin/cos equal (float)sin((double)x) on the reference's sample design (20k U[-8, 8], 5k
    U[-300, 300], +-0, pi; tests/box2d/test_box2d_parity.py:44-50) plus 4M uniform samples in [-100, 100]."""
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.uniform(-8, 8, 20000), rng.uniform(-300, 300, 5000), [0.0, -0.0, np.pi],
                        rng.uniform(-100, 100, 4_000_000)]).astype(np.float32)
    s, c = b2.sincos(torch.from_numpy(x).cuda())
    rs, rc = oracle.sincos(x)
    gs, gc = s.cpu().numpy(), c.cpu().numpy()
    assert np.signbit(gs[25001])  # sin(-0) = -0, as C
    assert np.array_equal(gs[:25003], rs[:25003]) and np.array_equal(gc[:25003], rc[:25003])
    bad = int((gs != rs).sum() + (gc != rc).sum())
    assert bad <= 4, f"{bad} of {2 * x.size} values differ from (float)sin((double)x)"


def test_full_size_config4_properties():
    """16384 worlds (the headline workload), 20 steps: finite state, contact-table overflow rare (the 32-slot table
    drops new contacts only in worlds whose fat AABBs sweep across many terrain pieces), TOI events happen, keys of
    live slots unique per world, no manifold points on free slots."""
    s, m, st, cfg = b2.scenes.make_config(4)
    dev = b2.layout.to_device(st, "cuda")
    rng = np.random.default_rng(11)
    events = 0
    for k in range(20):
        b2.scenes.apply_actions(dev.joints.motor_speed, dev.joints.max_motor,
                                torch.from_numpy(b2.scenes.actions(rng, st.bodies.type.shape[0])).cuda())
        b2.step_(m, dev, s, cfg.dt)
        events += int(dev.toi.events.sum())
    h = b2.layout.to_host(dev)
    assert np.isfinite(h.bodies.c).all() and np.isfinite(h.bodies.v).all()
    assert int((h.overflow > 0).sum()) < 0.01 * h.overflow.shape[0]
    assert events > 0
    live = h.contacts.pair >= 0
    keys = np.where(live, h.contacts.key, -1 - np.arange(live.shape[1])[None, :])
    assert all(len(set(r)) == len(r) for r in keys[:512])
    assert (h.contacts.count[~live] == 0).all()


def test_step_returns_new_state(oracle):
    """step() (the reference signature, step.py:28) leaves its input untouched and returns the stepped copy."""
    s, m, st, cfg = b2.scenes.make_config(4, 64)
    dev = b2.layout.to_device(st, "cuda")
    out = b2.step(m, dev, s, cfg.dt, axis_name="worlds")
    assert leaf_mismatches(st, b2.layout.to_host(dev)) == []
    assert leaf_mismatches(oracle.step(m, st, s, cfg.dt), b2.layout.to_host(out)) == []


def test_malformed_device_state_is_rejected():
    """A leaf with the wrong shape, dtype, layout or device never reaches the kernels."""
    s, m, st, cfg = b2.scenes.make_config(1, 8)
    dev = b2.layout.to_device(st, "cuda")
    bad = dev._replace(contacts=dev.contacts._replace(key=dev.contacts.key[:, :16]))
    with pytest.raises(ValueError):
        b2.step_(m, bad, s, cfg.dt)
    bad = dev._replace(bodies=dev.bodies._replace(v=dev.bodies.v.contiguous()))
    with pytest.raises(ValueError):
        b2.step_(m, bad, s, cfg.dt)
    bad = dev._replace(bodies=dev.bodies._replace(w=dev.bodies.w.double()))
    with pytest.raises(TypeError):
        b2.step_(m, bad, s, cfg.dt)
    bad = dev._replace(bodies=dev.bodies._replace(w=dev.bodies.w.cpu()))
    with pytest.raises(ValueError):
        b2.step_(m, bad, s, cfg.dt)


def test_new_fixture_forces_full_search(oracle):
    """A State edited outside step (here: live contacts removed from the table) gets a full FindNewContacts when
    new_fixture is set, as Box2D's e_newFixture asks: the device step then matches the oracle's full scan bit for
    bit, and the removed contacts come back."""
    s, m, st, cfg = b2.scenes.make_config(4, 256)
    ref = oracle.copy(st)
    for _ in range(5):
        oracle.step_(m, ref, s, cfg.dt)
    live = np.asarray(ref.contacts.pair) >= 0
    drop = live & (np.arange(live.shape[1])[None, :] % 2 == 0)
    assert drop.sum() > 100
    ref.contacts.pair[drop] = -1
    ref.contacts.touching[drop] = False
    ref.contacts.count[drop] = 0
    ref.new_fixture[...] = True
    dev = b2.layout.to_device(ref, "cuda")
    for k in range(3):
        b2.step_(m, dev, s, cfg.dt)
        oracle.step_(m, ref, s, cfg.dt)
        assert leaf_mismatches(ref, b2.layout.to_host(dev)) == [], k
    assert (np.asarray(ref.contacts.pair) >= 0).sum() > live.sum() - drop.sum()  # the search re-created contacts


@pytest.mark.parametrize("case,wpw,k", [("config4", None, 4), ("rig", "8", 3), ("pile", None, 5)])
def test_step_n_equals_repeated_steps(oracle, monkeypatch, case, wpw, k):
    """step_n_(k) (k steps in one launch, the workspaces kept in LDS between them) leaves the State k calls of
    step_ leave, and the oracle's after k steps, bit for bit; three launches in a row."""
    if wpw is not None:
        monkeypatch.setenv("GOI_WORLDS_PER_WAVE", wpw)
    if case == "pile":
        s, m, st = b2.scenes.build_test_scene("pile", iterations=(8, 3))
        st, dt = perturbed(st, 64, seed=7), 1.0 / 60.0
    else:
        s, m, st, cfg = b2.scenes.make_config(4, 512 if case == "config4" else 1024)
        dt = cfg.dt
    fused = b2.layout.to_device(st, "cuda")
    single = b2.layout.to_device(st, "cuda")
    ref = oracle.copy(st)
    for launch in range(3):
        b2.step_n_(m, fused, s, dt, k)
        for _ in range(k):
            b2.step_(m, single, s, dt)
            oracle.step_(m, ref, s, dt)
        got_f, got_s = b2.layout.to_host(fused), b2.layout.to_host(single)
        assert leaf_mismatches(got_s, got_f) == [], f"launch {launch}"
        assert leaf_mismatches(ref, got_f) == [], f"launch {launch}"


@pytest.mark.parametrize("edges", ["quad", "native"])
def test_rig_kernel_parity(oracle, monkeypatch, edges):
    """The step instance compiled for the rig's dimensions (5 bodies, 32 slots, 3 joints, 4 rows, 8 worlds per
    wavefront), which the launch picks for the benchmark workload: config 4, 1024 worlds, 40 steps with actions."""
    monkeypatch.setenv("GOI_WORLDS_PER_WAVE", "8")
    s, m, st, cfg = b2.scenes.make_config(4, 1024, edges=edges)
    assert wd.dims(st) == (5, 4, 3, 32)
    rng = np.random.default_rng(22)
    ref = _run(m, st, s, cfg.dt, 40, oracle, [b2.scenes.actions(rng, 1024) for _ in range(40)])
    assert int(np.asarray(ref.toi.events).sum()) > 0


@pytest.mark.parametrize("wpw", [1, 2, 4, 8, 32, 64])
def test_worlds_per_wave_variants(oracle, monkeypatch, wpw):
    """The block-cooperative passes (manifolds, TOIs) for other world counts per wavefront than the default (the
    library reads GOI_WORLDS_PER_WAVE at every call): config 4, 256 worlds, 10 steps with actions, bit for bit."""
    monkeypatch.setenv("GOI_WORLDS_PER_WAVE", str(wpw))
    s, m, st, cfg = b2.scenes.make_config(4, 256)
    rng = np.random.default_rng(21)
    _run(m, st, s, cfg.dt, 10, oracle, [b2.scenes.actions(rng, 256) for _ in range(10)])


@pytest.mark.parametrize("auto_clear", [True, False])
def test_applied_forces_parity(oracle, auto_clear):
    """Forces and torques written into the State between steps (every 5th step, random per world and body), with
    and without auto_clear_forces."""
    from dataclasses import replace
    s, m, st = b2.scenes.build_test_scene("pile", iterations=(8, 3))
    s = replace(s, auto_clear_forces=auto_clear)
    st = perturbed(st, 32, seed=9)
    dyn = np.asarray(st.bodies.type) == wd.DYNAMIC
    rng = np.random.default_rng(11)
    dev = b2.layout.to_device(st, "cuda")
    ref = oracle.copy(st)
    for k in range(40):
        if k % 5 == 0:
            f = np.where(dyn[..., None], rng.normal(0, 20, ref.bodies.force.shape), 0).astype(np.float32)
            t = np.where(dyn, rng.normal(0, 5, ref.bodies.torque.shape), 0).astype(np.float32)
            ref.bodies.force[...] = f
            ref.bodies.torque[...] = t
            dev.bodies.force.copy_(torch.from_numpy(f))
            dev.bodies.torque.copy_(torch.from_numpy(t))
        b2.step_(m, dev, s, 1.0 / 60.0)
        oracle.step_(m, ref, s, 1.0 / 60.0)
        bad = leaf_mismatches(ref, b2.layout.to_host(dev))
        assert bad == [], f"step {k + 1}: {bad[:4]}"
    assert np.abs(np.asarray(ref.bodies.force)).sum() == 0 if auto_clear else np.abs(ref.bodies.force).sum() > 0
