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
import scene_defs

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _run(model, state, settings, dt, steps, oracle, actions=None, every=1, on_step=None, nan_equal=False, pitch=None):
    """Steps the device and the oracle side by side from the same State (and actions), comparing every leaf bit for
    bit after every `every`-th step and after the last (nan_equal: any two NaNs equal). on_step(k, ref, dev) runs
    after each step; pitch: the device State's pitch (the world count by default)."""
    dev = b2.layout.to_device(state, "cuda", pitch)
    ref = oracle.copy(state)
    for k in range(steps):
        if actions is not None:
            a = actions[k]
            b2.scenes.apply_actions(ref.joints.motor_speed, ref.joints.max_motor, a)
            b2.scenes.apply_actions(dev.joints.motor_speed, dev.joints.max_motor, torch.from_numpy(a).cuda())
        b2.step_(model, dev, settings, dt)
        oracle.step_(model, ref, settings, dt)
        if on_step is not None:
            on_step(k, ref, dev)
        if (k + 1) % every == 0 or k + 1 == steps:
            got = b2.layout.to_host(dev)
            bad = leaf_mismatches(ref, got, nan_equal)
            assert bad == [], f"step {k + 1}: {bad[:4]}"
    return ref


@pytest.mark.parametrize("name", list(scene_defs.TEST_SCENES))
def test_scene_parity(name, oracle):
    """Every test scene, 64 perturbed copies, 90 steps, stock iteration counts."""
    s, m, st = scene_defs.build_test_scene(name, iterations=(8, 3))
    _run(m, perturbed(st, 64), s, 1.0 / 60.0, 90, oracle)


@pytest.mark.parametrize("name,wpw", [("pile", 2), ("pile", 8), ("joints", 16), ("polygons", 16), ("misc", 8)])
def test_islands_side_by_side_parity(name, wpw, oracle, monkeypatch):
    """Scenes of several islands (pile up to 12, polygons 9, joints 8 with every joint type, misc 6) at wave shapes
    whose lane groups hold fewer lanes than the world has islands (2 to 32 lanes), so lanes take several islands
    each: 64 perturbed copies, 60 steps."""
    monkeypatch.setenv("GOI_WORLDS_PER_WAVE", str(wpw))
    s, m, st = scene_defs.build_test_scene(name, iterations=(8, 3))

    def used(k, ref, dev):
        assert b2.last_launch()["worlds_per_wave"] == wpw
    _run(m, perturbed(st, 64), s, 1.0 / 60.0, 60, oracle, on_step=used)


@pytest.mark.parametrize("name", ["pile", "hammer_chain", "island_walk", "joints"])
def test_scene_parity_game_iterations(name, oracle):
    """The game's 300 / 30 iterations on the heavier scenes."""
    s, m, st = scene_defs.build_test_scene(name)
    _run(m, perturbed(st, 16, seed=3), s, b2.GAME_DT, 60, oracle)


@pytest.mark.parametrize("k,n,steps,edges,every", [(1, 1, 500, "quad", 1), (3, 4096, 200, "quad", 5),
                                                    (4, 16384, 100, "quad", 10), (4, 512, 30, "native", 1),
                                                    (5, 128, 60, "native", 1)])
def test_config_parity(k, n, steps, edges, every, oracle):
    """The benchmark configurations, configs 1, 3 and 4 at their full world and step counts; "native" builds the
    terrain chain from b2EdgeShape children instead of thin quads (parity with the oracle only: the reference has no
    edge shape). The contact tables (40 slots for the rig, 128 with the boxes) never overflow."""
    s, m, st, cfg = b2.scenes.make_config(k, n, edges=edges)
    rng = np.random.default_rng(5)
    acts = [b2.scenes.actions(rng, n) for _ in range(steps)]
    ref = _run(m, st, s, cfg.dt, steps, oracle, acts, every=every)
    assert np.isfinite(np.asarray(ref.bodies.c)).all()
    assert int(np.asarray(ref.overflow).sum()) == 0


def _islands(dbg, n):
    """(bodies, touching contacts) per (world, island) from GoiDebug-style arrays body_island [B, n] and
    contact_island [C, n]."""
    bi, ci = np.asarray(dbg["body_island"]), np.asarray(dbg["contact_island"])
    nb = np.zeros((n, bi.shape[0] + 1), int)
    nc = np.zeros((n, bi.shape[0] + 1), int)
    wb, wc = np.broadcast_to(np.arange(n), bi.shape), np.broadcast_to(np.arange(n), ci.shape)
    np.add.at(nb, (wb[bi >= 0], bi[bi >= 0]), 1)
    np.add.at(nc, (wc[ci >= 0], ci[ci >= 0]), 1)
    return nb, nc


def test_config5_large_islands(oracle):
    """The large-island configuration over its 300 steps (1,024 worlds): first the regime it is defined by (an
    island of all 16 dynamic bodies, more than 40 live contacts in a world, and more than 64, so the contact list is
    walked in more than one 64-position chunk; overflow 0 with 128 slots), then the device against the oracle bit
    for bit, island ids and solve order included, every 10 steps."""
    n, steps = 1024, 300
    s, m, st, cfg = b2.scenes.make_config(5, n)
    B, R, J, C = wd.dims(st)
    rng = np.random.default_rng(5)
    acts = [b2.scenes.actions(rng, n) for _ in range(steps)]
    seen = {"island16": 0, "live": 0}
    # the regime, on the oracle alone (with island outputs every step)
    x = oracle.copy(st)
    for k in range(steps):
        b2.scenes.apply_actions(x.joints.motor_speed, x.joints.max_motor, acts[k])
        d = dict(body_island=np.full((B, n), -1, np.int32), contact_island=np.full((C, n), -1, np.int32),
                 contact_order=np.full((C, n), -1, np.int32), n_islands=np.zeros(n, np.int32))
        oracle.step_(m, x, s, cfg.dt, debug=d)
        nb, _ = _islands(d, n)
        seen["island16"] += int((nb >= 16).any(1).sum())
        seen["live"] = max(seen["live"], int((np.asarray(x.contacts.pair) >= 0).sum(1).max()))
    assert seen["island16"] > 0, "no island of 16 bodies formed"
    assert seen["live"] > 64, f"at most {seen['live']} live contacts in a world"
    assert int(np.asarray(x.overflow).sum()) == 0
    # the device against the oracle, with the island outputs compared every 10 steps
    dev = b2.layout.to_device(st, "cuda")
    ref = oracle.copy(st)
    for k in range(steps):
        b2.scenes.apply_actions(ref.joints.motor_speed, ref.joints.max_motor, acts[k])
        b2.scenes.apply_actions(dev.joints.motor_speed, dev.joints.max_motor, torch.from_numpy(acts[k]).cuda())
        if k % 10 == 9:
            dbg, t = b2.make_debug(n, (B, R, J, C), pitch=b2.layout.pitch_of(dev))
            b2.step_(m, dev, s, cfg.dt, debug=dbg)
            d = {key: np.zeros(v.shape[:-1] + (n,), np.int32) for key, v in t.items()}
            oracle.step_(m, ref, s, cfg.dt, debug=d)
            torch.cuda.synchronize()
            for key in d:
                assert np.array_equal(d[key], t[key][..., :n].cpu().numpy()), (k + 1, key)
            bad = leaf_mismatches(ref, b2.layout.to_host(dev))
            assert bad == [], f"step {k + 1}: {bad[:4]}"
        else:
            b2.step_(m, dev, s, cfg.dt)
            oracle.step_(m, ref, s, cfg.dt)
    assert leaf_mismatches(ref, x) == []  # the same run as the regime pass


@pytest.mark.parametrize("oldest", [False, True])
@pytest.mark.parametrize("max_events", [1, None])
def test_toi_tie_parity(oracle, oldest, max_events):
    """scene_toi_tie over 64 worlds that keep its mirror symmetry (only the fall speed varies, 40 to 80 m/s), so
    every world's two TOIs tie to the bit and the device's pick must follow the tie rule as the oracle does
    (toi.py:552-556); max_events=1 leaves the rule's contact as the one with toi.count 1."""
    s = b2.Settings.stock(gravity=(0.0, 0.0), continuous_physics=True, toi_tie_oldest=oldest,
                          max_events=max_events)
    model, state = scene_defs.scene_toi_tie(s).build(8)
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
    model, state = scene_defs.scene_wake_cascade(s, xy_newer).build(8)
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
    s, m, st = scene_defs.build_test_scene("pile", iterations=(8, 3))
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
    s, m, st = scene_defs.build_test_scene("pile", iterations=(8, 3))
    st = perturbed(st, 64, seed=9)
    dev = b2.layout.to_device(st, "cuda")
    ref = oracle.copy(st)
    B, R, J, C = wd.dims(st)
    for _ in range(40):
        dbg, t = b2.make_debug(64, (B, R, J, C), pitch=b2.layout.pitch_of(dev))
        b2.step_(m, dev, s, 1.0 / 60.0, debug=dbg)
        d = {k: np.zeros(v.shape[:-1] + (64,), np.int32) for k, v in t.items()}
        oracle.step_(m, ref, s, 1.0 / 60.0, debug=d)
        torch.cuda.synchronize()
        for k in d:
            assert np.array_equal(d[k], t[k][..., :64].cpu().numpy()), k


def _debug_parity(m, st, s, dt, steps, oracle, actions=None):
    """Steps device and oracle side by side with GoiDebug outputs, comparing every debug array and every leaf after
    each step; returns the number of TOI events traced."""
    n = st.bodies.type.shape[0]
    dims = wd.dims(st)
    dev = b2.layout.to_device(st, "cuda")
    ref = oracle.copy(st)
    traced = 0
    for k in range(steps):
        if actions is not None:
            b2.scenes.apply_actions(ref.joints.motor_speed, ref.joints.max_motor, actions[k])
            b2.scenes.apply_actions(dev.joints.motor_speed, dev.joints.max_motor, torch.from_numpy(actions[k]).cuda())
        dbg, t = b2.make_debug(n, dims, pitch=b2.layout.pitch_of(dev))
        b2.step_(m, dev, s, dt, debug=dbg)
        d = {key: np.full(v.shape[:-1] + (n,), -9, np.int32) for key, v in t.items()}
        oracle.step_(m, ref, s, dt, debug=d)
        torch.cuda.synchronize()
        for key in d:
            assert np.array_equal(d[key], t[key][..., :n].cpu().numpy()), (k + 1, key)
        assert leaf_mismatches(ref, b2.layout.to_host(dev)) == [], k + 1
        traced += int((d["toi_event_slot"] >= 0).sum())
    return traced


def test_toi_event_traces(oracle):
    """The TOI events of each step, traced through GoiDebug (the event's slot and alpha, its island's size and its
    rows in walk order) on the device and in the oracle: config 4 (256 worlds, 15 steps with actions, thousands of
    events) and the plank falling onto 40 bumps, whose event walk stops at the 32-contact cap."""
    s, m, st, cfg = b2.scenes.make_config(4, 256)
    rng = np.random.default_rng(8)
    acts = [b2.scenes.actions(rng, 256) for _ in range(15)]
    assert _debug_parity(m, st, s, cfg.dt, 15, oracle, acts) > 500
    from test_oracle_pins import plank_over_bumps
    s, m, st = plank_over_bumps()
    st = wd.batch(wd.from_leaves([np.asarray(x)[0] for x in wd.leaves(st)]), 8)
    assert _debug_parity(m, st, s, np.float32(1 / 60), 3, oracle) >= 8


@pytest.mark.parametrize("n_steps", [1, 4])
def test_packed_and_unpacked_states_agree(n_steps, monkeypatch):
    """The 4-body rig on a packed State (one buffer, every leaf at its packed offset: the fixed-dimension kernel of
    goi_b2_rig.hip) and on the same State with one buffer per leaf (the general kernel) step to identical States, for
    single steps and for goi_step_n."""
    monkeypatch.setenv("GOI_WORLDS_PER_WAVE", "8")  # the rig kernel's 8 worlds per wave at this batch size
    s, m, st, cfg = b2.scenes.make_config(4, 512)
    rng = np.random.default_rng(3)
    acts = np.stack([b2.scenes.actions(rng, 512) for _ in range(24)])
    devs = [b2.layout.to_device(st, "cuda", packed=p) for p in (True, False)]
    for k in range(0, 24, n_steps):
        for d in devs:
            b2.scenes.apply_actions(d.joints.motor_speed, d.joints.max_motor, torch.from_numpy(acts[k]).cuda())
            if n_steps == 1:
                b2.step_(m, d, s, cfg.dt)
            else:
                b2.step_n_(m, d, s, cfg.dt, n_steps)
    torch.cuda.synchronize()
    a, b = (b2.layout.to_host(d) for d in devs)
    assert leaf_mismatches(a, b) == []
    assert int(np.asarray(a.toi.events).sum()) > 0  # the steps ran TOI events


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
    bad = np.nonzero((gs != rs) | (gc != rc))[0]
    assert bad.size == 0, f"{bad.size} inputs differ from (float)sin((double)x), e.g. {x[bad[:8]].tolist()}"


def _first(state, n):
    return wd.from_leaves([np.ascontiguousarray(np.asarray(x)[:n]) for x in wd.leaves(state)])


@pytest.mark.parametrize("k", [4, 5])
def test_full_size_properties(oracle, k):
    """The full-size run (16,384 worlds x 100 steps for config 4, 65,536 x 300 for config 5), checked through
    properties that do not need an oracle run of every world: finite state, no contact-table overflow, TOI events,
    keys of live slots unique per world, no manifold points on free slots; and, since worlds are independent, its
    first 256 worlds equal an oracle run of those 256 worlds alone, bit for bit."""
    s, m, st, cfg = b2.scenes.make_config(k)
    n = st.bodies.type.shape[0]
    dev = b2.layout.to_device(st, "cuda")
    rng = np.random.default_rng(11)
    acts = [b2.scenes.actions(rng, n) for _ in range(cfg.steps)]
    events = 0
    for a in acts:
        b2.scenes.apply_actions(dev.joints.motor_speed, dev.joints.max_motor, torch.from_numpy(a).cuda())
        b2.step_(m, dev, s, cfg.dt)
        events += int(dev.toi.events.sum())
    h = b2.layout.to_host(dev)
    assert np.isfinite(h.bodies.c).all() and np.isfinite(h.bodies.v).all()
    assert int(h.overflow.sum()) == 0
    assert events > 0
    live = h.contacts.pair >= 0
    keys = np.where(live, h.contacts.key, -1 - np.arange(live.shape[1])[None, :])
    assert all(len(set(r)) == len(r) for r in keys[:2048])
    assert (h.contacts.count[~live] == 0).all()
    sub = oracle.copy(_first(st, 256))
    for a in acts:
        b2.scenes.apply_actions(sub.joints.motor_speed, sub.joints.max_motor, a[:256])
        oracle.step_(m, sub, s, cfg.dt)
    assert leaf_mismatches(sub, _first(h, 256)) == []


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


@pytest.mark.parametrize("case,wpw,k", [("config4", None, 4), ("rig", "8", 3), ("pile", None, 5), ("island", "4", 3)])
def test_step_n_equals_repeated_steps(oracle, monkeypatch, case, wpw, k):
    """step_n_(k) (k steps in one launch, the workspaces kept in LDS between them) leaves the State k calls of
    step_ leave, and the oracle's after k steps, bit for bit; three launches in a row. "rig" and "island" run the
    multi-step instances for the rig's and the island workload's dimensions."""
    if wpw is not None:
        monkeypatch.setenv("GOI_WORLDS_PER_WAVE", wpw)
    if case == "pile":
        s, m, st = scene_defs.build_test_scene("pile", iterations=(8, 3))
        st, dt = perturbed(st, 64, seed=7), 1.0 / 60.0
    elif case == "island":
        s, m, st, cfg = b2.scenes.make_config(5, 256, edges="quad")
        assert wd.dims(st) == (17, 16, 3, 128)
        dt = cfg.dt
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


@pytest.mark.parametrize("case", ["island", "rig4"])
def test_multi_round_launches(oracle, monkeypatch, case):
    """Launches with more blocks than the GPU holds at once run their blocks in the order k_group_order gives (the
    world groups with the most TOI events of the previous step first): config 5 at 8,192 worlds (2,048 blocks of the
    island instance, 5 a CU) and config 4 at 16,384 worlds with 4 worlds a wave (4,096 blocks of the generic kernel,
    8 a CU). 6 steps with actions, bit for bit."""
    if case == "island":
        monkeypatch.setenv("GOI_WORLDS_PER_WAVE", "4")
        s, m, st, cfg = b2.scenes.make_config(5, 8192, edges="quad")
        n, kernel = 8192, "island"
    else:
        monkeypatch.setenv("GOI_WORLDS_PER_WAVE", "4")
        s, m, st, cfg = b2.scenes.make_config(4, 16384)
        n, kernel = 16384, "generic"
    rng = np.random.default_rng(37)

    def used(k, ref, dev):
        info = b2.last_launch()
        assert info["worlds_per_wave"] == 4 and info["blocks"] == n // 4 and info["kernel"] == kernel, info
    ref = _run(m, st, s, cfg.dt, 6, oracle, [b2.scenes.actions(rng, n) for _ in range(6)], on_step=used, every=3)
    assert int(np.asarray(ref.toi.events).sum()) > 0


@pytest.mark.parametrize("case", ["island", "native_edges"])
def test_other_kernels_with_lanes_without_a_world(oracle, monkeypatch, case):
    """A partly filled last block on the island instance (config 5, 250 worlds at 4 a wave on a packed State of pitch
    256: its SolveTOI re-derives its views in each event iteration) and on the generic kernel with native edge shapes
    (config 4 with a b2ChainShape terrain, 250 worlds at 8 a wave). 8 steps with actions, bit for bit."""
    if case == "island":
        monkeypatch.setenv("GOI_WORLDS_PER_WAVE", "4")
        s, m, st, cfg = b2.scenes.make_config(5, 250, edges="quad")
        pitch, wpw, kernel = 256, 4, "island"
    else:
        monkeypatch.setenv("GOI_WORLDS_PER_WAVE", "8")
        s, m, st, cfg = b2.scenes.make_config(4, 250, edges="native")
        pitch, wpw, kernel = None, 8, "generic"
    rng = np.random.default_rng(31)

    def used(k, ref, dev):
        info = b2.last_launch()
        assert info["worlds_per_wave"] == wpw and info["blocks"] == -(-250 // wpw), info
        assert info["kernel"] == kernel, info
    _run(m, st, s, cfg.dt, 8, oracle, [b2.scenes.actions(rng, 250) for _ in range(8)], on_step=used, pitch=pitch)


@pytest.mark.parametrize("wpw,n,pitch", [(8, 250, 256), (20, 256, None), (13, 250, None)])
def test_step_n_lanes_without_a_world(oracle, monkeypatch, wpw, n, pitch):
    """step_n_ (3 steps a launch, two launches) on blocks with lanes that run no world: the multi-step path sets up
    each step's cooperative views afresh as the single step does. The rig's multi-step instance on a packed State of
    pitch 256 with 250 worlds, the generic kernel at 20 and 13 worlds per wave. Config 4 with actions, bit for bit."""
    monkeypatch.setenv("GOI_WORLDS_PER_WAVE", str(wpw))
    s, m, st, cfg = b2.scenes.make_config(4, n, capacity=40)
    rng = np.random.default_rng(29)
    dev = b2.layout.to_device(st, "cuda", pitch)
    ref = oracle.copy(st)
    for launch in range(2):
        a = b2.scenes.actions(rng, n)
        b2.scenes.apply_actions(ref.joints.motor_speed, ref.joints.max_motor, a)
        b2.scenes.apply_actions(dev.joints.motor_speed, dev.joints.max_motor, torch.from_numpy(a).cuda())
        b2.step_n_(m, dev, s, cfg.dt, 3)
        info = b2.last_launch()
        assert info["worlds_per_wave"] == wpw and info["blocks"] == -(-n // wpw), info
        assert info["kernel"] == ("rig" if pitch == 256 else "generic"), info
        for _ in range(3):
            oracle.step_(m, ref, s, cfg.dt)
        assert leaf_mismatches(ref, b2.layout.to_host(dev)) == [], f"launch {launch}"


@pytest.mark.parametrize("edges", ["quad", "native"])
def test_rig_kernel_parity(oracle, monkeypatch, edges):
    """The step instance compiled for the rig's dimensions (5 bodies, 40 slots, 3 joints, 4 rows, 8 worlds per
    wavefront), which the launch picks for the benchmark workload: config 4, 1024 worlds, 40 steps with actions."""
    monkeypatch.setenv("GOI_WORLDS_PER_WAVE", "8")
    s, m, st, cfg = b2.scenes.make_config(4, 1024, edges=edges)
    assert wd.dims(st) == (5, 4, 3, 40)
    rng = np.random.default_rng(22)
    ref = _run(m, st, s, cfg.dt, 40, oracle, [b2.scenes.actions(rng, 1024) for _ in range(40)])
    assert int(np.asarray(ref.toi.events).sum()) > 0


def test_island_kernel_parity(oracle, monkeypatch):
    """The step instance compiled for config 5's dimensions (17 bodies, 128 slots, 3 joints, 16 rows, 4 worlds per
    wavefront, plain Model), which the launch picks for the island workload at full size: 512 worlds, 30 steps with
    actions, on the thin-quad terrain."""
    monkeypatch.setenv("GOI_WORLDS_PER_WAVE", "4")
    s, m, st, cfg = b2.scenes.make_config(5, 512, edges="quad")
    assert wd.dims(st) == (17, 16, 3, 128)
    rng = np.random.default_rng(23)
    ref = _run(m, st, s, cfg.dt, 30, oracle, [b2.scenes.actions(rng, 512) for _ in range(30)], every=5)
    assert int(np.asarray(ref.overflow).sum()) == 0


@pytest.mark.parametrize("wpw", ["4", "8"])
def test_nonfinite_islands_parity(oracle, monkeypatch, wpw):
    """Worlds of several islands, whose lanes solve the islands side by side, with a NaN or infinite value in one
    island (test_host_sanitized.nonfinite_islands_case, 64 worlds): Box2D's order carries it through the terrain into
    the other islands, which the device must follow by solving those worlds' islands one after another. 20 steps,
    NaN for NaN, on the island instance (4 worlds per wave) and the general kernel (8)."""
    from test_host_sanitized import nonfinite_islands_case
    monkeypatch.setenv("GOI_WORLDS_PER_WAVE", wpw)
    m, st, s, dt = nonfinite_islands_case(oracle, n=64)

    def used(k, ref, dev):
        assert b2.last_launch()["kernel"] == ("island" if wpw == "4" else "generic")
    ref = _run(m, st, s, dt, 20, oracle, on_step=used, nan_equal=True)
    assert np.isnan(ref.bodies.v[1]).any() and not np.isnan(ref.bodies.v[0]).any()


@pytest.mark.parametrize("wpw,capacity", [(1, 40), (2, 40), (4, 40), (8, 40), (16, 40), (27, 40), (32, 6), (64, 6)])
def test_worlds_per_wave_variants(oracle, monkeypatch, wpw, capacity):
    """The block-cooperative passes (manifolds, TOIs) for other world counts per wavefront than the default (the
    library reads GOI_WORLDS_PER_WAVE at every call): config 4, 256 worlds, 10 steps with actions, bit for bit. Each
    launch must have run the requested count (goi_last_launch): 27 is the most the rig's 40-slot workspace fits in a
    block's LDS (27 worlds on 2 lanes each, 10 lanes idle); 32 and 64 run the rig with 6 slots, whose workspaces fit
    64 to a block. At 8 worlds per wave the rig's packed State runs the instance compiled for it."""
    monkeypatch.setenv("GOI_WORLDS_PER_WAVE", str(wpw))
    s, m, st, cfg = b2.scenes.make_config(4, 256, capacity=capacity)
    rng = np.random.default_rng(21)

    def used(k, ref, dev):
        info = b2.last_launch()
        assert info["worlds_per_wave"] == wpw and info["blocks"] == -(-256 // wpw), info
        assert info["kernel"] == ("rig" if (wpw, capacity) == (8, 40) else "generic"), info
    _run(m, st, s, cfg.dt, 10, oracle, [b2.scenes.actions(rng, 256) for _ in range(10)], on_step=used)


@pytest.mark.parametrize("wpw,n,pitch,max_events", [(8, 250, 256, -1), (8, 250, 256, 0), (8, 250, None, -1),
                                                    (4, 250, None, -1), (16, 250, None, 0), (20, 256, None, -1),
                                                    (20, 256, None, 0), (13, 256, None, 0)])
def test_lanes_without_a_world(oracle, monkeypatch, wpw, n, pitch, max_events):
    """Blocks with lanes that run no world take part in every cooperative phase (manifolds, TOI searches, the block
    copies) after phases that only the lanes with a world run: a world count that leaves the last block partly filled
    (250 worlds at 8, 4 or 16 a block; the rig instance at 8 on a packed State of pitch 256, the generic kernel on one
    of pitch 250), or one that leaves lanes idle in every block (20 and 13 worlds per wave). max_events 0 stops every
    world's TOI walk before its first event, so the block's searches follow the solver directly. Config 4, 4 steps
    with actions, bit for bit."""
    from dataclasses import replace
    monkeypatch.setenv("GOI_WORLDS_PER_WAVE", str(wpw))
    s, m, st, cfg = b2.scenes.make_config(4, n, capacity=40)
    s = replace(s, max_events=max_events)
    rng = np.random.default_rng(21)

    def used(k, ref, dev):
        info = b2.last_launch()
        assert info["worlds_per_wave"] == wpw and info["blocks"] == -(-n // wpw), info
        assert info["kernel"] == ("rig" if pitch == 256 else "generic"), info
    _run(m, st, s, cfg.dt, 4, oracle, [b2.scenes.actions(rng, n) for _ in range(4)], on_step=used, pitch=pitch)


@pytest.mark.parametrize("auto_clear", [True, False])
def test_applied_forces_parity(oracle, auto_clear):
    """Forces and torques written into the State between steps (every 5th step, random per world and body), with
    and without auto_clear_forces."""
    from dataclasses import replace
    s, m, st = scene_defs.build_test_scene("pile", iterations=(8, 3))
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


@pytest.mark.parametrize("wpw", [None, "8"])
@pytest.mark.parametrize("capacity", [6, 10])
def test_contact_table_overflow_parity(oracle, monkeypatch, capacity, wpw):
    """Config 4 with too few contact slots (6 or 10 per world): FindNewContacts drops the pairs that find no free
    slot and counts them in `overflow` (world.py:173, pairs.py:176-178), and a world that ever dropped one keeps
    searching every candidate after Solve and after each TOI event (a dropped pair may find a slot later). 256
    worlds, 40 steps with actions, the default wave size and 8 worlds per wave; first the regime (the oracle drops
    contacts in many worlds), then the device bit for bit."""
    if wpw is not None:
        monkeypatch.setenv("GOI_WORLDS_PER_WAVE", wpw)
    n, steps = 256, 40
    s, m, st, cfg = b2.scenes.make_config(4, n, capacity=capacity)
    assert wd.dims(st) == (5, 4, 3, capacity)
    rng = np.random.default_rng(31)
    acts = [b2.scenes.actions(rng, n) for _ in range(steps)]
    ref = _run(m, st, s, cfg.dt, steps, oracle, acts)
    ovf = np.asarray(ref.overflow)
    assert int((ovf > 0).sum()) > 50 and int(ovf.sum()) > 5000
    assert int(np.asarray(ref.toi.events).sum()) > 0


def _full_layout_case(case, n):
    """(settings, full-layout Model, batched full-layout State, dt) as WorldDef.build returns them."""
    from dataclasses import replace
    if case == "config4":
        cfg = b2.scenes.CONFIGS[4]
        s = b2.scenes.settings_for(cfg)
        model, state, pts = b2.scenes.build_world(cfg, s)
        return s, model, b2.scenes.place_worlds(cfg, model, state, pts, n), np.float32(cfg.dt)
    fn, sfn, cap = scene_defs.TEST_SCENES[case]
    s = replace(sfn(), velocity_iterations=8, position_iterations=3)
    model, state = fn(s).build(contact_capacity=cap)
    return s, model, perturbed(state, n, seed=13), np.float32(1.0 / 60.0)


@pytest.mark.parametrize("case", ["config4", "joints", "circles"])
def test_full_layout_parity(oracle, case):
    """step_ on WorldDef.build's own Model and State, the full fixture layout (a row per fixture), as the reference's
    step takes them (world.py:400-434, pairs.py:184-188): the Model is compacted from the State's static rows once,
    the State stays in the full layout and its static rows are never written. Compared with the oracle stepping the
    same full-layout State, every leaf bit for bit; config 4 with actions (its non-static fixtures are the last
    rows), "joints" and "circles" with static fixtures between the non-static ones. step() with a compact Model and a
    full State gives the same."""
    n = 256 if case == "config4" else 64
    s, model, st, dt = _full_layout_case(case, n)
    assert model.fixture_slot is None and wd.dims(st)[1] == model.fixture_body.shape[0]
    rng = np.random.default_rng(17)
    acts = [b2.scenes.actions(rng, n) for _ in range(30)] if case == "config4" else None
    ref = _run(model, st, s, dt, 30, oracle, acts, every=5)
    assert int(np.asarray(ref.toi.events).sum()) > 0 or case != "config4"
    cm = wd.compact_model(model, st)
    out = b2.step(cm, b2.layout.to_device(st, "cuda"), s, dt)
    assert leaf_mismatches(oracle.step(model, st, s, dt), b2.layout.to_host(out)) == []


@pytest.mark.parametrize("wpw", [None, "8"])
def test_nonfinite_worlds_parity(oracle, monkeypatch, wpw):
    """NaN and infinite values written into a few worlds of config 4 (a NaN velocity, an infinite spin, a NaN
    position, 1e30 m/s, a NaN force; the failure inputs of the reference's bench, bench_gpu.py:135-136): the other
    worlds stay bit-exact and the poisoned ones follow the oracle, NaN for NaN (a box with a NaN coordinate overlaps
    every box under b2TestOverlap, so their tables fill and overflow). 64 worlds, 30 steps, the general kernel and the
    rig instance (8 worlds per wave). The same scenario runs first under the sanitizers on the CPU
    (test_host_sanitized.py::test_nonfinite_worlds_sanitized)."""
    from test_host_sanitized import nonfinite_case
    if wpw is not None:
        monkeypatch.setenv("GOI_WORLDS_PER_WAVE", wpw)
    m, st, s, dt, acts = nonfinite_case()
    bad = [3, 5, 7, 11]  # world 9's 1e30 m/s is scaled to rest by the max-translation clamp (h v squared is inf)
    ref = _run(m, st, s, dt, 30, oracle, list(acts), nan_equal=True)
    c = np.asarray(ref.bodies.c)
    finite = np.isfinite(c).reshape(c.shape[0], -1).all(1)
    assert not finite[bad].any() and finite[np.setdiff1d(np.arange(64), bad)].all()
    assert (np.asarray(ref.overflow)[bad] > 0).any()


@pytest.mark.parametrize("dt", [0.0, -0.02])
def test_non_positive_dt_parity(oracle, dt):
    """dt <= 0 (step.py:35-40, toi.py:841): Solve runs, SolveTOI is skipped, inv_dt0 is left as it was."""
    s, m, st, cfg = b2.scenes.make_config(4, 256)
    rng = np.random.default_rng(41)
    ref = _run(m, st, s, np.float32(dt), 6, oracle, [b2.scenes.actions(rng, 256) for _ in range(6)])
    assert int(np.asarray(ref.toi.events).sum()) == 0


@pytest.mark.parametrize("max_events", [1, 2, 3])
def test_max_events_parity(oracle, monkeypatch, max_events):
    """SolveTOI stops after max_events events a step (toi.py:838-842): config 4, 1,024 worlds, 20 steps, on the rig
    instance; some worlds reach the cap."""
    from dataclasses import replace
    monkeypatch.setenv("GOI_WORLDS_PER_WAVE", "8")
    s, m, st, cfg = b2.scenes.make_config(4, 1024)
    s = replace(s, max_events=max_events)
    rng = np.random.default_rng(43)
    capped = []
    ref = _run(m, st, s, cfg.dt, 20, oracle, [b2.scenes.actions(rng, 1024) for _ in range(20)],
               on_step=lambda k, r, d: capped.append(int((np.asarray(r.toi.events) == max_events).sum())))
    assert sum(capped) > 0 and int(np.asarray(ref.toi.events).max()) <= max_events


def test_status_word_parity(oracle):
    """GoiDebug.status (the step's failure counters as one word per world) on the device equals the oracle's at every
    step, with every bit raised somewhere: non-finite worlds (which also overflow their tables), max_events 2
    (SolveTOI capped) and one step of dt 0 (SolveTOI skipped). Config 4, 64 worlds, 12 steps, the general kernel (a
    launch with debug arrays takes it); the other debug arrays and every leaf are compared too, NaN for NaN."""
    from dataclasses import replace
    from test_host_sanitized import nonfinite_case
    A = b2._abi
    m, st, s, dt, acts = nonfinite_case(steps=12)
    s = replace(s, max_events=2)
    n, dims = 64, wd.dims(st)
    dev = b2.layout.to_device(st, "cuda")
    ref = oracle.copy(st)
    seen = 0
    for k in range(12):
        b2.scenes.apply_actions(ref.joints.motor_speed, ref.joints.max_motor, acts[k])
        b2.scenes.apply_actions(dev.joints.motor_speed, dev.joints.max_motor, torch.from_numpy(acts[k]).cuda())
        dtk = np.float32(0.0) if k == 5 else dt
        dbg, t = b2.make_debug(n, dims, pitch=b2.layout.pitch_of(dev))
        b2.step_(m, dev, s, dtk, debug=dbg)
        d = {key: np.full(v.shape[:-1] + (n,), -9, np.int32) for key, v in t.items()}
        oracle.step_(m, ref, s, dtk, debug=d)
        torch.cuda.synchronize()
        for key in d:
            assert np.array_equal(d[key], t[key][..., :n].cpu().numpy()), (k + 1, key)
        assert leaf_mismatches(ref, b2.layout.to_host(dev), nan_equal=True) == [], k + 1
        seen |= int(np.bitwise_or.reduce(d["status"]))
    assert seen == A.STATUS_OVERFLOW | A.STATUS_NONFINITE | A.STATUS_TOI_CAPPED | A.STATUS_TOI_SKIPPED


@pytest.mark.parametrize("variant", ["no_warm_start", "clamps_per_second", "no_position_iterations", "damping",
                                     "tangent_speed"])
def test_settings_variants_parity(oracle, variant):
    """The Settings switches and State inputs the benchmark configurations leave at their defaults: warm starting
    off, per-second clamps, no position iteration (islands never position-solved, so never asleep), angular and
    linear damping with a gravity scale, and a conveyor tangent speed on every live contact. Config 4, 256 worlds, 25
    steps with actions (the tangent speed on the pile scene, 32 worlds), bit for bit."""
    from dataclasses import replace
    s, m, st, cfg = b2.scenes.make_config(4, 256)
    dt, n, steps = cfg.dt, 256, 25
    if variant == "no_warm_start":
        s = replace(s, warm_starting=False)
    elif variant == "clamps_per_second":
        s = replace(s, clamps_per_second=True, max_translation=np.float32(60.0), max_rotation=np.float32(40.0))
    elif variant == "no_position_iterations":
        s = replace(s, position_iterations=0)
    elif variant == "damping":
        st.bodies.linear_damping[...] = np.float32(0.3)
        st.bodies.angular_damping[...] = np.float32(0.7)
        st.bodies.gravity_scale[:, 2] = np.float32(0.5)
    else:
        s, m, st = scene_defs.build_test_scene("pile", iterations=(8, 3))
        st, dt, n, steps = perturbed(st, 32, seed=5), np.float32(1 / 60), 32, 40
        ref = oracle.copy(st)
        for _ in range(10):
            oracle.step_(m, ref, s, dt)
        live = np.asarray(ref.contacts.pair) >= 0
        ref.contacts.tangent_speed[...] = np.where(live, np.random.default_rng(2).uniform(-2, 2, live.shape), 0)
        st = ref
    rng = np.random.default_rng(29)
    acts = [b2.scenes.actions(rng, n) for _ in range(steps)] if variant != "tangent_speed" else None
    _run(m, st, s, dt, steps, oracle, acts)


@pytest.mark.parametrize("case", ["cage", "walk_restore"])
def test_toi_bookkeeping_parity(oracle, case):
    """The TOI scenes of the oracle pins on the device, 64 worlds with varied speeds: a ball between two walls (up to
    18 events a step, each wall's contact capped at 9 sub-steps, the moved ball's contacts searched again after each
    event) and a bullet passing a box it shares a contact with but never touches (the island walk advances and
    restores it)."""
    from test_oracle_pins import _ball_between_walls
    rng = np.random.default_rng(37)
    if case == "cage":
        s, m, st = _ball_between_walls(700.0)
        st = wd.batch(wd.from_leaves([np.asarray(x)[0] for x in wd.leaves(st)]), 64)
        st.bodies.v[:, 1, 0] = rng.uniform(150.0, 900.0, 64).astype(np.float32) * rng.choice([-1, 1], 64)
    else:
        s = b2.Settings.stock(gravity=(0.0, 0.0), continuous_physics=True, max_translation=100.0)
        d = wd.WorldDef(s)
        g = d.add_body(wd.STATIC, (0.0, 0.0))
        d.add_box(g, (0.05, 2.0), center=(4.0, 0.0))
        ball = d.add_body(wd.DYNAMIC, (0.0, 0.0), velocity=(300.0, 0.0), mass=1.0, inertia=1.0, bullet=True)
        d.add_circle(ball, 0.1)
        box = d.add_body(wd.DYNAMIC, (2.0, 0.25), velocity=(0.0, 1.0), mass=1.0, inertia=1.0)
        d.add_box(box, (0.5, 0.1))
        model, state = d.build(8)
        m = wd.compact_model(model, state)
        st = wd.batch(wd.compact_state(m, state), 64)
        st.bodies.v[:, 1, 0] = rng.uniform(200.0, 400.0, 64).astype(np.float32)
        st.bodies.v[:, 2, 1] = rng.uniform(-2.0, 2.0, 64).astype(np.float32)
    events = []
    _run(m, st, s, np.float32(1 / 60), 4, oracle, on_step=lambda k, r, d: events.append(int(r.toi.events.sum())))
    assert events[0] > (64 if case == "cage" else 32)
