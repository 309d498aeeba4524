// SPDX-License-Identifier: Apache-2.0
// Restates game logic of cuju (Copyright 2026 The cuju Authors), a reimplementation of Google
// Research Football (Copyright 2019 Google LLC); see NOTICE.
// The ball momentum and spin of a touch, by kind (ball control, trap, shot, pass), and the aiming
// of passes and shots. Semantics: include/cuju/simulation/touch.h:15-400 (results depend on the
// number and order of the RNG draws), include/cuju/simulation/ai_functions.h:27-190. The float
// operations and the draws are GRF's; the organisation (a difficulty record, a control intent, a
// kick toward a planned point, shot power, ease and scatter, pass receivers and biases) is this
// engine's own.
#pragma once

#include "control.h"
#include "select.h"

namespace eng {

// The velocity the player's controller asks for: the gamer's keyboard, or the AI's last command.
HD float ControllerFloatVelocity(World &w, int p) {
    if (ExternalControllerActive(w, p)) return HumanGetFloatVelocity(w, p);
    return w.match.players[p].controller.lastDesiredVelocity;
}

// A touch's momentum and spin.
struct Kick {
    Vec3 momentum;
    float xRot = 0, yRot = 0;
};

// How hard a touch is, from 0 to 1 in three respects: where the ball goes (distance), how high it
// pops up (height) and how much of its incoming momentum it keeps (ball movement).
struct TouchDifficulty {
    float distance = 0, height = 0, ballMovement = 0;
};
// Player p's touch difficulty: an off-balance body (position offset up to 10 cm), a velocity gap
// to the ball (10 to 50 m/s), a ball beyond the foot (0.7 to 1.3 m), an opponent's touch just
// before (recovered from faster with reaction); scaled by ball control and one draw in 0.5..1.
HDN TouchDifficulty TouchDifficultyOf(World &w, const Ctx &c, int p, const Vec3 &offset) {
    const Ball &b = w.match.ball;
    const SpatialState &s = Sp(w, p);
    const float offBalance = NormalizedClamp(offset.Length(), 0.0f, 0.1f) * 2.0f;
    const float speedGap = libm::powf(NormalizedClamp((s.movement - b.momentum).Length(), 10.0f, 50.0f), 1.5f) * 5.0f;
    const float reachGap = NormalizedClamp(((s.position + s.directionVec * 0.2f) - BallPredict(b, 0).Get2D()).Length(), 0.7f, 1.3f);
    const float beyondFoot = reachGap * reachGap * 2.0f;
    TouchDifficulty d;
    d.distance = offBalance * 2.0f + speedGap + beyondFoot * 4.0f;
    d.height = offBalance * 0.5f + speedGap * 2.0f + beyondFoot;
    const int teamID = w.playerTeamID[p];
    if (w.match.lastTouchTeamID != teamID) {
        const int opponent = TeamByID(w, 1 - teamID).lastTouchPlayer;
        if (opponent >= 0) {
            const int recovery = TruncToInt32(1000 - GetStatistic(w, c, p, kStatReaction) * 500);
            const float surprise = libm::powf(GetLastTouchBias(w, opponent, recovery), 0.6f) * 5.0f;
            d.distance += surprise;
            d.height += surprise;
            d.ballMovement = surprise * 0.1f;
        }
    }
    d.ballMovement = Clamp(d.ballMovement, 0.0f, 0.9f);
    const float skill = (1.0f - GetStatistic(w, c, p, kStatBallControl) * 0.5f) * RandomInRange(w, 0.5f, 1.0f);
    d.distance = Clamp(d.distance * skill, 0.0f, 1.0f);
    d.height = Clamp(d.height * skill, 0.0f, 1.0f);
    d.ballMovement = Clamp(d.ballMovement * skill, 0.0f, 1.0f);
    return d;
}

// ---- ball control and traps --------------------------------------------------------------------

// How the humanoid moves through a controlled touch: the physics share (0.7 with the ball, 0.9
// without, 1 for an animation that ends idle); its speed, the command's blended with the
// controller's (stretched to the player's top speed above the walk-sprint switch), held between
// the animation's outgoing speed and up to 0.6 m/s (walking) or 1.2 m/s (sprinting) above it as
// far as the humanoid faces the command's direction; and two movements at that speed, along the
// command's direction and straight ahead of the next start angle.
struct ControlIntent {
    float physicsBias = 0, speed = 0;
    Vec3 desired, ahead;
};
HD ControlIntent BallControlIntent(World &w, const Ctx &c, int p, const Humanoid &h, const Anim &a, const Vec3 &outMov) {
    const PlayerCommand &cmd = h.anim.originatingCommand;
    const SpatialState &s = h.spatial;
    const bool endsIdle = VelocityCat(a.outgoingVelocity) == kVelIdle;
    ControlIntent in;
    in.physicsBias = endsIdle ? 1.0f : w.match.players[p].hasPossession ? 0.7f : 0.9f;
    const float explosiveness = 0.6f;
    float overdrive = 1.0f * explosiveness;
    if (cmd.desiredVelocityFloat < kDribbleWalkSwitch) overdrive = 0.0f;
    if (cmd.desiredVelocityFloat > kWalkSprintSwitch) overdrive = 2.0f * explosiveness;
    const Vec3 straight = Vec3(0, -1, 0).Rotated2D(h.nextStartAngle.value());
    const float facing = s.directionVec.Dot(cmd.desiredDirection) * 0.5f + 0.5f;
    const float facingNext = straight.Dot(cmd.desiredDirection) * 0.5f + 0.5f;
    overdrive *= Clamp(MinF(facing, facingNext), 0.0f, 1.0f);
    if (endsIdle) overdrive = 0.0f;
    const float own = 0.7f;
    Vec3 move = cmd.desiredDirection * (cmd.desiredVelocityFloat * own + ControllerFloatVelocity(w, p) * (1.0f - own));
    if (move.Length() > kWalkSprintSwitch)
        move = move.Normalized(0) * StretchSprint(move.Length(), kSprintVelocity, GetMaximumVelocity(*c.sd, p));
    in.speed = Clamp(move.Length(), outMov.Length(), outMov.Length() + overdrive);
    in.desired = move.Normalized(straight) * in.speed;
    in.ahead = straight * in.speed;
    return in;
}

// Where the foot meets the ball, relative to the body: the reach at the speed ahead, pushed out by
// `extra` and by up to 3 m of annoyance (an opponent within 1.5 m of a fast animation, less with
// calm and balance), along the next body direction; shifted toward the reach offset and the body
// direction for a ball 0.5 to 1 m up.
HD Vec3 ControlFoot(World &w, const Ctx &c, int p, const Humanoid &h, const Anim &a, float nextBodyAngle, float aheadSpeed,
                    float extra) {
    const SpatialState &s = h.spatial;
    const float ballHeight = BallPredict(w.match.ball, 0).v[2];
    const Vec3 reach = FootReachOffset(aheadSpeed, nextBodyAngle - s.angle.value(), ballHeight);
    const float hurry = Curve(NormalizedClamp(a.outgoingVelocity, kIdleVelocity, kSprintVelocity), 0.7f);
    const float annoy = (1.0f - NormalizedClamp(ClosestOpponentDistance(w, p), 0.5f, 1.5f)) *
                        (1.0f - (GetStatistic(w, c, p, kStatCalmness) * 0.5f + GetStatistic(w, c, p, kStatBalance) * 0.3f)) * hurry;
    Vec3 foot = Vec3(0, -1, 0).Rotated2D(nextBodyAngle) * (reach.Length() + extra + annoy * 3.0f);
    const float lift = NormalizedClamp(ballHeight, 0.5f, 1.0f) * 0.5f;
    foot += reach * lift * 0.5f + s.bodyDirectionVec * lift * 0.5f;
    return foot;
}

// The spin of a controlled touch: about the axis between the foot and the touch's direction, a
// roll of 2 pi per m/s less up to 30 of backspin.
HD void SpinAgainstFoot(Kick &k, const Vec3 &foot) {
    const float backspin = 30.0f;
    const float speed = k.momentum.Length();
    const float damping = libm::powf(NormalizedClamp(k.momentum.Length(), 0.0f, 10.0f), 0.7f);
    const Vec3 axis = (foot.Normalized(0) * 0.6f + k.momentum.Normalized(0) * 0.4f).Normalized(0);
    k.xRot = axis.v[1] * ((2 * PI * speed) - (backspin * damping));
    k.yRot = axis.v[0] * ((2 * PI * speed) - (backspin * damping));
}

// A controlled touch of humanoid p: the ball goes toward a point ahead of the foot where the
// humanoid will be after a speed-dependent delay (0.25 to 0.85 s) on each of its two movements,
// blended by the physics share, in the time left in the animation plus that delay and the touch
// offset. Power is the distance over a dribble-scaled time, to the 0.7; the height grows with it;
// a fast player touches up to 20% harder, less with ball control.
HDN Kick BallControlKick(World &w, const Ctx &c, int p, const Humanoid &h, float nextBodyAngle, const Vec3 &outMov,
                         float extraFoot = 0.0f) {
    const AnimationState &cur = h.anim;
    const Anim &a = c.A(cur.anim);
    const ControlIntent in = BallControlIntent(w, c, p, h, a, outMov);
    const float desiredSpeed = in.desired.Length(), aheadSpeed = in.ahead.Length();
    const Vec3 foot = ControlFoot(w, c, p, h, a, nextBodyAngle, aheadSpeed, extraFoot);
    const float desiredFast = NormalizedClamp(desiredSpeed, 0.0f, kSprintVelocity);
    const float desiredDelay = desiredFast * desiredFast * 0.60f + 0.25f;
    const float aheadFast = NormalizedClamp(aheadSpeed, 0.0f, kSprintVelocity);
    const float aheadDelay = aheadFast * aheadFast * 0.60f + 0.25f;
    Vec3 viaDesired = h.nextStartPos, viaAhead = h.nextStartPos;
    viaDesired += in.desired * desiredDelay + foot;
    viaAhead += in.ahead * aheadDelay + foot;
    const Vec3 point = viaAhead * in.physicsBias + viaDesired * (1.0f - in.physicsBias);
    const Vec3 toPoint = point - BallPredict(w.match.ball, 0).Get2D();
    float timeLeft = (((a.frameCount - 1) - cur.frameNum) * 10) * 0.001f;
    timeLeft += aheadDelay * in.physicsBias + desiredDelay * (1.0f - in.physicsBias);
    timeLeft += kDefaultTouchOffsetMs * 0.001f;
    float divisor = timeLeft * (0.38f + 0.02f * GetStatistic(w, c, p, kStatDribble));
    divisor *= 1.1f;
    const float power = libm::powf((toPoint.Length() / divisor), 0.7f);
    const Vec3 direction = toPoint.Normalized(Vec3(0, -1, 0).Rotated2D(nextBodyAngle));
    const float height = Clamp(0.1f + 1.5f * libm::powf(power / 10.0f, 1.6f), 0.0f, 1.5f);
    const float fast = NormalizedClamp(in.speed, kWalkVelocity, kSprintVelocity - 0.8f);
    const float harder = 1.0f * (1.0f - fast) + (1.2f - (GetStatistic(w, c, p, kStatBallControl) * 0.03f)) * fast;
    Kick k;
    k.momentum = direction * power * harder + Vec3(0, 0, height);
    SpinAgainstFoot(k, foot);
    return k;
}

// A trap: a controlled touch with the foot pushed out by the touch's distance difficulty, lifted
// by its height difficulty (more for a falling ball) and keeping part of the ball's momentum.
HDN Kick TrapKick(World &w, const Ctx &c, int p, const Humanoid &h, float nextBodyAngle, const Vec3 &outMov) {
    const TouchDifficulty d = TouchDifficultyOf(w, c, p, h.decayingPositionOffset);
    Kick k = BallControlKick(w, c, p, h, nextBodyAngle, outMov, d.distance);
    const Vec3 incoming = w.match.ball.momentum;
    k.momentum.v[2] += incoming.v[2] * d.height * 1.0f + d.height * 4.0f;
    k.momentum = k.momentum * (1.0f - d.ballMovement) + incoming * d.ballMovement;
    return k;
}

// ---- shots -----------------------------------------------------------------------------------------

// The humanoid's movement at the touch frame, on the pitch, its direction (the facing when idle)
// and speed.
struct ShotTouch {
    Vec3 movement, direction;
    float speed = 0;
};
HD ShotTouch ShotTouchOf(const Ctx &c, const AnimationState &cur, const SpatialState &s) {
    const Anim &a = c.A(cur.anim);
    ShotTouch t;
    t.movement = MovementAtFrame(c.t->positions + a.posFirst, a.posCount, cur.frameNum, 0).Rotated2D(s.angle.value());
    t.direction = t.movement.Normalized(s.directionVec);
    t.speed = t.movement.Length();
    if (VelocityCat(t.speed) == kVelIdle) t.direction = s.directionVec;
    return t;
}
// How well the touch lines up with the shot: 1 when it runs 0.2 pi off the desired direction on
// either side, curving down to 0 a half turn from there.
HD float ShotAlignment(const ShotTouch &t, const Vec3 &desired) {
    const float ideal = 0.2f * PI;
    const float left = fabsf(t.direction.Angle2D(desired.Rotated2D(-ideal)));
    const float right = fabsf(t.direction.Angle2D(desired.Rotated2D(ideal)));
    const float off = (right < left) ? right : left;
    return Curve(1.0f - Clamp(off / PI, 0.0f, 1.0f), 0.8f);
}
// The shot's strength: the desired power (45 m/s at full, to the 0.5) cut by a misaligned touch, a
// slow approach and an off-balance body; capped by shot power and the animation's touch power;
// raised by up to 20% by the gap to the ball's momentum (`ballGap`, 0 to 1 over 10 m/s).
HD float ShotPower(World &w, const Ctx &c, int p, const ShotTouch &t, float fromLine, float fromBalance, const AnimDerived &d,
                   float desiredPower, const Vec3 &ballMomentum, float &ballGap) {
    const float fromSpeed = libm::powf(NormalizedClamp(t.speed, 0.0f, kSprintVelocity), 0.3f);
    const float share =
        Clamp(1.0f * (0.7f + fromLine * 0.3f) * (0.7f + fromSpeed * 0.3f) * (0.4f + fromBalance * 0.6f), 0.0f, 1.0f);
    const float asked = 45.0f * (0.7f + libm::powf(desiredPower, 0.5f) * 0.3f);
    float animationMax = d.touchMaxPowerFactor;
    if (animationMax == 0.0f) animationMax = 1.0f;
    float power = Clamp(share * asked, 0.0f, (32.0f + GetStatistic(w, c, p, kStatShotPower) * 13.0f) * (0.2f + animationMax * 0.8f));
    ballGap = NormalizedClamp((t.movement - ballMomentum).Length(), 0.0f, 10.0f);
    power *= 1.0f + ballGap * 0.2f;
    return power;
}
// The shot's difficulty, 1 less its ease: a product of the alignment, a touch near dribble speed,
// the body's balance, a small gap to the ball's momentum (volleys are easier with the volley
// statistic) and a moderate power (30 to 100 m/s).
HD float ShotDifficulty(World &w, const Ctx &c, int p, const ShotTouch &t, float fromLine, float fromBalance, float ballGap,
                        float power) {
    const float nearDribble = 1.0f - NormalizedClamp(fabsf(t.speed - kDribbleVelocity), 0.0f, 4.0f);
    const float steadyBall = 1.0f - ballGap * (0.5f - GetStatistic(w, c, p, kStatVolley) * 0.3f);
    const float moderate = Curve(1.0f - NormalizedClamp(power, 30.0f, 100.0f), 1.0f);
    const float ease = 1.0f * (0.4f + fromLine * 0.6f) * (0.7f + nearDribble * 0.3f) * (0.3f + fromBalance * 0.7f) *
                       (0.6f + steadyBall * 0.4f) * (0.6f + moderate * 0.4f);
    return Clamp(1.0f - ease, 0.0f, 1.0f);
}
// The shot between the desired one (lifted 0.05) and a worst one: the touch's direction mixed in
// by the difficulty, scattered by three draws (z, y, x: GRF evaluates the arguments right to
// left), lifted and weakened with the difficulty. One more draw, to the power of 0.7 times the
// shot statistic, is how far toward the worst the shot goes (`worstShare`).
HD Vec3 ScatterShot(World &w, const Ctx &c, int p, const ShotTouch &t, const Vec3 &desired, float power, float difficulty,
                    float &worstShare) {
    const Vec3 desiredShot = (desired.Get2D() + Vec3(0, 0, 0.05f)).Normalized() * power;
    const float lag = difficulty * 0.8f;
    Vec3 worst = (t.direction * lag + desired.Get2D() * (1.0f - lag)).Normalized(0);
    const float rz = RandomInRange(w, -1, 1);
    const float ry = RandomInRange(w, -1, 1);
    const float rx = RandomInRange(w, -1, 1);
    worst = worst + (Vec3(rx, ry, rz) * 0.5f * difficulty);
    worst.Normalize();
    const float worstLift = Curve(libm::powf(difficulty, 0.7f), 0.7f) * 0.7f;
    const float worstPower = power * (1.0f - libm::powf(difficulty, 0.7f) * 0.5f);
    const Vec3 worstShot = (worst + Vec3(0, 0, worstLift)).Normalized() * worstPower;
    worstShare = libm::powf(RandomInRange(w, 0.0f, 1.0f), GetStatistic(w, c, p, kStatShot) * 0.7f);
    return desiredShot * (1.0f - worstShare) + worstShot * worstShare;
}
// How far a kick curls away from the body direction: the angle between them in half turns,
// folded so that a kick behind the body counts from the back, doubled, a quarter of that.
HD float CurlAmount(const Vec3 &body, const Vec3 &kick) {
    float across = body.Angle2D(kick) / PI;
    if (fabsf(across) > 0.5f) across = (1.0f - fabsf(across)) * SignSide(across);
    across *= 2.0f;
    return across * 0.25f;
}
// Turns a kick by its curl, more for a harder kick (to 70 m/s).
HD void CurlKick(Vec3 &kick, float amount) { kick.Rotate2D(amount * (0.4f + 0.6f * NormalizedClamp(kick.Length(), 0.0f, 70.0f))); }

// A shot's momentum and spin (x and y against the desired direction, z with the curl), with a
// draw each, the x and y draws scaled up the nearer the shot comes to the worst one.
HDN Vec3 ShotKick(World &w, const Ctx &c, int p, const AnimationState &cur, const SpatialState &s, const Vec3 &offset,
                  float &xRot, float &yRot, float &zRot) {
    const PlayerCommand &cmd = cur.originatingCommand;
    const Vec3 desired = cmd.touchInfo.desiredDirection;
    const ShotTouch t = ShotTouchOf(c, cur, s);
    const float fromLine = libm::powf(ShotAlignment(t, desired), 0.8f);
    const float fromBalance = 1.0f - NormalizedClamp(offset.Length(), 0.0f, 0.1f);
    float ballGap = 0;
    const float power = ShotPower(w, c, p, t, fromLine, fromBalance, c.D(cur.anim), cmd.touchInfo.desiredPower,
                                  w.match.ball.momentum, ballGap);
    const float difficulty = ShotDifficulty(w, c, p, t, fromLine, fromBalance, ballGap, power);
    float worstShare = 0;
    Vec3 shot = ScatterShot(w, c, p, t, desired, power, difficulty, worstShare);
    const float spinScatter = 0.3f + worstShare * 0.7f, curlScatter = 0.7f;
    xRot = -desired.v[1] * 20.0f + (RandomInRange(w, -20, 20) * spinScatter);
    yRot = -desired.v[0] * 20.0f + (RandomInRange(w, -20, 20) * spinScatter);
    const float amount = CurlAmount(s.bodyDirectionVec, shot);
    CurlKick(shot, amount);
    zRot = amount * -420 + (RandomInRange(w, -20, 20) * curlScatter);
    return shot;
}

// ---- passes ------------------------------------------------------------------------------------

// A desired pass momentum within the animation's power: 30 m/s (42 for high passes) scaled by the
// animation's touch power and cut by up to a quarter for an off-balance body, plus half the
// ball's speed; the excess (up to 10 m/s) lifts the ball by a quarter of it.
HD Vec3 CapTouchPower(Vec3 r, int fn, const AnimDerived &d, const Vec3 &offset, const Vec3 &incoming) {
    float animation = d.touchMaxPowerFactor;
    if (animation == 0.0f) animation = 1.0f;
    animation = animation * 0.7f + 0.3f;
    float most = (fn == kFnHighPass ? 42.0f : 30.0f) * animation * (1.0f - Clamp(offset.Length() * 2.5f, 0.0f, 0.25f));
    most += incoming.Length() * 0.5f;
    if (r.Length() > most) {
        const float excess = r.Length() - most;
        r = r.Normalized(0) * most;
        r.v[2] += Clamp(excess, 0.0f, 10.0f) * 0.25f;
    }
    return r;
}
// The touch a player manages for a desired pass momentum: within the animation's power, turned
// toward the animation's own ball direction by the touch's difficulty (without one, by a draw of
// up to a quarter turn either way), weakened and lifted by it, keeping some of the ball's
// momentum, and lifted by one more draw scaled by the pass's own difficulty (less with the pass
// statistics).
HDN Vec3 AttainableTouch(World &w, const Ctx &c, int p, const Vec3 &desired, int fn) {
    Humanoid &h = Hum(w, p);
    const AnimationState &cur = h.anim;
    const AnimDerived &d = c.D(cur.anim);
    const Vec3 incoming = w.match.ball.momentum;
    Vec3 r = CapTouchPower(desired, fn, d, h.decayingPositionOffset, incoming);
    float passDifficulty = d.touchDifficultyFactor;
    if (fn == kFnShortPass || fn == kFnLongPass) passDifficulty *= (1.0f - GetStatistic(w, c, p, kStatShortPass) * 0.5f);
    if (fn == kFnHighPass) passDifficulty *= (1.0f - GetStatistic(w, c, p, kStatHighPass) * 0.5f);
    const TouchDifficulty td = TouchDifficultyOf(w, c, p, h.decayingPositionOffset);
    const float wobble = td.distance * 0.15f + td.height * 0.15f + td.ballMovement * 0.3f + passDifficulty * 0.5f;
    const Vec3 own = d.ballDirection.Rotated2D(h.startAngle.value() + cur.rotationSmuggleOffset.value());
    if (own.Length() > 0.01f) {
        const float bias = Clamp(wobble * 1.5f, 0.0f, 1.0f);
        const Vec3 native = own.Normalized(r).Get2D() * r.Length() + r * Vec3(0, 0, 1);
        r = r * (1.0f - bias) + native * bias;
    } else {
        r.Rotate2D(RandomInRange(w, -0.5f * PI, 0.5f * PI) * MinF(wobble, 0.5f));
    }
    r *= 1.0f - td.distance * 0.3f;
    r.v[2] += td.distance * 1.5f;
    r.v[2] += incoming.v[2] * td.height * 0.5f + td.height * 1.0f;
    r = r * (1.0f - td.ballMovement) + incoming * td.ballMovement;
    r.v[2] += passDifficulty * 5.0f * RandomInRange(w, 0.2f, 1.0f);
    return r;
}

// The direction and power of a pass along `v`: lifted 0.11 (a high pass 0.45, less up to 0.15 with
// distance); power the distance over 60 m to the 1.4, times 1.8 (1.15 for a high pass).
HDN void PassForVector(int passType, const Vec3 &v, Vec3 &dir, float &power) {
    const bool high = passType == kFnHighPass;
    const float lift = high ? 0.45f - NormalizedClamp(v.Length(), 0.0f, 60.0f) * 0.15f : 0.11f;
    dir = (v.Normalized(0) + Vec3(0, 0, lift)).Normalized(0);
    power = libm::powf(NormalizedClamp(v.Length(), 0.0f, 60.0f), 1.4f) * (high ? 1.15f : 1.8f);
}

// Where a pass leaves from: the touch position during a touch, else 20 cm ahead along the movement.
HD Vec3 PassOrigin(const World &w, int p) {
    const SpatialState &s = Sp(w, p);
    const AnimationState &cur = Hum(w, p).anim;
    if (cur.touchFrame != -1) return cur.touchPos.Get2D();
    return s.position + s.movement.Normalized(0) * 0.2f;
}
// Where a teammate will be when a pass from `origin` arrives: ahead along its movement by 0.3 s
// plus 0.05 s per metre (at most 1 s), to the 0.7, times 0.7.
HD Vec3 LeadPoint(const SpatialState &mate, const Vec3 &origin) {
    float lead = 0.3f + (mate.position - origin).Length() * 0.05f;
    lead = libm::powf(Clamp(lead, 0.0f, 1.0f), 0.7f) * 0.7f;
    return mate.position + mate.movement * lead;
}
// The teammate a pass toward `manual` (input direction `inDir`) goes to, and where: the lowest
// rating of distance from the manual target (over 70 m, to the 0.8, times 0.8) plus angle off the
// input direction (in half turns); the passer, at the origin, without teammates.
HD int PassReceiver(const World &w, int p, const PlayerList &players, const Vec3 &origin, const Vec3 &manual, const Vec3 &inDir,
                    Vec3 &aim) {
    int best = p;
    float bestRating = 10000;
    aim = origin;
    for (int mate : players) {
        if (mate == p) continue;
        const Vec3 lead = LeadPoint(Sp(w, mate), origin);
        const float fromManual = libm::powf(NormalizedClamp((lead - manual).Length(), 0.0f, 70.0f), 0.8f) * 0.8f;
        const float offInput = fabsf((lead - origin).Normalized(0).Angle2D(inDir) / (1.0f * PI)) * 1.0f;
        if (fromManual + offInput < bestRating) {
            bestRating = fromManual + offInput;
            best = mate;
            aim = lead;
        }
    }
    return best;
}
// A pass's direction, power and receiver. The receiver is the forced one or the best-rated
// teammate; the pass blends the manual target (the input direction, 60 m per unit of input power,
// 1 to 100 m) with the receiver's lead point, by direction and by distance, with the auto biases
// cut as the two targets part (to 50 m) and, for direction, raised toward 1 near the receiver
// (within 12 m). A forced receiver or a gamer-controlled passer passes fully automatically; a
// player without teammates fully manually. Long passes aim 20% of their length further upfield.
HDN void AimPass(const World &w, int p, int passType, const Vec3 &inDir, float inPower, float autoDirBias, float autoPowerBias,
                 Vec3 &outDir, float &outPower, int &target, int forcedTarget = -1) {
    const int teamID = w.playerTeamID[p];
    const Vec3 origin = PassOrigin(w, p);
    const Vec3 manual = origin + inDir * Clamp(inPower * 60.0f, 1.0f, 100.0f);
    const PlayerList players = TeamActivePlayers(w, teamID);
    const bool alone = players.size() < 2;
    const bool automatic = ExternalControllerActive(w, p) && !alone;
    float dirBias = alone ? 0.0f : autoDirBias, powerBias = alone ? 0.0f : autoPowerBias;
    Vec3 aim;
    if (forcedTarget >= 0) {
        target = forcedTarget;
        aim = LeadPoint(Sp(w, forcedTarget), origin);
    } else {
        target = PassReceiver(w, p, players, origin, manual, inDir, aim);
    }
    Vec3 autoRel = aim - origin, manualRel = manual - origin;
    if (forcedTarget >= 0 || automatic) {
        dirBias = 1.0f;
        powerBias = 1.0f;
    } else {
        // The subtraction from 1 runs in double and rounds once.
        const float agreement = (float)(1.0 - (double)libm::powf(Clamp((autoRel - manualRel).Length() / 50.0f, 0.0f, 1.0f), 1.5f));
        const float near = libm::powf(1.0f - NormalizedClamp((origin - aim).Length(), 0.0f, 12.0f), 0.5f);
        dirBias *= agreement;
        dirBias = libm::powf(dirBias, 1.0f - near * 0.9f);
        powerBias *= agreement;
        powerBias = Clamp((float)((double)powerBias * (1.0 + (double)near)), 0.0f, 1.0f);
    }
    if (passType == kFnLongPass) {
        const float length = autoRel.Length() * dirBias + manualRel.Length() * (1.0f - dirBias);
        const Vec3 upfield = Vec3(-TeamDynamicSide(w, teamID) * length * 0.2f, 0, 0);
        autoRel += upfield;
        manualRel += upfield;
    }
    Vec3 pass = (autoRel.Normalized(0) * dirBias + manualRel.Normalized(0) * (1.0f - dirBias)).Normalized(manual);
    pass *= float(autoRel.Length() * powerBias + manualRel.Length() * (1.0f - powerBias));
    PassForVector(passType, pass, outDir, outPower);
}

// A shot's direction: the input direction blended by the auto bias with a direction at the goal,
// aimed across its mouth (up to 90% of its half width) as far as the input points away from the
// goal's centre (a quarter turn reaches the post; the offset to the 0.7).
HDN Vec3 AimShot(const World &w, int p, const Vec3 &inDir, float autoDirBias) {
    const SpatialState &s = Sp(w, p);
    const int side = TeamDynamicSide(w, w.playerTeamID[p]);
    const Vec3 from = s.position + s.movement * 0.12f;
    Vec3 goal = Vec3(side * -kPitchHalfLength, 0, 0);
    float across = Clamp(((goal - from).Normalized(0).Angle2D(inDir) / PI) / 0.5f, -1.0f, 1.0f);
    across = libm::powf(fabsf(across), 0.7f) * SignSide(across);
    goal.v[1] = across * kGoalHalfWidth * 0.9f * side;
    return (inDir * (1.0f - autoDirBias) + (goal - from).Normalized(0) * autoDirBias).Normalized(inDir);
}

}  // namespace eng
