# A finishing drill written for the tests: three attackers against a defender and a keeper, the
# ball 25 m from goal (x = (55 - 25) / 54.4), its side switching with the episode's parity.
from . import *


def build_scenario(builder):
    config = builder.config()
    config.game_duration = 400
    config.deterministic = False
    config.offsides = False
    config.end_episode_on_score = True
    config.end_episode_on_out_of_play = True
    config.end_episode_on_possession_change = True
    side = 1 if builder.EpisodeNumber() % 2 == 0 else -1
    builder.SetBallPosition(0.55, 0.12 * side)

    builder.SetTeam(Team.e_Left)
    builder.AddPlayer(-1.0, 0.0, e_PlayerRole_GK)
    builder.AddPlayer(0.53, 0.12 * side, e_PlayerRole_CF)
    builder.AddPlayer(0.45, -0.2 * side, e_PlayerRole_LM)
    builder.AddPlayer(0.4, 0.3 * side, e_PlayerRole_RM)

    builder.SetTeam(Team.e_Right)
    builder.AddPlayer(-1.0, 0.0, e_PlayerRole_GK)
    builder.AddPlayer(-0.8, 0.05, e_PlayerRole_CB)
