# A deterministic one-on-one written for the tests: a forward against the keeper, with a seed of
# its own, a lazy defender and a team that starts the match from the right.
from . import *


def build_scenario(builder):
    config = builder.config()
    config.game_duration = 200
    config.deterministic = True
    config.game_engine_random_seed = 1234
    config.left_team_difficulty = 0.25
    config.right_team_difficulty = 0.8
    config.end_episode_on_score = True
    builder.SetBallPosition(0.7, -0.05)

    builder.SetTeam(Team.e_Left)
    builder.AddPlayer(-1.0, 0.0, e_PlayerRole_GK, controllable=False)
    builder.AddPlayer(0.68, -0.05, e_PlayerRole_CF)

    builder.SetTeam(Team.e_Right)
    builder.AddPlayer(-1.0, 0.0, e_PlayerRole_GK)
    builder.AddPlayer(-0.5, 0.3, e_PlayerRole_CB, lazy=True)
